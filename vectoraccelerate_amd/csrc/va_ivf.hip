// va_ivf.hip — IVF-Flat (L2^2) build, coarse probe and list-major scan.
//
// Build (IVFStructure.assignToCluster / prepareGPUStructure, Index/Internal/IVFStructure.swift:
// 280-307, 347-467): nearest-centroid assignment on the fp32 MFMA distance kernel (k = 1,
// ties to the lower centroid id), CSR offsets and row ids built on the host in centroid order
// with insertion order inside each list (as the reference does), and the list vectors gathered
// into CSR order by a device copy kernel (the reference memcpy-gathers on the host).
//
// Search (IVFSearchPipeline.search, Index/Kernels/IVF/IVFSearchPipeline.swift:197-568), queued
// without any host read-back:
//   probe : the nprobe nearest centroids by (L2^2, id) through the exact top-k scan;
//   plan  : on the device, from the probes: the queries probing each list and, per tile shape,
//           the prefix of the lists' tile counts (the scan kernels decode their tiles from it);
//   scan  : list-major — every (list, block of the queries that probe it, block of its rows)
//           is one MFMA tile of the distance kernel, so a list's rows are read once per block
//           of up to 128 probing queries instead of once per query (ivf_list_search,
//           Metal/Shaders/IVFListSearch.metal:199-339, streams each query's lists separately);
//           persistent launches, one per tile shape;
//   top-k : a prefix sample of each probed list gives each query an upper bound tau_q of its
//           k-th distance; the full scan appends only keys <= tau_q; exact (L2^2, row id)
//           selection follows.  Queries whose candidate list overflows are finished by the
//           device fallback over their probed lists, with each list's own arithmetic.
// The reference's per-thread heap (K_PRIVATE = 8) is only exact for k <= 8; this is exact
// for every k <= VA_MAX_K.
#include <algorithm>
#include <vector>

#include "va_fallback.hpp"
#include "va_internal.hpp"
#include "va_screen_bound.hpp"

struct va_ivf {
    int device = 0;
    uint32_t C = 0, D = 0, N = 0;
    float* centroids = nullptr;     // [C x D]
    float* list_vectors = nullptr;  // [N x D] in CSR order
    uint32_t* ids = nullptr;        // [N] original row id of every CSR position
    uint32_t* offsets = nullptr;    // [C + 1]
    // fp16 shadow of list_vectors (rows of va::shadow_pitch(D) halves) and per row {|x|^2, an
    // upper bound of |fp16(x) - x|}, for the screened list scan; nullptr when D % 4 != 0 or the
    // allocation failed
    _Float16* shadow = nullptr;
    float2* norms = nullptr;
    std::vector<uint32_t> h_offsets;
    // host bounds of a search (from the list sizes, so a search reads nothing back): top_rows[p]
    // = rows of the p longest lists, top_sample[p] = their threshold-sample rows, max_len =
    // the longest list
    std::vector<uint64_t> top_rows, top_sample;
    uint32_t max_len = 0;
    uint64_t id_end = 0;  // one past the largest row id (ids of added rows are the caller's)
    uint32_t* probe_buf = nullptr;  // probes of va_ivf_search
    size_t probe_cap = 0;
    void refresh_bounds() {
        std::vector<uint32_t> len(C);
        for (uint32_t l = 0; l < C; ++l) len[l] = h_offsets[l + 1] - h_offsets[l];
        std::sort(len.begin(), len.end(), [](uint32_t a, uint32_t b) { return a > b; });
        top_rows.assign(C + 1, 0);
        top_sample.assign(C + 1, 0);
        for (uint32_t i = 0; i < C; ++i) {
            top_rows[i + 1] = top_rows[i] + len[i];
            top_sample[i + 1] = top_sample[i] + va::ivf_sample_rows(len[i]);
        }
        max_len = C ? len[0] : 0;
    }
};

namespace va {
namespace {

// va_ivf_add: old CSR position p of list c moves to p + pre[c] (the new rows of earlier lists
// come before it)
__global__ __launch_bounds__(256) void ivf_merge_old(const float* __restrict__ vecs, const uint32_t* __restrict__ ids,
                                                     const uint32_t* __restrict__ off, const uint32_t* __restrict__ pre,
                                                     uint32_t C, uint32_t N, uint32_t D, float* __restrict__ out_vecs,
                                                     uint32_t* __restrict__ out_ids) {
    for (uint32_t p = blockIdx.x; p < N; p += gridDim.x) {
        uint32_t lo = 0, hi = C - 1;  // list of p: the last c with off[c] <= p
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) >> 1;
            if (off[mid] <= p) lo = mid;
            else hi = mid - 1;
        }
        const uint32_t dst = p + pre[lo];
        for (uint32_t d = threadIdx.x; d < D; d += 256) out_vecs[uint64_t(dst) * D + d] = vecs[uint64_t(p) * D + d];
        if (threadIdx.x == 0) out_ids[dst] = ids[p];
    }
}

// new row at grouped position s of list c goes after list c's old rows: off[c + 1] + s
__global__ __launch_bounds__(256) void ivf_place_new(const float* __restrict__ x, const uint32_t* __restrict__ order,
                                                     const uint32_t* __restrict__ pre,
                                                     const uint32_t* __restrict__ off, uint32_t C, uint32_t n,
                                                     uint32_t D, uint32_t first_id, float* __restrict__ out_vecs,
                                                     uint32_t* __restrict__ out_ids) {
    for (uint32_t s = blockIdx.x; s < n; s += gridDim.x) {
        uint32_t lo = 0, hi = C - 1;  // the last c with pre[c] <= s
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) >> 1;
            if (pre[mid] <= s) lo = mid;
            else hi = mid - 1;
        }
        const uint32_t dst = off[lo + 1] + s, r = order[s];
        for (uint32_t d = threadIdx.x; d < D; d += 256) out_vecs[uint64_t(dst) * D + d] = x[uint64_t(r) * D + d];
        if (threadIdx.x == 0) out_ids[dst] = first_id + r;
    }
}

__global__ __launch_bounds__(256) void ivf_new_offsets(const uint32_t* __restrict__ off, const uint32_t* __restrict__ pre,
                                                       uint32_t C, uint32_t* __restrict__ out) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c <= C) out[c] = off[c] + pre[c];
}

__global__ __launch_bounds__(256) void gather_rows(const float* __restrict__ x, const uint32_t* __restrict__ ids,
                                                   uint32_t N, uint32_t D, float* __restrict__ out) {
    for (uint32_t p = blockIdx.x; p < N; p += gridDim.x) {
        const float* src = x + uint64_t(ids[p]) * D;
        float* dst = out + uint64_t(p) * D;
        if ((D & 3) == 0) {
            for (uint32_t d = threadIdx.x * 4; d < D; d += 1024)
                *reinterpret_cast<float4*>(dst + d) = *reinterpret_cast<const float4*>(src + d);
        } else {
            for (uint32_t d = threadIdx.x; d < D; d += 256) dst[d] = src[d];
        }
    }
}

// The fp16 shadow of n list rows for the screened scan.  None (both nullptr) when D % 4 != 0
// or memory is short: the index then searches with the fp32 list scan alone.
va_status make_list_shadow(va_context* ctx, const float* vecs, uint32_t n, uint32_t D, _Float16** sh, float2** nr) {
    *sh = nullptr;
    *nr = nullptr;
    if (D % 4 != 0 || n == 0) return VA_OK;
    void* a = nullptr;
    void* b = nullptr;
    if (hipMalloc(&a, uint64_t(n) * shadow_pitch(D) * 2) != hipSuccess ||
        hipMalloc(&b, uint64_t(n) * 8) != hipSuccess) {
        (void)hipGetLastError();
        if (a) (void)hipFree(a);
        return VA_OK;
    }
    *sh = static_cast<_Float16*>(a);
    *nr = static_cast<float2*>(b);
    return build_shadow(ctx, vecs, n, D, *sh, nullptr, *nr);
}

struct F32Keys final : KeyProducer {
    va_context* ctx;
    const float* q;
    const float* x;
    uint32_t Q, N, D;
    va_status fallback_pass(const FbArgs& a, int pass) override {
        return fb_launch_pass(ctx, FbF32{q, int64_t(D), x, int64_t(D), N, D, int(OP_L2SQ)}, a, pass);
    }
    va_status dense(const uint32_t* qrow, uint32_t q0, uint32_t nq, uint32_t c0, uint32_t cols, uint32_t stride,
                    uint32_t* out_k, int64_t ldo) override {
        DistArgs a;
        a.q = qrow ? q : q + int64_t(q0) * D;
        a.qrow = qrow;
        a.q_rows = Q;
        a.ldq = D;
        a.x = x + int64_t(c0) * D;
        a.ldx = int64_t(stride) * D;
        a.Q = nq;
        a.N = cols;
        a.D = D;
        a.op = OP_L2SQ;
        a.out = OUT_KEYS;
        a.out_k = out_k;
        a.ldo = ldo;
        return launch_dist(ctx, a);
    }
    va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) override {
        DistArgs a;
        a.q = q;
        a.ldq = D;
        a.x = x;
        a.ldx = D;
        a.Q = Q;
        a.N = N;
        a.D = D;
        a.op = OP_L2SQ;
        a.out = OUT_FILTER;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        return launch_dist(ctx, a);
    }
};

// ---------------------------------------------------------------------------------------
// Lists probed by few queries: 16-query tiles
// ---------------------------------------------------------------------------------------
// Most probed lists of an IVF search are probed by a handful of queries (configs[4]: 2,000 of
// 2,550 lists by at most 16), so a 32-query MFMA tile of the distance kernel is mostly
// padding there, and such a list's rows are read once per search anyway: the scan of these
// lists is bound by streaming their rows from HBM, not by the MFMA.  This kernel covers a
// tile of 16 queries x 128 rows per wave with v_mfma_f32_16x16x4f32 (8 blocks of 16 rows),
// loads both operands straight from global memory into registers (no LDS staging, no
// barrier: the four waves of a workgroup are independent tiles), and prefetches the next
// 16-float k-chunk while the current one runs.  K mapping: in k-chunk c, lane l (query or
// row l % 16, group g = l / 16) holds elements 16c + 4g .. 16c + 4g + 3 of its row as one
// 16-byte load, and MFMA e of the chunk takes element e of it from both operands, so the four
// lanes of a row read 64 contiguous bytes.  Squared norms accumulate on the VALU from the same
// registers.  Filter epilogue as in the distance kernel (L2^2 keys, key <= tau).  Keys differ
// in rounding from the 32-query kernel's, so a list takes the same kernel in every pass of a
// search (its probing-query count decides).
namespace ivfs {
constexpr uint32_t TQ = 16, TN = 128, WAVES = 4;
}
typedef float f32x4s __attribute__((ext_vector_type(4)));

// One wave's tile: queries qrow[qs + i] (i < qc) x row positions rs + r (r < rc).
__device__ __forceinline__ void small_tile(const DistArgs& a, float (*xnorm)[ivfs::TN], int wave, uint32_t qs,
                                           uint32_t qc, uint32_t rs, uint32_t rc) {
    using namespace ivfs;
    const int lane = threadIdx.x & 63;
    const int j = lane & 15, g = lane >> 4;
    const uint32_t D = a.D;
    // this lane's query row (zeros past the tile's queries)
    const bool qv = uint32_t(j) < qc;
    const uint32_t qi = qv ? a.qrow[qs + j] : 0u;
    const float* qp = a.q + int64_t(qi) * a.ldq;
    // the tile's rows through a buffer descriptor: rows past rc read as zeros
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a.x + int64_t(rs) * a.ldx), 0, int(uint32_t(rc) * uint32_t(a.ldx) * 4u), 0x00020000);
    const uint32_t rowoff = uint32_t(j) * uint32_t(a.ldx) * 4u;  // byte offset of row j
    const uint32_t blkoff = 16u * uint32_t(a.ldx) * 4u;          // 16 rows further
    const uint32_t nch = (D + 31) / 32 * 2;  // even; chunks past D load zeros
    f32x4s qa, qb, ra[8], rb[8];
    // Branch-free loads (the compiler's wait counts stay exact, so chunk c+1 stays in flight
    // while chunk c computes): past D or the tile's queries a load reads a valid address and
    // is zeroed, past the tile's rows the descriptor returns zeros.
    auto load = [&](uint32_t c, f32x4s& qv4, f32x4s(&rv)[8]) {
        const uint32_t k = 16 * c + 4 * uint32_t(g);
        const bool kin = k < D;  // D % 4 == 0: a 4-element group is whole or absent
        const f32x4s t = *reinterpret_cast<const f32x4s*>(qp + (kin ? k : 0u));
        const bool use = qv && kin;
        qv4 = f32x4s{use ? t[0] : 0.f, use ? t[1] : 0.f, use ? t[2] : 0.f, use ? t[3] : 0.f};
        const uint32_t vo = kin ? rowoff + 4 * k : 0x80000000u;
#pragma unroll
        for (int b = 0; b < 8; ++b)
            rv[b] = __builtin_bit_cast(f32x4s, __builtin_amdgcn_raw_buffer_load_b128(
                                                   xr, kin ? vo + uint32_t(b) * blkoff : vo, 0, 0));
    };
    f32x4s acc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] = f32x4s{0.f, 0.f, 0.f, 0.f};
    float xs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, qsum = 0.f;
    auto compute = [&](const f32x4s& qv4, const f32x4s(&rv)[8]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            qsum = fmaf(qv4[e], qv4[e], qsum);
#pragma unroll
            for (int b = 0; b < 8; ++b) xs[b] = fmaf(rv[b][e], rv[b][e], xs[b]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int b = 0; b < 8; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(rv[b][e], qv4[e], acc[b], 0, 0, 0);
    };
    // two register sets: the loads of chunk c+1 are in flight while chunk c computes (the
    // scheduling barriers keep the compiler from hoisting a third set's loads)
    load(0, qa, ra);
    for (uint32_t c = 0; c < nch; c += 2) {
        load(c + 1, qb, rb);
        compute(qa, ra);
        __builtin_amdgcn_sched_barrier(0);
        load(c + 2, qa, ra);  // past the end: zeros, unused
        compute(qb, rb);
        __builtin_amdgcn_sched_barrier(0);
    }
    // norms: the four k groups of a row or query hold partial sums
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        xs[b] += __shfl_xor(xs[b], 16);
        xs[b] += __shfl_xor(xs[b], 32);
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
    if (g == 0) {
#pragma unroll
        for (int b = 0; b < 8; ++b) xnorm[wave][16 * b + j] = xs[b];
    }
    // (one wave writes and reads its own LDS row: in order, no barrier)
    if (!qv) return;
    // lane (j, g) holds query j's dots with rows 16b + 4g + v, v < 4; two halves of four
    // blocks keep the epilogue's registers within the main loop's
    const uint32_t thr = a.thr[qi];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t keys[16];
        uint32_t pass = 0;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const int b = 4 * h + bb;
            const f32x4s xx = *reinterpret_cast<const f32x4s*>(&xnorm[wave][16 * b + 4 * g]);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float d = qsum + xx[v] - 2.0f * acc[b][v];  // L2^2; cancellation can leave a tiny negative
                d = (d < 0.0f) ? 0.0f : d;
                const uint32_t key = key_of_float(d);
                keys[4 * bb + v] = key;
                const bool p = (uint32_t(16 * b + 4 * g + v) < rc) & (key <= thr);
                pass |= uint32_t(p) << (4 * bb + v);
            }
        }
        if (!pass) continue;
        uint32_t pos = atomicAdd(a.cnt + qi, uint32_t(__popc(pass)));
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            if (!((pass >> t) & 1)) continue;
            if (pos < a.cap) {
                const uint32_t r = rs + uint32_t(16 * (4 * h + (t >> 2)) + 4 * g + (t & 3));
                const int64_t o = int64_t(qi) * a.cap + pos;
                a.cand_key[o] = keys[t];
                a.cand_id[o] = a.ids ? a.ids[r] : a.id_base + r;
            }
            ++pos;
        }
    }
}

// A planned launch (a.plan): every wave loops over the plan's tiles on its own (the waves are
// independent tiles, no barrier).
__global__ __launch_bounds__(256) void ivf_small_kernel(DistArgs a) {
    using namespace ivfs;
    __shared__ __attribute__((aligned(16))) float xnorm[WAVES][TN];
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const uint32_t total = a.plan.pre[a.plan.C];
    for (uint32_t t = blockIdx.x * WAVES + uint32_t(wave); t < total; t += gridDim.x * WAVES) {
        uint32_t qs, qc, rs, rc;
        plan_tile(a.plan, t, TQ, TN, qs, qc, rs, rc);
        small_tile(a, xnorm, wave, qs, qc, rs, rc);
    }
}

// ---------------------------------------------------------------------------------------
// The screened list scan: fp16 shadow rows on the fp16 MFMA
// ---------------------------------------------------------------------------------------
// The rows stream from the index's fp16 shadow (half the bytes of the fp32 rows) and every pair
// is screened with the flat screen's proven bound (va_screen_bound.hpp): a pair becomes a
// candidate when the lower end of the interval that contains its fp32 key can be <= tau_q (the
// linear pre-test on the scaled fp16 dot).  The exact keys of the few rows that can reach the
// top-k are then recomputed with the arithmetic of the kernel that scans the list in the fp32
// list scan, so the result is the fp32 list scan's, bit for bit.
//
// One wave per tile (no LDS staging, no barrier), persistent over the device plan:
//   narrow : 16 queries x 128 rows, v_mfma_f32_16x16x32_f16 (lists probed by <= 16 queries);
//   wide<W>: 32W queries x 128 rows, v_mfma_f32_32x32x16_f16 (W = 1: 17-32 queries, 2: more).
// Both operands load straight into registers.  A dot is the same sum whatever the order of its
// terms (the bound does not depend on it), so the k order inside a 64-value chunk follows the
// loads: a narrow lane loads 32 and a wide lane 64 contiguous bytes of its row or query, and
// the two lanes that meet in an MFMA hold the same k indices.  The pre-test's constants come
// from the query's threshold; the appended (dot, |x|^2, position) triples become intervals in
// screen_list_bounds.
namespace iv16 {
constexpr uint32_t TN = 128, WAVES = 4;
constexpr int kGroupsUsed = 3;  // narrow, wide<1>, wide<2>
__host__ __device__ inline int group_of(uint32_t nq) { return nq <= 16 ? 0 : (nq <= 32 ? 1 : 2); }
__host__ __device__ inline uint32_t group_tq(int g) { return g == 0 ? 16u : 32u * uint32_t(g); }
}  // namespace iv16

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16s __attribute__((ext_vector_type(16)));

struct Ivf16Args {
    const _Float16* qh = nullptr;    // [Q x Dp] scaled fp16 queries (screen_prepare_queries)
    uint32_t nq = 0;                 // Q
    const float4* qinfo = nullptr;   // {|q|^2, |q|, 2^-scale, c0q}
    const float* qerr = nullptr;     // [Q] bound of |fp16(q) - q| (unscaled)
    const uint32_t* qrow = nullptr;  // the plan's query lists
    const _Float16* xh = nullptr;    // [N x Dp] fp16 list rows, CSR order
    const float2* xn = nullptr;      // [N] {|x|^2, bound of |fp16(x) - x|}
    uint32_t Dp = 0;
    BoundV bnd{};
    const uint32_t* thr = nullptr;   // tau_q as keys (~0: every pair passes)
    uint32_t* cnt = nullptr;
    float* cand_dot = nullptr;       // unscaled fp16 dots
    uint32_t* cand_pos = nullptr;    // CSR positions
    uint32_t cap = 0;
    ListPlan plan;
    // per plan slot (qlist order): {A, B, E, C} and {2^-scale, query id} (ivf16_big_kernel)
    const float4* gpt = nullptr;
    const float2* gqv = nullptr;
};

// pre-test inputs of a row: rows whose entries can leave the fp16 range are flagged NaN (their
// right-hand side is NaN, so they always pass)
__device__ __forceinline__ void screen_norms(float2 n, float& xxp, float& nxp, float& exp) {
    const bool flag = !(n.x < 4.29e9f);
    xxp = flag ? __builtin_nanf("") : n.x;
    nxp = flag ? __builtin_nanf("") : __builtin_amdgcn_sqrtf(n.x);
    exp = flag ? __builtin_nanf("") : n.y;
}
__device__ __forceinline__ float pretest_rhs(const PreTestV& p, float xxp, float nxp, float exp) {
    return fmaf(p.A, xxp, fmaf(p.B, nxp, fmaf(p.E, exp, p.C)));
}

__device__ __forceinline__ h8v masked_h8(const _Float16* p, bool use) {
    u32x4 t = __builtin_bit_cast(u32x4, *reinterpret_cast<const h8v*>(p));
    t &= use ? 0xFFFFFFFFu : 0u;
    return __builtin_bit_cast(h8v, t);
}

// The wave's rows' {|x|^2, error bound} into its LDS slot xs[0 .. 128) (zeros past rc); read back
// by the same wave after the main loop (one wave's LDS accesses are in order).
__device__ __forceinline__ void stage_norms(const Ivf16Args& a, float2* xs, uint32_t rs, uint32_t rc, int lane) {
    xs[lane] = uint32_t(lane) < rc ? a.xn[rs + uint32_t(lane)] : make_float2(0.0f, 0.0f);
    xs[64 + lane] = uint32_t(64 + lane) < rc ? a.xn[rs + 64u + uint32_t(lane)] : make_float2(0.0f, 0.0f);
}

// Appends the set bits of mask (bit t = element t of vals / rows[t]) to query qi's list from
// position pos.
template <int NB>
__device__ __forceinline__ void append_pairs(const Ivf16Args& a, uint32_t qi, uint32_t pos, uint32_t mask,
                                             const float (&vals)[NB], const uint32_t (&rows)[NB], uint32_t rs,
                                             float inv) {
#pragma unroll
    for (int t = 0; t < NB; ++t) {
        if (!((mask >> t) & 1u)) continue;
        if (pos < a.cap) {
            const int64_t o = int64_t(qi) * a.cap + pos;
            a.cand_dot[o] = vals[t] * inv;
            a.cand_pos[o] = rs + rows[t];
        }
        ++pos;
    }
}

// narrow tiles: lane (j, g) = (lane % 16, lane / 16) loads 16 halves at 64c + 16g of row j of
// each 16-row block and of query j; MFMA u of chunk c takes halves 8u .. 8u + 7 of them.  The
// result: lane (j, g) holds query j against rows 16b + 4g + v in acc[b][v].
struct NarrowTile {
    uint32_t qs = 0, qc = 0, rs = 0, rc = 0;
    uint32_t qi = 0;                 // the lane's query (query j of the tile; query 0 of it past qc)
    __amdgpu_buffer_rsrc_t xr;       // the tile's rows (loads past rc read zeros)
    bool valid = false;              // false: every load of the tile reads zeros
};
// wide tile: lane (l32, hh) loads 32 halves at 64c + 32hh of row l32 of each 32-row block and of
// query l32 of each 32-query block; MFMA u of chunk c takes halves 8u .. 8u + 7.  The result:
// lane (l32, hh) holds query 32n + l32 against rows 32m + 8i + 4hh + e in acc[n][m][4i + e].
template <int W>
__device__ __forceinline__ void wide_tile(const Ivf16Args& a, float2* xs, uint32_t qs, uint32_t qc, uint32_t rs,
                                          uint32_t rc) {
    const int lane = threadIdx.x & 63, l32 = lane & 31, hh = lane >> 5;
    bool qv[W];
    uint32_t qi[W];
    const _Float16* qp[W];
#pragma unroll
    for (int n = 0; n < W; ++n) {
        qv[n] = uint32_t(32 * n + l32) < qc;
        qi[n] = a.qrow[qs + (qv[n] ? uint32_t(32 * n + l32) : 0u)];
        qp[n] = a.qh + int64_t(qi[n]) * a.Dp + 32 * hh;
    }
    const uint32_t rowb = a.Dp * 2u;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a.xh + int64_t(rs) * a.Dp), 0, int(rc * rowb), 0x00020000);
    const uint32_t lo = uint32_t(l32) * rowb + 64u * uint32_t(hh);
    const uint32_t nch = a.Dp / 64;
    stage_norms(a, xs, rs, rc, lane);
    h8v qa[W][4], qb[W][4], ra[4][4], rb[4][4];
    auto load = [&](uint32_t c, h8v(&q4)[W][4], h8v(&r4)[4][4]) {
        const bool in = c < nch;
        const uint32_t k = in ? 64u * c : 0u;
#pragma unroll
        for (int n = 0; n < W; ++n)
#pragma unroll
            for (int u = 0; u < 4; ++u) q4[n][u] = masked_h8(qp[n] + k + 8 * u, qv[n] && in);
        const uint32_t vo = in ? lo + 2u * k : 0x80000000u;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                r4[m][u] = __builtin_bit_cast(
                    h8v, __builtin_amdgcn_raw_buffer_load_b128(xr, vo + uint32_t(m) * 32u * rowb + 16u * uint32_t(u), 0, 0));
    };
    f32x16s acc[W][4];
#pragma unroll
    for (int n = 0; n < W; ++n)
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[n][m][v] = 0.0f;
    auto compute = [&](const h8v(&q4)[W][4], const h8v(&r4)[4][4]) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int n = 0; n < W; ++n)
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    acc[n][m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(r4[m][u], q4[n][u], acc[n][m], 0, 0, 0);
    };
#ifndef VA_IVF16_RING
#define VA_IVF16_RING 2
#endif
    constexpr int RG = VA_IVF16_RING;
    h8v qr[RG][W][4], rr[RG][4][4];
#pragma unroll
    for (int r = 0; r < RG - 1; ++r) {
        load(uint32_t(r), qr[r], rr[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (uint32_t c = 0; c < nch; c += RG) {
#pragma unroll
        for (int r = 0; r < RG; ++r) {
            load(c + uint32_t(r + RG - 1), qr[(r + RG - 1) % RG], rr[(r + RG - 1) % RG]);
            compute(qr[r], rr[r]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    (void)qa; (void)qb; (void)ra; (void)rb;
    PreTestV pt[W];
    float inv[W];
#pragma unroll
    for (int n = 0; n < W; ++n) {
        const float4 inf = a.qinfo[qi[n]];
        pt[n] = pretest_v(a.bnd, inf.x, inf.y, a.qerr[qi[n]], inf.z, a.thr[qi[n]]);
        inv[n] = inf.z;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        float xxp[16], nxp[16], exp[16];
        uint32_t rows[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            rows[t] = uint32_t(32 * m + 8 * (t >> 2) + 4 * hh + (t & 3));
            screen_norms(xs[rows[t]], xxp[t], nxp[t], exp[t]);
        }
#pragma unroll
        for (int n = 0; n < W; ++n) {
            float vals[16];
            uint32_t mask = 0;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                vals[t] = acc[n][m][t];
                mask |= uint32_t((rows[t] < rc) & !(vals[t] < pretest_rhs(pt[n], xxp[t], nxp[t], exp[t]))) << t;
            }
            mask = qv[n] ? mask : 0u;
            // lanes l32 and l32 + 32 hold the same query: one atomic reserves both lanes' places
            const uint32_t c = uint32_t(__popc(mask));
            const uint32_t other = uint32_t(__shfl_xor(int(c), 32));
            uint32_t base = 0;
            if (hh == 0 && c + other) base = atomicAdd(a.cnt + qi[n], c + other);
            base = uint32_t(__shfl(int(base), l32));
            if (mask) append_pairs<16>(a, qi[n], hh ? base + other : base, mask, vals, rows, rs, inv[n]);
        }
    }
}

// Candidate lists of the screened scan, in place: (unscaled fp16 dot, position) -> the key of the
// pair's upper bound (over the dot) and of its lower bound (into lo), for i < min(cnt[q], cap).
// Pairs that cannot be bounded get [0, the NaN key].
__global__ __launch_bounds__(256) void ivf_bound_kernel(BoundV b, const float4* __restrict__ qinfo,
                                                        const float* __restrict__ qerr, const float2* __restrict__ xn,
                                                        float* __restrict__ dot, const uint32_t* __restrict__ pos,
                                                        uint32_t* __restrict__ lo, const uint32_t* __restrict__ cnt,
                                                        uint32_t cap) {
    const uint32_t q = blockIdx.y;
    const float4 inf = qinfo[q];
    const float eq = qerr[q];
    const uint32_t m = min(cnt[q], cap);
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < m; i += gridDim.x * 256) {
        const int64_t o = int64_t(q) * cap + i;
        const float2 n = xn[pos[o]];
        float l, h;
        uint32_t klo = 0u, khi = 0xFFFFFFFEu;
        if (screen_bounds_v(b, dot[o], inf.x, inf.y, eq, n.x, sqrtf(n.x), n.y, l, h)) {
            klo = key_of_float(l);
            khi = key_of_float(h);
        }
        reinterpret_cast<uint32_t*>(dot)[o] = khi;
        lo[o] = klo;
    }
}

// The 16-query tiles, one independent tile per wave, software-pipelined across the wave's tiles:
// the next tile is located, and its first 64-value chunk requested, while the current one is
// scanned, so the chunk's HBM latency overlaps the current tile's last chunk and epilogue; the
// epilogue's inputs (the rows' {|x|^2, error bound}, the query's pre-test constants) are loaded
// at the tile's start and used after its main loop.  Every wait for a load also waits for the
// loads issued before it, so each wait is placed where those are due anyway.
__global__ __launch_bounds__(256, 2) void ivf16_narrow_kernel(Ivf16Args a) {
    __shared__ __attribute__((aligned(16))) float2 xs_all[iv16::WAVES][iv16::TN];
    // a tile's 32 values per lane, kept for its appends ([b][lane]: conflict-free 16-byte accesses)
    __shared__ __attribute__((aligned(16))) f32x4s dump_all[iv16::WAVES][8 * 64];
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    float2* xs = xs_all[wave];
    f32x4s* dump = dump_all[wave];
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const uint32_t total = a.plan.pre[a.plan.C];
    const uint32_t stride = gridDim.x * iv16::WAVES;
    uint32_t t = blockIdx.x * iv16::WAVES + uint32_t(wave);
    if (t >= total) return;
    const uint32_t rowb = a.Dp * 2u;
    const uint32_t nch = a.Dp / 64, nce = (nch + 1) & ~1u;
    const uint32_t lo = uint32_t(j) * rowb + 32u * uint32_t(g);
    uint32_t h = 0;  // the list of the wave's last located tile
    auto setup = [&](uint32_t tt, NarrowTile& T) {
        T.valid = tt < total;
        if (!T.valid) {
            // no tile: a zero-length descriptor (every row load out of range); the query loads
            // (of query 0) are zeroed by the mask
            T.qs = T.qc = T.rs = T.rc = T.qi = 0;
            T.xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.xh), 0, 0, 0x00020000);
            return;
        }
        h = plan_tile_wave(a.plan, tt, h, 16, iv16::TN, T.qs, T.qc, T.rs, T.rc);
        T.qi = a.qrow[T.qs + (uint32_t(j) < T.qc ? uint32_t(j) : 0u)];
        T.xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.xh + int64_t(T.rs) * a.Dp), 0,
                                                 int(T.rc * rowb), 0x00020000);
    };
    // chunk c of tile T (c past the last chunk, or an invalid tile: zeros, no memory traffic)
    auto load = [&](const NarrowTile& T, uint32_t c, h8v(&q2)[2], h8v(&r2)[8][2]) {
        const bool in = T.valid && c < nch;
        const bool qv = uint32_t(j) < T.qc && in;
        const uint32_t k = in ? 64u * c : 0u;
        const _Float16* qp = a.qh + int64_t(T.qi) * a.Dp + 16 * g + k;
        q2[0] = masked_h8(qp, qv);
        q2[1] = masked_h8(qp + 8, qv);
        const uint32_t vo = in ? lo + 2u * k : 0x80000000u;
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int u = 0; u < 2; ++u)
                r2[b][u] = __builtin_bit_cast(
                    h8v, __builtin_amdgcn_raw_buffer_load_b128(T.xr, vo + uint32_t(b) * 16u * rowb + 16u * uint32_t(u), 0, 0));
    };
    f32x4s acc[8];
    auto compute = [&](const h8v(&q2)[2], const h8v(&r2)[8][2]) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int b = 0; b < 8; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r2[b][u], q2[u], acc[b], 0, 0, 0);
    };
    // The appends of a tile wait for their atomic's result, and the wait for a returning atomic
    // also waits for every load issued before it (the next tile's chunk 0, in flight during the
    // epilogue), so they run one tile late: the epilogue keeps the tile's values in LDS and issues
    // the atomic; the stores follow at the next tile's first chunk step, where chunk 0 is due.
    uint32_t p_mask = 0, p_qi = 0, p_rs = 0, p_pos = 0;
    float p_inv = 0.0f;
    const float* dumpf = reinterpret_cast<const float*>(dump);
    auto flush = [&]() {
        if (!__ballot(p_mask != 0u)) return;
        uint32_t pos = p_pos, m = p_mask;
        const int64_t ob = int64_t(p_qi) * a.cap;
        while (m && pos < a.cap) {
            const uint32_t tt = uint32_t(__builtin_ctz(m));  // value tt = 4 b + v: row 16 b + 4 g + v
            m &= m - 1;
            a.cand_dot[ob + pos] = dumpf[((tt >> 2) * 64 + uint32_t(lane)) * 4 + (tt & 3)] * p_inv;
            a.cand_pos[ob + pos] = p_rs + 16 * (tt >> 2) + 4 * uint32_t(g) + (tt & 3);
            ++pos;
        }
        p_mask = 0;
    };
    NarrowTile cur, nxt;
    setup(t, cur);
    h8v qa[2], qb[2], ra[8][2], rb[8][2];
    load(cur, 0, qa, ra);
    while (true) {
        // this tile's epilogue inputs, used after its main loop
        const float2 xn0 = uint32_t(lane) < cur.rc ? a.xn[cur.rs + uint32_t(lane)] : make_float2(0.0f, 0.0f);
        const float2 xn1 = uint32_t(64 + lane) < cur.rc ? a.xn[cur.rs + 64u + uint32_t(lane)] : make_float2(0.0f, 0.0f);
        const float4 inf = a.qinfo[cur.qi];
        const float eq = a.qerr[cur.qi];
        const uint32_t th = a.thr[cur.qi];
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[b] = f32x4s{0.f, 0.f, 0.f, 0.f};
        // an even number of chunks (one of zeros when nch is odd), so the next tile's chunk 0
        // always lands in the first register set
        for (uint32_t c = 0; c < nce; c += 2) {
            if (c == 0) flush();  // the previous tile's appends (chunk 0, older than their atomic, is due now)
            load(cur, c + 1, qb, rb);
            compute(qa, ra);
            __builtin_amdgcn_sched_barrier(0);
            // the next tile (its chunk 0 is requested during this tile's last step), located while
            // chunk 1 is in flight: the lookup's waits also wait for chunk 1, which is due next
            if (c == 0) setup(t + stride, nxt);
            if (c + 2 < nce) load(cur, c + 2, qa, ra);
            else load(nxt, 0, qa, ra);
            compute(qb, rb);
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- epilogue of this tile (the next tile's chunk 0 in flight)
        xs[lane] = xn0;
        xs[64 + lane] = xn1;  // (read back by this wave only: in order, no barrier)
        if (uint32_t(j) < cur.qc) {
            const PreTestV pt = pretest_v(a.bnd, inf.x, inf.y, eq, inf.z, th);
            uint32_t mask = 0;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t row = uint32_t(16 * b + 4 * g + v);
                    float xxp, nxp, exp;
                    screen_norms(xs[row], xxp, nxp, exp);
                    mask |= uint32_t((row < cur.rc) & !(acc[b][v] < pretest_rhs(pt, xxp, nxp, exp))) << (4 * b + v);
                }
            }
            if (mask) {
#pragma unroll
                for (int b = 0; b < 8; ++b) dump[b * 64 + lane] = acc[b];
                p_pos = atomicAdd(a.cnt + cur.qi, uint32_t(__popc(mask)));  // (awaited in flush)
                p_mask = mask;
                p_qi = cur.qi;
                p_rs = cur.rs;
                p_inv = inf.z;
            }
        }
        if (!nxt.valid) break;
        t += stride;
        cur = nxt;
    }
    flush();  // the last tile's appends
}

template <int W>
__global__ __launch_bounds__(256, W == 1 ? 2 : 1) void ivf16_wide_kernel(Ivf16Args a) {
    __shared__ __attribute__((aligned(16))) float2 xs[iv16::WAVES][iv16::TN];
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const uint32_t total = a.plan.pre[a.plan.C];
    uint32_t h = 0;  // the list of the wave's previous tile
    for (uint32_t t = blockIdx.x * iv16::WAVES + uint32_t(wave); t < total; t += gridDim.x * iv16::WAVES) {
        uint32_t qs, qc, rs, rc;
        h = plan_tile_wave(a.plan, t, h, 32u * W, iv16::TN, qs, qc, rs, rc);
        wide_tile<W>(a, xs[wave], qs, qc, rs, rc);
    }
}

// ---- lists probed by more than 32 queries: resident queries, rows straight into registers ------
// A workgroup (8 waves, one per CU) takes a tile of 64 of a list's queries x 1024 of its rows:
// the queries (gathered through the plan) and the rows' {|x|^2, error} go to LDS once per tile,
// and each wave walks its 32 rows of each of the tile's four 256-row sub-tiles against all 64
// queries on v_mfma_f32_16x16x32_f16 (2 x 4 blocks).  The rows move from HBM straight into a
// ring of R register slots of one 32-value k-step each (the wave's four lanes of a row read 64
// contiguous bytes per instruction), R - 1 k-steps ahead and across the sub-tiles of the tile;
// the query fragments come from LDS (chunk-major: each fragment read serves two MFMAs).  Passes
// are staged per wave in LDS and appended when the stage fills and at the end, so no global
// atomic or store waits inside the stream.  The wide tiles reloaded their queries with every
// 128 rows and kept one 64-value chunk in flight per wave.
namespace ivr {
constexpr int NW = 8, MB = 2;
constexpr int WR = 16 * MB;               // rows per wave per sub-tile
constexpr int SUB = NW * WR;              // rows per sub-tile
constexpr uint32_t DPMAX = 1024;          // the queries' LDS share: 64 x 1024 halves = 128 KiB
// Two shapes: 96 queries x 1024 rows where 96 fp16 query rows fit (padded d <= 768: a third
// fewer row fetches for a list probed by 97-192 queries, half for 65-96), else 64 x 1024.
template <int NQB>
struct Shape {
    static constexpr int TQ = 16 * NQB;
    static constexpr int NSUB = 4;  // sub-tiles per tile
    static constexpr uint32_t TN = uint32_t(SUB * NSUB);
    // staged passes per wave: at least 64, the most one ballot adds after a flush
    static constexpr int LCAP = NQB == 6 ? 64 : 128;
    static_assert(LCAP >= 64, "a flush must leave room for a whole wave's passes");
    static_assert(TQ <= 256, "a staged pass keeps its query's tile index in one byte");
    // LDS: queries [TQ x Dp halves], row norms [TN float2], per query {A, B, E, C} and {inv, qi},
    // the stage lists
    // (a staged pass: its value and CSR position, 4 bytes each, and its query's tile index, 1 byte)
    static constexpr uint32_t lds_bytes(uint32_t Dp) { return TQ * Dp * 2 + TN * 8 + TQ * 16 + TQ * 8 + NW * LCAP * 9; }
};
static_assert(Shape<6>::lds_bytes(768) <= 160 * 1024 && Shape<4>::lds_bytes(DPMAX) <= 160 * 1024,
              "one workgroup's LDS at the largest padded d of each shape");
inline int nqb_for(uint32_t Dp) { return Dp <= 768 ? 6 : 4; }
}  // namespace ivr

template <int R, int NQB>
__global__ __launch_bounds__(512, 2) void ivf16_resq_kernel(Ivf16Args a) {
    using namespace ivr;
    using Sh = Shape<NQB>;
    constexpr int TQ = Sh::TQ, NSUB = Sh::NSUB, LCAP = Sh::LCAP;
    constexpr uint32_t TN = Sh::TN;
    constexpr uint32_t CS = TQ * 16;  // bytes of one 16-byte chunk column of the queries
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int tid = threadIdx.x, lane = tid & 63, r16 = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t Dp = a.Dp, rowb = Dp * 2u;
    const uint32_t nsl = Dp / 64;  // ring slots (128 bytes of each row) per sub-tile, a multiple of R
    char* nrm_b = lds8 + TQ * rowb;
    const float2* s_nrm = reinterpret_cast<const float2*>(nrm_b);
    float4* s_pt = reinterpret_cast<float4*>(nrm_b + TN * 8);
    float2* s_qv = reinterpret_cast<float2*>(nrm_b + TN * 8 + TQ * 16);
    uint32_t* s_val = reinterpret_cast<uint32_t*>(nrm_b + TN * 8 + TQ * 24 + wave * 9 * LCAP);
    uint32_t* s_pos = s_val + LCAP;
    uint8_t* s_ql = reinterpret_cast<uint8_t*>(s_pos + LCAP);  // the pass's query in the tile (< TQ)
    const uint32_t lds0 = lds_addr_of(lds8);
    uint32_t lc = 0;  // staged passes (wave-uniform)
    // Appends the staged passes: count every pass, keep a query's first cap.
    auto flush = [&]() {
        for (uint32_t b0 = 0; b0 < lc; b0 += 64) {
            const uint32_t e = b0 + uint32_t(lane);
            if (e < lc) {
                const uint32_t qi = __builtin_bit_cast(uint32_t, s_qv[s_ql[e]].y);
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    a.cand_dot[int64_t(qi) * a.cap + pos] = __builtin_bit_cast(float, s_val[e]);
                    a.cand_pos[int64_t(qi) * a.cap + pos] = s_pos[e];
                }
            }
        }
        lc = 0;
    };
    // query block u of k-step t: chunk 4 t + g of query 16 u + r16
    const char* qrd = lds8 + g * CS + r16 * 16;
    auto rd_q = [&](uint32_t t, int u) { return *reinterpret_cast<const h8v*>(qrd + t * (4 * CS) + u * 256); };
    uint32_t voff[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) voff[j] = uint32_t(16 * j + r16) * rowb + 16u * uint32_t(g);
    const __amdgpu_buffer_rsrc_t qres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.qh), 0, int(a.nq * rowb), 0x00020000);

    // XCD-aware order: XCD x (workgroups b with b % 8 == x; gridDim.x is a multiple of 8) takes
    // the x-th eighth of the plan's tiles, which its workgroups walk together, so the query
    // blocks of one row block (consecutive tiles) meet in the XCD's L2 and the rows come from
    // HBM about once.
    const uint32_t total = a.plan.pre[a.plan.C];
    const uint32_t tpx = (total + kXcds - 1) / kXcds, xcd = blockIdx.x % kXcds;
    const uint32_t tend = min(total, (xcd + 1) * tpx);
    uint32_t lh = 0;  // the list of this workgroup's previous tile
    uint32_t pqs = 0xFFFFFFFFu, pqc = 0;  // the query block the LDS holds (a list's row tiles share one)
    for (uint32_t t = xcd * tpx + blockIdx.x / kXcds; t < tend; t += gridDim.x / kXcds) {
        uint32_t qs, qc, rs, rc;
        lh = plan_tile_after_wave(a.plan, t, lh, TQ, TN, qs, qc, rs, rc);
        // the queries and their constants stay in LDS from the previous tile when it had the same
        // query block (consecutive tiles of a workgroup often are row blocks of one list)
        const bool newq = qs != pqs || qc != pqc;
        pqs = qs;
        pqc = qc;
        __syncthreads();  // every wave is done with the previous tile's LDS
        // the tile's rows' {|x|^2, error} (past rc: zeros) by direct loads, and its queries,
        // chunk-major (16-byte chunk m of query r at m * CS + r * 16; past qc: zeros): thread
        // t < 5 TQ holds query t % TQ and copies chunks t / TQ, + 5, ...
        {
            if (uint32_t(wave) < TN * 8 / 1024) {
                const dma_rsrc nres = make_dma_rsrc(a.xn + rs, rc * 8u);
                lds_dma16(nres, uint32_t(tid) * 16u, lds0 + TQ * rowb + uint32_t(wave) * 1024u);
            }
            constexpr uint32_t QS = 512 / TQ, QT = QS * TQ;  // threads that copy queries
            if (newq && uint32_t(tid) < QT) {
                const uint32_t r = uint32_t(tid) % TQ;
                const bool qv = r < qc;
                // buffer loads over all the fp16 queries (Q Dp 2 < 2^31 bytes): a query past qc or
                // a chunk past the row reads zeros through the range check, so the loads are
                // issued without branches and all in flight before their stores
                const uint32_t qoff = qv ? a.qrow[qs + r] * rowb : kDmaSkip;
                // (24 loads a thread cover a row at every shape: one round trip)
                constexpr int NB = 24;
                static_assert(NB * QS * 8 >= (TQ == 96 ? 768 : int(DPMAX)), "one batch per query row");
                for (uint32_t m0 = uint32_t(tid) / TQ; m0 < Dp / 8; m0 += NB * QS) {
                    uint4 v[NB];
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const uint32_t m = m0 + uint32_t(b) * QS;
                        v[b] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                             qres, m < Dp / 8 ? qoff + m * 16u : kDmaSkip, 0, 0));
                    }
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const uint32_t m = m0 + uint32_t(b) * QS;
                        if (m < Dp / 8) *reinterpret_cast<uint4*>(lds8 + m * CS + r * 16u) = v[b];
                    }
                }
            }
        }
        if (newq && tid < TQ) {
            float4 p = {0.0f, 0.0f, 0.0f, 0.0f};
            float2 v = {0.0f, 0.0f};
            if (uint32_t(tid) < qc) {
                const uint32_t qi = a.qrow[qs + uint32_t(tid)];
                const float4 inf = a.qinfo[qi];
                const PreTestV pt = pretest_v(a.bnd, inf.x, inf.y, a.qerr[qi], inf.z, a.thr[qi]);
                p = make_float4(pt.A, pt.B, pt.E, pt.C);
                v = make_float2(inf.z, __builtin_bit_cast(float, qi));
            }
            s_pt[tid] = p;
            s_qv[tid] = v;
        }
        wait_vmcnt<0>();
        __syncthreads();  // queries, norms and constants visible

        // ---- this wave's rows: sub-tiles j with rows j SUB + wave WR .. (+ WR) of the tile ------
        const uint32_t w0 = uint32_t(wave) * WR;
        const uint32_t nsub = rc > w0 ? min(uint32_t(NSUB), (rc - w0 + SUB - 1) / SUB) : 0u;
        if (nsub == 0) continue;
        uint32_t lsub = 0, lsl = 0;  // sub-tile and slot of the next load (wave-uniform)
        // The descriptor covers this wave's rows of the sub-tile being loaded; a lane's row
        // offset fails its range check for rows past the tile (and every load past the last
        // sub-tile reads zeros).
        // A slot is the 128 bytes of each row that one cache line holds: both 64-byte halves of
        // a row block are requested back to back (one instruction per half and row block).
        auto load = [&](h8v(&dst)[2][MB]) {
            const bool ok = lsub < nsub;
            const uint32_t o = lsub * SUB + w0;
            const uint32_t rows = __builtin_amdgcn_readfirstlane(ok ? min(uint32_t(WR), rc - o) : 0u);
            const uint64_t base = reinterpret_cast<uint64_t>(a.xh + int64_t(rs + (ok ? o : 0u)) * Dp);
            const uint64_t bs = (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(base >> 32)))) << 32) |
                                uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(base)));
            const __amdgpu_buffer_rsrc_t xres =
                __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(bs), 0, int(rows * rowb), 0x00020000);
            const uint32_t skip = rows ? 0u : kDmaSkip;
#pragma unroll
            for (int j = 0; j < MB; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    dst[h][j] = __builtin_bit_cast(
                        h8v, __builtin_amdgcn_raw_buffer_load_b128(xres, voff[j] | skip, int(lsl * 128u + 64u * h), 0));
            if (++lsl == nsl) {
                lsl = 0;
                ++lsub;
            }
        };
        f32x4s acc[NQB][MB];
#pragma unroll
        for (int u = 0; u < NQB; ++u)
#pragma unroll
            for (int j = 0; j < MB; ++j) acc[u][j] = f32x4s{0.f, 0.f, 0.f, 0.f};
        h8v xr[R][2][MB], qf[NQB];
        static_assert(NQB <= 8, "query fragments in registers");
#pragma unroll
        for (int r = 0; r < R - 1; ++r) {
            load(xr[r]);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int u = 0; u < NQB; ++u) qf[u] = rd_q(0, u);
        uint32_t mst = 0, msub = 0;  // k-step (32 values) and sub-tile of the MFMAs
        const uint32_t nst = 2 * nsl;
        auto mma = [&](const h8v(&x)[2][MB]) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t nks = mst + 1 == nst ? 0u : mst + 1;
#pragma unroll
                for (int u = 0; u < NQB; ++u) {
#pragma unroll
                    for (int j = 0; j < MB; ++j)
                        acc[u][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[h][j], qf[u], acc[u][j], 0, 0, 0);
                    qf[u] = rd_q(nks, u);
                    __builtin_amdgcn_sched_group_barrier(0x008, MB, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                mst = nks;
            }
        };
        // A sub-tile's passes: lane (r16, g) holds query 16 u + r16 against rows 16 j + 4 g + v of
        // the wave's 32 in acc[u][j][v]; the pre-test of the flat screen (flagged rows pass).  The
        // rows' pre-test inputs are read once for all query blocks; a block with passes is staged
        // by a loop over its eight values (one copy of the flush per block, not per value: the
        // fully unrolled staging made the kernel's code several times larger).
        auto epilogue = [&]() {
            const uint32_t o = msub * SUB + w0;  // the wave's first row in the tile
            float xxp[4 * MB], nxp[4 * MB], exp[4 * MB];
            bool rin[4 * MB];
#pragma unroll
            for (int t = 0; t < 4 * MB; ++t) {
                const uint32_t row = o + uint32_t(16 * (t >> 2) + 4 * g + (t & 3));
                screen_norms(s_nrm[row], xxp[t], nxp[t], exp[t]);
                rin[t] = row < rc;
            }
#pragma unroll
            for (int u = 0; u < NQB; ++u) {
                const int ql = 16 * u + r16;
                const float4 p = s_pt[ql];
                const PreTestV pt = {p.x, p.y, p.z, p.w};
                uint32_t mask = 0;
#pragma unroll
                for (int t = 0; t < 4 * MB; ++t) {
                    const bool pass = rin[t] && !(acc[u][t >> 2][t & 3] < pretest_rhs(pt, xxp[t], nxp[t], exp[t]));
                    mask |= uint32_t(pass) << t;
                }
                mask = uint32_t(ql) < qc ? mask : 0u;
                if (!__ballot(mask != 0u)) continue;
                const float2 qv = s_qv[ql];
                float vals[4 * MB];
#pragma unroll
                for (int t = 0; t < 4 * MB; ++t) vals[t] = acc[u][t >> 2][t & 3] * qv.x;
#pragma unroll 1
                for (int t = 0; t < 4 * MB; ++t) {
                    const bool pass = (mask >> t) & 1u;
                    const uint64_t mk = __ballot(pass);
                    if (!mk) continue;
                    const uint32_t n = uint32_t(__popcll(mk));
                    if (lc + n > uint32_t(LCAP)) flush();  // wave-uniform
                    if (pass) {
                        const uint32_t e = lc + __builtin_amdgcn_mbcnt_hi(uint32_t(mk >> 32),
                                                                         __builtin_amdgcn_mbcnt_lo(uint32_t(mk), 0u));
                        s_ql[e] = uint8_t(ql);
                        s_val[e] = __builtin_bit_cast(uint32_t, vals[t]);
                        s_pos[e] = rs + o + uint32_t(16 * (t >> 2) + 4 * g + (t & 3));
                    }
                    lc += n;
                }
            }
        };
        const uint32_t steps = nsub * nsl;
        for (uint32_t s = 0; s < steps; s += R) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                load(xr[(r + R - 1) % R]);  // the slot the previous k-step consumed
                mma(xr[r]);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (mst == 0) {
                epilogue();
                ++msub;
#pragma unroll
                for (int u = 0; u < NQB; ++u)
#pragma unroll
                    for (int j = 0; j < MB; ++j) acc[u][j] = f32x4s{0.f, 0.f, 0.f, 0.f};
            }
        }
        // a staged pass names its query by the tile's index, which the next tile's setup
        // reassigns: the stage empties with the tile
        flush();
    }
}

// ---- lists probed by many queries: LDS-staged 32x32x16 tiles ------------------------------------
// A list probed by more than ivb::kMinQueries queries is, for its probing queries, a small flat
// database, so the full pass gives it the flat screen's layout (screen16_kernel): a workgroup tile
// of 192 of its queries x 256 of its rows, twelve waves of 64 x 64 (2 x 2 blocks of
// v_mfma_f32_32x32x16_f16, three waves per SIMD), both operands moved global -> LDS by direct
// loads, the queries gathered through the plan's list of the list's probing queries.  One row
// fetch serves up to 192 queries (configs[4]'s 642K-row list probed by ~170 queries is read once
// instead of twice by the 96-query tiles).  Unlike the flat screen's rows, which its neighbouring
// query blocks share through L2, a list's rows come from HBM once, so the stages are a ring of
// NSLOT slots of KC d-values with NSLOT - 1 stages in flight while one computes.  The tile's
// pre-test constants come from the plan-slot table (ivf_slot_pretest_kernel: one load per query,
// no gather) and its rows' {|x|^2, error bound} with one load per row, both loaded at the tile's
// start and used after its main loop.  The epilogue tests every value from registers against the
// list pre-test A|x|^2 + B|x| + E ex + C (a lane reads each 4-row group's inputs from LDS once for
// both of its queries) and appends (value, CSR position).
namespace ivb {
constexpr int NQB = 2, MB = 2;  // a wave: 32 NQB queries x 32 MB rows
template <int WAVES, int TQ, int KC, int NSLOT>
struct Shape {
    static constexpr int WQ = 32 * NQB, WN = 32 * MB;
    static constexpr int QW = TQ / WQ;            // waves along the queries
    static constexpr int TN = WN * (WAVES / QW);  // rows per tile
    static constexpr int ROWB = KC * 2;           // bytes of a row in a stage
    static constexpr int CPR = KC / 8;            // 16-byte chunks per row
    static constexpr int RPG = 64 / CPR;          // rows per 1 KiB direct-load group (one per lane chunk)
    // chunk swizzle: the rows that share a 256-byte LDS line (16 / CPR of them) spread one chunk
    // column over the line, so a fragment read of 16 lanes touches every bank once
    static constexpr int SWS = CPR == 8 ? 1 : CPR == 4 ? 2 : 3;  // log2(16 / CPR)
    static constexpr int OPQ = TQ * ROWB, OPX = TN * ROWB, STAGE = OPQ + OPX, LDS = NSLOT * STAGE;
    // 1 KiB direct-load groups per stage: GQ of queries, GX of rows; a wave issues up to LPW of
    // each and at least LMIN loads in all
    static constexpr int GQ = OPQ / 1024, GX = OPX / 1024;
    static constexpr int LPW = ((GQ > GX ? GQ : GX) + WAVES - 1) / WAVES, LMIN = GQ / WAVES + GX / WAVES;
    // the next tile's first EARLY stages load during the epilogue; the epilogue's dump (4 KiB per
    // wave) takes the slots after them
    static constexpr int EARLY = NSLOT - (WAVES * 4096 + STAGE - 1) / STAGE;
    static_assert(KC % 16 == 0 && (CPR == 8 || CPR == 4 || CPR == 2), "stage width");
    static_assert(QW * WQ == TQ && WAVES % QW == 0 && TN % RPG == 0 && TQ % RPG == 0, "wave layout");
    static_assert(64 * WAVES >= TN && 64 * WAVES >= TQ, "one thread per row and query");
    static_assert(EARLY >= 1 && NSLOT >= 2 && NSLOT <= 4, "ring: the epilogue's dump and one early stage");
    static_assert(LMIN >= 1 && 3 * LMIN < 64, "wait counts");
};
constexpr int kWaves = 12, kTQ = 192, kKC = 32, kSlots = 4;
using Big = Shape<kWaves, kTQ, kKC, kSlots>;
constexpr uint32_t kMinQueries = 96;  // (the 96-query tiles read a list once up to 96 queries)
}  // namespace ivb

// {A, B, E, C} and {2^-scale, query id} of every slot of the plan's query lists (qlist order), so
// a tile of a list's queries loads its constants with one load per query.
__global__ __launch_bounds__(256) void ivf_slot_pretest_kernel(BoundV b, const uint32_t* __restrict__ qlist,
                                                              const uint32_t* __restrict__ total, uint32_t n,
                                                              const float4* __restrict__ qinfo,
                                                              const float* __restrict__ qerr,
                                                              const uint32_t* __restrict__ thr, float4* __restrict__ gpt,
                                                              float2* __restrict__ gqv) {
    const uint32_t m = min(*total, n);
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < m; j += gridDim.x * 256) {
        const uint32_t qi = qlist[j];
        const float4 inf = qinfo[qi];
        const PreTestV pt = pretest_v(b, inf.x, inf.y, qerr[qi], inf.z, thr[qi]);
        gpt[j] = make_float4(pt.A, pt.B, pt.E, pt.C);
        gqv[j] = make_float2(inf.z, __builtin_bit_cast(float, qi));
    }
}

// wait until at most m stages' loads (LMIN per stage and wave) are in flight, m < 4
template <int LMIN>
__device__ __forceinline__ void wait_stages(uint32_t m) {
    if (m >= 3) wait_vmcnt<3 * LMIN>();
    else if (m == 2) wait_vmcnt<2 * LMIN>();
    else if (m == 1) wait_vmcnt<LMIN>();
    else wait_vmcnt<0>();
}

template <int WAVES, int TQ, int KC, int NSLOT>
__global__ __launch_bounds__(64 * WAVES, 1) void ivf16_big_kernel(Ivf16Args a) {
    using namespace ivb;
    using Sh = Shape<WAVES, TQ, KC, NSLOT>;
    constexpr int WQ = Sh::WQ, WN = Sh::WN, QW = Sh::QW, TN = Sh::TN, ROWB = Sh::ROWB, CPR = Sh::CPR;
    constexpr int RPG = Sh::RPG, SWS = Sh::SWS, OPQ = Sh::OPQ, STAGE = Sh::STAGE, GQ = Sh::GQ, GX = Sh::GX;
    constexpr int LPW = Sh::LPW, LMIN = Sh::LMIN, EARLY = Sh::EARLY;
    constexpr int KS = KC / 16;  // k-steps per stage
    typedef float f32x16v __attribute__((ext_vector_type(16)));
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    __shared__ __attribute__((aligned(16))) float norms[3 * TN];  // pre-test inputs xx, nx, ex (NaN: flagged)
    __shared__ float4 ptl[TQ];       // {A, B, E, C} of the tile's queries
    __shared__ float2 pqv[TQ];       // {2^-scale, query id}
    __shared__ uint32_t tcount[TQ];  // the tile's passes per query (zero between tiles)
    __shared__ uint32_t tbase[TQ];   // their first position in the query's candidate list
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave % QW, wn = wave / QW, l32 = lane & 31, hh = lane >> 5;
    const uint32_t nst = a.Dp / KC, rowb = a.Dp * 2u;
    if (tid < TQ) tcount[tid] = 0u;  // (published by the tile loop's barriers)
    float* xxp = norms;
    float* nxp = norms + TN;
    float* exq = norms + 2 * TN;

    // Tiles: XCD x (workgroups b with b % 8 == x; gridDim.x is a multiple of 8) walks the x-th
    // eighth of the group's plan tiles, so the row blocks of a list run on one XCD and the list's
    // queries stay in its L2.
    const uint32_t total = a.plan.pre[a.plan.C];
    const uint32_t tpx = (total + kXcds - 1) / kXcds, xcd = blockIdx.x % kXcds;
    const uint32_t tend = min(total, (xcd + 1) * tpx), tstep = gridDim.x / kXcds;
    // The list of the last tile located (wave-uniform, the same in every wave): a tile of the
    // same list is located without a load.
    uint32_t cl = 0, cpre0 = 0, cpre1 = 0, cq0 = 0, cnq = 0, cr0 = 0, cn = 0;
    auto locate = [&](uint32_t t, uint32_t& qs, uint32_t& qc, uint32_t& rs, uint32_t& rc) {
        if (t >= cpre1) {  // (t only grows; the first call: cpre1 = 0)
            uint32_t q_, c_, r_, n_;
            cl = __builtin_amdgcn_readfirstlane(plan_tile_after_wave(a.plan, t, cl, TQ, TN, q_, c_, r_, n_));
            cpre0 = __builtin_amdgcn_readfirstlane(a.plan.pre[cl]);
            cpre1 = __builtin_amdgcn_readfirstlane(a.plan.pre[cl + 1]);
            cq0 = __builtin_amdgcn_readfirstlane(a.plan.qoff[cl]);
            cnq = __builtin_amdgcn_readfirstlane(a.plan.qoff[cl + 1]) - cq0;
            cr0 = __builtin_amdgcn_readfirstlane(a.plan.roff[cl]);
            const uint32_t len = __builtin_amdgcn_readfirstlane(a.plan.roff[cl + 1]) - cr0;
            cn = a.plan.sample ? ivf_sample_rows(len) : len;
        }
        const uint32_t local = t - cpre0, nqb = (cnq + TQ - 1) / TQ;
        const uint32_t rb = local / nqb, qb = local % nqb;
        qs = cq0 + qb * uint32_t(TQ);
        qc = min(uint32_t(TQ), cnq - qb * uint32_t(TQ));
        rs = cr0 + rb * uint32_t(TN);
        rc = min(uint32_t(TN), cn - rb * uint32_t(TN));
    };

    // Direct loads: wave w fills 1 KiB groups g = w + WAVES i (rows RPG g .. RPG g + RPG - 1) of
    // each operand; lane L loads row RPG g + L / CPR at physical chunk L % CPR = logical chunk
    // (L % CPR) ^ ((row >> SWS) % CPR).  Query rows past qc and list rows past rc read nothing
    // (zeros).
    auto swz_of = [](uint32_t row) { return (row >> SWS) & uint32_t(CPR - 1); };
    uint32_t xoff[LPW], qoff[LPW], qnext[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const uint32_t row = uint32_t(RPG * (wave + WAVES * i) + lane / CPR);
        xoff[i] = row * rowb + 16u * ((uint32_t(lane) % CPR) ^ swz_of(row));
    }
    // the query rows' offsets of a tile (qrow loads; used when its stages are issued)
    auto query_offsets = [&](uint32_t qs, uint32_t qc, uint32_t(&o)[LPW]) {
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int g = wave + WAVES * i;
            const uint32_t row = uint32_t(RPG * g + lane / CPR);
            const bool in = (GQ == LPW * WAVES || g < GQ) && row < qc;
            o[i] = in ? a.qrow[qs + row] * rowb + 16u * ((uint32_t(lane) % CPR) ^ swz_of(row)) : kDmaSkip;
        }
    };
    const dma_rsrc qres = make_dma_rsrc(a.qh, a.nq * rowb);
    const uint32_t lds0 = lds_addr_of(lds);
    // stage s of a tile into slot s % NSLOT (stages past the row's end are not issued)
    auto issue_with = [&](const dma_rsrc& xr, const uint32_t(&qo)[LPW], uint32_t s) {
        const uint32_t d0 = s * KC;
        const uint32_t sb = lds0 + (s % NSLOT) * uint32_t(STAGE);
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int g = wave + WAVES * i;  // wave-uniform
            if (GQ == LPW * WAVES || g < GQ)
                lds_dma16(qres, qo[i] != kDmaSkip ? qo[i] + d0 * 2u : kDmaSkip, sb + uint32_t(g) * 1024u);
            if (GX == LPW * WAVES || g < GX) lds_dma16(xr, xoff[i] + d0 * 2u, sb + uint32_t(OPQ + g * 1024));
        }
    };
    // fragment rows start at multiples of 32, a multiple of the swizzle's period
    const uint32_t swz = swz_of(uint32_t(l32));
    const uint32_t a_off = uint32_t(OPQ + (wn * WN + l32) * ROWB);
    const uint32_t b_off = uint32_t((wq * WQ + l32) * ROWB);
    f32x16v acc[MB][NQB];
    h8v fa[2][MB], fb[2][NQB];
    auto read_frags = [&](int buf, uint32_t slot, int t) {
        const char* base = lds + slot * STAGE;
        const uint32_t ko = 16u * ((uint32_t(2 * t + hh)) ^ swz);
#pragma unroll
        for (int m = 0; m < MB; ++m) fa[buf][m] = *reinterpret_cast<const h8v*>(base + a_off + m * 32 * ROWB + ko);
#pragma unroll
        for (int n = 0; n < NQB; ++n) fb[buf][n] = *reinterpret_cast<const h8v*>(base + b_off + n * 32 * ROWB + ko);
    };
    auto mma = [&](int buf) {
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int n = 0; n < NQB; ++n)
                acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[buf][m], fb[buf][n], acc[m][n], 0, 0, 0);
    };
    auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < MB * NQB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < MB + NQB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    };
    // workgroup barrier without the release fence of __syncthreads (which would also wait for
    // the direct loads in flight); this wave's LDS reads are complete before it
    auto barrier = [&]() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    auto row_of = [&](int t) { return wn * WN + 32 * (t >> 4) + 8 * ((t >> 2) & 3) + 4 * hh + (t & 3); };
    using Mask = uint32_t;  // bit t: value t of a query block (16 MB values)
    static_assert(16 * MB <= 32, "one mask word per query block");
    // the epilogue's LDS: 4 KiB per wave in the slots after the EARLY ones
    f32x4v* dump = reinterpret_cast<f32x4v*>(lds + EARLY * STAGE + wave * 4096) + lane;  // [c][lane], c < 4

    uint32_t t = xcd * tpx + blockIdx.x / kXcds;
    if (t >= tend) return;
    uint32_t qs, qc, rs, rc;
    locate(t, qs, qc, rs, rc);
    query_offsets(qs, qc, qoff);
    dma_rsrc xres = make_dma_rsrc(a.xh + int64_t(rs) * a.Dp, rc * rowb);
    // later tiles: stages 0 .. EARLY - 1 are loaded during the previous epilogue
    for (uint32_t s = 0; s < uint32_t(EARLY) && s < nst; ++s) issue_with(xres, qoff, s);
    while (t < tend) {
        // the next tile (located now: a tile of another list waits for its plan entries here,
        // where this tile's first stages are in flight anyway) and its query rows' offsets,
        // loaded during this tile
        const uint32_t tn = t + tstep;
        uint32_t nqs = 0, nqc = 0, nrs = 0, nrc = 0;
        if (tn < tend) {
            locate(tn, nqs, nqc, nrs, nrc);
            query_offsets(nqs, nqc, qnext);
        }
        // this tile's pre-test inputs: loaded now, used after the main loop
        const float2 xn_t = tid < TN && uint32_t(tid) < rc ? a.xn[rs + uint32_t(tid)] : make_float2(0.0f, 0.0f);
        const bool qin = tid < TQ && uint32_t(tid) < qc;
        const float4 pt_t = qin ? a.gpt[qs + uint32_t(tid)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float2 qv_t = qin ? a.gqv[qs + uint32_t(tid)] : make_float2(0.0f, 0.0f);
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int n = 0; n < NQB; ++n)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[m][n][v] = 0.0f;
        // every wave is past the previous tile's epilogue (its dump is read)
        barrier();
        const uint32_t ahead = min(uint32_t(NSLOT), nst);  // stages in flight before the main loop
        for (uint32_t s = uint32_t(EARLY); s < ahead; ++s) issue_with(xres, qoff, s);
        wait_stages<LMIN>(ahead - 1);  // stage 0 (the oldest)
        barrier();
        read_frags(0, 0, 0);
        for (uint32_t s = 0; s < nst; ++s) {
            const uint32_t slot = s % NSLOT;
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const int cur = k & 1;
                if (k < KS - 1) {
                    read_frags(cur ^ 1, slot, k + 1);
                    mma(cur);
                    interleave();
                } else {
                    // this k-step's fragments are in registers: wait for stage s + 1 (the stages
                    // after it stay in flight), publish it, and refill slot s with stage s + NSLOT
                    const uint32_t after = s + 2 < nst ? min(nst - (s + 2), uint32_t(NSLOT - 2)) : 0u;
                    wait_stages<LMIN>(after);
                    barrier();
                    if (s + NSLOT < nst) issue_with(xres, qoff, s + NSLOT);
                    read_frags(cur ^ 1, (s + 1) % NSLOT, 0);
                    mma(cur);
                    interleave();
                }
            }
        }
        wait_vmcnt<0>();

        if (tid < TN) {
            float x2, x1, xe;
            screen_norms(xn_t, x2, x1, xe);
            xxp[tid] = x2;
            nxp[tid] = x1;
            exq[tid] = xe;
        }
        if (tid < TQ) {
            ptl[tid] = pt_t;
            pqv[tid] = qv_t;
        }
        __syncthreads();  // every wave is past the main loop: every slot is free

        // ---- epilogue: lane (l32, hh) holds query wq*WQ + 32n + l32 against rows
        // wn*WN + 32m + 8j + 4hh + e in acc[m][n][4j + e]; t = 16m + 4j + e indexes its 16 MB values.
        // 1. the passes of each query block as a bit mask; 2. each lane pair's count added to its query's tile
        //    count in LDS (the returned value is the pair's offset in the query's share of the tile);
        // 3. one global atomic per query of the tile reserves its share of the candidate list (a
        //    list probed by many queries appends for most of them in every tile, so per-wave atomics
        //    and their waits were most of the tile's time); 4. the next tile's first stages; 5. the
        //    appends.  No returning global operation is waited for after the next tile's loads are
        //    issued (that wait would also wait for them).
        Mask valid = ~Mask(0);
        if (rc < uint32_t(TN)) {
            valid = 0;
#pragma unroll 1
            for (int v = 0; v < 16 * MB; ++v) valid |= Mask(uint32_t(row_of(v)) < rc) << v;
        }
        // row block m of query block n into the dump (for the appends): values 16m .. 16m + 15
        auto dump_half = [&](auto NC, auto MC) {
            constexpr int n = decltype(NC)::value, m = decltype(MC)::value;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                f32x4v v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[m][n][4 * c + e];
                dump[c * 64] = v;
            }
            asm volatile("" ::: "memory");  // re-read the dump from LDS below
        };
        // 1. the passes of the lane's two queries over its 32 rows, tested from registers: each 4-row
        //    group's pre-test inputs are read once for both queries (a list probed by this many
        //    queries has candidates in most row blocks, so no quick rejection precedes the test)
        static_assert(NQB == 2, "two query blocks per wave");
        Mask mk0 = 0, mk1 = 0;
        {
            const uint32_t qt0 = uint32_t(wq * WQ + l32), qt1 = qt0 + 32u;
            const float4 p0 = ptl[qt0], p1 = ptl[qt1];
            const PreTestV pt0 = {p0.x, p0.y, p0.z, p0.w}, pt1 = {p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int m = 0; m < MB; ++m)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int r = row_of(16 * m + 4 * c);  // rows r .. r + 3
                    const f32x4v x2 = *reinterpret_cast<const f32x4v*>(xxp + r);
                    const f32x4v x1 = *reinterpret_cast<const f32x4v*>(nxp + r);
                    const f32x4v xe = *reinterpret_cast<const f32x4v*>(exq + r);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = 16 * m + 4 * c + e;
                        mk0 |= Mask(!(acc[m][0][4 * c + e] < pretest_rhs(pt0, x2[e], x1[e], xe[e]))) << t;
                        mk1 |= Mask(!(acc[m][1][4 * c + e] < pretest_rhs(pt1, x2[e], x1[e], xe[e]))) << t;
                    }
                }
            mk0 &= qt0 < qc ? valid : Mask(0);
            mk1 &= qt1 < qc ? valid : Mask(0);
        }
        // 2. the pair's offset in its query's share of the tile (lane l32 adds both halves' passes)
        uint32_t off0 = 0, off1 = 0;
        {
            const uint32_t c0 = uint32_t(__popc(mk0)), c1 = uint32_t(__popc(mk1));
            const uint32_t o0 = uint32_t(__shfl_xor(int(c0), 32)), o1 = uint32_t(__shfl_xor(int(c1), 32));
            uint32_t b0 = 0, b1 = 0;
            if (hh == 0 && c0 + o0) b0 = atomicAdd(&tcount[wq * WQ + l32], c0 + o0);
            if (hh == 0 && c1 + o1) b1 = atomicAdd(&tcount[wq * WQ + 32 + l32], c1 + o1);
            off0 = uint32_t(__shfl(int(b0), l32)) + (hh ? o0 : 0u);
            off1 = uint32_t(__shfl(int(b1), l32)) + (hh ? o1 : 0u);
        }
        __syncthreads();
        // 3. the tile's share of each query's candidate list
        if (tid < TQ) {
            const uint32_t n = tcount[tid];
            uint32_t base = 0;
            if (n) base = atomicAdd(a.cnt + __builtin_bit_cast(uint32_t, pqv[tid].y), n);
            tbase[tid] = base;
            tcount[tid] = 0u;  // (read above; cleared for the next tile)
        }
        __syncthreads();
        // 4. the next tile's first stages, during the appends
        if (tn < tend) {
#pragma unroll
            for (int i = 0; i < LPW; ++i) qoff[i] = qnext[i];
            xres = make_dma_rsrc(a.xh + int64_t(nrs) * a.Dp, nrc * rowb);
            for (uint32_t s = 0; s < uint32_t(EARLY) && s < nst; ++s) issue_with(xres, qoff, s);
        }
        // 5. the appends (stores only)
        auto append = [&](auto NC, Mask mk, uint32_t off) {
            constexpr int n = decltype(NC)::value;
            if (!__ballot(mk != 0u)) return;
            const uint32_t qt = uint32_t(wq * WQ + 32 * n + l32);
            const float2 qv = pqv[qt];
            const uint32_t qi = __builtin_bit_cast(uint32_t, qv.y);
            uint32_t pos = tbase[qt] + off;
            const float* src = reinterpret_cast<const float*>(dump);
            auto append_half = [&](auto MC) {
                constexpr int m = decltype(MC)::value;
                uint32_t mh = (mk >> (16 * m)) & 0xFFFFu;
                if (!__ballot(mh != 0u)) return;
                dump_half(NC, MC);
                while (mh && pos < a.cap) {
                    const int c16 = __builtin_ctz(mh);
                    mh &= mh - 1;
                    const int r = row_of(16 * m + c16);
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_dot[o] = src[(c16 >> 2) * 256 + (c16 & 3)] * qv.x;
                    a.cand_pos[o] = rs + uint32_t(r);
                    ++pos;
                }
            };
            append_half(std::integral_constant<int, 0>());
            append_half(std::integral_constant<int, 1>());
        };
        append(std::integral_constant<int, 0>(), mk0, off0);
        append(std::integral_constant<int, 1>(), mk1, off1);
        t = tn;
        qs = nqs;
        qc = nqc;
        rs = nrs;
        rc = nrc;
    }
    wait_vmcnt<0>();
}

// Tile shapes and their cost model: shape_for / group_tile (va_plan.hpp, shared with the host
// planning tests).
static_assert(ivfs::TQ == kSmallTileQueries && ivfs::TN == kSmallTileRows, "16-query tile of ivf_small_kernel");

// ---- device plan of a list-major search ----------------------------------------------------
// From the probes alone, on the device: every (query, list) pair once (a list probed twice by a
// query is scanned once; sentinel / out-of-range probes are skipped, IVFListSearch.metal:
// 249-251), the queries probing each list grouped by list (qlist, offsets qoff), and for each
// pass (0: threshold sample, 1: full scan) and tile group the exclusive prefix over the lists of
// their tile counts.  The scan kernels decode their tiles from these prefixes.
struct DevPlan {
    const uint32_t* probes = nullptr;  // [Q x np]
    uint32_t Q = 0, np = 0, C = 0;
    const uint32_t* roff = nullptr;    // list offsets [C + 1]
    uint32_t small_ok = 0;
    uint32_t screen = 0;        // tile groups of the screened scan (iv16) instead of the fp32 shapes
    uint32_t wide_tn = 0;       // screened scan: rows and queries per tile of the last group in the
    uint32_t wide_tq = 0;       // full pass (ivf16_resq_kernel's tiles; 0: the wide tiles' 128 x 64)
    uint32_t big_tq = 0;        // screened scan, full pass: lists probed by more than ivb::kMinQueries
    uint32_t big_tn = 0;        // queries go to group 3 (ivf16_big_kernel's tiles; 0: off)
    uint32_t* P = nullptr;      // [Q x np] probes with repeats / sentinels replaced by ~0
    uint32_t* qcnt = nullptr;   // [C] queries per list
    uint32_t* qoff = nullptr;   // [C + 1]
    uint32_t* qfill = nullptr;  // [C] fill cursors
    uint32_t* qlist = nullptr;  // [Q x np] (the first qoff[C] are used)
    uint32_t* counts = nullptr; // [2][kGroups][C] tiles per list
    uint32_t* pre = nullptr;    // [2][kGroups][C + 1]
};

__global__ __launch_bounds__(256) void plan_probes_kernel(DevPlan p) {
    const uint32_t q = blockIdx.x;
    const uint32_t* pr = p.probes + int64_t(q) * p.np;
    for (uint32_t i = threadIdx.x; i < p.np; i += 256) {
        const uint32_t l = pr[i];
        bool ok = l < p.C;
        for (uint32_t j = 0; ok && j < i; ++j) ok = pr[j] != l;
        p.P[int64_t(q) * p.np + i] = ok ? l : 0xFFFFFFFFu;
        if (ok) atomicAdd(p.qcnt + l, 1u);
    }
}

// Exclusive prefix of in[0..n) into out[0..n] (out[n] = total), one workgroup of 1024 threads;
// copy (may be null) receives out[0..n) as well.  Workgroup b scans array b of a batch.
__global__ __launch_bounds__(1024) void plan_scan_kernel(const uint32_t* in, uint32_t n, uint32_t* out, uint32_t* copy,
                                                        int64_t in_stride, int64_t out_stride) {
    __shared__ uint32_t part[1024];
    in += int64_t(blockIdx.x) * in_stride;
    out += int64_t(blockIdx.x) * out_stride;
    const uint32_t t = threadIdx.x, per = (n + 1023) / 1024;
    const uint32_t b0 = min(n, t * per), b1 = min(n, b0 + per);
    uint32_t s = 0;
    for (uint32_t i = b0; i < b1; ++i) s += in[i];
    part[t] = s;
    __syncthreads();
    for (uint32_t w = 1; w < 1024; w <<= 1) {  // inclusive Hillis-Steele scan of the partial sums
        const uint32_t v = t >= w ? part[t - w] : 0u;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    uint32_t run = part[t] - s;
    for (uint32_t i = b0; i < b1; ++i) {
        out[i] = run;
        if (copy) copy[i] = run;
        run += in[i];
    }
    if (t == 1023) out[n] = part[1023];
}

__global__ __launch_bounds__(256) void plan_fill_kernel(DevPlan p) {
    const uint64_t total = uint64_t(p.Q) * p.np;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += uint64_t(gridDim.x) * 256) {
        const uint32_t l = p.P[i];
        if (l == 0xFFFFFFFFu) continue;
        const uint32_t pos = atomicAdd(p.qfill + l, 1u);
        p.qlist[pos] = uint32_t(i / p.np);
    }
}

__global__ __launch_bounds__(256) void plan_counts_kernel(DevPlan p) {
    for (uint32_t l = blockIdx.x * 256 + threadIdx.x; l < p.C; l += gridDim.x * 256) {
        const uint32_t nq = p.qcnt[l], n = p.roff[l + 1] - p.roff[l];
        int g;
        uint32_t TQ, TN;
        if (p.screen) {
            g = iv16::group_of(nq);
            TQ = iv16::group_tq(g);
            TN = iv16::TN;
        } else {
            g = (p.small_ok && nq <= kSmallListQueries) ? kSmallGroup : shape_for(nq, n);
            group_tile(g, TQ, TN);
        }
        for (int pass = 0; pass < 2; ++pass) {
            if (p.screen && pass == 1 && p.big_tq && nq > ivb::kMinQueries) {
                g = 3;
                TN = p.big_tn;
                TQ = p.big_tq;
            } else if (p.screen && g == 2 && pass == 1 && p.wide_tn) {
                TN = p.wide_tn;
                TQ = p.wide_tq;
            }
            const uint32_t rows = pass == 0 ? ivf_sample_rows(n) : n;
            const uint32_t tiles = (nq == 0 || rows == 0) ? 0u : ((nq + TQ - 1) / TQ) * ((rows + TN - 1) / TN);
            for (int gi = 0; gi < kGroups; ++gi)
                p.counts[(int64_t(pass) * kGroups + gi) * p.C + l] = gi == g ? tiles : 0u;
        }
    }
}

// Enqueues the device plan (probes -> lists -> tile prefixes).
va_status plan_on_device(va_context* ctx, const DevPlan& p) {
    VA_CHECK_STATUS(fill_u32(ctx, p.qcnt, p.C, 0));
    plan_probes_kernel<<<dim3(p.Q), dim3(256), 0, ctx->stream>>>(p);
    VA_CHECK_LAUNCH(ctx);
    plan_scan_kernel<<<dim3(1), dim3(1024), 0, ctx->stream>>>(p.qcnt, p.C, p.qoff, p.qfill, 0, 0);
    VA_CHECK_LAUNCH(ctx);
    const uint64_t pairs = uint64_t(p.Q) * p.np;
    plan_fill_kernel<<<dim3(uint32_t(std::min<uint64_t>(4096, (pairs + 255) / 256))), dim3(256), 0, ctx->stream>>>(p);
    VA_CHECK_LAUNCH(ctx);
    plan_counts_kernel<<<dim3(std::min<uint32_t>(1024, (p.C + 255) / 256)), dim3(256), 0, ctx->stream>>>(p);
    VA_CHECK_LAUNCH(ctx);
    plan_scan_kernel<<<dim3(2 * kGroups), dim3(1024), 0, ctx->stream>>>(p.counts, p.C, p.pre, nullptr, p.C,
                                                                          int64_t(p.C) + 1);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// Runs one list-major filter pass over the device plan: one persistent launch per tile group
// (each exits at once when its group has no tile).  The groups are independent (they meet only
// in the per-query atomics of the candidate lists), so the 32-query groups run on the context's
// stream and the others on the auxiliary streams: the smaller launches leave most of the chip
// idle on their own, and the 16-query tiles stream their rows from HBM while the larger tiles
// are MFMA-bound.
va_status run_planned_pass(va_context* ctx, const DevPlan& dp, int pass, const float* q, const va_ivf* ivf,
                           const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) {
    VA_CHECK_STATUS(aux_fork(ctx));
    hipStream_t const main_stream = ctx->stream;
    va_status st = VA_OK;
    for (int g = 0; g < kGroups && st == VA_OK; ++g) {
        DistArgs a;
        a.q = q;
        a.qrow = dp.qlist;
        a.q_rows = dp.Q;
        a.ldq = ivf->D;
        a.x = ivf->list_vectors;
        a.ldx = ivf->D;
        a.D = ivf->D;
        a.op = OP_L2SQ;
        a.out = OUT_FILTER;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        a.ids = ivf->ids;
        a.plan.pre = dp.pre + (int64_t(pass) * kGroups + g) * (int64_t(dp.C) + 1);
        a.plan.qoff = dp.qoff;
        a.plan.roff = dp.roff;
        a.plan.C = dp.C;
        a.plan.sample = pass == 0 ? 1u : 0u;
        // shapes 0 (4x1) and 1 (2x2) carry most of the work: the context's stream; the rest
        // spread over the auxiliary streams
        const hipStream_t s = g <= 1 ? main_stream : ctx->aux[(g - 2) % va_context::kAux];
        if (g == kSmallGroup) {
            a.plan.grid = uint32_t(ctx->num_cus) * 4;
            ivf_small_kernel<<<dim3(a.plan.grid), dim3(64 * ivfs::WAVES), 0, s>>>(a);
            if (hipGetLastError() != hipSuccess) st = fail(ctx, VA_ERR_HIP, "ivf_small_kernel launch failed");
        } else {
            a.wq = shape_wq(g);
            a.wn = shape_wn(g);
            // 4x1 and 2x2 run up to four workgroups per CU, the others two
            a.plan.grid = uint32_t(ctx->num_cus) * (g <= 2 ? 4u : 2u);
            ctx->stream = s;  // launch_dist enqueues on the context's stream
            st = launch_dist(ctx, a);
            ctx->stream = main_stream;
        }
    }
    const va_status j = aux_join(ctx);
    return st != VA_OK ? st : j;
}

// One screened pass over the device plan: the three tile groups as persistent launches, the
// narrow tiles on the context's stream and the wide ones on auxiliary streams (they meet only
// in the per-query atomics of the candidate lists).
va_status run_screen_pass(va_context* ctx, const DevPlan& dp, int pass, Ivf16Args a) {
    static_assert(kGroups > 3, "group 3 of the plan: the lists of ivf16_big_kernel");
    a.qrow = dp.qlist;
    a.plan.qoff = dp.qoff;
    a.plan.roff = dp.roff;
    a.plan.C = dp.C;
    a.plan.sample = pass == 0 ? 1u : 0u;
    va_status st = VA_OK;
    // the groups after the first run on aux streams 0 .. kGroupsUsed - 2 (each fork and join is a
    // barrier packet on the context's stream: only the streams used)
    constexpr int kAuxUsed = iv16::kGroupsUsed - 1;
    static_assert(kAuxUsed <= va_context::kAux, "one aux stream per group after the first");
    VA_CHECK_STATUS(aux_fork(ctx, kAuxUsed));
    if (pass == 1 && dp.big_tq) {
        // on the context's stream, ahead of the narrow tiles, while the wide groups start on the
        // auxiliary streams
        using Big = ivb::Big;
        Ivf16Args b = a;
        b.plan.pre = dp.pre + (int64_t(pass) * kGroups + 3) * (int64_t(dp.C) + 1);
        auto kern = &ivf16_big_kernel<ivb::kWaves, ivb::kTQ, ivb::kKC, ivb::kSlots>;
        const uint32_t lds = uint32_t(Big::LDS);
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                int(lds)) != hipSuccess)
            st = fail(ctx, VA_ERR_HIP, "ivf16_big_kernel: %u bytes of LDS refused", lds);
        else
            kern<<<dim3(std::max<uint32_t>(kXcds, uint32_t(ctx->num_cus) / kXcds * kXcds)), dim3(64 * ivb::kWaves), lds,
               ctx->stream>>>(b);
        if (hipGetLastError() != hipSuccess) st = fail(ctx, VA_ERR_HIP, "ivf16_big_kernel launch failed");
    }
    for (int g = 0; g < iv16::kGroupsUsed && st == VA_OK; ++g) {
        a.plan.pre = dp.pre + (int64_t(pass) * kGroups + g) * (int64_t(dp.C) + 1);
        const hipStream_t s = g == 0 ? ctx->stream : ctx->aux[g - 1];
        if (g == 0) {
            ivf16_narrow_kernel<<<dim3(uint32_t(ctx->num_cus) * 2), dim3(256), 0, s>>>(a);
        } else if (g == 1) {
            // two workgroups per CU (two waves per SIMD: one chunk in flight per wave)
            ivf16_wide_kernel<1><<<dim3(uint32_t(ctx->num_cus) * 2), dim3(256), 0, s>>>(a);
        } else if (pass == 1 && dp.wide_tn) {
            // one workgroup per CU (the LDS); the ring depth divides the slots of a sub-tile
            const int nqb = ivr::nqb_for(a.Dp);
            const uint32_t nsl = a.Dp / 64,
                           lds = nqb == 6 ? ivr::Shape<6>::lds_bytes(a.Dp) : ivr::Shape<4>::lds_bytes(a.Dp);
            auto go = [&](auto kern) {
                if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                        int(lds)) != hipSuccess) {
                    st = fail(ctx, VA_ERR_HIP, "ivf16_resq_kernel: %u bytes of LDS refused", lds);
                    return;
                }
                kern<<<dim3(std::max<uint32_t>(kXcds, uint32_t(ctx->num_cus) / kXcds * kXcds)), dim3(512), lds, s>>>(a);
            };
            auto pick = [&](auto NC) {
                constexpr int NQB = decltype(NC)::value;
                if (nsl % 6 == 0) go(&ivf16_resq_kernel<6, NQB>);
                else if (nsl % 4 == 0) go(&ivf16_resq_kernel<4, NQB>);
                else if (nsl % 3 == 0) go(&ivf16_resq_kernel<3, NQB>);
                else if (nsl % 2 == 0) go(&ivf16_resq_kernel<2, NQB>);
                else go(&ivf16_resq_kernel<1, NQB>);
            };
            if (nqb == 6) pick(std::integral_constant<int, 6>());
            else pick(std::integral_constant<int, 4>());
            if (st != VA_OK) break;
        } else {
            ivf16_wide_kernel<2><<<dim3(uint32_t(ctx->num_cus)), dim3(256), 0, s>>>(a);
        }
        if (hipGetLastError() != hipSuccess) st = fail(ctx, VA_ERR_HIP, "screened list scan launch failed");
    }
    const va_status j = aux_join(ctx, kAuxUsed);
    return st != VA_OK ? st : j;
}

// ---- device-side overflow fallback of the list scan -----------------------------------------
// The keys of ivf_small_kernel for one query (supplied by the lanes of column 0) against 32 rows
// xr[b] = row 16b + (lane % 16), b < 2 (nullptr: zeros): v_mfma_f32_16x16x4_f32 over 16-value
// chunks (lane group g = lane / 16 holds values 16c + 4g .. 16c + 4g + 3, MFMA e takes value e
// of each group), ceil(D / 32) * 2 chunks, squared norms as per-group fmaf chains combined by
// xor-16 then xor-32 shuffles, d = qq + xx - 2 dot clamped at 0.  Lane (j, g) gets rows
// 16b + 4g + v in keys[4b + v].  Needs D % 4 == 0 and 16-byte aligned rows.
__device__ inline void small_keys32(const float* qp, const float* xr0, const float* xr1, uint32_t D, int lane,
                                    uint32_t* keys) {
    const int g = lane >> 4;
    const float* xr[2] = {xr0, xr1};
    f32x4s acc[2] = {f32x4s{0.f, 0.f, 0.f, 0.f}, f32x4s{0.f, 0.f, 0.f, 0.f}};
    float xs[2] = {0.f, 0.f}, qsum = 0.f;
    const uint32_t nch = (D + 31) / 32 * 2;
    for (uint32_t c = 0; c < nch; ++c) {
        const uint32_t k = 16 * c + 4 * uint32_t(g);
        const bool kin = k < D;
        const f32x4s zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4s qv = (qp && kin) ? *reinterpret_cast<const f32x4s*>(qp + k) : zero;
        f32x4s rv[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) rv[b] = (xr[b] && kin) ? *reinterpret_cast<const f32x4s*>(xr[b] + k) : zero;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            qsum = fmaf(qv[e], qv[e], qsum);
#pragma unroll
            for (int b = 0; b < 2; ++b) xs[b] = fmaf(rv[b][e], rv[b][e], xs[b]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int b = 0; b < 2; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(rv[b][e], qv[e], acc[b], 0, 0, 0);
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        xs[b] += __shfl_xor(xs[b], 16);
        xs[b] += __shfl_xor(xs[b], 32);
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float xx = __shfl(xs[b], 4 * g + v);  // the norm of row 16b + 4g + v
            float d = qsum + xx - 2.0f * acc[b][v];
            d = (d < 0.0f) ? 0.0f : d;
            keys[4 * b + v] = key_of_float(d);
        }
}

struct FbIvf {
    const float* q;
    const float* x;         // list vectors, CSR order
    const uint32_t* ids;    // row id of every CSR position
    const uint32_t* roff;   // [C + 1]
    const uint32_t* P;      // deduplicated probes [Q x np] (~0: skipped)
    const uint32_t* qcnt;   // queries per list (which kernel scanned the list)
    uint32_t np, D, tmax, small_ok;
};

// Work items (overflowed query slot, probe, 32-row tile of the probed list), one per wave: the
// keys with the arithmetic of the kernel that scanned the list in the full pass, then the
// fallback pass's action for each.
template <bool VEC>
__global__ __launch_bounds__(256) void fb_ivf_pass_kernel(FbIvf v, FbArgs a, int pass) {
    const uint32_t n = fb_count(a);
    if (n == 0) return;  // nothing overflowed: every workgroup leaves at once
    const int lane = threadIdx.x & 63;
    const uint64_t items = uint64_t(n) * v.np * v.tmax;
    const uint32_t nw = gridDim.x * 4;
    for (uint64_t it = blockIdx.x * 4 + (threadIdx.x >> 6); it < items; it += nw) {
        const uint32_t t = uint32_t(it % v.tmax);
        const uint64_t sp = it / v.tmax;
        const uint32_t p = uint32_t(sp % v.np), s = uint32_t(sp / v.np);
        const uint32_t qi = a.rows[s];
        const uint32_t l = v.P[int64_t(qi) * v.np + p];
        if (l == 0xFFFFFFFFu) continue;
        const uint32_t len = v.roff[l + 1] - v.roff[l];
        if (t * 32 >= len) continue;  // (uniform)
        FbSlot sl;
        if (!fb_slot_begin(a, pass, s, sl)) continue;
        const uint32_t base = v.roff[l] + t * 32, rc = min(32u, len - t * 32);
        const float* qrow = v.q + int64_t(qi) * v.D;
        if (v.small_ok && v.qcnt[l] <= kSmallListQueries) {
            const int j = lane & 15, g = lane >> 4;
            uint32_t keys[8];
            small_keys32(j == 0 ? qrow : nullptr, uint32_t(j) < rc ? v.x + int64_t(base + j) * v.D : nullptr,
                         uint32_t(16 + j) < rc ? v.x + int64_t(base + 16 + j) * v.D : nullptr, v.D, lane, keys);
            if (j == 0) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t m = uint32_t(16 * (i >> 2) + 4 * g + (i & 3));
                    if (m < rc) {
                        const uint32_t id = v.ids[base + m];
                        fb_consume(a, pass, sl, (a.skip && a.skip[id]) ? kAbsentKey : keys[i], id);
                    }
                }
            }
        } else {
            const int l32 = lane & 31, hh = lane >> 5;
            uint32_t keys[16];
            f32_block_keys<VEC>(l32 == 0 ? qrow : nullptr,
                                uint32_t(l32) < rc ? v.x + int64_t(base + l32) * v.D : nullptr, v.D, int(OP_L2SQ),
                                lane, keys);
            if (l32 == 0) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t m = uint32_t(8 * (i >> 2) + 4 * hh + (i & 3));
                    if (m < rc) {
                        const uint32_t id = v.ids[base + m];
                        fb_consume(a, pass, sl, (a.skip && a.skip[id]) ? kAbsentKey : keys[i], id);
                    }
                }
            }
        }
        sl.run.flush();
    }
    fb_pass_done(a, pass, n);
}

// ---- exact keys of the screened scan's rerank lists ------------------------------------------
// One wave per (64-row chunk of a query's rerank list, query), persistent and chunk-major.  The
// rows hold CSR positions; lane l scores row 64c + l on the VALU with the per-element sequence of
// the kernel that scans its list in the fp32 list scan (SmallChain: ivf_small_kernel's, for lists
// probed by at most 16 queries; GemmChain: the distance GEMM's, otherwise), so every key equals
// the fp32 list scan's, and the row's id replaces its position.  The rows pass through the wave's
// LDS slot in coalesced 128-byte lines (rows_through_lds).
__global__ __launch_bounds__(256) void ivf_rerank_kernel(const float* __restrict__ q, const float* __restrict__ x,
                                                         const uint32_t* __restrict__ ids,
                                                         const uint32_t* __restrict__ roff, uint32_t C,
                                                         const uint32_t* __restrict__ qcnt, uint32_t D,
                                                         const uint32_t* __restrict__ rr,
                                                         const uint32_t* __restrict__ rcount, uint32_t rcap, uint32_t Q,
                                                         uint32_t* __restrict__ rkey, uint32_t* __restrict__ rid) {
    __shared__ fb_f32x4 slots[4][64 * 8];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nch = (rcap + 63) / 64;
    const uint64_t items = uint64_t(Q) * nch;
    const uint32_t nw = gridDim.x * 4;
    for (uint64_t it = uint64_t(blockIdx.x) * 4 + wave; it < items; it += nw) {
        const uint32_t c = uint32_t(it / Q), qi = uint32_t(it % Q);
        const uint32_t n = min(rcount[qi], rcap);
        if (c * 64 >= n) continue;  // (uniform)
        const uint32_t* rl = rr + int64_t(qi) * rcap + c * 64;
        const uint32_t m = min(64u, n - c * 64);
        uint32_t pos8[8];
        bool rv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t r = uint32_t(8 * i + (lane >> 3));
            rv[i] = r < m;
            pos8[i] = rv[i] ? rl[r] : 0u;
        }
        // this lane's own row: its list decides the arithmetic
        const bool mine = uint32_t(lane) < m;
        const uint32_t pos = mine ? rl[lane] : 0u;
        bool small = false;
        if (mine) {
            uint32_t lo = 0, hi = C - 1;  // the list of pos: the last l with roff[l] <= pos
            while (lo < hi) {
                const uint32_t mid = (lo + hi + 1) >> 1;
                if (roff[mid] <= pos) lo = mid;
                else hi = mid - 1;
            }
            small = qcnt[lo] <= kSmallListQueries;
        }
        GemmChain gc;
        SmallChain sc;
        rows_through_lds(q + int64_t(qi) * D, x, pos8, rv, D, slots[wave],
                         [&](uint32_t j, const fb_f32x4(&xv)[8], const fb_f32x4(&qv)[8]) {
                             if (small) sc.group(xv, qv);
                             else gc.group(xv, qv, j, D);
                         });
        if (mine) {
            rkey[int64_t(qi) * rcap + c * 64 + lane] = small ? sc.key() : gc.key(int(OP_L2SQ));
            rid[int64_t(qi) * rcap + c * 64 + lane] = ids[pos];
        }
    }
}

// Exact top-k, on the device, of the queries listed in fb (their candidates outgrew a list):
// their probed lists walked with the arithmetic of the kernel that scans each list.  The passes
// read only the queries, the lists, the plan and fb's list of queries, and write only fb's
// buffers; the selection writes the listed queries' results.
va_status ivf_fallback_passes(va_context* ctx, const va_ivf* ivf, const float* queries, const DevPlan& dp, uint32_t np,
                              const FbArgs& fb) {
    VA_CHECK_STATUS(fb_init(ctx, fb));
    FbIvf v;
    v.q = queries;
    v.x = ivf->list_vectors;
    v.ids = ivf->ids;
    v.roff = ivf->offsets;
    v.P = dp.P;
    v.qcnt = dp.qcnt;
    v.np = np;
    v.D = ivf->D;
    v.tmax = std::max<uint32_t>(1, (ivf->max_len + 31) / 32);
    v.small_ok = dp.small_ok;
    const bool vec = ivf->D % 4 == 0 && (reinterpret_cast<uintptr_t>(queries) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(ivf->list_vectors) & 15) == 0;
    for (int pass = 0; pass < kFbPasses; ++pass) {
        if (vec)
            fb_ivf_pass_kernel<true><<<dim3(fb.grid), dim3(256), 0, ctx->stream>>>(v, fb, pass);
        else
            fb_ivf_pass_kernel<false><<<dim3(fb.grid), dim3(256), 0, ctx->stream>>>(v, fb, pass);
        VA_CHECK_LAUNCH(ctx);
    }
    return VA_OK;
}
va_status ivf_fallback(va_context* ctx, const va_ivf* ivf, const float* queries, const DevPlan& dp, uint32_t np,
                       const FbArgs& fb, const SelectArgs& base) {
    VA_CHECK_STATUS(ivf_fallback_passes(ctx, ivf, queries, dp, np, fb));
    return fb_select(ctx, fb, base, 32);
}

// A list takes 16-query tiles when few queries probe it (decided once per search from the
// full probe lists, so every pass of the search scans the list with the same kernel).  Needs
// whole, aligned 16-byte groups (D % 4 == 0) and 32-bit byte offsets within a tile.
bool small_tiles_ok(const va_ivf* ivf, const float* q) {
#ifndef VA_IVF_SMALL
#define VA_IVF_SMALL 1
#endif
    return VA_IVF_SMALL && ivf->D % 4 == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(ivf->list_vectors) & 15) == 0 &&
           uint64_t(ivfs::TN) * ivf->D * 4 + 16 <= 0x7FFFFFF0ull;
}
// The lists probed by more than 32 queries take ivf16_resq_kernel in the full pass when the 64
// queries' fp16 rows fit the kernel's LDS share and every query row lies within a 31-bit
// descriptor offset.
bool ivf_resq_applies(const va_context* ctx, uint32_t Q, uint32_t Dp) {
#ifndef VA_IVF_RESQ
#define VA_IVF_RESQ 1
#endif
    return VA_IVF_RESQ && ctx->opt_screen != 1 && Dp <= ivr::DPMAX && uint64_t(Q) * Dp * 2 <= kDmaMaxBytes;
}
// The full pass of the screened scan sends lists probed by more than ivb::kMinQueries queries to
// ivf16_big_kernel (its direct loads address every fp16 query through one descriptor).
bool ivf_big_applies(const va_context* ctx, uint32_t Q, uint32_t Dp) {
#ifndef VA_IVF_BIG
#define VA_IVF_BIG 1
#endif
    return VA_IVF_BIG && ctx->opt_screen != 1 && Q > ivb::kMinQueries && uint64_t(Q) * Dp * 2 <= kDmaMaxBytes &&
           Dp % uint32_t(ivb::kKC) == 0;
}

// The screened list scan serves an index with an fp16 shadow whose lists can take the 16-query
// tiles (their keys are replayed in the rerank), unless VA_OPT_SCREEN turns it off.
bool ivf_screen_applies(const va_context* ctx, const va_ivf* ivf, const float* q) {
    return ctx->opt_screen != 1 && ivf->shadow && ivf->norms && small_tiles_ok(ivf, q);
}

// The IVF list scan with the fp16 screen (the same steps as the flat screened scan, over the
// device plan's list tiles):
//   prep    : queries -> scaled fp16 + {|q|^2, |q|, 2^-scale, c0q};
//   sample  : every pair of each probed list's sample prefix as an interval; tau_q = the k-th
//             smallest upper bound (>= the k-th fp32 key of the probed lists);
//   screen  : the pairs whose interval can reach below tau_q, as intervals;
//   bound   : U_q = k-th smallest upper bound among them (>= the k-th fp32 key again);
//   compact : the rows whose lower bound is <= U_q (they hold the fp32 top-k);
//   rerank  : their exact fp32 keys, with each list's fp32 arithmetic, and their ids;
//   select  : exact (key, id) top-k.  Overflowed queries take the device fallback.
va_status ivf_scan_screened(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t Q,
                            const uint32_t* probes, uint32_t np, uint32_t k, uint32_t* out_idx, float* out_dist,
                            const uint8_t* skip) {
    const uint32_t C = ivf->C, D = ivf->D, Dp = shadow_pitch(D);
    const uint32_t npc = std::min(np, C);
    const uint64_t cap_s = std::max<uint64_t>(1, ivf->top_sample[npc]);
    // The screen's candidates are the fp32 scan's (about 64 x k per query) plus the rows within
    // the bound's width of tau_q, several times as many on long lists (configs[4]: up to ~16,000
    // for k = 10 against ~640 exact); the capacity is the fp32 scan's plus 7x it (at most 16,384
    // of it per 7): queries that outgrow it take the device fallback.
    const uint64_t cap = ivf_screen_cap(ctx->opt_candidate_cap, k, ivf->top_rows[npc]);
    const uint64_t cand = std::max(cap_s, cap);
    const uint64_t rcap = ivf_rerank_cap(k, cap, ivf->top_rows[npc]);
    const uint64_t pairs = uint64_t(Q) * np;
    const uint32_t id_span = uint32_t(std::min<uint64_t>(ivf->id_end, 0xFFFFFFFFull));
    const Bound bnd = make_bound(D);

    Scratch s(ctx);
    const size_t q4 = Scratch::round(uint64_t(Q) * 4);
    const size_t need = q4 * 5 + Scratch::round(uint64_t(Q) * 8) + Scratch::round(256) + Scratch::round(uint64_t(Q) * 16) +
                        Scratch::round(uint64_t(Q) * Dp * 2) + Scratch::round(pairs * 4) * 2 +
                        Scratch::round(uint64_t(C) * 4) * 2 + Scratch::round((uint64_t(C) + 1) * 4) +
                        Scratch::round(uint64_t(2 * kGroups) * C * 4) +
                        Scratch::round(uint64_t(2 * kGroups) * (uint64_t(C) + 1) * 4) +
                        Scratch::round(uint64_t(Q) * cand * 4) * 3 + Scratch::round(uint64_t(Q) * rcap * 4) * 3 +
                        fb_bytes(Q, id_span, k, ivf->N) +
                        (ivf_big_applies(ctx, Q, Dp) ? Scratch::round(pairs * 16) + Scratch::round(pairs * 8) : 0);
    VA_CHECK_STATUS(s.reserve(need));
    uint32_t* thr = s.carve<uint32_t>(Q);
    // list counts: [0, Q) the sample pass's, [Q, 2Q) the full pass's (both cleared by the prep)
    uint32_t* const cnt2 = s.carve<uint32_t>(uint64_t(Q) * 2);
    uint32_t* cnt = cnt2;
    uint32_t* ubound = s.carve<uint32_t>(Q);
    uint32_t* rcount = s.carve<uint32_t>(Q);
    uint32_t* ovf_rows = s.carve<uint32_t>(Q);
    uint32_t* ovf_cnt = s.carve<uint32_t>(64);
    float4* qinfo = s.carve<float4>(Q);
    float* qerr = s.carve<float>(Q);
    _Float16* qh = s.carve<_Float16>(uint64_t(Q) * Dp);
    DevPlan dp;
    dp.probes = probes;
    dp.Q = Q;
    dp.np = np;
    dp.C = C;
    dp.roff = ivf->offsets;
    dp.small_ok = 1;
    dp.screen = 1;
    if (ivf_resq_applies(ctx, Q, Dp)) {
        const bool n6 = ivr::nqb_for(Dp) == 6;
        dp.wide_tn = n6 ? ivr::Shape<6>::TN : ivr::Shape<4>::TN;
        dp.wide_tq = n6 ? uint32_t(ivr::Shape<6>::TQ) : uint32_t(ivr::Shape<4>::TQ);
    }
    if (ivf_big_applies(ctx, Q, Dp)) {
        dp.big_tq = uint32_t(ivb::kTQ);
        dp.big_tn = uint32_t(ivb::Big::TN);
    }
    dp.P = s.carve<uint32_t>(pairs);
    dp.qlist = s.carve<uint32_t>(pairs);
    dp.qcnt = s.carve<uint32_t>(C);
    dp.qfill = s.carve<uint32_t>(C);
    dp.qoff = s.carve<uint32_t>(uint64_t(C) + 1);
    dp.counts = s.carve<uint32_t>(uint64_t(2 * kGroups) * C);
    dp.pre = s.carve<uint32_t>(uint64_t(2 * kGroups) * (uint64_t(C) + 1));
    float* cdot = s.carve<float>(uint64_t(Q) * cand);  // becomes the keys of the upper bounds
    uint32_t* clo = s.carve<uint32_t>(uint64_t(Q) * cand);
    uint32_t* cpos = s.carve<uint32_t>(uint64_t(Q) * cand);
    uint32_t* rr = s.carve<uint32_t>(uint64_t(Q) * rcap);
    uint32_t* rkey = s.carve<uint32_t>(uint64_t(Q) * rcap);
    uint32_t* rid = s.carve<uint32_t>(uint64_t(Q) * rcap);
    FbArgs fb = fb_carve(s, Q, id_span, k, ivf->N);
    fb.n_rows = ovf_cnt;
    fb.rows = ovf_rows;
    fb.skip = skip;
    float4* gpt = dp.big_tq ? s.carve<float4>(pairs) : nullptr;
    float2* gqv = dp.big_tq ? s.carve<float2>(pairs) : nullptr;
    VA_CHECK_STATUS(s.verify(need));
    uint32_t* chi = reinterpret_cast<uint32_t*>(cdot);
    auto bounds = [&](uint64_t cp) -> va_status {
        const uint32_t bx = uint32_t(std::min<uint64_t>(4, (cp + 255) / 256));
        ivf_bound_kernel<<<dim3(bx, Q), dim3(256), 0, ctx->stream>>>(make_bound_v(D), qinfo, qerr, ivf->norms, cdot,
                                                                     cpos, clo, cnt, uint32_t(cp));
        VA_CHECK_LAUNCH(ctx);
        // excluded rows (an index's deletions) become absent keys before every selection
        return mask_list_keys(ctx, chi, clo, cpos, cnt, Q, uint32_t(cp), int64_t(cp), skip, ivf->ids);
    };

    ScanPhaseMarks pm(ctx);
    ctx->last_scan = va_scan_timings{};
    VA_CHECK_STATUS(pm.mark(0));
    // ---- 0. plan and queries --------------------------------------------------------------------
    VA_CHECK_STATUS(plan_on_device(ctx, dp));
    VA_CHECK_STATUS(screen_prepare_queries(ctx, queries, Q, D, qh, qinfo, bnd.c0, qerr, cnt2, 2 * Q, ovf_cnt, 2));
    Ivf16Args a;
    a.qh = qh;
    a.nq = Q;
    a.qinfo = qinfo;
    a.qerr = qerr;
    a.xh = ivf->shadow;
    a.xn = ivf->norms;
    a.Dp = Dp;
    a.bnd = make_bound_v(D);
    a.thr = thr;
    a.cnt = cnt;
    a.cand_dot = cdot;
    a.cand_pos = cpos;
    // ---- 1. sample: tau_q = k-th smallest upper bound of the sampled pairs ----------------------
    VA_CHECK_STATUS(fill_u32(ctx, thr, Q, 0xFFFFFFFFu));
    a.cap = uint32_t(cap_s);
    VA_CHECK_STATUS(run_screen_pass(ctx, dp, 0, a));
    VA_CHECK_STATUS(bounds(cap_s));
    {
        SelectArgs sel;
        sel.keys = chi;
        sel.ids = cpos;
        sel.counts = cnt;
        sel.ld = int64_t(cap_s);
        sel.n = uint32_t(cap_s);
        sel.rows = Q;
        sel.k = k;
        sel.out_kth = thr;
        VA_CHECK_STATUS(launch_select(ctx, sel));
    }
    // ---- 2. screen, 3. U_q (overflowed queries are listed) ---------------------------------------
    cnt = cnt2 + Q;
    a.cnt = cnt;
    a.cap = uint32_t(cap);
    if (dp.big_tq) {
        // the pre-test constants of every plan slot, for the tiles of ivf16_big_kernel
        const uint32_t blocks = uint32_t(std::min<uint64_t>(1024, (pairs + 255) / 256));
        ivf_slot_pretest_kernel<<<dim3(blocks), dim3(256), 0, ctx->stream>>>(make_bound_v(D), dp.qlist, dp.qoff + C,
                                                                            uint32_t(pairs), qinfo, qerr, thr, gpt, gqv);
        VA_CHECK_LAUNCH(ctx);
        a.gpt = gpt;
        a.gqv = gqv;
    }
    VA_CHECK_STATUS(pm.mark(1));
    VA_CHECK_STATUS(run_screen_pass(ctx, dp, 1, a));
    VA_CHECK_STATUS(pm.mark(2));
    VA_CHECK_STATUS(bounds(cap));
    {
        SelectArgs sel;
        sel.keys = chi;
        sel.ids = cpos;
        sel.counts = cnt;
        sel.ld = int64_t(cap);
        sel.n = uint32_t(cap);
        sel.rows = Q;
        sel.k = k;
        sel.out_kth = ubound;
        sel.overflow_count = ovf_cnt;
        sel.overflow_rows = ovf_rows;
        VA_CHECK_STATUS(launch_select(ctx, sel));
    }
    // ---- 4. rerank lists, 5. exact keys ----------------------------------------------------------
    VA_CHECK_STATUS(screen_compact(ctx, cnt, clo, cpos, ubound, uint32_t(cap), Q, rr, rcount, uint32_t(rcap), ovf_cnt,
                                   ovf_rows));
    // ---- 7a. the overflowed queries (listed by the U_q selection and the compaction) take the
    // device fallback's passes on an aux stream, beside the rerank and the selection (a search
    // with none still pays their launches, off the critical path here)
    VA_CHECK_STATUS(aux_fork(ctx, 1));
    AuxJoinGuard fb_join(ctx, 1);
    {
        StreamScope on_aux(ctx, ctx->aux[0]);
        VA_CHECK_STATUS(ivf_fallback_passes(ctx, ivf, queries, dp, np, fb));
    }
    {
        const uint64_t items = uint64_t(Q) * ((rcap + 63) / 64);
        const uint32_t blocks = uint32_t(std::min<uint64_t>(2048, (items + 3) / 4));
        ivf_rerank_kernel<<<dim3(blocks), dim3(256), 0, ctx->stream>>>(queries, ivf->list_vectors, ivf->ids,
                                                                       ivf->offsets, C, dp.qcnt, D, rr, rcount,
                                                                       uint32_t(rcap), Q, rkey, rid);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_STATUS(mask_list_keys(ctx, rkey, nullptr, rid, rcount, Q, uint32_t(rcap), int64_t(rcap), skip));
    }
    // ---- 6. exact (key, id) top-k, 7. overflowed queries -----------------------------------------
    SelectArgs base;
    base.k = k;
    base.out_idx = out_idx;
    base.out_f = out_dist;
    {
        SelectArgs sel = base;
        sel.keys = rkey;
        sel.ids = rid;
        sel.counts = rcount;
        sel.ld = int64_t(rcap);
        sel.n = uint32_t(rcap);
        sel.rows = Q;
        VA_CHECK_STATUS(launch_select(ctx, sel));
    }
    ctx->last_scan.scan_launches = iv16::kGroupsUsed + (dp.big_tq ? 1 : 0);
    ctx->last_scan.candidate_cap = uint32_t(cap);
    ctx->last_scan.screened = 1;
    VA_CHECK_STATUS(pm.count_sum(rcount, Q));
    VA_CHECK_STATUS(pm.count_overflow(ovf_cnt));
    VA_CHECK_STATUS(pm.mark(3));
    // ---- 7b. their exact top-k over the rows the selection wrote
    VA_CHECK_STATUS(fb_join.join());
    VA_CHECK_STATUS(fb_select(ctx, fb, base, 32));
    return pm.finish(true, true);
}
}  // namespace
}  // namespace va

extern "C" {

va_status va_ivf_build(va_context* ctx, const float* centroids, uint32_t num_centroids, const float* x,
                       uint32_t num_vectors, uint32_t dim, va_ivf** out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, centroids && x && out, "va_ivf_build: NULL pointer");
    // IVFSearchConfiguration.validate (Index/Kernels/IVF/IVFKernels.swift:68-82)
    VA_REQUIRE(ctx, num_centroids >= 1, "numCentroids must be at least 1, got %u", num_centroids);
    VA_REQUIRE(ctx, dim >= 1 && dim <= 4096, "dimension must be 1-4096, got %u", dim);
    VA_REQUIRE(ctx, num_vectors >= 1, "va_ivf_build: no vectors");
    va::DeviceGuard g(ctx->device);
    *out = nullptr;
    va_ivf* ivf = new va_ivf();
    ivf->device = ctx->device;
    ivf->C = num_centroids;
    ivf->D = dim;
    ivf->N = num_vectors;
    auto cleanup = [&](va_status st) {
        va_ivf_destroy(ivf);
        return st;
    };
    const uint64_t cbytes = uint64_t(num_centroids) * dim * 4, xbytes = uint64_t(num_vectors) * dim * 4;
    if (hipMalloc(&ivf->centroids, cbytes) != hipSuccess || hipMalloc(&ivf->list_vectors, xbytes) != hipSuccess ||
        hipMalloc(&ivf->ids, uint64_t(num_vectors) * 4) != hipSuccess ||
        hipMalloc(&ivf->offsets, uint64_t(num_centroids + 1) * 4) != hipSuccess) {
        (void)hipGetLastError();
        return cleanup(va::fail(ctx, VA_ERR_OOM, "va_ivf_build: device allocation failed"));
    }
    if (hipMemcpyAsync(ivf->centroids, centroids, cbytes, hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess)
        return cleanup(va::fail(ctx, VA_ERR_HIP, "va_ivf_build: centroid copy failed"));

    // nearest-centroid assignment (fp32 MFMA argmin; ties -> lower id, IVFStructure.findNearestCentroid),
    // then the CSR lists on the device: centroid order, insertion order inside each list
    // (IVFStructure.swift:370-381) from a stable radix sort of the assignments
    uint32_t* assign = nullptr;
    unsigned long long* best = nullptr;
    if (hipMalloc(&assign, uint64_t(num_vectors) * 4) != hipSuccess ||
        hipMalloc(&best, uint64_t(num_vectors) * 8) != hipSuccess) {
        (void)hipGetLastError();
        if (assign) (void)hipFree(assign);
        return cleanup(va::fail(ctx, VA_ERR_OOM, "va_ivf_build: assignment buffers"));
    }
    va_status st = va::nearest_centroids(ctx, x, ivf->centroids, num_vectors, num_centroids, dim, best, assign);
    if (st == VA_OK) st = va::csr_from_assignments(ctx, assign, num_vectors, num_centroids, ivf->ids, ivf->offsets);
    (void)hipFree(best);
    (void)hipFree(assign);
    if (st != VA_OK) return cleanup(st);
    ivf->h_offsets.assign(num_centroids + 1, 0);
    if (hipMemcpy(ivf->h_offsets.data(), ivf->offsets, uint64_t(num_centroids + 1) * 4, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return cleanup(va::fail(ctx, VA_ERR_HIP, "va_ivf_build: offsets read-back failed"));
    ivf->refresh_bounds();
    ivf->id_end = num_vectors;
    va::gather_rows<<<dim3(std::min<uint32_t>(num_vectors, 65536)), dim3(256), 0, ctx->stream>>>(
        x, ivf->ids, num_vectors, dim, ivf->list_vectors);
    if (hipGetLastError() != hipSuccess) return cleanup(va::fail(ctx, VA_ERR_HIP, "va_ivf_build: gather failed"));
    st = va::make_list_shadow(ctx, ivf->list_vectors, num_vectors, dim, &ivf->shadow, &ivf->norms);
    if (st != VA_OK) return cleanup(st);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess)
        return cleanup(va::fail(ctx, VA_ERR_HIP, "va_ivf_build: gather failed"));
    *out = ivf;
    return VA_OK;
}

va_status va_ivf_add(va_context* ctx, va_ivf* ivf, const float* x, uint32_t num_vectors, uint32_t dim,
                     uint32_t first_id) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ivf && x, "va_ivf_add: NULL pointer");
    VA_REQUIRE(ctx, dim == ivf->D, "va_ivf_add: dimension %u, index has %u", dim, ivf->D);
    VA_REQUIRE(ctx, uint64_t(ivf->N) + num_vectors < 0xFFFFFFFFull, "va_ivf_add: too many vectors");
    if (num_vectors == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    const uint32_t C = ivf->C, D = ivf->D, No = ivf->N, n = num_vectors, Nn = No + n;
    struct Bufs {
        void* p[9] = {};
        ~Bufs() {
            for (void* q : p)
                if (q) (void)hipFree(q);
        }
    } b;
    auto get = [&](int i, size_t bytes) -> bool {
        if (hipMalloc(&b.p[i], std::max<size_t>(bytes, 256)) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        return true;
    };
    if (!get(0, size_t(n) * 4) || !get(1, size_t(n) * 8) || !get(2, size_t(n) * 4) || !get(3, size_t(C + 1) * 4) ||
        !get(4, size_t(Nn) * D * 4) || !get(5, size_t(Nn) * 4) || !get(6, size_t(C + 1) * 4))
        return va::fail(ctx, VA_ERR_OOM, "va_ivf_add: device allocation failed");
    uint32_t* assign = static_cast<uint32_t*>(b.p[0]);
    auto* best = static_cast<unsigned long long*>(b.p[1]);
    uint32_t* order = static_cast<uint32_t*>(b.p[2]);  // new rows grouped by list, row order inside
    uint32_t* pre = static_cast<uint32_t*>(b.p[3]);    // new rows in lists before c
    float* vecs = static_cast<float*>(b.p[4]);
    uint32_t* ids = static_cast<uint32_t*>(b.p[5]);
    uint32_t* offs = static_cast<uint32_t*>(b.p[6]);
    // IVFStructure.assignToCluster (Index/Internal/IVFStructure.swift:280-287) for every new row:
    // appended to its nearest list after the rows already there
    VA_CHECK_STATUS(va::nearest_centroids(ctx, x, ivf->centroids, n, C, D, best, assign));
    VA_CHECK_STATUS(va::csr_from_assignments(ctx, assign, n, C, order, pre));
    va::ivf_merge_old<<<dim3(std::min<uint32_t>(std::max<uint32_t>(No, 1), 65536)), dim3(256), 0, ctx->stream>>>(
        ivf->list_vectors, ivf->ids, ivf->offsets, pre, C, No, D, vecs, ids);
    VA_CHECK_LAUNCH(ctx);
    va::ivf_place_new<<<dim3(std::min<uint32_t>(n, 65536)), dim3(256), 0, ctx->stream>>>(
        x, order, pre, ivf->offsets, C, n, D, first_id, vecs, ids);
    VA_CHECK_LAUNCH(ctx);
    va::ivf_new_offsets<<<dim3((C + 1 + 255) / 256), dim3(256), 0, ctx->stream>>>(ivf->offsets, pre, C, offs);
    VA_CHECK_LAUNCH(ctx);
    _Float16* sh = nullptr;
    float2* nr = nullptr;
    {
        const va_status st = va::make_list_shadow(ctx, vecs, Nn, D, &sh, &nr);
        b.p[7] = sh;
        b.p[8] = nr;
        VA_CHECK_STATUS(st);
    }
    std::vector<uint32_t> h(C + 1);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(h.data(), offs, size_t(C + 1) * 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // the new arrays replace the index's; the old ones are freed with the scratch
    b.p[4] = ivf->list_vectors;
    b.p[5] = ivf->ids;
    b.p[6] = ivf->offsets;
    b.p[7] = ivf->shadow;
    b.p[8] = ivf->norms;
    ivf->list_vectors = vecs;
    ivf->ids = ids;
    ivf->offsets = offs;
    ivf->shadow = sh;
    ivf->norms = nr;
    ivf->h_offsets = std::move(h);
    ivf->refresh_bounds();
    ivf->id_end = std::max<uint64_t>(ivf->id_end, uint64_t(first_id) + n);
    ivf->N = Nn;
    return VA_OK;
}

va_status va_ivf_destroy(va_ivf* ivf) {
    if (!ivf) return VA_ERR_INVALID_ARG;
    va::DeviceGuard g(ivf->device);
    (void)hipDeviceSynchronize();
    if (ivf->centroids) (void)hipFree(ivf->centroids);
    if (ivf->list_vectors) (void)hipFree(ivf->list_vectors);
    if (ivf->ids) (void)hipFree(ivf->ids);
    if (ivf->offsets) (void)hipFree(ivf->offsets);
    if (ivf->shadow) (void)hipFree(ivf->shadow);
    if (ivf->norms) (void)hipFree(ivf->norms);
    if (ivf->probe_buf) (void)hipFree(ivf->probe_buf);
    delete ivf;
    return VA_OK;
}

va_status va_ivf_get_lists(va_context* ctx, const va_ivf* ivf, uint32_t* host_offsets, uint32_t* host_ids) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ivf && host_offsets && host_ids, "va_ivf_get_lists: NULL pointer");
    va::DeviceGuard g(ctx->device);
    std::copy(ivf->h_offsets.begin(), ivf->h_offsets.end(), host_offsets);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(host_ids, ivf->ids, uint64_t(ivf->N) * 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VA_OK;
}

va_status va_ivf_probe(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                       uint32_t nprobe, uint32_t* probes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ivf && queries && probes, "va_ivf_probe: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "Queries cannot be empty");
    VA_REQUIRE(ctx, nprobe >= 1 && nprobe <= VA_MAX_K, "nprobe must be in [1, %u], got %u", VA_MAX_K, nprobe);
    va::DeviceGuard g(ctx->device);
    va::F32Keys kp;
    kp.ctx = ctx;
    kp.q = queries;
    kp.x = ivf->centroids;
    kp.Q = num_queries;
    kp.N = ivf->C;
    kp.D = ivf->D;
    va::ScanOutputs o;
    o.idx = probes;
    return va::exact_topk_scan(ctx, kp, num_queries, ivf->C, nprobe, o);
}

}  // extern "C"

namespace va {

// va_ivf_scan with an exclusion mask: rows whose skip byte (indexed by row id) is set never take
// a place in a result or hold a threshold down (nullptr: none excluded).
va_status ivf_scan_masked(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                          const uint32_t* probes, uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist,
                          const uint8_t* skip) {
    using va::Scratch;
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ivf && queries && probes && out_idx, "va_ivf_scan: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "Queries cannot be empty");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    VA_REQUIRE(ctx, nprobe >= 1, "nprobe must be at least 1, got %u", nprobe);
    va::DeviceGuard g(ctx->device);
    if (va::ivf_screen_applies(ctx, ivf, queries))
        return va::ivf_scan_screened(ctx, ivf, queries, num_queries, probes, nprobe, k, out_idx, out_dist, skip);
    const uint32_t Q = num_queries, C = ivf->C, np = nprobe;

    // ---- sizes from the list lengths alone (nothing is read back) --------------------------------
    // A query's lists are at most its np longest: its threshold sample never outgrows cap_s (the
    // sample pass cannot overflow); the full pass keeps about 64 x k candidates per query, and
    // queries that outgrow cap are finished by the device fallback.
    const uint32_t npc = std::min(np, C);
    const uint64_t cap_s = std::max<uint64_t>(1, ivf->top_sample[npc]);
    const uint64_t cap = va::ivf_fp32_cap(ctx->opt_candidate_cap, k, ivf->top_rows[npc]);
    const uint64_t cand = std::max(cap_s, cap);
    const uint64_t pairs = uint64_t(Q) * np;
    // the fallback's tie-id histogram covers the ids of the index
    const uint32_t id_span = uint32_t(std::min<uint64_t>(ivf->id_end, 0xFFFFFFFFull));

    Scratch s(ctx);
    const size_t need = Scratch::round(uint64_t(Q) * 4) * 3 + Scratch::round(256) + Scratch::round(pairs * 4) * 2 +
                        Scratch::round(uint64_t(C) * 4) * 2 + Scratch::round((uint64_t(C) + 1) * 4) +
                        Scratch::round(uint64_t(2 * va::kGroups) * C * 4) +
                        Scratch::round(uint64_t(2 * va::kGroups) * (uint64_t(C) + 1) * 4) +
                        Scratch::round(uint64_t(Q) * cand * 4) * 2 + va::fb_bytes(Q, id_span, k, ivf->N);
    VA_CHECK_STATUS(s.reserve(need));
    uint32_t* thr = s.carve<uint32_t>(Q);
    uint32_t* cnt = s.carve<uint32_t>(Q);
    uint32_t* ovf_rows = s.carve<uint32_t>(Q);
    uint32_t* ovf_cnt = s.carve<uint32_t>(64);
    va::DevPlan dp;
    dp.probes = probes;
    dp.Q = Q;
    dp.np = np;
    dp.C = C;
    dp.roff = ivf->offsets;
    dp.small_ok = va::small_tiles_ok(ivf, queries) ? 1u : 0u;
    dp.P = s.carve<uint32_t>(pairs);
    dp.qlist = s.carve<uint32_t>(pairs);
    dp.qcnt = s.carve<uint32_t>(C);
    dp.qfill = s.carve<uint32_t>(C);
    dp.qoff = s.carve<uint32_t>(uint64_t(C) + 1);
    dp.counts = s.carve<uint32_t>(uint64_t(2 * va::kGroups) * C);
    dp.pre = s.carve<uint32_t>(uint64_t(2 * va::kGroups) * (uint64_t(C) + 1));
    uint32_t* ckey = s.carve<uint32_t>(uint64_t(Q) * cand);
    uint32_t* cid = s.carve<uint32_t>(uint64_t(Q) * cand);
    va::FbArgs fb = va::fb_carve(s, Q, id_span, k, ivf->N);
    fb.n_rows = ovf_cnt;
    fb.rows = ovf_rows;
    fb.skip = skip;
    VA_CHECK_STATUS(s.verify(need));

    va::ScanPhaseMarks pm(ctx);
    ctx->last_scan = va_scan_timings{};
    VA_CHECK_STATUS(pm.mark(0));
    // ---- 0. plan: the queries of every probed list, tile prefixes per group and pass ------------
    VA_CHECK_STATUS(va::plan_on_device(ctx, dp));
    // ---- 1. sample pass: every sampled candidate, then tau = k-th smallest ----------------------
    VA_CHECK_STATUS(va::fill_u32(ctx, thr, Q, 0xFFFFFFFFu));
    VA_CHECK_STATUS(va::fill_u32(ctx, cnt, Q, 0));
    VA_CHECK_STATUS(va::run_planned_pass(ctx, dp, 0, queries, ivf, thr, cnt, ckey, cid, uint32_t(cap_s)));
    VA_CHECK_STATUS(va::mask_list_keys(ctx, ckey, nullptr, cid, cnt, Q, uint32_t(cap_s), int64_t(cap_s), skip));
    {
        va::SelectArgs a;
        a.keys = ckey;
        a.ids = cid;
        a.counts = cnt;
        a.ld = int64_t(cap_s);
        a.n = uint32_t(cap_s);
        a.rows = Q;
        a.k = k;
        a.out_kth = thr;
        VA_CHECK_STATUS(va::launch_select(ctx, a));
    }
    // ---- 2. full pass with the thresholds, 3. exact selection -----------------------------------
    VA_CHECK_STATUS(va::fill_u32(ctx, cnt, Q, 0));
    VA_CHECK_STATUS(va::fill_u32(ctx, ovf_cnt, 1, 0));
    VA_CHECK_STATUS(pm.mark(1));
    VA_CHECK_STATUS(va::run_planned_pass(ctx, dp, 1, queries, ivf, thr, cnt, ckey, cid, uint32_t(cap)));
    VA_CHECK_STATUS(pm.mark(2));
    VA_CHECK_STATUS(va::mask_list_keys(ctx, ckey, nullptr, cid, cnt, Q, uint32_t(cap), int64_t(cap), skip));
    va::SelectArgs base;
    base.k = k;
    base.out_idx = out_idx;
    base.out_f = out_dist;
    {
        va::SelectArgs a = base;
        a.keys = ckey;
        a.ids = cid;
        a.counts = cnt;
        a.ld = int64_t(cap);
        a.n = uint32_t(cap);
        a.rows = Q;
        a.overflow_count = ovf_cnt;
        a.overflow_rows = ovf_rows;
        VA_CHECK_STATUS(va::launch_select(ctx, a));
    }
    ctx->last_scan.scan_launches = va::kGroups;
    ctx->last_scan.candidate_cap = uint32_t(cap);
    VA_CHECK_STATUS(pm.count_overflow(ovf_cnt));
    VA_CHECK_STATUS(pm.mark(3));
    // ---- 4. queries whose candidates outgrew cap: exact top-k on the device ----------------------
    VA_CHECK_STATUS(va::ivf_fallback(ctx, ivf, queries, dp, np, fb, base));
    return pm.finish(true, true);
}

// va_ivf_search with an exclusion mask (see ivf_scan_masked)
va_status ivf_search_masked(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                            uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist, const uint8_t* skip) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ivf && queries && out_idx, "va_ivf_search: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "Queries cannot be empty");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    // IVFSearchConfiguration clamps nprobe to numCentroids (IVFKernels.swift:62)
    VA_REQUIRE(ctx, nprobe >= 1, "nprobe must be at least 1, got %u", nprobe);
    nprobe = std::min(nprobe, ivf->C);
    va::DeviceGuard g(ctx->device);
    va_ivf* m = const_cast<va_ivf*>(ivf);
    const size_t need = uint64_t(num_queries) * nprobe * 4;
    if (m->probe_cap < need) {
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (m->probe_buf) (void)hipFree(m->probe_buf);
        m->probe_buf = nullptr;
        m->probe_cap = 0;
        VA_CHECK_HIP(ctx, hipMalloc(&m->probe_buf, need));
        m->probe_cap = need;
    }
    VA_CHECK_STATUS(va_ivf_probe(ctx, ivf, queries, num_queries, nprobe, m->probe_buf));
    return ivf_scan_masked(ctx, ivf, queries, num_queries, m->probe_buf, nprobe, k, out_idx, out_dist, skip);
}

uint32_t ivf_num_lists(const va_ivf* ivf) { return ivf->C; }

}  // namespace va

extern "C" {

va_status va_ivf_scan(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                      const uint32_t* probes, uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist) {
    return va::ivf_scan_masked(ctx, ivf, queries, num_queries, probes, nprobe, k, out_idx, out_dist, nullptr);
}

va_status va_ivf_search(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                        uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist) {
    return va::ivf_search_masked(ctx, ivf, queries, num_queries, nprobe, k, out_idx, out_dist, nullptr);
}

}  // extern "C"
