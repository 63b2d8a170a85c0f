// va_ivf.hip — IVF-Flat (L2^2) build, coarse probe and list-major scan.
//
// Build (IVFStructure.assignToCluster / prepareGPUStructure, Index/Internal/IVFStructure.swift:
// 280-307, 347-467): nearest-centroid assignment on the fp32 MFMA distance kernel (k = 1,
// ties to the lower centroid id), CSR offsets and row ids built on the host in centroid order
// with insertion order inside each list (as the reference does), and the list vectors gathered
// into CSR order by a device copy kernel (the reference memcpy-gathers on the host).
//
// Search (IVFSearchPipeline.search, Index/Kernels/IVF/IVFSearchPipeline.swift:197-568):
//   probe : the nprobe nearest centroids by (L2^2, id) through the exact top-k scan;
//   scan  : list-major — every (list, block of the queries that probe it, block of its rows)
//           is one MFMA tile of the distance kernel, so a list's rows are read once per block
//           of up to 128 probing queries instead of once per query (ivf_list_search,
//           Metal/Shaders/IVFListSearch.metal:199-339, streams each query's lists separately);
//   top-k : a strided in-list sample (every 64th row of each probed list) gives each query an
//           upper bound tau_q of its k-th distance; the full scan appends only keys <= tau_q;
//           exact (L2^2, row id) selection follows.  Queries whose candidate list overflows
//           are rescanned with room for every candidate they have.
// The reference's per-thread heap (K_PRIVATE = 8) is only exact for k <= 8; this is exact
// for every k <= VA_MAX_K.
#include <algorithm>
#include <vector>

#include "va_fallback.hpp"
#include "va_internal.hpp"

struct va_ivf {
    int device = 0;
    uint32_t C = 0, D = 0, N = 0;
    float* centroids = nullptr;     // [C x D]
    float* list_vectors = nullptr;  // [N x D] in CSR order
    uint32_t* ids = nullptr;        // [N] original row id of every CSR position
    uint32_t* offsets = nullptr;    // [C + 1]
    std::vector<uint32_t> h_offsets;
    uint32_t* probe_buf = nullptr;  // probes of va_ivf_search
    size_t probe_cap = 0;
};

namespace va {
namespace {

// Threshold sample: a prefix of every probed list (rows are in insertion order, so a prefix is
// an unbiased subset) of at least 1/kSampleRate of its rows and at least kSampleMin rows.
// Every list is sampled at rate >= 1/kSampleRate, so a query's candidate count stays within
// about kSampleRate x k; the floor keeps small lists' sample tiles full.
constexpr uint32_t kSampleRate = 64;
constexpr uint32_t kSampleMin = 128;
inline uint32_t sample_rows(uint32_t n) {
    return std::min(n, std::max((n + kSampleRate - 1) / kSampleRate, kSampleMin));
}

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

__global__ __launch_bounds__(256) void gather_queries(const float* __restrict__ q, const uint32_t* __restrict__ rows,
                                                      uint32_t R, uint32_t D, float* __restrict__ out) {
    for (uint32_t r = blockIdx.x; r < R; r += gridDim.x) {
        const float* src = q + uint64_t(rows[r]) * D;
        for (uint32_t d = threadIdx.x; d < D; d += 256) out[uint64_t(r) * D + d] = src[d];
    }
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

__global__ __launch_bounds__(256) void ivf_small_kernel(DistArgs a) {
    using namespace ivfs;
    __shared__ __attribute__((aligned(16))) float xnorm[WAVES][TN];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const uint32_t tile = blockIdx.x * WAVES + uint32_t(wave);
    if (tile >= a.ntiles) return;  // whole wave; the waves never synchronise
    const uint32_t qs = a.tiles[4 * tile], qc = a.tiles[4 * tile + 1];
    const uint32_t rs = a.tiles[4 * tile + 2], rc = a.tiles[4 * tile + 3];
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

// Tile descriptors {qs, qc, rs, rc} of one list-major pass, grouped by tile shape.  A tile of
// wq x wn waves covers 32*wq queries x 128*wn rows.  A list with nq probing queries and n
// rows gets the shape with the least estimated time: tiles x waves x the measured cost of
// one wave tile (32 x 128) in that shape on MI355X (shapes with more waves share their LDS
// stages across more MFMA work and run more workgroups per CU, except 1 x 4, whose 87 KB of
// LDS leaves one workgroup per CU).  The one- and two-wave shapes keep lists with few
// queries or few rows from paying for a 4-wave tile.
struct TilePlan {
    static constexpr int NS = 5;
    static constexpr int WQ[NS] = {4, 2, 2, 1, 1};
    static constexpr int WN[NS] = {1, 2, 1, 1, 4};
    static constexpr uint32_t COST[NS] = {100, 120, 135, 175, 195};  // per wave tile, relative
    std::vector<uint32_t> t[NS];
    std::vector<uint32_t> small;  // 16-query tiles (ivf_small_kernel)
    // every group back to back, as uploaded by run_pass (kept with the plan, which outlives
    // the asynchronous copy)
    mutable std::vector<uint32_t> packed;
    static int shape_for(uint32_t nq, uint32_t nrows) {
        int best = 0;
        uint64_t best_cost = ~0ull;
        for (int i = 0; i < NS; ++i) {
            const uint64_t cost = uint64_t((nq + 32 * WQ[i] - 1) / (32 * WQ[i])) *
                                  ((nrows + 128 * WN[i] - 1) / (128 * WN[i])) * (WQ[i] * WN[i]) * COST[i];
            if (cost < best_cost) {
                best = i;
                best_cost = cost;
            }
        }
        return best;
    }
    // rows of a list: positions off + j, j < nrows; small_list: the list takes 16-query tiles
    void add(uint32_t lq_start, uint32_t nq, uint32_t off, uint32_t nrows, bool small_list = false) {
        if (nq == 0 || nrows == 0) return;
        if (small_list) {
            for (uint32_t qb = 0; qb < nq; qb += ivfs::TQ)
                for (uint32_t r = 0; r < nrows; r += ivfs::TN) {
                    small.push_back(lq_start + qb);
                    small.push_back(std::min(ivfs::TQ, nq - qb));
                    small.push_back(off + r);
                    small.push_back(std::min(ivfs::TN, nrows - r));
                }
            return;
        }
        const int sh = shape_for(nq, nrows);
        const uint32_t TQ = dist_tile_queries(WQ[sh]), TN = dist_tile_rows(WN[sh]);
        auto& v = t[sh];
        for (uint32_t qb = 0; qb < nq; qb += TQ)
            for (uint32_t r = 0; r < nrows; r += TN) {
                v.push_back(lq_start + qb);
                v.push_back(std::min(TQ, nq - qb));
                v.push_back(off + r);
                v.push_back(std::min(TN, nrows - r));
            }
    }
    size_t words() const {
        size_t w = small.size();
        for (const auto& v : t) w += v.size();
        return w;
    }
};

// Runs one list-major filter pass; tiles hold "rs" as an index into the strided row space
// (the kernel multiplies j by rstride; rs must already be the first position).
va_status run_pass(va_context* ctx, const TilePlan& plan, uint32_t* dev_tiles, const float* q, uint32_t q_rows,
                   const uint32_t* lq, const va_ivf* ivf, uint32_t rstride, const uint32_t* thr, uint32_t* cnt,
                   uint32_t* ckey, uint32_t* cid, uint32_t cap) {
    // One upload of every group's tile descriptors, then one launch per group.  The groups are
    // independent (they meet only in the per-query atomics of the candidate lists), so the
    // largest runs on the context's stream and the others on the auxiliary streams: the
    // smaller launches leave most of the chip idle on their own, and the 16-query tiles stream
    // their rows from HBM while the larger tiles are MFMA-bound.
    constexpr int NG = TilePlan::NS + 1;  // group NS: the 16-query tiles
    const std::vector<uint32_t>* groups[NG];
    for (int sh = 0; sh < TilePlan::NS; ++sh) groups[sh] = &plan.t[sh];
    groups[TilePlan::NS] = &plan.small;
    std::vector<uint32_t>& all = plan.packed;
    all.clear();
    all.reserve(plan.words());
    size_t goff[NG];
    int ngroups = 0, biggest = -1;
    for (int gi = 0; gi < NG; ++gi) {
        goff[gi] = all.size();
        all.insert(all.end(), groups[gi]->begin(), groups[gi]->end());
        if (groups[gi]->empty()) continue;
        ++ngroups;
        if (biggest < 0 || groups[gi]->size() > groups[biggest]->size()) biggest = gi;
    }
    if (ngroups == 0) return VA_OK;
    VA_CHECK_HIP(ctx, hipMemcpyAsync(dev_tiles, all.data(), all.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    if (ngroups > 1) VA_CHECK_STATUS(aux_fork(ctx));
    hipStream_t const main_stream = ctx->stream;
    int next_aux = 0;
    va_status st = VA_OK;
    for (int gi = 0; gi < NG && st == VA_OK; ++gi) {
        const auto& v = *groups[gi];
        if (v.empty()) continue;
        hipStream_t s = main_stream;
        if (gi != biggest) s = ctx->aux[next_aux++ % va_context::kAux];
        DistArgs a;
        a.q = q;
        a.qrow = lq;
        a.q_rows = q_rows;
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
        a.tiles = dev_tiles + goff[gi];
        a.ntiles = uint32_t(v.size() / 4);
        a.rstride = rstride;
        a.ids = ivf->ids;
        if (gi == TilePlan::NS) {
            const uint32_t blocks = (a.ntiles + ivfs::WAVES - 1) / ivfs::WAVES;
            ivf_small_kernel<<<dim3(blocks), dim3(64 * ivfs::WAVES), 0, s>>>(a);
            if (hipGetLastError() != hipSuccess) st = fail(ctx, VA_ERR_HIP, "ivf_small_kernel launch failed");
        } else {
            a.wq = TilePlan::WQ[gi];
            a.wn = TilePlan::WN[gi];
            ctx->stream = s;  // launch_dist enqueues on the context's stream
            st = launch_dist(ctx, a);
            ctx->stream = main_stream;
        }
    }
    if (ngroups > 1) {
        const va_status j = aux_join(ctx);
        if (st == VA_OK) st = j;
    }
    return st;
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
constexpr uint32_t kSmallListQueries = 16;

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
    va::gather_rows<<<dim3(std::min<uint32_t>(num_vectors, 65536)), dim3(256), 0, ctx->stream>>>(
        x, ivf->ids, num_vectors, dim, ivf->list_vectors);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess)
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
        void* p[7] = {};
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
    std::vector<uint32_t> h(C + 1);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(h.data(), offs, size_t(C + 1) * 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // the new arrays replace the index's; the old ones are freed with the scratch
    b.p[4] = ivf->list_vectors;
    b.p[5] = ivf->ids;
    b.p[6] = ivf->offsets;
    ivf->list_vectors = vecs;
    ivf->ids = ids;
    ivf->offsets = offs;
    ivf->h_offsets = std::move(h);
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

va_status va_ivf_scan(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                      const uint32_t* probes, uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist) {
    using va::Scratch;
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ivf && queries && probes && out_idx, "va_ivf_scan: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "Queries cannot be empty");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    VA_REQUIRE(ctx, nprobe >= 1, "nprobe must be at least 1, got %u", nprobe);
    va::DeviceGuard g(ctx->device);
    const uint32_t Q = num_queries, C = ivf->C;
    const auto& off = ivf->h_offsets;

    // ---- host plan: the queries probing every list, per-query candidate totals ------------------
    std::vector<uint32_t> P(uint64_t(Q) * nprobe);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(P.data(), probes, P.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    std::vector<uint32_t> lq_off(C + 1, 0), seen(C, 0xFFFFFFFFu);
    std::vector<uint64_t> total(Q, 0), sampled(Q, 0);
    for (uint32_t q = 0; q < Q; ++q)
        for (uint32_t p = 0; p < nprobe; ++p) {
            uint32_t& l = P[uint64_t(q) * nprobe + p];
            // sentinel / out-of-range probes are skipped (IVFListSearch.metal:249-251); a list
            // probed twice by one query is scanned once
            if (l >= C || seen[l] == q) {
                l = 0xFFFFFFFFu;
                continue;
            }
            seen[l] = q;
            lq_off[l + 1]++;
            const uint32_t n = off[l + 1] - off[l];
            total[q] += n;
            sampled[q] += va::sample_rows(n);
        }
    for (uint32_t l = 0; l < C; ++l) lq_off[l + 1] += lq_off[l];
    std::vector<uint32_t> lq(lq_off[C]), fillp(lq_off.begin(), lq_off.end() - 1);
    for (uint32_t q = 0; q < Q; ++q)
        for (uint32_t p = 0; p < nprobe; ++p) {
            const uint32_t l = P[uint64_t(q) * nprobe + p];
            if (l < C) lq[fillp[l]++] = q;
        }
    va::TilePlan sample_plan, main_plan;
    const bool small_ok = va::small_tiles_ok(ivf, queries);
    auto small_list = [&](uint32_t l) { return small_ok && lq_off[l + 1] - lq_off[l] <= va::kSmallListQueries; };
    for (uint32_t l = 0; l < C; ++l) {
        const uint32_t nq = lq_off[l + 1] - lq_off[l];
        const uint32_t n = off[l + 1] - off[l];
        main_plan.add(lq_off[l], nq, off[l], n, small_list(l));
    }
    for (uint32_t l = 0; l < C; ++l)
        sample_plan.add(lq_off[l], lq_off[l + 1] - lq_off[l], off[l], va::sample_rows(off[l + 1] - off[l]),
                        small_list(l));
    const uint64_t cap_s = std::max<uint64_t>(1, *std::max_element(sampled.begin(), sampled.end()));
    const uint64_t max_total = std::max<uint64_t>(1, *std::max_element(total.begin(), total.end()));
    // every list is sampled at rate >= 1/kSampleRate: a query's candidates stay near
    // kSampleRate x k; queries that still outgrow the list take the exact rescan below
    uint64_t cap = ctx->opt_candidate_cap ? ctx->opt_candidate_cap
                                          : std::max<uint64_t>(3ull * k, uint64_t(k) + 32) * va::kSampleRate + 1024;
    cap = std::min(cap, max_total);
    const uint64_t cand = std::max(cap_s, cap);

    Scratch s(ctx);
    const size_t tile_words = std::max(sample_plan.words(), main_plan.words());
    const size_t need = Scratch::round(uint64_t(Q) * 4) * 3 + Scratch::round(256) + Scratch::round(lq.size() * 4 + 4) +
                        Scratch::round(tile_words * 4 + 4) + Scratch::round(uint64_t(Q) * cand * 4) * 2;
    VA_CHECK_STATUS(s.reserve(need));
    uint32_t* thr = s.carve<uint32_t>(Q);
    uint32_t* cnt = s.carve<uint32_t>(Q);
    uint32_t* ovf_rows = s.carve<uint32_t>(Q);
    uint32_t* ovf_cnt = s.carve<uint32_t>(64);
    uint32_t* d_lq = s.carve<uint32_t>(lq.size() + 1);
    uint32_t* d_tiles = s.carve<uint32_t>(tile_words + 1);
    uint32_t* ckey = s.carve<uint32_t>(uint64_t(Q) * cand);
    uint32_t* cid = s.carve<uint32_t>(uint64_t(Q) * cand);
    if (!lq.empty())
        VA_CHECK_HIP(ctx, hipMemcpyAsync(d_lq, lq.data(), lq.size() * 4, hipMemcpyHostToDevice, ctx->stream));

    // ---- 1. sample pass: every sampled candidate, then tau = k-th smallest ----------------------
    VA_CHECK_STATUS(va::fill_u32(ctx, thr, Q, 0xFFFFFFFFu));
    VA_CHECK_STATUS(va::fill_u32(ctx, cnt, Q, 0));
    VA_CHECK_STATUS(va::run_pass(ctx, sample_plan, d_tiles, queries, Q, d_lq, ivf, 1, thr, cnt, ckey, cid,
                                 uint32_t(cap_s)));
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
    VA_CHECK_STATUS(va::run_pass(ctx, main_plan, d_tiles, queries, Q, d_lq, ivf, 1, thr, cnt, ckey, cid, uint32_t(cap)));
    {
        va::SelectArgs a;
        a.keys = ckey;
        a.ids = cid;
        a.counts = cnt;
        a.ld = int64_t(cap);
        a.n = uint32_t(cap);
        a.rows = Q;
        a.k = k;
        a.out_idx = out_idx;
        a.out_f = out_dist;
        a.overflow_count = ovf_cnt;
        a.overflow_rows = ovf_rows;
        VA_CHECK_STATUS(va::launch_select(ctx, a));
    }
    VA_CHECK_HIP(ctx, hipMemcpyAsync(ctx->host_word, ovf_cnt, 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const uint32_t n_ovf = ctx->host_word[0];
    if (n_ovf == 0) return VA_OK;

    // ---- 4. overflowed queries: rescan with room for all of their candidates ---------------------
    std::vector<uint32_t> rows(n_ovf), h_thr(Q);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(rows.data(), ovf_rows, uint64_t(n_ovf) * 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipMemcpyAsync(h_thr.data(), thr, uint64_t(Q) * 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    std::sort(rows.begin(), rows.end());
    std::vector<uint32_t> compact(Q, 0xFFFFFFFFu), c_thr(n_ovf);
    uint64_t cap2 = 1;
    for (uint32_t i = 0; i < n_ovf; ++i) {
        compact[rows[i]] = i;
        c_thr[i] = h_thr[rows[i]];
        cap2 = std::max<uint64_t>(cap2, total[rows[i]]);
    }
    std::vector<uint32_t> lq2_off(C + 1, 0), lq2;
    for (uint32_t l = 0; l < C; ++l) {
        for (uint32_t e = lq_off[l]; e < lq_off[l + 1]; ++e)
            if (compact[lq[e]] != 0xFFFFFFFFu) lq2.push_back(compact[lq[e]]);
        lq2_off[l + 1] = uint32_t(lq2.size());
    }
    va::TilePlan plan2;
    for (uint32_t l = 0; l < C; ++l)
        plan2.add(lq2_off[l], lq2_off[l + 1] - lq2_off[l], off[l], off[l + 1] - off[l], small_list(l));
    Scratch f(ctx);
    const size_t need2 = Scratch::round(uint64_t(n_ovf) * ivf->D * 4) + Scratch::round(uint64_t(n_ovf) * 4) * 3 +
                         Scratch::round(lq2.size() * 4 + 4) + Scratch::round(plan2.words() * 4 + 4) +
                         Scratch::round(uint64_t(n_ovf) * cap2 * 4) * 2;
    VA_CHECK_STATUS(f.reserve(need2));
    float* cq = f.carve<float>(uint64_t(n_ovf) * ivf->D);
    uint32_t* d_rows = f.carve<uint32_t>(n_ovf);
    uint32_t* d_thr = f.carve<uint32_t>(n_ovf);
    uint32_t* d_cnt = f.carve<uint32_t>(n_ovf);
    uint32_t* d_lq2 = f.carve<uint32_t>(lq2.size() + 1);
    uint32_t* d_t2 = f.carve<uint32_t>(plan2.words() + 1);
    uint32_t* k2 = f.carve<uint32_t>(uint64_t(n_ovf) * cap2);
    uint32_t* i2 = f.carve<uint32_t>(uint64_t(n_ovf) * cap2);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(d_rows, rows.data(), uint64_t(n_ovf) * 4, hipMemcpyHostToDevice, ctx->stream));
    VA_CHECK_HIP(ctx, hipMemcpyAsync(d_thr, c_thr.data(), uint64_t(n_ovf) * 4, hipMemcpyHostToDevice, ctx->stream));
    if (!lq2.empty())
        VA_CHECK_HIP(ctx, hipMemcpyAsync(d_lq2, lq2.data(), lq2.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    va::gather_queries<<<dim3(std::min<uint32_t>(n_ovf, 4096)), dim3(256), 0, ctx->stream>>>(queries, d_rows, n_ovf,
                                                                                            ivf->D, cq);
    VA_CHECK_LAUNCH(ctx);
    VA_CHECK_STATUS(va::fill_u32(ctx, d_cnt, n_ovf, 0));
    VA_CHECK_STATUS(va::run_pass(ctx, plan2, d_t2, cq, n_ovf, d_lq2, ivf, 1, d_thr, d_cnt, k2, i2, uint32_t(cap2)));
    va::SelectArgs a;
    a.keys = k2;
    a.ids = i2;
    a.counts = d_cnt;
    a.ld = int64_t(cap2);
    a.n = uint32_t(cap2);
    a.rows = n_ovf;
    a.k = k;
    a.row_map = d_rows;
    a.out_idx = out_idx;
    a.out_f = out_dist;
    VA_CHECK_STATUS(va::launch_select(ctx, a));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));  // host vectors above must outlive the copies
    return VA_OK;
}

va_status va_ivf_search(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                        uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist) {
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
    return va_ivf_scan(ctx, ivf, queries, num_queries, m->probe_buf, nprobe, k, out_idx, out_dist);
}

}  // extern "C"
