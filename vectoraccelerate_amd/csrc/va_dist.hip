// va_dist.hip — fp32 distance GEMM on CDNA4 MFMA (v_mfma_f32_32x32x2_f32).
//
// One kernel computes every Q x N distance family of the search path:
//   dist(q, x) from the contraction q.x and the squared norms |q|^2, |x|^2, where the
//   norms are accumulated on the VALU from the same LDS fragments that feed the MFMA
//   (no separate norm pass over the database).
// Replaces the reference's per-pair scalar loops: l2_distance_kernel
// (Metal/Shaders/L2Distance.metal:34-91), dot_product_kernel (DotProduct.metal:29-96) and the
// distance loop of fused_l2_topk (AdvancedTopK.metal:238-242).
//
// Tile geometry (256 threads = 4 wave64):
//   wave tile      = 32 queries x 128 database rows = 4 MFMA blocks of 32x32, 64 acc/lane
//   workgroup tile = (32*WQ) queries x (128*WN) rows, WQ*WN = 4
//   K loop         = LDS stages of KC=16 d-values, double buffered, one barrier per stage
// MFMA operand map: A = database rows (M), B = queries (N).  The contraction index is
// permuted so one ds_read_b128 per lane feeds four MFMA steps: at step s of an 8-wide
// d-group, lane half h supplies d = d0 + 4h + s for both A and B.
// Output map of a 32x32 block (lane l, acc v): row m = 8*(v/4) + 4*(l/32) + v%4,
// column n = l%32 — so each lane owns ONE query and 64 database rows.
#include <cfloat>

#include "va_internal.hpp"

namespace va {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int KC = 16;               // d-values per LDS stage
constexpr int LDS_STRIDE = KC + 4;   // 80-byte rows: conflict-free ds_read_b128 / ds_write_b128

// WQ x WN waves of 64 lanes; each wave owns 32 queries x 128 rows (4 MFMA blocks).
template <int WQ, int WN>
struct Tile {
    static constexpr int NW = WQ * WN;
    static constexpr int NT = 64 * NW;
    static constexpr int TQ = 32 * WQ;
    static constexpr int TN = 128 * WN;
    static constexpr int ROWS = TQ + TN;
    static constexpr int CHUNKS = ROWS * (KC / 4);
    static constexpr int CPT = (CHUNKS + NT - 1) / NT;
    static constexpr int STAGE = ROWS * LDS_STRIDE;
    static constexpr size_t LDS_BYTES = size_t(2 * STAGE + NW * 128) * sizeof(float);
};

__device__ __forceinline__ float apply_op(int op, float dot, float qq, float xx) {
    switch (op) {
        case OP_L2SQ:
        case OP_L2: {
            // cancellation can leave a tiny negative: clamp at 0, but let NaN through
            float v = qq + xx - 2.0f * dot;
            v = (v < 0.0f) ? 0.0f : v;
            return op == OP_L2 ? sqrtf(v) : v;
        }
        case OP_COS_SIM:
        case OP_COS_DIST: {
            // cosine_similarity finalisation (DistanceShaders.metal:300-319)
            float denom = sqrtf(qq) * sqrtf(xx);
            float raw = (denom < FLT_MIN) ? 0.0f : dot / denom;
            float s = (raw != raw) ? raw : fminf(fmaxf(raw, -1.0f), 1.0f);
            return op == OP_COS_SIM ? s : 1.0f - s;
        }
        case OP_DOT: return dot;
        case OP_ABS_DOT: return fabsf(dot);
        default: return -dot;
    }
}

template <int WQ, int WN, bool VEC, int OUT>
__global__ __launch_bounds__(64 * WQ * WN, 2) void dist_gemm_kernel(DistArgs a) {  // 2 waves per SIMD
    using T = Tile<WQ, WN>;
    extern __shared__ float lds[];
    float* nrm = lds + 2 * T::STAGE;  // [waves][128] squared norms of the wave's rows

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wq = wave % WQ;
    const int wn = wave / WQ;
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    // XCD-aware order: workgroup w runs on XCD w % 8.  XCD x takes database tiles x, x+8, ...
    // and runs every query block of a tile back to back, so each tile crosses the fabric once
    // and is reused from that XCD's L2 (the grid is padded to a multiple of 8 tiles).
    const uint32_t nqb = a.tiles ? 1u : (a.Q + T::TQ - 1) / T::TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t tb = (seq / nqb) * kXcds + xcd;
    if (!a.tiles && tb * uint32_t(T::TN) >= a.N) return;  // padding workgroup
    // Tile extent: queries qs + i (i < qc; through qrow when given) and database rows at
    // positions rs + j*rstride (j < rc).  Flat launches derive it from blockIdx; list-major
    // (IVF) launches read one descriptor {qs, qc, rs, rc} per workgroup.
    uint32_t qs = qb * T::TQ, rs = tb * T::TN, qc, rc, rstride = 1;
    if (a.tiles) {
        const uint32_t* td = a.tiles + 4 * int64_t(blockIdx.x);
        qs = td[0];
        qc = td[1];
        rs = td[2];
        rc = td[3];
        rstride = a.rstride;
    } else {
        qc = min(uint32_t(T::TQ), a.Q - qs);
        rc = min(uint32_t(T::TN), a.N - rs);
    }

    // source row pointers of this thread's load chunks (fixed across stages)
    const float* src[T::CPT];
    int ldsoff[T::CPT];
    uint32_t colv[T::CPT];
#pragma unroll
    for (int j = 0; j < T::CPT; ++j) {
        const int c = tid + T::NT * j;
        src[j] = nullptr;
        ldsoff[j] = -1;
        colv[j] = 0;
        if (c < T::CHUNKS) {
            const int row = c >> 2;
            const int col = (c & 3) * 4;
            ldsoff[j] = row * LDS_STRIDE + col;
            colv[j] = uint32_t(col);
            if (row < T::TQ) {
                if (uint32_t(row) < qc) {
                    const uint32_t r = a.qrow ? a.qrow[qs + row] : qs + row;
                    src[j] = a.q + int64_t(r) * a.ldq + col;
                }
            } else {
                const uint32_t jr = uint32_t(row - T::TQ);
                if (jr < rc) src[j] = a.x + int64_t(rs + jr * rstride) * a.ldx + col;
            }
        }
    }

    f32x4v pre[T::CPT];
    auto load = [&](uint32_t d0) {
#pragma unroll
        for (int j = 0; j < T::CPT; ++j) {
            f32x4v v = {0.0f, 0.0f, 0.0f, 0.0f};
            const uint32_t d = d0 + colv[j];
            if (src[j]) {
                if (VEC) {
                    if (d < a.D) v = *reinterpret_cast<const f32x4v*>(src[j] + d0);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d + e < a.D) v[e] = src[j][d0 + e];
                }
            }
            pre[j] = v;
        }
    };
    auto store = [&](float* stage) {
#pragma unroll
        for (int j = 0; j < T::CPT; ++j)
            if (ldsoff[j] >= 0) *reinterpret_cast<f32x4v*>(stage + ldsoff[j]) = pre[j];
    };

    f32x16 acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
    float qss = 0.0f;
    float xss[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    const int nstages = int((a.D + KC - 1) / KC);
    load(0);
    store(lds);
    __syncthreads();

    const int boff = (wq * 32 + l32) * LDS_STRIDE + hh * 4;
    const int aoff = (T::TQ + wn * 128 + l32) * LDS_STRIDE + hh * 4;

    for (int s = 0; s < nstages; ++s) {
        const bool more = (s + 1) < nstages;
        if (more) load(uint32_t(s + 1) * KC);
        const float* st = lds + (s & 1) * T::STAGE;
#pragma unroll
        for (int g = 0; g < KC / 8; ++g) {
            const f32x4v bv = *reinterpret_cast<const f32x4v*>(st + boff + g * 8);
            qss = fmaf(bv[0], bv[0], qss);
            qss = fmaf(bv[1], bv[1], qss);
            qss = fmaf(bv[2], bv[2], qss);
            qss = fmaf(bv[3], bv[3], qss);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const f32x4v av = *reinterpret_cast<const f32x4v*>(st + aoff + b * 32 * LDS_STRIDE + g * 8);
                xss[b] = fmaf(av[0], av[0], xss[b]);
                xss[b] = fmaf(av[1], av[1], xss[b]);
                xss[b] = fmaf(av[2], av[2], xss[b]);
                xss[b] = fmaf(av[3], av[3], xss[b]);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0], bv[0], acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[1], bv[1], acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[2], bv[2], acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[3], bv[3], acc[b], 0, 0, 0);
            }
        }
        if (more) store(lds + ((s + 1) & 1) * T::STAGE);
        __syncthreads();
    }

    // combine the two lane halves of every partial sum of squares
    const float qq = qss + __shfl_xor(qss, 32);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const float t = xss[b] + __shfl_xor(xss[b], 32);
        if (hh == 0) nrm[wave * 128 + b * 32 + l32] = t;
    }
    __syncthreads();

    const uint32_t li = uint32_t(wq * 32 + l32);  // query slot of this lane in the tile
    if (li >= qc) return;
    const uint32_t orow = qs + li;                                   // dense output row
    const uint32_t qi = (OUT == OUT_FILTER && a.qrow) ? a.qrow[orow] : orow;  // query id (filter)
    if (OUT == OUT_FILTER) {
        // Count this lane's passing keys, reserve them with one atomic, then write them.
        const uint32_t thr = a.thr[qi];
        uint64_t pass = 0;  // bit 16b + 4j + e
        uint32_t keys[64];
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int mloc = b * 32 + 8 * j + 4 * hh;
                const f32x4v xx = *reinterpret_cast<const f32x4v*>(nrm + wave * 128 + mloc);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t key = key_of_float(apply_op(a.op, acc[b][4 * j + e], qq, xx[e]));
                    keys[16 * b + 4 * j + e] = key;
                    const bool p = uint32_t(wn * 128 + mloc + e) < rc && key <= thr;
                    pass |= uint64_t(p) << (16 * b + 4 * j + e);
                }
            }
        if (pass) {
            uint32_t pos = atomicAdd(a.cnt + qi, uint32_t(__popcll(pass)));
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                if (!((pass >> t) & 1)) continue;
                if (pos < a.cap) {
                    const int b = t >> 4, j = (t >> 2) & 3, e = t & 3;
                    const uint32_t p = rs + uint32_t(wn * 128 + b * 32 + 8 * j + 4 * hh + e) * rstride;
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_key[o] = keys[t];
                    a.cand_id[o] = a.ids ? a.ids[p] : a.id_base + p;
                }
                ++pos;
            }
        }
        return;
    }

#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int mloc = b * 32 + 8 * j + 4 * hh;
            const f32x4v xx = *reinterpret_cast<const f32x4v*>(nrm + wave * 128 + mloc);
            float val[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) val[e] = apply_op(a.op, acc[b][4 * j + e], qq, xx[e]);
            const uint32_t jr = uint32_t(wn * 128 + mloc);  // row slot of acc element e = 0
            if (OUT == OUT_KEYS) {
                uint32_t* o = a.out_k + int64_t(orow) * a.ldo + rs + jr;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (jr + e < rc) o[e] = key_of_float(val[e]);
            } else {
                float* o = a.out_f + int64_t(orow) * a.ldo + rs + jr;
                if (jr + 3 < rc && ((a.ldo & 3) == 0) && ((reinterpret_cast<uintptr_t>(o) & 15) == 0)) {
                    f32x4v w = {val[0], val[1], val[2], val[3]};
                    *reinterpret_cast<f32x4v*>(o) = w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (jr + e < rc) o[e] = val[e];
                }
            }
        }
    }
}

template <int WQ, int WN, bool VEC, int OUT>
va_status launch_tile(va_context* ctx, const DistArgs& a) {
    using T = Tile<WQ, WN>;
    const uint64_t nqb = (a.Q + T::TQ - 1) / T::TQ;
    const uint64_t ntb = (a.N + T::TN - 1) / T::TN;
    const uint64_t grid = a.tiles ? a.ntiles : nqb * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (grid == 0) return VA_OK;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "distance grid too large (%llu tiles)", (unsigned long long)grid);
    auto kern = &dist_gemm_kernel<WQ, WN, VEC, OUT>;
    if (T::LDS_BYTES > 65536) {
        VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, int(T::LDS_BYTES)));
    }
    kern<<<dim3(uint32_t(grid)), dim3(T::NT), T::LDS_BYTES, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

}  // namespace

va_status launch_dist(va_context* ctx, const DistArgs& a) {
    if (a.tiles ? a.ntiles == 0 : (a.Q == 0 || a.N == 0)) return VA_OK;
    const bool vec = (a.D % 4 == 0) && (a.ldq % 4 == 0) && (a.ldx % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    const int wq = a.wq ? a.wq : (a.Q <= 32 ? 1 : (a.Q <= 64 ? 2 : 4));
    const int wn = a.wn ? a.wn : 4 / wq;
#define VA_DIST_CASE(W, N, O)                                                              \
    if (wq == W && wn == N && a.out == O)                                                  \
        return vec ? launch_tile<W, N, true, O>(ctx, a) : launch_tile<W, N, false, O>(ctx, a);
    VA_DIST_CASE(1, 4, OUT_VALUES) VA_DIST_CASE(1, 4, OUT_KEYS) VA_DIST_CASE(1, 4, OUT_FILTER)
    VA_DIST_CASE(2, 2, OUT_VALUES) VA_DIST_CASE(2, 2, OUT_KEYS) VA_DIST_CASE(2, 2, OUT_FILTER)
    VA_DIST_CASE(4, 1, OUT_VALUES) VA_DIST_CASE(4, 1, OUT_KEYS) VA_DIST_CASE(4, 1, OUT_FILTER)
    // small list-major tiles (one or two waves) for sparse IVF work
    VA_DIST_CASE(1, 1, OUT_FILTER) VA_DIST_CASE(2, 1, OUT_FILTER)
#undef VA_DIST_CASE
    return fail(ctx, VA_ERR_INVALID_ARG, "launch_dist: no %dx%d tile for output mode %d", wq, wn, int(a.out));
}

}  // namespace va
