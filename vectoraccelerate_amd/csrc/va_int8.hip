// va_int8.hip — scalar-int8 quantize-and-scan on CDNA4.
//
//   params   : per-dimension min/max (HBM-bound reduction, ordered-key atomics) and the
//              affine map of ScalarQuantizationKernel.computeQuantizationParams
//              (Kernels/Metal4/ScalarQuantizationKernel.swift:496-520), per dimension;
//   quantize : q = clamp(rint(x/scale + zp), -128, 127) exactly as quantize_int8_kernel
//              (Metal/Shaders/DataTransformations.metal:174-201) — IEEE division and rint,
//              so codes are bit-identical to the CPU rule;
//   scan     : int32 dot of int8 codes on v_mfma_i32_32x32x32_i8; distance = -dot; exact
//              top-k through the shared scan driver.
// Tile geometry of the scan mirrors the fp32 GEMM: A = database codes, B = query codes, wave
// tile 32 queries x 128 rows, LDS stages of 64 bytes per row.  Each lane feeds an MFMA with
// 16 contiguous bytes of its row; lane half h covers bytes [16h, 16h+16) of a 32-byte k-step,
// the same map for A and B, so the contraction pairs equal d on both sides.
#include <algorithm>

#include "va_internal.hpp"

namespace va {
namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------
// per-dimension min / max
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void minmax_kernel(const float* __restrict__ x, uint64_t N, uint32_t D,
                                                     uint64_t rows_per_block, uint32_t* kmin, uint32_t* kmax) {
    const uint32_t d = blockIdx.y * 256 + threadIdx.x;
    if (d >= D) return;
    const uint64_t r0 = uint64_t(blockIdx.x) * rows_per_block;
    const uint64_t r1 = std::min<uint64_t>(N, r0 + rows_per_block);
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    bool any = false;
    for (uint64_t r = r0; r < r1; ++r) {
        const float v = x[r * D + d];
        if (v != v) continue;  // NaN never wins a comparison (the CPU rule)
        const uint32_t k = key_of_float(v);
        lo = k < lo ? k : lo;
        hi = k > hi ? k : hi;
        any = true;
    }
    if (any) {
        atomicMin(kmin + d, lo);
        atomicMax(kmax + d, hi);
    }
}

__global__ void params_finalize(const uint32_t* kmin, const uint32_t* kmax, uint32_t D, float* mn, float* mx,
                                float* scale, int32_t* zp) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    const bool have = kmin[d] != 0xFFFFFFFFu;
    const float lo = have ? float_of_key(kmin[d]) : 0.0f;
    const float hi = have ? float_of_key(kmax[d]) : 0.0f;
    // ScalarQuantizationKernel.swift:513-518: scale = max(range / 255, 1e-8)
    const float range = hi - lo;
    float s = range / 255.0f;
    if (!(s > 1e-8f)) s = 1e-8f;
    // Swift round() and roundf(): half away from zero
    const float r = roundf(lo / s);
    if (mn) mn[d] = lo;
    if (mx) mx[d] = hi;
    scale[d] = s;
    zp[d] = -128 - int32_t(r);
}

// ---------------------------------------------------------------------------------------
// quantize / dequantize (one row per block-iteration, columns across threads)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int8_t quantize_one(float v, float s, int32_t z) {
    if (fabsf(s) < 1e-9f) return int8_t(z < -128 ? -128 : (z > 127 ? 127 : z));
    const float scaled = v / s + float(z);
    float r = rintf(scaled);
    r = r < -128.0f ? -128.0f : r;
    r = r > 127.0f ? 127.0f : r;
    if (r != r) r = 0.0f;
    return int8_t(r);
}

__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ x, uint64_t N, uint32_t D,
                                                       const float* __restrict__ scale,
                                                       const int32_t* __restrict__ zp, int8_t* __restrict__ out) {
    for (uint64_t r = blockIdx.x; r < N; r += gridDim.x) {
        const float* row = x + r * D;
        int8_t* o = out + r * D;
        for (uint32_t d = threadIdx.x; d < D; d += 256) o[d] = quantize_one(row[d], scale[d], zp[d]);
    }
}

// D % 4 == 0 and 16-byte aligned rows: float4 in, char4 out
__global__ __launch_bounds__(256) void quantize_kernel_v4(const float4* __restrict__ x, uint64_t N, uint32_t D4,
                                                          const float4* __restrict__ scale,
                                                          const int4* __restrict__ zp, char4* __restrict__ out) {
    for (uint64_t r = blockIdx.x; r < N; r += gridDim.x) {
        for (uint32_t c = threadIdx.x; c < D4; c += 256) {
            const float4 v = x[r * D4 + c];
            const float4 s = scale[c];
            const int4 z = zp[c];
            char4 q;
            q.x = quantize_one(v.x, s.x, z.x);
            q.y = quantize_one(v.y, s.y, z.y);
            q.z = quantize_one(v.z, s.z, z.z);
            q.w = quantize_one(v.w, s.w, z.w);
            out[r * D4 + c] = q;
        }
    }
}

__global__ __launch_bounds__(256) void dequantize_kernel(const int8_t* __restrict__ c, uint64_t N, uint32_t D,
                                                         const float* __restrict__ scale,
                                                         const int32_t* __restrict__ zp, float* __restrict__ out) {
    for (uint64_t r = blockIdx.x; r < N; r += gridDim.x)
        for (uint32_t d = threadIdx.x; d < D; d += 256)
            out[r * D + d] = (float(c[r * D + d]) - float(zp[d])) * scale[d];
}

// ---------------------------------------------------------------------------------------
// int8 MFMA scan
// ---------------------------------------------------------------------------------------
#ifndef VA_I8_KB
#define VA_I8_KB 64
#endif
constexpr int KB = VA_I8_KB;           // bytes of each row per LDS stage (32-byte k-steps)
constexpr int ROWB = KB + 16;          // +16 B pad: conflict-free ds_read_b128 across 16 rows

struct I8Args {
    const int8_t* q = nullptr;
    const uint32_t* qrow = nullptr;
    int64_t ldq = 0;
    const int8_t* x = nullptr;
    int64_t ldx = 0;
    uint32_t Q = 0, N = 0, D = 0;
    uint32_t* out_k = nullptr;
    int64_t ldo = 0;
    const uint32_t* thr = nullptr;
    uint32_t* cnt = nullptr;
    uint32_t* cand_key = nullptr;
    uint32_t* cand_id = nullptr;
    uint32_t cap = 0;
};

// Tile shapes: QBW query blocks of 32 per wave, WQ x WN waves; wave tile = 32*QBW queries x
// 128 rows; workgroup tile = 32*QBW*WQ queries x 128*WN rows.  The 8-wave 256 x 256 shape is
// used for large Q: it halves the L2-to-CU bytes per MFMA op of the 128 x 128 shape (the
// int8 MFMA rate otherwise outruns the ~64 B/clk/CU the L2 can deliver).
template <int QBW, int WQ, int WN>
struct I8Tile {
    static constexpr int THREADS = 64 * WQ * WN;
    static constexpr int TQ = 32 * QBW * WQ;
    static constexpr int TN = 128 * WN;
    static constexpr int ROWS = TQ + TN;
    static constexpr int CHUNKS = ROWS * (KB / 16);
    static constexpr int CPT = (CHUNKS + THREADS - 1) / THREADS;
    static constexpr int STAGE = ROWS * ROWB;  // bytes
    static constexpr size_t LDS_BYTES = size_t(2 * STAGE);
};

template <int QBW, int WQ, int WN, bool VEC, bool FILTER>
__global__ __launch_bounds__(64 * WQ * WN) void i8_scan_kernel(I8Args a) {
    using T = I8Tile<QBW, WQ, WN>;
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wq = wave % WQ;
    const int wn = wave / WQ;
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    // XCD-aware order (workgroup w runs on XCD w % 8): XCD x takes database tiles x, x+8, ...
    // and runs every query block of a tile back to back, so a tile crosses the fabric once.
    const uint32_t nqb = (a.Q + T::TQ - 1) / T::TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t tb = (seq / nqb) * kXcds + xcd;
    const uint32_t q0 = qb * T::TQ;
    const uint32_t n0 = tb * T::TN;
    if (n0 >= a.N) return;  // padding workgroup

    const int8_t* src[T::CPT];
    int ldsoff[T::CPT];
    uint32_t colv[T::CPT];
#pragma unroll
    for (int j = 0; j < T::CPT; ++j) {
        const int c = tid + T::THREADS * j;
        src[j] = nullptr;
        ldsoff[j] = -1;
        colv[j] = 0;
        if (c < T::CHUNKS) {
            const int row = c / (KB / 16);
            const int col = (c % (KB / 16)) * 16;
            ldsoff[j] = row * ROWB + col;
            colv[j] = uint32_t(col);
            if (row < T::TQ) {
                const uint32_t qi = q0 + row;
                if (qi < a.Q) src[j] = a.q + int64_t(a.qrow ? a.qrow[qi] : qi) * a.ldq + col;
            } else {
                const uint32_t ni = n0 + uint32_t(row - T::TQ);
                if (ni < a.N) src[j] = a.x + int64_t(ni) * a.ldx + col;
            }
        }
    }
    i32x4v pre[T::CPT];
    auto load = [&](uint32_t d0) {
#pragma unroll
        for (int j = 0; j < T::CPT; ++j) {
            i32x4v v = {0, 0, 0, 0};
            const uint32_t d = d0 + colv[j];
            if (src[j]) {
                if (VEC) {
                    if (d < a.D) v = *reinterpret_cast<const i32x4v*>(src[j] + d0);
                } else {
                    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (d + e < a.D) w[e >> 2] |= uint32_t(uint8_t(src[j][d0 + e])) << (8 * (e & 3));
                    v = i32x4v{int(w[0]), int(w[1]), int(w[2]), int(w[3])};
                }
            }
            pre[j] = v;
        }
    };
    auto store = [&](char* stage) {
#pragma unroll
        for (int j = 0; j < T::CPT; ++j)
            if (ldsoff[j] >= 0) *reinterpret_cast<i32x4v*>(stage + ldsoff[j]) = pre[j];
    };

    i32x16 acc[QBW][4];
#pragma unroll
    for (int u = 0; u < QBW; ++u)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[u][b][v] = 0;

    const int nstages = int((a.D + KB - 1) / KB);
    load(0);
    store(lds8);
    __syncthreads();
    const int boff = (wq * QBW * 32 + l32) * ROWB + hh * 16;
    const int aoff = (T::TQ + wn * 128 + l32) * ROWB + hh * 16;
    for (int s = 0; s < nstages; ++s) {
        const bool more = (s + 1) < nstages;
        if (more) load(uint32_t(s + 1) * KB);
        const char* st = lds8 + (s & 1) * T::STAGE;
#pragma unroll
        for (int g = 0; g < KB / 32; ++g) {
            i32x4v bv[QBW];
#pragma unroll
            for (int u = 0; u < QBW; ++u)
                bv[u] = *reinterpret_cast<const i32x4v*>(st + boff + u * 32 * ROWB + g * 32);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const i32x4v av = *reinterpret_cast<const i32x4v*>(st + aoff + b * 32 * ROWB + g * 32);
#pragma unroll
                for (int u = 0; u < QBW; ++u)
                    acc[u][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[u], acc[u][b], 0, 0, 0);
            }
        }
        if (more) store(lds8 + ((s + 1) & 1) * T::STAGE);
        __syncthreads();
    }

    const uint32_t nbase = n0 + uint32_t(wn * 128);
#pragma unroll
    for (int u = 0; u < QBW; ++u) {
        const uint32_t qi = q0 + uint32_t((wq * QBW + u) * 32 + l32);
        if (qi >= a.Q) continue;
        if (FILTER) {
            const uint32_t thr = a.thr[qi];
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t m = nbase + uint32_t(b * 32 + 8 * j + 4 * hh + e);
                        const uint32_t key = key_of_i32(-acc[u][b][4 * j + e]);
                        if (m < a.N && key <= thr) {
                            const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                            if (pos < a.cap) {
                                const int64_t o = int64_t(qi) * a.cap + pos;
                                a.cand_key[o] = key;
                                a.cand_id[o] = m;
                            }
                        }
                    }
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t m = nbase + uint32_t(b * 32 + 8 * j + 4 * hh);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e < a.N) a.out_k[int64_t(qi) * a.ldo + m + e] = key_of_i32(-acc[u][b][4 * j + e]);
                }
        }
    }
}

template <int QBW, int WQ, int WN, bool VEC, bool FILTER>
va_status launch_i8_tile(va_context* ctx, const I8Args& a) {
    using T = I8Tile<QBW, WQ, WN>;
    const uint64_t ntb = (a.N + T::TN - 1) / T::TN;
    const uint64_t grid = uint64_t((a.Q + T::TQ - 1) / T::TQ) * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (grid == 0) return VA_OK;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "int8 scan grid too large");
    auto kern = &i8_scan_kernel<QBW, WQ, WN, VEC, FILTER>;
    if (T::LDS_BYTES > 65536)
        VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, int(T::LDS_BYTES)));
    kern<<<dim3(uint32_t(grid)), dim3(T::THREADS), T::LDS_BYTES, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

template <int QBW, int WQ, int WN>
va_status launch_i8_shape(va_context* ctx, const I8Args& a, bool vec, bool filter) {
    if (filter) return vec ? launch_i8_tile<QBW, WQ, WN, true, true>(ctx, a) : launch_i8_tile<QBW, WQ, WN, false, true>(ctx, a);
    return vec ? launch_i8_tile<QBW, WQ, WN, true, false>(ctx, a) : launch_i8_tile<QBW, WQ, WN, false, false>(ctx, a);
}

va_status launch_i8(va_context* ctx, const I8Args& a, bool filter) {
    if (a.Q == 0 || a.N == 0) return VA_OK;
    const bool vec = (a.D % 16 == 0) && (a.ldq % 16 == 0) && (a.ldx % 16 == 0) &&
                     ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    if (a.Q <= 32) return launch_i8_shape<1, 1, 4>(ctx, a, vec, filter);
    if (a.Q <= 64) return launch_i8_shape<1, 2, 2>(ctx, a, vec, filter);
// Large-Q shape: 0 = 128 x 128 (4 waves), 1 = 128 x 256 (4 waves), 2 = 256 x 256 (8 waves).
// Measured on configs[2] (10M x 512, Q=4096): 0 is fastest with 64-byte register-staged
// stages (each stage's MFMA work is shorter than its load round trip).
#ifndef VA_I8_LARGE_SHAPE
#define VA_I8_LARGE_SHAPE 0
#endif
    if (a.Q <= 192 || VA_I8_LARGE_SHAPE == 0) return launch_i8_shape<1, 4, 1>(ctx, a, vec, filter);
    if (VA_I8_LARGE_SHAPE == 1) return launch_i8_shape<2, 2, 2>(ctx, a, vec, filter);
    return launch_i8_shape<2, 4, 2>(ctx, a, vec, filter);
}

struct I8Producer final : KeyProducer {
    va_context* ctx;
    const int8_t* q;
    const int8_t* x;
    uint32_t Q, N, D;
    va_status dense(const uint32_t* qrow, uint32_t q0, uint32_t nq, uint32_t c0, uint32_t cols, uint32_t stride,
                    uint32_t* out_k, int64_t ldo) override {
        I8Args a;
        a.q = qrow ? q : q + int64_t(q0) * D;
        a.qrow = qrow;
        a.ldq = D;
        a.x = x + int64_t(c0) * D;
        a.ldx = int64_t(stride) * D;
        a.Q = nq;
        a.N = cols;
        a.D = D;
        a.out_k = out_k;
        a.ldo = ldo;
        return launch_i8(ctx, a, false);
    }
    va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) override {
        I8Args a;
        a.q = q;
        a.ldq = D;
        a.x = x;
        a.ldx = D;
        a.Q = Q;
        a.N = N;
        a.D = D;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        return launch_i8(ctx, a, true);
    }
};

uint32_t grid_rows(uint64_t N) { return uint32_t(std::min<uint64_t>(N, 16384)); }

}  // namespace
}  // namespace va

extern "C" {

va_status va_sq_params_per_dim(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim, float* out_min,
                               float* out_max, float* out_scale, int32_t* out_zero_point) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, x && out_scale && out_zero_point, "va_sq_params_per_dim: NULL pointer");
    VA_REQUIRE(ctx, num_vectors > 0 && dim > 0, "Empty input data");
    va::DeviceGuard g(ctx->device);
    va::Scratch s(ctx);
    VA_CHECK_STATUS(s.reserve(va::Scratch::round(uint64_t(dim) * 4) * 2));
    uint32_t* kmin = s.carve<uint32_t>(dim);
    uint32_t* kmax = s.carve<uint32_t>(dim);
    VA_CHECK_STATUS(va::fill_u32(ctx, kmin, dim, 0xFFFFFFFFu));
    VA_CHECK_STATUS(va::fill_u32(ctx, kmax, dim, 0u));
    const uint32_t ycols = (dim + 255) / 256;
    // enough row blocks to cover the chip (about 2048 workgroups in total)
    uint64_t xblocks = std::max<uint64_t>(1, std::min<uint64_t>(num_vectors, 2048 / ycols + 1));
    const uint64_t rpb = (uint64_t(num_vectors) + xblocks - 1) / xblocks;
    xblocks = (uint64_t(num_vectors) + rpb - 1) / rpb;
    va::minmax_kernel<<<dim3(uint32_t(xblocks), ycols), dim3(256), 0, ctx->stream>>>(x, num_vectors, dim, rpb, kmin,
                                                                                       kmax);
    VA_CHECK_LAUNCH(ctx);
    va::params_finalize<<<dim3((dim + 255) / 256), dim3(256), 0, ctx->stream>>>(kmin, kmax, dim, out_min, out_max,
                                                                                 out_scale, out_zero_point);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_sq_quantize_i8(va_context* ctx, const float* x, uint64_t num_vectors, uint32_t dim, const float* scale,
                            const int32_t* zero_point, int8_t* codes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, x && scale && zero_point && codes, "va_sq_quantize_i8: NULL pointer");
    VA_REQUIRE(ctx, num_vectors > 0 && dim > 0, "Empty input data");
    va::DeviceGuard g(ctx->device);
    const bool v4 = dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(scale) |
                                      reinterpret_cast<uintptr_t>(zero_point)) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(codes) & 3) == 0;
    if (v4)
        va::quantize_kernel_v4<<<dim3(va::grid_rows(num_vectors)), dim3(256), 0, ctx->stream>>>(
            reinterpret_cast<const float4*>(x), num_vectors, dim / 4, reinterpret_cast<const float4*>(scale),
            reinterpret_cast<const int4*>(zero_point), reinterpret_cast<char4*>(codes));
    else
        va::quantize_kernel<<<dim3(va::grid_rows(num_vectors)), dim3(256), 0, ctx->stream>>>(x, num_vectors, dim,
                                                                                           scale, zero_point, codes);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_sq_dequantize_i8(va_context* ctx, const int8_t* codes, uint64_t num_vectors, uint32_t dim,
                              const float* scale, const int32_t* zero_point, float* out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, codes && scale && zero_point && out, "va_sq_dequantize_i8: NULL pointer");
    VA_REQUIRE(ctx, num_vectors > 0 && dim > 0, "Empty input data");
    va::DeviceGuard g(ctx->device);
    va::dequantize_kernel<<<dim3(va::grid_rows(num_vectors)), dim3(256), 0, ctx->stream>>>(codes, num_vectors, dim,
                                                                                         scale, zero_point, out);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_i8_scan_topk(va_context* ctx, const int8_t* query_codes, const int8_t* database_codes,
                          uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k, uint32_t* out_idx,
                          int32_t* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, query_codes && database_codes && out_idx, "va_i8_scan_topk: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0 && num_database > 0 && dim > 0, "va_i8_scan_topk: empty input");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    va::DeviceGuard g(ctx->device);
    va::I8Producer p;
    p.ctx = ctx;
    p.q = query_codes;
    p.x = database_codes;
    p.Q = num_queries;
    p.N = num_database;
    p.D = dim;
    va::ScanOutputs o;
    o.idx = out_idx;
    o.i32 = out_dist;
    o.key_kind = 2;
    return va::exact_topk_scan(ctx, p, num_queries, num_database, k, o);
}

}  // extern "C"
