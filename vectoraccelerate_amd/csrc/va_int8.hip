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

#include "va_fallback.hpp"
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

// D % 4 == 0 and 16-byte aligned rows: each thread owns 4 dimensions (one float4 column) of
// a row slab; a block covers 256 / (D/4) rows per step and strides over the rows, keeping
// four independent loads in flight per thread; partial min/max meet in LDS, then one atomic
// per dimension and block.  HBM-bound: every byte of x is read once.
__global__ __launch_bounds__(256) void minmax_kernel_v4(const float4* __restrict__ x, uint64_t N, uint32_t D4,
                                                        uint32_t* kmin, uint32_t* kmax) {
    __shared__ uint32_t smin[1024], smax[1024];
    const uint32_t t = threadIdx.x;
    const uint32_t rpb = 256 / D4;  // rows per block step (D4 <= 256)
    const uint32_t c = t % D4, r0 = t / D4;
    const bool active = r0 < rpb;
    uint32_t lo[4] = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu}, hi[4] = {0u, 0u, 0u, 0u};
    auto take = [&](const float4 v) {
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (e[i] != e[i]) continue;  // NaN never wins a comparison (the CPU rule)
            const uint32_t k = key_of_float(e[i]);
            lo[i] = k < lo[i] ? k : lo[i];
            hi[i] = k > hi[i] ? k : hi[i];
        }
    };
    if (active) {
        const uint64_t step = uint64_t(gridDim.x) * rpb;
        uint64_t r = uint64_t(blockIdx.x) * rpb + r0;
        for (; r + 3 * step < N; r += 4 * step) {
            const float4 a = x[r * D4 + c], b = x[(r + step) * D4 + c];
            const float4 cc = x[(r + 2 * step) * D4 + c], d = x[(r + 3 * step) * D4 + c];
            take(a);
            take(b);
            take(cc);
            take(d);
        }
        for (; r < N; r += step) take(x[r * D4 + c]);
    }
    // reduce the rpb partials of each column in LDS
    for (uint32_t i = t; i < 4 * D4; i += 256) {
        smin[i] = 0xFFFFFFFFu;
        smax[i] = 0u;
    }
    __syncthreads();
    if (active) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            atomicMin(smin + 4 * c + i, lo[i]);
            atomicMax(smax + 4 * c + i, hi[i]);
        }
    }
    __syncthreads();
    for (uint32_t i = t; i < 4 * D4; i += 256) {
        if (smin[i] == 0xFFFFFFFFu) continue;  // only NaN (or nothing) seen in this column
        atomicMin(kmin + i, smin[i]);
        atomicMax(kmax + i, smax[i]);
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

// D % 4 == 0 and 16-byte aligned rows: float4 in, char4 out.  Each thread owns one float4
// column of a row slab (256 / (D/4) rows per block step, D <= 1024), so the column's scale and
// zero point stay in registers and four rows are in flight per thread.
__global__ __launch_bounds__(256) void quantize_kernel_v4(const float4* __restrict__ x, uint64_t N, uint32_t D4,
                                                          const float4* __restrict__ scale,
                                                          const int4* __restrict__ zp, char4* __restrict__ out) {
    const uint32_t t = threadIdx.x;
    const uint32_t rpb = 256 / D4;
    const uint32_t c = t % D4, r0 = t / D4;
    if (r0 >= rpb) return;
    const float4 sc = scale[c];
    const int4 z = zp[c];
    auto q4 = [&](const float4 v) {
        char4 o;
        o.x = quantize_one(v.x, sc.x, z.x);
        o.y = quantize_one(v.y, sc.y, z.y);
        o.z = quantize_one(v.z, sc.z, z.z);
        o.w = quantize_one(v.w, sc.w, z.w);
        return o;
    };
    const uint64_t step = uint64_t(gridDim.x) * rpb;
    uint64_t r = uint64_t(blockIdx.x) * rpb + r0;
    for (; r + 3 * step < N; r += 4 * step) {
        const float4 a = x[r * D4 + c], b = x[(r + step) * D4 + c];
        const float4 e = x[(r + 2 * step) * D4 + c], f = x[(r + 3 * step) * D4 + c];
        out[r * D4 + c] = q4(a);
        out[(r + step) * D4 + c] = q4(b);
        out[(r + 2 * step) * D4 + c] = q4(e);
        out[(r + 3 * step) * D4 + c] = q4(f);
    }
    for (; r < N; r += step) out[r * D4 + c] = q4(x[r * D4 + c]);
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

// ---------------------------------------------------------------------------------------
// int8 scan with an LDS-DMA pipeline (large Q)
// ---------------------------------------------------------------------------------------
// Workgroup tile 256 queries x 128 rows; four waves as 2 x 2, wave tile 128 queries x 64 rows
// (4 x 2 MFMA blocks, 128 accumulators).  Stages of 64 bytes per row move global -> LDS by
// direct buffer loads (no register staging) into a ring of three slots, issued two stages
// ahead of the MFMAs that read them.  Rows and columns outside the tile load from an offset
// past the descriptor and land as zeros.  LDS rows are 64 bytes, unpadded: 16-byte chunk c of
// row r sits at chunk c ^ swz(r).  ds_read_b128 serves 16 lanes per clock from 64 banks, so the
// 16 rows read together must cover 16 distinct 16-byte bank groups: rows r..r+3 already do
// (64-byte stride), and swz = (r >> 2) & 3 shifts each following group of four by one chunk.
// 256 x 128 halves the L2-to-CU bytes per MFMA op of a 128 x 128 tile; 78 KiB of LDS (ring +
// candidate staging) leaves room for two workgroups per CU.
//
// At d = 512 a tile is only 16 MFMA k-steps deep, so the epilogue must cost far less than the
// MFMAs: the filter epilogue rejects with a per-lane max, tests surviving positions with one
// wave-wide compare each, and stages passes in LDS (see below).
namespace dmai8 {
constexpr int TQ = 256, TN = 128, ROWS = TQ + TN, SKB = 64, NS = 3;
constexpr int STAGE = ROWS * SKB;                  // 24 KiB per ring slot
constexpr int RING = NS * STAGE;                   // 72 KiB
// candidate staging: 512 (query, key, id) entries, a 128-entry slice per wave, + 4 counts
constexpr int STAGED = 512;
constexpr size_t LDS_BYTES = size_t(RING) + 3 * 4 * STAGED + 16;
constexpr int GPW = ROWS / 16 / 4;                 // 16-row DMA groups per wave and stage (6)
constexpr int QGPW = TQ / 16 / 4;                  // of which query groups (4)
__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }
}  // namespace dmai8

template <bool FILTER>
__global__ __launch_bounds__(256, 2) void i8_dma_kernel(I8Args a) {
    using namespace dmai8;
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, hh = lane >> 5;

    // XCD-aware order, as in i8_scan_kernel
    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t tb = (seq / nqb) * kXcds + xcd;
    const uint32_t q0 = qb * TQ;
    const uint32_t n0 = tb * TN;
    if (n0 >= a.N) return;  // padding workgroup
    const uint32_t rc = min(uint32_t(TN), a.N - n0);

    const dma_rsrc qres = make_dma_rsrc(a.q, uint32_t(int64_t(a.Q - 1) * a.ldq + a.D));
    const dma_rsrc xres = make_dma_rsrc(a.x + int64_t(n0) * a.ldx, uint32_t(int64_t(rc - 1) * a.ldx + a.D));

    // This lane's source offset and 16-byte column in each of the wave's DMA groups.
    uint32_t base[GPW], colb[GPW];
#pragma unroll
    for (int i = 0; i < GPW; ++i) {
        const int row = 16 * (wave + 4 * i) + (lane >> 2);
        const int col = 16 * ((lane & 3) ^ swz(row));
        colb[i] = uint32_t(col);
        if (i < QGPW) {
            const uint32_t qi = q0 + uint32_t(row);
            base[i] = qi < a.Q ? uint32_t(int64_t(qi) * a.ldq) + col : kDmaSkip;
        } else {
            const uint32_t jr = uint32_t(row - TQ);
            base[i] = jr < rc ? uint32_t(int64_t(jr) * a.ldx) + col : kDmaSkip;
        }
    }
    const uint32_t lds0 = lds_addr_of(lds8);
    auto issue = [&](uint32_t stage, uint32_t slot) {
        const uint32_t d0 = stage * SKB;
#pragma unroll
        for (int i = 0; i < GPW; ++i) {
            const uint32_t voff = (base[i] != kDmaSkip && d0 + colb[i] < a.D) ? base[i] + d0 : kDmaSkip;
            const uint32_t dst = lds0 + slot * STAGE + uint32_t(wave + 4 * i) * 1024u;
            lds_dma16(i < QGPW ? qres : xres, voff, dst);
        }
    };

    i32x16 acc[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[u][b][v] = 0;

    // fragment rows: bases are multiples of 32, so every fragment row has swz(row) == swz(l32)
    const int sw = swz(l32);
    const int qfrag = (wq * 128 + l32) * SKB;
    const int xfrag = (TQ + wn * 64 + l32) * SKB;
    int koff[SKB / 32];
#pragma unroll
    for (int g = 0; g < SKB / 32; ++g) koff[g] = ((2 * g + hh) ^ sw) * 16;

    // The filter's thresholds load before the stream starts, so their latency hides behind
    // the MFMA loop instead of stalling the epilogue.
    uint32_t thr0[4] = {0u, 0u, 0u, 0u};
    if (FILTER) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t qi = q0 + uint32_t(wq * 128 + u * 32 + l32);
            thr0[u] = a.thr[qi < a.Q ? qi : 0u];
        }
    }
    const uint32_t nst = (a.D + SKB - 1) / SKB;
    issue(0, 0);
    if (nst > 1) issue(1, 1);
    uint32_t slot = 0;
    for (uint32_t s = 0; s < nst; ++s) {
        if (s + 1 < nst) wait_vmcnt<GPW>();
        else wait_vmcnt<0>();
        __syncthreads();  // stage s visible; every wave is past the reads of slot (s + 2) % 3
        if (s + 2 < nst) issue(s + 2, slot == 0 ? 2u : slot - 1);
        const char* st = lds8 + slot * STAGE;
#pragma unroll
        for (int g = 0; g < SKB / 32; ++g) {
            i32x4v bq[4], ax[2];
#pragma unroll
            for (int u = 0; u < 4; ++u) bq[u] = *reinterpret_cast<const i32x4v*>(st + qfrag + u * 32 * SKB + koff[g]);
#pragma unroll
            for (int b = 0; b < 2; ++b) ax[b] = *reinterpret_cast<const i32x4v*>(st + xfrag + b * 32 * SKB + koff[g]);
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[u][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax[b], bq[u], acc[u][b], 0, 0, 0);
        }
        slot = slot == 2 ? 0u : slot + 1;
    }

    const uint32_t nbase = n0 + uint32_t(wn * 64);
    // rows of this lane's values that exist: offsets 32b + 8j + e (+4hh) below lim
    const int64_t lim = int64_t(a.N) - int64_t(nbase) - 4 * hh;
    if (FILTER) {
        // A value passes when its dot is >= the query's bound (the threshold key turned back
        // into an int32 dot).  A lane's 32 values of a query are reduced with max first, so a
        // wave skips a query column when no lane passes; otherwise each value position is
        // tested with one wave-wide compare, and where some lane passes the wave appends its
        // passes to its own slice of the LDS staging list.  Slots come from a wave-uniform
        // running count plus the lane's rank in the compare mask: no atomics (an LDS atomic
        // round trip per appending position cost as much as a third of the kernel).  After a
        // barrier the four slices are flushed with one global reservation per entry, all in
        // flight at once.
        uint32_t* s_qi = reinterpret_cast<uint32_t*>(lds8 + RING);
        uint32_t* s_key = s_qi + STAGED;
        uint32_t* s_id = s_key + STAGED;
        uint32_t* s_cnt = s_id + STAGED;  // per-wave entry counts
        constexpr uint32_t WCAP = STAGED / 4;
        const uint32_t wbase = uint32_t(wave) * WCAP;
        if (nbase + 64 > a.N) {  // last tile: rows past N never pass
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        if (int64_t(b * 32 + 8 * (v >> 2) + (v & 3)) >= lim) acc[u][b][v] = INT32_MIN;
        }
        int32_t bound[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t qi = q0 + uint32_t(wq * 128 + u * 32 + l32);
            const int32_t t = i32_of_key(thr0[u]);  // pass iff -dot <= t
            bound[u] = (qi >= a.Q || t == INT32_MIN) ? INT32_MAX : -t;
        }
        __syncthreads();  // every wave is done with the ring before the staging area is used
        uint32_t wc = 0;  // entries this wave has staged (wave-uniform)
        // Branches are the cost here (a wave-uniform branch per value position took as long as
        // the MFMAs), so the test is hierarchical: the maximum of a lane's 32 values, then of
        // each group of 8, and only then single positions.
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int32_t m8[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                m8[g] = acc[u][(8 * g) >> 4][(8 * g) & 15];
#pragma unroll
                for (int w = 8 * g + 1; w < 8 * g + 8; ++w) m8[g] = max(m8[g], acc[u][w >> 4][w & 15]);
            }
            const int32_t m = max(max(m8[0], m8[1]), max(m8[2], m8[3]));
            if (!__ballot(m >= bound[u])) continue;  // no lane of the wave passes
            const uint32_t qloc = uint32_t(wq * 128 + u * 32 + l32);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (!__ballot(m8[g] >= bound[u])) continue;
#pragma unroll
                for (int w = 8 * g; w < 8 * g + 8; ++w) {
                    const int b = w >> 4, v = w & 15;
                    const bool p = acc[u][b][v] >= bound[u];
                    const uint64_t mk = __ballot(p);  // lanes passing at this position
                    if (!mk) continue;
                    if (p) {
                        const uint32_t e =
                            wc + __builtin_amdgcn_mbcnt_hi(uint32_t(mk >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mk), 0u));
                        const uint32_t key = key_of_i32(-acc[u][b][v]);
                        const uint32_t id = nbase + uint32_t(b * 32 + 8 * (v >> 2) + 4 * hh + (v & 3));
                        if (e < WCAP) {
                            s_qi[wbase + e] = qloc;
                            s_key[wbase + e] = key;
                            s_id[wbase + e] = id;
                        } else {  // slice full: reserve and write directly
                            const uint32_t qi = q0 + qloc;
                            const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                            if (pos < a.cap) {
                                a.cand_key[int64_t(qi) * a.cap + pos] = key;
                                a.cand_id[int64_t(qi) * a.cap + pos] = id;
                            }
                        }
                    }
                    wc += uint32_t(__popcll(mk));
                }
            }
        }
        if (lane == 0) s_cnt[wave] = min(wc, WCAP);
        __syncthreads();  // staged entries and counts visible
        for (uint32_t e = uint32_t(tid); e < uint32_t(STAGED); e += 256) {
            if (e % WCAP >= s_cnt[e / WCAP]) continue;
            const uint32_t qi = q0 + s_qi[e];
            const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
            if (pos < a.cap) {
                a.cand_key[int64_t(qi) * a.cap + pos] = s_key[e];
                a.cand_id[int64_t(qi) * a.cap + pos] = s_id[e];
            }
        }
    } else {
        // Dense keys leave through LDS: each wave writes a 32-query x 64-row block of keys (rows
        // padded to 65 words, conflict-free both ways), then stores it row by row with the 64
        // lanes on consecutive rows of the output, 256 contiguous bytes per store instead of
        // 64 scattered words.
        __syncthreads();  // every wave is past its last read of the ring
        uint32_t* tile = reinterpret_cast<uint32_t*>(lds8) + wave * (32 * 65);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        tile[l32 * 65 + b * 32 + 8 * j + 4 * hh + e] = key_of_i32(-acc[u][b][4 * j + e]);
            __syncthreads();
            const uint32_t m = nbase + uint32_t(lane);
            for (int q = 0; q < 32; ++q) {
                const uint32_t qi = q0 + uint32_t(wq * 128 + u * 32 + q);
                if (qi < a.Q && m < a.N) a.out_k[int64_t(qi) * a.ldo + m] = tile[q * 65 + lane];
            }
            __syncthreads();  // the block is read before the next one overwrites it
        }
    }
}

template <bool FILTER>
va_status launch_i8_dma(va_context* ctx, const I8Args& a) {
    using namespace dmai8;
    const uint64_t ntb = (a.N + TN - 1) / TN;
    const uint64_t grid = uint64_t((a.Q + TQ - 1) / TQ) * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "int8 scan grid too large");
    auto kern = &i8_dma_kernel<FILTER>;
    VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, int(LDS_BYTES)));
    kern<<<dim3(uint32_t(grid)), dim3(256), LDS_BYTES, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// ---------------------------------------------------------------------------------------
// int8 filter scan with resident queries (large Q, d <= 512)
// ---------------------------------------------------------------------------------------
// A workgroup keeps 256 queries resident in LDS for its whole life and streams a contiguous
// range of database tiles past them.  Each of its eight waves owns 32 rows of a 256-row tile
// and moves them through a private 3-slot LDS ring (a slot is one 32-byte k-step of its 32
// rows, 1 KiB) by direct buffer loads issued two k-steps ahead.  Nothing but the initial
// query load is shared between waves, so the main loop has no workgroup barrier: with one
// 8-wave workgroup per CU (the queries take 128 KiB of the 160 KiB LDS) a barrier per k-step
// cost about a third of the MFMA rate.  Wave tile 256 queries x 32 rows = 8 MFMA blocks (128
// accumulators); the operands of k-step t+1 are read from LDS while the MFMAs of step t run.
// Workgroup w runs on XCD w % 8 and the q-blocks that share a database range sit on one XCD,
// so a range comes from HBM once per XCD L2 and then from L2 for the other q-blocks.
// Filter passes are staged in a per-wave LDS list and appended to the per-query candidate
// lists only when the list fills (and at the end): a global reservation is an atomic whose
// result the wave must wait for, and even plain stores count in the same in-order wait
// counter as the stage loads, so writing passes out at every tile stalled the stream.
namespace resq {
constexpr int TQ = 256, NW = 8, WR = 32, NS = 3, SLOT = WR * 32;
constexpr int TN = NW * WR;           // rows per tile
constexpr int RING = NW * NS * SLOT;  // 24 KiB
constexpr int LCAP = 80;              // staged passes per wave
constexpr int STAGE = NW * LCAP * 12;
template <int QS>
constexpr int lds_bytes() { return TQ * QS + RING + STAGE; }
}  // namespace resq

// FULL: d % 64 == 0, so every k-step of a tile reads real bytes (no zero padding step).
template <int QS, bool FULL>
__global__ __launch_bounds__(512, 2) void i8_resq_kernel(I8Args a, uint32_t R) {
    using namespace resq;
    constexpr int QBYTES = TQ * QS;
    constexpr int CPR = QS / 16;    // 16-byte chunks per resident query row
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hh = lane >> 5;

    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t range = (seq / nqb) * kXcds + xcd;
    const uint32_t ntiles = (a.N + TN - 1) / TN;
    const uint32_t tpr = (ntiles + R - 1) / R;
    const uint32_t t0 = range * tpr;
    if (t0 >= ntiles) return;  // the whole workgroup: no range left
    const uint32_t tcount = min(tpr, ntiles - t0);
    const uint32_t q0 = qb * TQ;
    const uint32_t qn = min(uint32_t(TQ), a.Q - q0);
    const uint32_t lds0 = lds_addr_of(lds8);

    // Resident queries, chunk-major: 16-byte chunk c of query r at c * 4096 + r * 16.  The 32
    // queries of a block read one chunk as 512 contiguous bytes (no bank conflicts, no swizzle)
    // and the 8 blocks of a k-step lie within a 16-bit DS offset of one address.  A load
    // instruction fills chunk m / 4 of 64 consecutive queries.  Queries past Q and chunks past
    // D load as zeros.
    {
        const dma_rsrc qres = make_dma_rsrc(a.q + int64_t(q0) * a.ldq, uint32_t(int64_t(qn - 1) * a.ldq + a.D));
        for (int m = wave; m < 4 * CPR; m += NW) {
            const int row = (m & 3) * 64 + lane;
            const int c = m >> 2;
            const uint32_t voff = (uint32_t(row) < qn && uint32_t(16 * c) < a.D)
                                      ? uint32_t(int64_t(row) * a.ldq) + uint32_t(16 * c)
                                      : kDmaSkip;
            lds_dma16(qres, voff, lds0 + uint32_t(m) * 1024u);
        }
    }
    // A value passes when its dot is >= the query's bound (the threshold key turned back into
    // an int32 dot); padding queries never pass.
    int32_t bound[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const uint32_t ql = uint32_t(u * 32 + l32);
        const int32_t t = i32_of_key(a.thr[q0 + (ql < qn ? ql : 0u)]);
        bound[u] = (ql >= qn || t == INT32_MIN) ? INT32_MAX : -t;
    }
    wait_vmcnt<0>();
    __syncthreads();  // resident queries visible; the only workgroup barrier

    // ---- this wave's database stream ------------------------------------------------------
    const uint32_t nst = (a.D + 63) / 64 * 2;  // k-steps per tile, even (a padding step loads zeros)
    const uint32_t steps = tcount * nst;
    const uint32_t ring = lds0 + uint32_t(QBYTES) + uint32_t(wave) * uint32_t(NS * SLOT);
    const char* ringp = lds8 + QBYTES + wave * (NS * SLOT);
    // DMA lane map: row lane / 2; slot position lane & 1 holds the row's 16-byte chunk
    // (lane & 1) ^ ((row >> 3) & 1), which keeps rows r and r + 8 apart in the banks.
    const int drow = lane >> 1;
    const uint32_t dcol = 16u * uint32_t((lane & 1) ^ ((drow >> 3) & 1));
    const uint32_t drow_off = uint32_t(int64_t(drow) * a.ldx);
    uint32_t ltile = 0, lst = 0, lslot = 0;
    // The descriptor covers this wave's 32 rows of the tile being loaded; it is rebuilt from
    // scalars at every load (a few scalar ops), which keeps it out of vector registers.  With
    // FULL rows the k-step's column goes in the scalar offset and a lane's vector offset is
    // fixed; rows past N fail the range check through it.
    auto issue = [&]() {
        // 32-bit row arithmetic (N <= 2^32 - 256): a 64-bit compare would run on the VALU
        const uint32_t r0 = (t0 + ltile) * uint32_t(TN) + uint32_t(wave) * uint32_t(WR);
        const uint32_t rows = r0 < a.N ? min(uint32_t(WR), a.N - r0) : 0u;
        const dma_rsrc xres =
            make_dma_rsrc(a.x + int64_t(r0) * a.ldx, rows ? uint32_t(int64_t(rows - 1) * a.ldx + a.D) : 0u);
        if (FULL) {
            lds_dma16_so(xres, drow_off + dcol, lst * 32, ring + lslot * uint32_t(SLOT));
        } else {
            const uint32_t d = lst * 32 + dcol;
            lds_dma16(xres, d < a.D ? drow_off + d : kDmaSkip, ring + lslot * uint32_t(SLOT));
        }
        lslot = lslot == NS - 1 ? 0u : lslot + 1;
        if (++lst == nst) {
            lst = 0;
            ++ltile;
        }
    };

    // Operand reads: query block u row 32u + l32, database row l32, k-chunk 2 * step + hh.
    // One register set: the query fragment u of k-step t+1 is read right after the MFMA of
    // step t that consumed fragment u (eight MFMAs cover the read latency); the database
    // fragment alternates between two registers.  The first k-step of a tile starts from a
    // zero accumulator (inline constant), so tiles need no clearing pass.
    const char* qrd = lds8 + hh * 4096 + l32 * 16;
    const int xrd = l32 * 32 + 16 * (hh ^ ((l32 >> 3) & 1));
    auto rd_q = [&](uint32_t st, int u) { return *reinterpret_cast<const i32x4v*>(qrd + st * 8192 + u * 512); };
    auto rd_x = [&](uint32_t slot) { return *reinterpret_cast<const i32x4v*>(ringp + slot * SLOT + xrd); };

    i32x16 acc[8];

    // ---- filter epilogue ------------------------------------------------------------------
    uint32_t* s_qi = reinterpret_cast<uint32_t*>(lds8 + QBYTES + RING) + wave * 3 * LCAP;
    uint32_t* s_key = s_qi + LCAP;
    uint32_t* s_id = s_key + LCAP;
    uint32_t lc = 0;  // staged passes (wave-uniform)
    uint32_t mtile = 0;
    // Appends the staged passes to the candidate lists: count every pass, keep a query's first
    // cap.  The reservations are waited for once per 64 entries.
    auto flush = [&]() {
        for (uint32_t b0 = 0; b0 < lc; b0 += 64) {
            const uint32_t e = b0 + uint32_t(lane);
            if (e < lc) {
                const uint32_t qi = s_qi[e];
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    a.cand_key[int64_t(qi) * a.cap + pos] = s_key[e];
                    a.cand_id[int64_t(qi) * a.cap + pos] = s_id[e];
                }
            }
        }
        lc = 0;
    };
    // Lane value v of an MFMA block is row 8 * (v >> 2) + 4 * hh + (v & 3) of the wave's 32.
    // Passes are rare, so the test is cheap first (a lane's 16 values of a query reduced to a
    // maximum, one wave-wide vote per query block) and exact only where that vote passes: one
    // vote per value position, then a rolled loop over the positions some lane passes at (a
    // wave-uniform position, so the value is read with an indexed register move).  Rows past
    // N hold zero dots and are rejected there.  The code stays compact: an unrolled test of all
    // 128 positions with the append logic inlined in each outgrew the instruction cache and the
    // register budget.
    auto epilogue = [&]() {
        const uint64_t r64 = uint64_t(t0 + mtile) * TN + uint32_t(wave) * WR;
        const uint32_t r0 = uint32_t(r64);  // ids of rows below N fit 32 bits
        const int32_t lim = int32_t(r64 < a.N ? min(uint64_t(a.N) - r64, uint64_t(WR)) : 0) - 4 * hh;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int32_t b = bound[u];
            int32_t m = acc[u][0];
#pragma unroll
            for (int v = 1; v < 16; ++v) m = max(m, acc[u][v]);
            if (!__ballot(m >= b)) continue;
            const uint32_t qi = q0 + uint32_t(u * 32 + l32);
            // value positions where some lane passes (wave-uniform bits)
            uint32_t vm = 0;
#pragma unroll
            for (int v = 0; v < 16; ++v) vm |= __ballot(acc[u][v] >= b) ? (1u << v) : 0u;
#pragma unroll 1
            while (vm) {
                const uint32_t v = __builtin_ctz(vm);
                vm &= vm - 1;
                const int32_t dot = acc[u][v];
                const uint32_t roff = 8 * (v >> 2) + (v & 3);
                const bool p = dot >= b && int32_t(roff) < lim;
                const uint64_t mk = __ballot(p);
                if (!mk) continue;
                const uint32_t n = uint32_t(__popcll(mk));
                if (lc + n > uint32_t(LCAP)) flush();  // wave-uniform
                if (p) {
                    const uint32_t e =
                        lc + __builtin_amdgcn_mbcnt_hi(uint32_t(mk >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mk), 0u));
                    s_qi[e] = qi;
                    s_key[e] = key_of_i32(-dot);
                    s_id[e] = r0 + roff + 4 * uint32_t(hh);
                }
                lc += n;
            }
        }
    };

    // ---- main loop ------------------------------------------------------------------------
    // k-steps run in pairs; nst is even, so a tile ends only after the second of a pair and the
    // epilogue has one call site.
    for (int i = 0; i < NS - 1; ++i)
        if (uint32_t(i) < steps) issue();
    i32x4v bq[8], xa, xb;
#pragma unroll
    for (int u = 0; u < 8; ++u) bq[u] = rd_q(0, u);
    {
        const uint32_t after = min(uint32_t(NS - 1), steps) - 1;  // stages issued after stage 0
        if (after >= 1) wait_vmcnt<1>();
        else wait_vmcnt<0>();
    }
    xa = rd_x(0);
    uint32_t mst = 0;  // k-step within the tile
    // k-step t with database fragment cx; reads the next step's operands: the database
    // fragment first (a whole step ahead of its use), then each query fragment right after the
    // MFMA that consumed its register.
    auto step = [&](uint32_t t, const i32x4v& cx, i32x4v& nx, bool first) {
        // Refills the slot of stage t-1, read at the start of step t-2; 17 LDS reads were
        // issued after that one and at most 15 can be outstanding, so it has completed.
        if (t + NS - 1 < steps) issue();
        if (t + 1 < steps) {
            const uint32_t after = min(t + NS, steps) - (t + 2);  // stages issued after stage t+1
            if (after >= 1) wait_vmcnt<1>();
            else wait_vmcnt<0>();
            nx = rd_x((t + 1) % NS);
        }
        const uint32_t nst1 = mst + 1 == nst ? 0u : mst + 1;  // k-step of t+1 within its tile
        if (first) {
            const i32x16 z = {};
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cx, bq[u], z, 0, 0, 0);
                bq[u] = rd_q(nst1, u);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cx, bq[u], acc[u], 0, 0, 0);
                bq[u] = rd_q(nst1, u);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
        mst = nst1;
    };
    for (uint32_t t = 0; t < steps; t += 2) {
        if (mst == 0) step(t, xa, xb, true);
        else step(t, xa, xb, false);
        step(t + 1, xb, xa, false);
        if (mst == 0) {
            epilogue();
            ++mtile;
        }
    }
    flush();
}

// ---- resident queries on the 16x16x64 MFMA, rows straight into registers ----------------------
// The filter scan for d = 256, 512, 768 and 1024.  A workgroup (8 waves, one per CU) holds TQ
// queries in LDS (256 at d <= 512, 128 above) and streams a range of 256-row tiles past them; a
// wave's part of a tile is 32 database rows x the TQ queries = 2 x TQ/16 blocks of
// v_mfma_i32_16x16x64_i8.  Its rows go from global memory straight into a ring of R register
// slots (one 64-byte k-step of its 32 rows each; R = 4 at d <= 512, a whole tile of d / 64
// k-steps above): the slot a k-step consumed is refilled at once, R - 1 k-steps ahead, and no
// LDS write, wait or barrier sits between a load and its MFMA.  LDS carries the query fragments
// (each read once per k-step and used by two MFMAs).  Load and fragment map: lane (r, g) =
// (lane % 16, lane / 16) holds bytes 64 t + 16 g .. + 15 of row r of a row block (and of query r
// of a query block) at k-step t, so the four lanes of a row read 64 contiguous bytes per
// instruction, and both operands pair the same d.  Rows past N, and the loads past a wave's
// last tile, use an offset beyond the descriptor's range (zeros; every lane's offset carries its
// row, so this does not depend on whether the range check includes the scalar column offset).
// Measured on one box against the kernels it replaced (Q = 4096, random int8 rows, scan time):
// d = 512 15.6 ms against i8_resq_kernel's 19.9 (0.53 of the int8 peak), d = 256 8.2 against
// 10.7, d = 768 and 1024 18.4 and 18.3 against i8_dma_kernel's 22.2 and 22.7.  What moved it:
// the bytes each CU pulls from L2 per MFMA (a row fetched once per 256 queries instead of 128:
// 18.5 -> 15.6 ms at d = 512) and loads kept in flight (the register ring).  What did not:
// cutting the LDS bytes per MFMA to a third (64-row wave tiles), 16-row wave tiles, two
// workgroups per CU, 192 resident queries at d = 768 (blocks of 192 do not tile 256 CUs).
namespace resq16 {
constexpr int NW = 8, MB = 2;  // waves, row blocks of 16 per wave
constexpr int WR = 16 * MB;    // rows per wave
constexpr int TN = NW * WR;    // rows per tile
constexpr int TQMAX = 256;     // resident queries at most
constexpr int LCAP = 80;       // staged passes per wave
constexpr int STAGE = NW * LCAP * 12;
template <int QS, int NQB>
constexpr int lds_bytes() { return 16 * NQB * QS + STAGE; }
}  // namespace resq16

// QS = D, a multiple of 256; NQB query blocks of 16 (TQ = 16 NQB resident queries); a ring of
// R k-steps, R dividing the tile's D / 64.
template <int QS, int NQB, int R>
__global__ __launch_bounds__(512, 2) void i8_resq16_kernel(I8Args a, uint32_t NR) {
    using namespace resq16;
    static_assert((QS / 64) % R == 0, "the ring's slots must repeat tile by tile");
    constexpr int TQ = 16 * NQB;
    constexpr int CS = TQ * 16;  // bytes per 16-byte chunk column of the resident queries
    constexpr int QBYTES = TQ * QS;
    constexpr int CPR = QS / 16;  // 16-byte chunks per resident query row
    extern __shared__ __attribute__((aligned(16))) char lds8[];
    const int tid = threadIdx.x;
    const int lane = tid & 63, r16 = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Workgroup w runs on XCD w % 8; the query blocks of one range of tiles share an XCD, so
    // the range comes from HBM about once and from that XCD's L2 for the other blocks.  (Giving
    // each XCD one range that its streams interleave over, tile by tile, measured 5 % slower.)
    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t range = (seq / nqb) * kXcds + xcd;
    const uint32_t ntiles = (a.N + TN - 1) / TN;
    const uint32_t tpr = (ntiles + NR - 1) / NR;
    const uint32_t t0 = range * tpr;
    if (t0 >= ntiles) return;  // the whole workgroup: no range left
    const uint32_t tcount = min(tpr, ntiles - t0);
    const uint32_t q0 = qb * TQ;
    const uint32_t qn = min(uint32_t(TQ), a.Q - q0);
    const uint32_t lds0 = lds_addr_of(lds8);

    // Resident queries, chunk-major: 16-byte chunk c of query r at c * CS + r * 16 (a query
    // block's 16 queries read 256 contiguous bytes per lane group).  One load fills one chunk of
    // 64 consecutive queries; queries past Q load as zeros.
    {
        constexpr int G64 = TQ / 64;  // loads per chunk column
        const dma_rsrc qres = make_dma_rsrc(a.q + int64_t(q0) * a.ldq, uint32_t(int64_t(qn - 1) * a.ldq + a.D));
        for (int m = wave; m < G64 * CPR; m += NW) {
            const int row = (m % G64) * 64 + lane;
            const int c = m / G64;
            const uint32_t voff = uint32_t(row) < qn ? uint32_t(int64_t(row) * a.ldq) + uint32_t(16 * c) : kDmaSkip;
            lds_dma16(qres, voff, lds0 + uint32_t(m) * 1024u);
        }
    }
    // A value passes when its dot is >= the query's bound (the threshold key turned back into
    // an int32 dot); padding queries never pass.
    int32_t bound[NQB];
#pragma unroll
    for (int u = 0; u < NQB; ++u) {
        const uint32_t ql = uint32_t(u * 16 + r16);
        const int32_t t = i32_of_key(a.thr[q0 + (ql < qn ? ql : 0u)]);
        bound[u] = (ql >= qn || t == INT32_MIN) ? INT32_MAX : -t;
    }
    wait_vmcnt<0>();
    __syncthreads();  // resident queries visible; the only workgroup barrier

    // ---- this wave's row stream ---------------------------------------------------------------
    constexpr uint32_t nst = QS / 64;  // k-steps per tile
    uint32_t voff[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) voff[j] = uint32_t(16 * j + r16) * uint32_t(a.ldx) + 16u * uint32_t(g);
    uint32_t ltile = 0, lst = 0;  // tile and k-step of the next load (wave-uniform)
    // The descriptor covers this wave's rows of the tile being loaded ((rows - 1) strides plus
    // one row), rebuilt from scalars at every load; a lane's row offset fails its range check
    // for rows past N.
    auto load = [&](i32x4v(&dst)[MB]) {
        // (wave-uniform values; readfirstlane keeps the descriptor in scalar registers where the
        // compiler's divergence analysis cannot prove it, which would otherwise loop over lanes)
        const bool ok = ltile < tcount;
        const uint32_t r0 =
            __builtin_amdgcn_readfirstlane(ok ? (t0 + ltile) * uint32_t(TN) + uint32_t(wave) * uint32_t(WR) : 0u);
        const uint32_t rows = __builtin_amdgcn_readfirstlane(ok && r0 < a.N ? min(uint32_t(WR), a.N - r0) : 0u);
        const uint64_t base = reinterpret_cast<uint64_t>(a.x + int64_t(r0) * a.ldx);
        const uint64_t bs = (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(base >> 32)))) << 32) |
                            uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(base)));
        const int nrec = __builtin_amdgcn_readfirstlane(rows ? int(int64_t(rows - 1) * a.ldx + a.D) : 0);
        const __amdgpu_buffer_rsrc_t xres =
            __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(bs), 0, nrec, 0x00020000);
        const uint32_t skip = rows ? 0u : kDmaSkip;  // (offsets are below 2^31: OR-ing it in puts them out of range)
#pragma unroll
        for (int j = 0; j < MB; ++j)
            dst[j] = __builtin_bit_cast(
                i32x4v, __builtin_amdgcn_raw_buffer_load_b128(xres, voff[j] | skip, int(lst * 64u), 0));
        if (++lst == nst) {
            lst = 0;
            ++ltile;
        }
    };

    // query block u of k-step t: chunk 4 t + g of query 16 u + r16
    const char* qrd = lds8 + g * CS + r16 * 16;
    auto rd_q = [&](uint32_t t, int u) { return *reinterpret_cast<const i32x4v*>(qrd + t * (4 * CS) + u * 256); };

    // acc[u][j]: lane (r16, g) holds query 16 u + r16 against rows 16 j + 4 g + v in value v
    i32x4v acc[NQB][MB];

    // ---- filter epilogue ----------------------------------------------------------------------
    uint32_t* s_qi = reinterpret_cast<uint32_t*>(lds8 + QBYTES) + wave * 3 * LCAP;
    uint32_t* s_key = s_qi + LCAP;
    uint32_t* s_id = s_key + LCAP;
    uint32_t lc = 0;  // staged passes (wave-uniform)
    uint32_t mtile = 0;
    // Appends the staged passes to the candidate lists: count every pass, keep a query's first
    // cap.  The reservations are waited for once per 64 entries.
    auto flush = [&]() {
        for (uint32_t b0 = 0; b0 < lc; b0 += 64) {
            const uint32_t e = b0 + uint32_t(lane);
            if (e < lc) {
                const uint32_t qi = s_qi[e];
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    a.cand_key[int64_t(qi) * a.cap + pos] = s_key[e];
                    a.cand_id[int64_t(qi) * a.cap + pos] = s_id[e];
                }
            }
        }
        lc = 0;
    };
    // Passes are rare: a lane's 4 MB values of a query block reduced to a maximum and one wave
    // vote per block, then one vote per value position and a rolled loop over the positions
    // some lane passes at (wave-uniform, the value picked by a select chain).  Rows past N hold
    // zero dots and are rejected by their position.
    auto epilogue = [&]() {
        const uint64_t r64 = uint64_t(t0 + mtile) * TN + uint32_t(wave) * WR;
        const uint32_t r0 = uint32_t(r64);  // ids of rows below N fit 32 bits
        const int32_t lim = int32_t(r64 < a.N ? min(uint64_t(a.N) - r64, uint64_t(WR)) : 0) - 4 * g;
#pragma unroll
        for (int u = 0; u < NQB; ++u) {
            const int32_t b = bound[u];
            int32_t m = acc[u][0][0];
#pragma unroll
            for (int j = 0; j < MB; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) m = max(m, acc[u][j][v]);
            if (!__ballot(m >= b)) continue;
            const uint32_t qi = q0 + uint32_t(u * 16 + r16);
            uint32_t vm = 0;  // bit 4 j + v: some lane passes there (wave-uniform)
#pragma unroll
            for (int j = 0; j < MB; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) vm |= __ballot(acc[u][j][v] >= b) ? (1u << (4 * j + v)) : 0u;
#pragma unroll 1
            while (vm) {
                const uint32_t p = __builtin_ctz(vm);
                vm &= vm - 1;
                int32_t dot = 0;
#pragma unroll
                for (int j = 0; j < MB; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v) dot = p == uint32_t(4 * j + v) ? acc[u][j][v] : dot;
                const uint32_t roff = 16 * (p >> 2) + (p & 3);
                const bool pass = dot >= b && int32_t(roff) < lim;
                const uint64_t mk = __ballot(pass);
                if (!mk) continue;
                const uint32_t n = uint32_t(__popcll(mk));
                if (lc + n > uint32_t(LCAP)) flush();  // wave-uniform
                if (pass) {
                    const uint32_t e =
                        lc + __builtin_amdgcn_mbcnt_hi(uint32_t(mk >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mk), 0u));
                    s_qi[e] = qi;
                    s_key[e] = key_of_i32(-dot);
                    s_id[e] = r0 + roff + 4 * uint32_t(g);
                }
                lc += n;
            }
        }
    };

    // ---- main loop: groups of R k-steps (a tile is a whole number of groups) -----------------
    i32x4v xr[R][MB];
    // four query fragments in turn: block u uses qf[u % 4], refilled after its two MFMAs with
    // block u + 4 of this k-step or block u + 4 - NQB of the next (eight MFMAs cover the read)
    constexpr int QF = 4;
    i32x4v qf[QF];
    // (in order: the compiler's wait counts follow the issue order, and the first k-step's slot
    // must be the oldest load in flight)
#pragma unroll
    for (int r = 0; r < R - 1; ++r) {
        load(xr[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < QF; ++u) qf[u] = rd_q(0, u);
    uint32_t mst = 0;  // k-step within the tile
    auto mma = [&](const i32x4v(&x)[MB]) {
        const uint32_t nks = mst + 1 == nst ? 0u : mst + 1;
#pragma unroll
        for (int u = 0; u < NQB; ++u) {
#pragma unroll
            for (int j = 0; j < MB; ++j)
                acc[u][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[j], qf[u % QF], acc[u][j], 0, 0, 0);
            qf[u % QF] = u + QF < NQB ? rd_q(mst, u + QF) : rd_q(nks, u + QF - NQB);
            __builtin_amdgcn_sched_group_barrier(0x008, MB, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        mst = nks;
    };
#pragma unroll
    for (int u = 0; u < NQB; ++u)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[u][j] = i32x4v{0, 0, 0, 0};
    for (uint32_t t = 0; t < tcount; ++t) {
        // The whole ring has landed before a tile starts (its first k-step needs only the oldest
        // slot): measured 2-4 % faster than waiting slot by slot (d = 512 and 1024).
        wait_vmcnt<0>();
#pragma unroll
        for (int r = 0; r < int(nst); ++r) {
            load(xr[(r + R - 1) % R]);  // the slot the previous k-step consumed
            mma(xr[r % R]);
            __builtin_amdgcn_sched_barrier(0);
        }
        epilogue();
        ++mtile;
#pragma unroll
        for (int u = 0; u < NQB; ++u)
#pragma unroll
            for (int j = 0; j < MB; ++j) acc[u][j] = i32x4v{0, 0, 0, 0};
    }
    flush();
}

// The resident-query scan needs dense 16-byte query and database rows, d <= 512, enough
// queries to fill a 256-query block reasonably, and 32-bit descriptor offsets within a
// 256-query block and within a wave's 32 rows.
bool resq_ok(const I8Args& a, bool vec) {
#ifndef VA_I8_RESQ
#define VA_I8_RESQ 1
#endif
    return VA_I8_RESQ && vec && !a.qrow && a.Q > 192 && a.D <= 512 && a.N <= 0xFFFFFF00u &&
           uint64_t(resq::TQ - 1) * uint64_t(a.ldq) + a.D <= kDmaMaxBytes &&
           uint64_t(resq::WR - 1) * uint64_t(a.ldx) + a.D <= kDmaMaxBytes;
}

// The 16x16x64 layout: d in {256, 512, 768, 1024} (at most 128 KiB of resident queries and a
// register ring of 16 k-steps), and 32-bit descriptor offsets within a 128-query block and a
// wave's 32 rows.
bool resq16_ok(const I8Args& a, bool vec) {
#ifndef VA_I8_RESQ16
#define VA_I8_RESQ16 1
#endif
    return VA_I8_RESQ16 && vec && !a.qrow && a.Q > 192 && a.D % 256 == 0 && a.D <= 1024 &&
           a.N <= 0xFFFFFE00u && uint64_t(resq16::TQMAX - 1) * uint64_t(a.ldq) + a.D <= kDmaMaxBytes &&
           uint64_t(resq16::WR - 1) * uint64_t(a.ldx) + a.D <= kDmaMaxBytes;
}

va_status launch_i8_resq16(va_context* ctx, const I8Args& a) {
    using namespace resq16;
    // 256 resident queries where they fit beside the stage lists (d <= 512), else 128
    const uint32_t TQ = a.D <= 512 ? 256u : 128u;
    // one workgroup per CU (the registers of 8 waves), the number of ranges a multiple of the
    // XCD count
    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t per = (uint32_t(std::max(ctx->num_cus, 8)) + nqb - 1) / nqb;
    const uint32_t NR = std::max<uint32_t>(kXcds, (per + kXcds - 1) / kXcds * kXcds);
    const uint64_t grid = uint64_t(nqb) * NR;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "int8 scan grid too large");
    auto go = [&](auto kern, int lds) -> va_status {
        VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, lds));
        kern<<<dim3(uint32_t(grid)), dim3(512), lds, ctx->stream>>>(a, NR);
        return VA_OK;
    };
    va_status st;
    switch (a.D) {
        case 256: st = go(&i8_resq16_kernel<256, 16, 4>, lds_bytes<256, 16>()); break;
        case 512: st = go(&i8_resq16_kernel<512, 16, 4>, lds_bytes<512, 16>()); break;
        case 768: st = go(&i8_resq16_kernel<768, 8, 12>, lds_bytes<768, 8>()); break;
        default: st = go(&i8_resq16_kernel<1024, 8, 16>, lds_bytes<1024, 8>());
    }
    if (st != VA_OK) return st;
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status launch_i8_resq(va_context* ctx, const I8Args& a) {
    using namespace resq;
    // one workgroup per CU (LDS-bound), the number of ranges a multiple of the XCD count
    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t per = (uint32_t(std::max(ctx->num_cus, 8)) + nqb - 1) / nqb;
    const uint32_t R = std::max<uint32_t>(kXcds, (per + kXcds - 1) / kXcds * kXcds);
    const uint64_t grid = uint64_t(nqb) * R;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "int8 scan grid too large");
    const bool full = a.D % 64 == 0;
    auto go = [&](auto kern, int lds) -> va_status {
        VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, lds));
        kern<<<dim3(uint32_t(grid)), dim3(512), lds, ctx->stream>>>(a, R);
        return VA_OK;
    };
    va_status st;
    if (a.D <= 256)
        st = full ? go(&i8_resq_kernel<256, true>, lds_bytes<256>()) : go(&i8_resq_kernel<256, false>, lds_bytes<256>());
    else
        st = full ? go(&i8_resq_kernel<512, true>, lds_bytes<512>()) : go(&i8_resq_kernel<512, false>, lds_bytes<512>());
    if (st != VA_OK) return st;
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

template <int QBW, int WQ, int WN>
va_status launch_i8_shape(va_context* ctx, const I8Args& a, bool vec, bool filter) {
    if (filter) return vec ? launch_i8_tile<QBW, WQ, WN, true, true>(ctx, a) : launch_i8_tile<QBW, WQ, WN, false, true>(ctx, a);
    return vec ? launch_i8_tile<QBW, WQ, WN, true, false>(ctx, a) : launch_i8_tile<QBW, WQ, WN, false, false>(ctx, a);
}

// whole, aligned 16-byte chunks in every query and database row
bool i8_vec(const I8Args& a) {
    return (a.D % 16 == 0) && (a.ldq % 16 == 0) && (a.ldx % 16 == 0) &&
           ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
}

va_status launch_i8(va_context* ctx, const I8Args& a, bool filter) {
    if (a.Q == 0 || a.N == 0) return VA_OK;
    const bool vec = i8_vec(a);
    if (filter && resq16_ok(a, vec)) return launch_i8_resq16(ctx, a);
    if (filter && resq_ok(a, vec)) return launch_i8_resq(ctx, a);
#ifndef VA_I8_DMA
#define VA_I8_DMA 1
#endif
    // The DMA pipeline needs whole 16-byte chunks, dense query rows (no indirection) and
    // descriptor offsets below 2^31.
    const bool dma_ok = VA_I8_DMA && vec && !a.qrow && a.Q > 192 && a.D <= 131071 &&
                        uint64_t(a.Q - 1) * uint64_t(a.ldq) + a.D <= kDmaMaxBytes &&
                        uint64_t(dmai8::TN - 1) * uint64_t(a.ldx) + a.D <= kDmaMaxBytes;
    if (dma_ok) return filter ? launch_i8_dma<true>(ctx, a) : launch_i8_dma<false>(ctx, a);
    if (a.Q <= 32) return launch_i8_shape<1, 1, 4>(ctx, a, vec, filter);
    if (a.Q <= 64) return launch_i8_shape<1, 2, 2>(ctx, a, vec, filter);
// Large-Q shape: 0 = 128 x 128 (4 waves), 1 = 128 x 256 (4 waves), 2 = 256 x 256 (8 waves).
// Measured on configs[2] (10M x 512, Q=4096): 0 is fastest with 64-byte register-staged
// stages (each stage's MFMA work is shorter than its load round trip, so a bigger tile only
// waits longer per stage).
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
    va_status fallback_pass(const FbArgs& a, int pass) override {
        return fb_launch_pass(ctx, FbI8{q, int64_t(D), x, int64_t(D), N, D}, a, pass);
    }
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
    I8Args filter_args() const {
        I8Args a;
        a.q = q;
        a.ldq = D;
        a.x = x;
        a.ldx = D;
        a.Q = Q;
        a.N = N;
        a.D = D;
        return a;
    }
    va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) override {
        I8Args a = filter_args();
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
    if (dim % 4 == 0 && dim <= 1024 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const uint32_t rows_per_step = 256 / (dim / 4);
        const uint64_t blocks = std::max<uint64_t>(
            1, std::min<uint64_t>(2048, (uint64_t(num_vectors) + rows_per_step - 1) / rows_per_step));
        va::minmax_kernel_v4<<<dim3(uint32_t(blocks)), dim3(256), 0, ctx->stream>>>(
            reinterpret_cast<const float4*>(x), num_vectors, dim / 4, kmin, kmax);
    } else {
        const uint32_t ycols = (dim + 255) / 256;
        // enough row blocks to cover the chip (about 2048 workgroups in total)
        uint64_t xblocks = std::max<uint64_t>(1, std::min<uint64_t>(num_vectors, 2048 / ycols + 1));
        const uint64_t rpb = (uint64_t(num_vectors) + xblocks - 1) / xblocks;
        xblocks = (uint64_t(num_vectors) + rpb - 1) / rpb;
        va::minmax_kernel<<<dim3(uint32_t(xblocks), ycols), dim3(256), 0, ctx->stream>>>(x, num_vectors, dim, rpb,
                                                                                           kmin, kmax);
    }
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
    const bool v4 = dim % 4 == 0 && dim <= 1024 &&
                    ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(scale) |
                      reinterpret_cast<uintptr_t>(zero_point)) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(codes) & 3) == 0;
    if (v4) {
        const uint32_t rows_per_step = 256 / (dim / 4);
        const uint64_t blocks = std::max<uint64_t>(
            1, std::min<uint64_t>(8192, (num_vectors + rows_per_step - 1) / rows_per_step));
        va::quantize_kernel_v4<<<dim3(uint32_t(blocks)), dim3(256), 0, ctx->stream>>>(
            reinterpret_cast<const float4*>(x), num_vectors, dim / 4, reinterpret_cast<const float4*>(scale),
            reinterpret_cast<const int4*>(zero_point), reinterpret_cast<char4*>(codes));
    } else
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
    // the int32 dot of two code vectors lies in [-16256 dim, 16384 dim]: exact below 2^31
    VA_REQUIRE(ctx, dim <= VA_I8_MAX_DIM, "va_i8_scan_topk: dim %u exceeds %u (int32 accumulation)", dim,
               VA_I8_MAX_DIM);
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
