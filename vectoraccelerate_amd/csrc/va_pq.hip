// va_pq.hip — product quantization: codebook training, encoding and the ADC (asymmetric distance)
// top-k scan.
//
// Replaces Metal4ProductQuantizationKernel (Kernels/Metal4/ProductQuantizationKernel.swift:221-560)
// and its shaders (Metal/Shaders/ProductQuantization.metal): pq_assignment_or_encoding (:61-101),
// pq_train_update_accumulate / _finalize (:103-189), pq_precompute_distance_table (:191-213) and
// pq_compute_distances_adc (:215-254).  A vector of dimension D is cut into M sub-vectors of
// D_sub = D / M values; sub-vector m is coded by the nearest of the K <= 256 centroids of codebook
// m (one byte).  The distance of a query to a coded row is sum_m table[m][code_m], table[m][k] =
// |q_m - c_mk|^2.
//
// Sub-vector distances follow the shader's calculate_l2_sq_dist order exactly: four fp32 lanes
// accumulate fma(diff, diff, acc) over the float4 blocks, the lanes add as ((x + y) + z) + w, the
// D_sub % 4 tail adds diff * diff one by one; so codes and tables equal the oracle's bit for bit.
// The ADC sum adds the M table entries in subspace order, as the shader does.
//
// Layout: codebooks [M x K x D_sub] fp32, codes [N x M] bytes (row-major, as the reference),
// tables [Q x M x K] fp32.  The ADC scan keeps the tables of a group of queries in LDS (up to
// 160 KB) and streams the code rows: every code row is read once per query group, and each
// (query, row) pair costs M LDS lookups, which bound the scan.
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>
#include <vector>

#include "va_fallback.hpp"
#include "va_internal.hpp"

namespace va {
namespace {

constexpr uint32_t kPQChunk = 256;  // points per partial centroid sum (fixed summation order)

__device__ __forceinline__ float sub_l2sq(const float* __restrict__ v, const float* __restrict__ c, uint32_t n) {
#pragma clang fp contract(off)  // the tail's diff * diff + s rounds twice, as in the shader
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    const uint32_t n4 = n / 4;
    for (uint32_t d = 0; d < n4; ++d) {
        const float e0 = v[4 * d] - c[4 * d], e1 = v[4 * d + 1] - c[4 * d + 1];
        const float e2 = v[4 * d + 2] - c[4 * d + 2], e3 = v[4 * d + 3] - c[4 * d + 3];
        a0 = __builtin_fmaf(e0, e0, a0);
        a1 = __builtin_fmaf(e1, e1, a1);
        a2 = __builtin_fmaf(e2, e2, a2);
        a3 = __builtin_fmaf(e3, e3, a3);
    }
    float s = ((a0 + a1) + a2) + a3;
    for (uint32_t d = n4 * 4; d < n; ++d) {
        const float e = v[d] - c[d];
        s = s + e * e;  // not fused: the pragma above covers expressions written here
    }
    return s;
}

// codes[n * M + m] = argmin_k |x_nm - c_mk|^2 (strict <: the lowest k on ties); one thread per
// (row, subspace), grid.y = subspace.  Centroids go in chunks of kAssignChunk: the thread's four
// values of a float4 block are loaded once and used for the whole chunk (4 accumulators per
// centroid, the sub_l2sq order), the centroids' values are the same for the whole wave.
constexpr uint32_t kAssignChunk = 16;
__global__ __launch_bounds__(256) void pq_assign(const float* __restrict__ x, uint32_t N, uint32_t D, uint32_t M,
                                                 uint32_t K, const float* __restrict__ cb, uint8_t* __restrict__ codes) {
#pragma clang fp contract(off)  // the tail's diff * diff + s rounds twice, as in the shader
    const uint32_t n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
    if (n >= N) return;
    const uint32_t ds = D / M, n4 = ds / 4;
    const float* v = x + int64_t(n) * D + int64_t(m) * ds;
    const float* cm = cb + int64_t(m) * K * ds;
    float best = __builtin_inff();
    uint32_t bk = 0;
    for (uint32_t k0 = 0; k0 < K; k0 += kAssignChunk) {
        const uint32_t kn = min(kAssignChunk, K - k0);
        float acc[kAssignChunk][4];
#pragma unroll
        for (uint32_t kk = 0; kk < kAssignChunk; ++kk) acc[kk][0] = acc[kk][1] = acc[kk][2] = acc[kk][3] = 0.0f;
        for (uint32_t d = 0; d < n4; ++d) {
            const float x0 = v[4 * d], x1 = v[4 * d + 1], x2 = v[4 * d + 2], x3 = v[4 * d + 3];
#pragma unroll
            for (uint32_t kk = 0; kk < kAssignChunk; ++kk) {
                if (kk < kn) {
                    const float* c = cm + int64_t(k0 + kk) * ds + 4 * d;
                    const float e0 = x0 - c[0], e1 = x1 - c[1], e2 = x2 - c[2], e3 = x3 - c[3];
                    acc[kk][0] = __builtin_fmaf(e0, e0, acc[kk][0]);
                    acc[kk][1] = __builtin_fmaf(e1, e1, acc[kk][1]);
                    acc[kk][2] = __builtin_fmaf(e2, e2, acc[kk][2]);
                    acc[kk][3] = __builtin_fmaf(e3, e3, acc[kk][3]);
                }
            }
        }
#pragma unroll
        for (uint32_t kk = 0; kk < kAssignChunk; ++kk) {
            if (kk < kn) {
                float t = ((acc[kk][0] + acc[kk][1]) + acc[kk][2]) + acc[kk][3];
                const float* c = cm + int64_t(k0 + kk) * ds;
                for (uint32_t d = n4 * 4; d < ds; ++d) {
                    const float e = v[d] - c[d];
                    t = t + e * e;
                }
                if (t < best) {
                    best = t;
                    bk = k0 + kk;
                }
            }
        }
    }
    codes[int64_t(n) * M + m] = uint8_t(bk);
}

// tables[q][m][k] = |q_m - c_mk|^2 (pq_precompute_distance_table)
__global__ __launch_bounds__(256) void pq_tables(const float* __restrict__ q, uint32_t D, uint32_t M, uint32_t K,
                                                 const float* __restrict__ cb, float* __restrict__ tables) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y, qi = blockIdx.z;
    if (k >= K) return;
    const uint32_t ds = D / M;
    tables[(int64_t(qi) * M + m) * K + k] =
        sub_l2sq(q + int64_t(qi) * D + int64_t(m) * ds, cb + (int64_t(m) * K + k) * ds, ds);
}

// ---- training: fixed-order sums per (subspace, centroid) -------------------------------------

__global__ __launch_bounds__(256) void pq_column(const uint8_t* __restrict__ codes, uint32_t N, uint32_t M, uint32_t m,
                                                 uint8_t* __restrict__ col, uint32_t* __restrict__ iota) {
    const uint32_t n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    col[n] = codes[int64_t(n) * M + m];
    iota[n] = n;
}

// first[k], counts[k], chunk counts of subspace m's sorted codes
__global__ __launch_bounds__(256) void pq_ranges(const uint8_t* __restrict__ sorted, uint32_t N, uint32_t K,
                                                 uint32_t* __restrict__ first, uint32_t* __restrict__ counts,
                                                 uint32_t* __restrict__ chunks) {
    const uint32_t k = blockIdx.x * 256 + threadIdx.x;
    if (k >= K) return;
    auto lower = [&](uint32_t v) {
        uint32_t lo = 0, hi = N;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (uint32_t(sorted[mid]) < v) lo = mid + 1;
            else hi = mid;
        }
        return lo;
    };
    const uint32_t a = lower(k), b = lower(k + 1);
    first[k] = a;
    counts[k] = b - a;
    chunks[k] = (b - a + kPQChunk - 1) / kPQChunk;
}

// chunk sums of subspace m: chunk b (cluster from the inclusive scan chunk_end) sums its points'
// sub-vectors in point order
__global__ __launch_bounds__(256) void pq_chunk_sums(const float* __restrict__ x, uint32_t D, uint32_t ds, uint32_t m,
                                                     uint32_t K, const uint32_t* __restrict__ members,
                                                     const uint32_t* __restrict__ first,
                                                     const uint32_t* __restrict__ counts,
                                                     const uint32_t* __restrict__ chunk_end,
                                                     float* __restrict__ partial) {
    __shared__ uint32_t rows[kPQChunk];
    const uint32_t b = blockIdx.x;
    if (b >= chunk_end[K - 1]) return;
    uint32_t lo = 0, hi = K - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (chunk_end[mid] > b) hi = mid;
        else lo = mid + 1;
    }
    const uint32_t c = lo, n = counts[c];
    const uint32_t nch = (n + kPQChunk - 1) / kPQChunk;
    const uint32_t t = b - (chunk_end[c] - nch);
    const uint32_t p0 = first[c] + t * kPQChunk, cnt = min(kPQChunk, n - t * kPQChunk);
    if (threadIdx.x < cnt) rows[threadIdx.x] = members[p0 + threadIdx.x];
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < ds; d += 256) {
        float s = 0.0f;
        for (uint32_t i = 0; i < cnt; ++i) s += x[int64_t(rows[i]) * D + int64_t(m) * ds + d];
        partial[int64_t(b) * ds + d] = s;
    }
}

// new centroid = (chunk sums in order) * (1/count) (pq_train_update_finalize); empty keeps its
// value; movement_sq[m * K + k] = sum_d (old - new)^2 (0 when empty)
__global__ __launch_bounds__(64) void pq_finalize(uint32_t ds, uint32_t m, uint32_t K,
                                                  const uint32_t* __restrict__ counts,
                                                  const uint32_t* __restrict__ chunk_end,
                                                  const float* __restrict__ partial, float* __restrict__ cb,
                                                  float* __restrict__ movement) {
#pragma clang fp contract(off)  // movement rounds diff * diff and the add separately
    const uint32_t k = blockIdx.x * 64 + threadIdx.x;
    if (k >= K) return;
    const uint32_t n = counts[k];
    float mv = 0.0f;
    if (n > 0) {
        const uint32_t nch = (n + kPQChunk - 1) / kPQChunk, b0 = chunk_end[k] - nch;
        const float inv = 1.0f / float(n);
        float* c = cb + (int64_t(m) * K + k) * ds;
        for (uint32_t d = 0; d < ds; ++d) {
            float s = 0.0f;
            for (uint32_t t = 0; t < nch; ++t) s += partial[int64_t(b0 + t) * ds + d];
            const float nv = s * inv, ov = c[d];
            c[d] = nv;
            const float diff = ov - nv;
            mv = mv + diff * diff;
        }
    }
    movement[int64_t(m) * K + k] = mv;
}

// total movement sqrt(sum / (M K)), summed in index order by one thread
__global__ void pq_movement(const float* __restrict__ movement, uint32_t n, float* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float t = 0.0f;
    for (uint32_t i = 0; i < n; ++i) t += movement[i];
    *out = sqrtf(t / float(n));
}

__global__ __launch_bounds__(256) void pq_init(const float* __restrict__ x, uint32_t D, uint32_t M, uint32_t K,
                                               const uint32_t* __restrict__ rows, float* __restrict__ cb) {
    const uint32_t mk = blockIdx.x, m = mk / K;
    const uint32_t ds = D / M;
    for (uint32_t d = threadIdx.x; d < ds; d += 256)
        cb[int64_t(mk) * ds + d] = x[int64_t(rows[mk]) * D + int64_t(m) * ds + d];
}

// ---- ADC scan ----------------------------------------------------------------------------------

struct AdcArgs {
    const uint8_t* codes = nullptr;
    const float* tables = nullptr;  // [Q x M x K]
    uint32_t M = 0, K = 0;
    uint32_t QB = 1;                // queries per workgroup (tables in LDS)
    // queries q0 + i (or qrow[i]), i < nq; rows c0 + j * stride, j < cols
    const uint32_t* qrow = nullptr;
    uint32_t q0 = 0, nq = 0;
    uint32_t c0 = 0, cols = 0, stride = 1;
    // dense keys (or the fp32 sums themselves when out_f is set)
    uint32_t* out_k = nullptr;
    float* out_f = nullptr;
    int64_t ldo = 0;
    bool words = false;  // code rows 4-byte aligned (M % 4 == 0, aligned base): word loads
    // filter
    const uint32_t* thr = nullptr;
    uint32_t* cnt = nullptr;
    uint32_t* cand_key = nullptr;
    uint32_t* cand_id = nullptr;
    uint32_t cap = 0;
};

// grid: x = row blocks (each strides over the rows), y = query groups of QB
template <bool FILTER>
__global__ __launch_bounds__(256) void pq_adc_kernel(AdcArgs a) {
    extern __shared__ float tab[];  // [QB x M x K]
    const uint32_t g0 = blockIdx.y * a.QB;
    const uint32_t nqg = min(a.QB, a.nq - g0);
    const uint32_t MK = a.M * a.K;
    for (uint32_t i = 0; i < nqg; ++i) {
        const uint32_t qi = a.qrow ? a.qrow[g0 + i] : a.q0 + g0 + i;
        const float* src = a.tables + int64_t(qi) * MK;
        for (uint32_t e = threadIdx.x; e < MK; e += 256) tab[i * MK + e] = src[e];
    }
    __syncthreads();
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < a.cols; j += gridDim.x * 256) {
        const uint32_t row = a.c0 + j * a.stride;
        const uint8_t* cr = a.codes + int64_t(row) * a.M;
        for (uint32_t i = 0; i < nqg; ++i) {
            const float* t = tab + i * MK;
            float s = 0.0f;
            uint32_t m = 0;
            if (a.words)
            for (; m + 4 <= a.M; m += 4) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(cr + m);
                s += t[m * a.K + (w & 0xFF)];
                s += t[(m + 1) * a.K + ((w >> 8) & 0xFF)];
                s += t[(m + 2) * a.K + ((w >> 16) & 0xFF)];
                s += t[(m + 3) * a.K + (w >> 24)];
            }
            for (; m < a.M; ++m) s += t[m * a.K + cr[m]];
            const uint32_t key = key_of_float(s);
            if (FILTER) {
                const uint32_t qi = a.q0 + g0 + i;
                if (key <= a.thr[qi]) {
                    const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                    if (pos < a.cap) {
                        const int64_t o = int64_t(qi) * a.cap + pos;
                        a.cand_key[o] = key;
                        a.cand_id[o] = row;
                    }
                }
            } else if (a.out_f) {
                a.out_f[int64_t(g0 + i) * a.ldo + j] = s;
            } else {
                a.out_k[int64_t(g0 + i) * a.ldo + j] = key;
            }
        }
    }
}

// K = 256 and M in {8, 16, 32, 64}: M and the query group QB = 64 / M are compile-time, so the
// table entry of (query i, subspace m, code c) is LDS byte 4 c + a constant offset: one
// ds_read_b32 with an immediate offset and one add per lookup, the code bytes unpacked once per
// row for all QB queries.  QB x M x 1 KB = 64 KB of tables: two workgroups per CU, of kAdcThreads
// threads each (one row per thread).
constexpr int kAdcThreads = 512;
template <int M, bool FILTER>
__global__ __launch_bounds__(kAdcThreads) void pq_adc_fast(AdcArgs a) {
    constexpr int QB = 64 / M;
    constexpr int MK = M * 256;
    __shared__ float tab[QB * MK];
    const uint32_t g0 = blockIdx.y * QB;
    const uint32_t nqg = min(uint32_t(QB), a.nq - g0);
    for (uint32_t i = 0; i < uint32_t(QB); ++i) {
        const uint32_t qi = i < nqg ? (a.qrow ? a.qrow[g0 + i] : a.q0 + g0 + i) : 0u;
        const float* src = a.tables + int64_t(qi) * MK;
        for (uint32_t e = threadIdx.x; e < uint32_t(MK); e += kAdcThreads) tab[i * MK + e] = i < nqg ? src[e] : 0.0f;
    }
    __syncthreads();
    // the next row's codes are loaded while the current row's lookups run (two workgroups per CU
    // leave too few waves to hide a load per row otherwise)
    constexpr int NW4 = M / 4;
    auto load_codes = [&](uint32_t j, uint32_t (&w)[NW4]) {
        const uint32_t row = a.c0 + j * a.stride;
        const uint4* cr = reinterpret_cast<const uint4*>(a.codes + int64_t(row) * M);
        if constexpr (M == 8) {
            const uint2 v = *reinterpret_cast<const uint2*>(cr);
            w[0] = v.x;
            w[1] = v.y;
        } else {
#pragma unroll
            for (int b = 0; b < M / 16; ++b) {
                const uint4 v = cr[b];
                w[4 * b] = v.x;
                w[4 * b + 1] = v.y;
                w[4 * b + 2] = v.z;
                w[4 * b + 3] = v.w;
            }
        }
    };
    const uint32_t step = gridDim.x * kAdcThreads;
    uint32_t wn[NW4];
    uint32_t j = blockIdx.x * kAdcThreads + threadIdx.x;
    if (j < a.cols) load_codes(j, wn);
    for (; j < a.cols; j = uint64_t(j) + step < a.cols ? j + step : a.cols) {
        const uint32_t row = a.c0 + j * a.stride;
        uint32_t w[NW4];
#pragma unroll
        for (int b = 0; b < NW4; ++b) w[b] = wn[b];
        if (uint64_t(j) + step < a.cols) load_codes(j + step, wn);
        uint32_t off[M];
#pragma unroll
        for (int m = 0; m < M; ++m) off[m] = (w[m / 4] >> (8 * (m % 4))) & 0xFFu;
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            if (uint32_t(i) >= nqg) break;
            float s = 0.0f;
#pragma unroll
            for (int m = 0; m < M; ++m) s += tab[i * MK + m * 256 + off[m]];
            const uint32_t key = key_of_float(s);
            if (FILTER) {
                const uint32_t qi = a.q0 + g0 + i;
                if (key <= a.thr[qi]) {
                    const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                    if (pos < a.cap) {
                        const int64_t o = int64_t(qi) * a.cap + pos;
                        a.cand_key[o] = key;
                        a.cand_id[o] = row;
                    }
                }
            } else if (a.out_f) {
                a.out_f[int64_t(g0 + i) * a.ldo + j] = s;
            } else {
                a.out_k[int64_t(g0 + i) * a.ldo + j] = key;
            }
        }
    }
}

template <int M, bool FILTER>
va_status launch_adc_fast(va_context* ctx, const AdcArgs& a) {
    constexpr uint32_t QB = 64 / M;
    const uint32_t groups = (a.nq + QB - 1) / QB;
    const uint32_t rb = std::max<uint32_t>(
        1, uint32_t(std::min<uint64_t>((uint64_t(a.cols) + kAdcThreads - 1) / kAdcThreads,
                                       std::max<uint64_t>(1, 4096 * 256 / kAdcThreads / groups))));
    pq_adc_fast<M, FILTER><<<dim3(rb, groups), dim3(kAdcThreads), 0, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// ---- fp16-screened ADC filter (va_pq_search's filter pass; K = 256, M in {8, 16, 32, 64}) ----
// Two queries' tables share one 32-bit LDS word per (subspace, code), as fp16 halves: each
// query's table is scaled by a power of two 2^e_q that puts its largest entry in [2^14, 2^15).
// One lookup then serves two queries, which halves the LDS instructions of a scan bound by their
// bank conflicts (random code bytes), and each half is added to an fp32 sum.  The entries are
// squared distances (>= 0), so with tau_q the query's threshold and S the fp32 scan's sum
// (S <= tau_q): the exact real sum R <= tau_q / (1 - g) (g = M 2^-24 bounds the fp32 rounding of
// a sum of M non-negative terms), the fp16 entries h_m satisfy |h_m - 2^e R_m| <= 2^-11 2^e R_m
// + 2^-14 (normal range; below 2^-14 even a flush to zero stays within 2^-14), and the screened
// fp32 sum A <= (1 + g)(sum h_m).  Together
//     A <= 2^e tau_q (1 + 2^-10) + M 2^-14 (1 + g)  <  thr'_q = fma(2^e tau_q, 1 + 2^-9, M 2^-13),
// so no pair with key <= tau_q is screened out.  A pair that passes is re-scored from the fp32
// tables in the fp32 scan's order and kept only if its exact key is <= tau_q, so the candidate
// lists are the fp32 scan's.  A query whose table holds a negative or non-finite entry, or one
// too large for fp16 after scaling, gets scale 0, which makes its screen pass every row.
__global__ __launch_bounds__(256) void pq_pack_pairs(const float* __restrict__ tables, uint32_t Q, uint32_t MK,
                                                     uint32_t* __restrict__ packed, float* __restrict__ scale) {
    const uint32_t p = blockIdx.x;
    __shared__ float rmax[2][256];
    __shared__ uint32_t rbad[2][256];
    float s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t q = 2 * p + h;
        float mx = 0.0f;
        uint32_t bad = 0;
        if (q < Q)
            for (uint32_t e = threadIdx.x; e < MK; e += 256) {
                const float v = tables[int64_t(q) * MK + e];
                bad |= !(v >= 0.0f && v <= 3.0e38f);  // negative, NaN or near overflow
                mx = fmaxf(mx, v);
            }
        rmax[h][threadIdx.x] = mx;
        rbad[h][threadIdx.x] = bad;
    }
    __syncthreads();
    for (uint32_t w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                rmax[h][threadIdx.x] = fmaxf(rmax[h][threadIdx.x], rmax[h][threadIdx.x + w]);
                rbad[h][threadIdx.x] |= rbad[h][threadIdx.x + w];
            }
        __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float mx = rmax[h][0];
        int x = 0;
        (void)frexpf(mx, &x);  // mx in [2^(x-1), 2^x)
        const int e = mx > 0.0f ? min(100, max(-100, 15 - x)) : 0;
        const float sc = ldexpf(1.0f, e);
        s[h] = (rbad[h][0] || !(mx * sc < 65504.0f)) ? 0.0f : sc;
        if (threadIdx.x == 0 && 2 * p + h < Q) scale[2 * p + h] = s[h];
    }
    for (uint32_t e = threadIdx.x; e < MK; e += 256) {
        uint32_t w = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t q = 2 * p + h;
            // a flagged query (scale 0) packs zeros: its screened sums are 0 and pass (NaN * 0 would not)
            const float v = q < Q && s[h] != 0.0f ? tables[int64_t(q) * MK + e] * s[h] : 0.0f;
            w |= uint32_t(__builtin_bit_cast(uint16_t, _Float16(v))) << (16 * h);
        }
        packed[int64_t(p) * MK + e] = w;
    }
}

// acc + the fp16 value in the low (HI = 0) or high half of v, in one VALU op (v_fma_mix_f32:
// half x 1.0 + acc, rounded once, so the same value as a conversion and an fp32 add)
template <int HI>
__device__ __forceinline__ float add_half(float acc, uint32_t v) {
    float d;
    if (HI)
        asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(v), "v"(acc));
    else
        asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(v), "v"(acc));
    return d;
}

// The workgroup's QP query pairs sit entry-major in LDS: entry e (subspace m, centroid c) of
// pair i at word e * QP + i, so one wide read (128 bits for QP >= 4) at a row's code fetches that
// entry for every pair: a random address costs the same bank conflicts whatever its width, and
// the lookups per conflict grow with the pairs per read (one word per pair, two queries per
// word).
template <int QP>
struct PairWords {
    uint32_t w[QP];
};
template <int QP>
__device__ __forceinline__ PairWords<QP> read_pairs(const uint32_t* p) {
    PairWords<QP> r;
    if constexpr (QP % 4 == 0) {
#pragma unroll
        for (int b = 0; b < QP / 4; ++b) {
            const uint4 v = reinterpret_cast<const uint4*>(p)[b];
            r.w[4 * b] = v.x;
            r.w[4 * b + 1] = v.y;
            r.w[4 * b + 2] = v.z;
            r.w[4 * b + 3] = v.w;
        }
    } else if constexpr (QP == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        r.w[0] = v.x;
        r.w[1] = v.y;
    } else {
        r.w[0] = p[0];
    }
    return r;
}

template <int M>
__global__ __launch_bounds__(kAdcThreads) void pq_adc_screen(AdcArgs a, const uint32_t* __restrict__ packed,
                                                              const float* __restrict__ scale) {
    constexpr int QP = 64 / M;  // query pairs per workgroup: QP x M x 1 KB = 64 KB of LDS
    constexpr int MK = M * 256;
    __shared__ __attribute__((aligned(16))) uint32_t tab[QP * MK];
    const uint32_t p0 = blockIdx.y * QP;
    const uint32_t np = min(uint32_t(QP), (a.nq + 1) / 2 - p0);
    for (uint32_t e = threadIdx.x; e < uint32_t(MK); e += kAdcThreads)
#pragma unroll
        for (uint32_t i = 0; i < uint32_t(QP); ++i) tab[e * QP + i] = i < np ? packed[int64_t(p0 + i) * MK + e] : 0u;
    // screen thresholds (query index past nq: never passes)
    float thr[2 * QP];
#pragma unroll
    for (int i = 0; i < 2 * QP; ++i) {
        const uint32_t q = 2 * p0 + uint32_t(i);
        float t = -INFINITY;
        if (q < a.nq) {
            const uint32_t tk = a.thr[q];
            const float sc = scale[q];
            t = (sc == 0.0f || tk >= key_of_float(INFINITY))
                    ? INFINITY
                    : fmaf(float_of_key(tk) * sc, 1.0f + 0x1p-9f, float(M) * 0x1p-13f);
        }
        thr[i] = t;
    }
    __syncthreads();
    constexpr int NW4 = M / 4;
    auto load_codes = [&](uint32_t j, uint32_t (&w)[NW4]) {
        const uint4* cr = reinterpret_cast<const uint4*>(a.codes + int64_t(j) * M);
        if constexpr (M == 8) {
            const uint2 v = *reinterpret_cast<const uint2*>(cr);
            w[0] = v.x;
            w[1] = v.y;
        } else {
#pragma unroll
            for (int b = 0; b < M / 16; ++b) {
                const uint4 v = cr[b];
                w[4 * b] = v.x;
                w[4 * b + 1] = v.y;
                w[4 * b + 2] = v.z;
                w[4 * b + 3] = v.w;
            }
        }
    };
    // exact re-score of (query q, row j) in the fp32 scan's order; appended if key <= tau_q
    auto rescore = [&](uint32_t q, uint32_t j, const uint32_t (&off)[M]) {
        const float* t = a.tables + int64_t(q) * MK;
        float s = 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) s += t[m * 256 + off[m]];
        const uint32_t key = key_of_float(s);
        if (key <= a.thr[q]) {
            const uint32_t pos = atomicAdd(a.cnt + q, 1u);
            if (pos < a.cap) {
                const int64_t o = int64_t(q) * a.cap + pos;
                a.cand_key[o] = key;
                a.cand_id[o] = j;
            }
        }
    };
    const uint32_t step = gridDim.x * kAdcThreads;
    uint32_t wn[NW4];
    uint32_t j = blockIdx.x * kAdcThreads + threadIdx.x;
    if (j < a.cols) load_codes(j, wn);
    for (; j < a.cols; j = uint64_t(j) + step < a.cols ? j + step : a.cols) {
        uint32_t w[NW4];
#pragma unroll
        for (int b = 0; b < NW4; ++b) w[b] = wn[b];
        if (uint64_t(j) + step < a.cols) load_codes(j + step, wn);
        uint32_t off[M];
#pragma unroll
        for (int m = 0; m < M; ++m) off[m] = (w[m / 4] >> (8 * (m % 4))) & 0xFFu;
        if constexpr (QP == 1) {
            // one pair: one word per read either way
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t v = tab[m * 256 + off[m]];
                s0 = add_half<0>(s0, v);
                s1 = add_half<1>(s1, v);
            }
            if (s0 <= thr[0]) rescore(2 * p0, j, off);
            if (s1 <= thr[1]) rescore(2 * p0 + 1, j, off);
        } else {
            // every pair's sums (pairs past np have zero tables and thresholds that never pass)
            float s0[QP], s1[QP];
#pragma unroll
            for (int i = 0; i < QP; ++i) s0[i] = s1[i] = 0.0f;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const PairWords<QP> v = read_pairs<QP>(tab + (m * 256 + off[m]) * QP);
#pragma unroll
                for (int i = 0; i < QP; ++i) {
                    s0[i] = add_half<0>(s0[i], v.w[i]);
                    s1[i] = add_half<1>(s1[i], v.w[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < QP; ++i) {
                if (s0[i] <= thr[2 * i]) rescore(2 * (p0 + i), j, off);
                if (s1[i] <= thr[2 * i + 1]) rescore(2 * (p0 + i) + 1, j, off);
            }
        }
    }
}

// The screened filter of a whole search (queries 0..nq-1, rows 0..cols-1, dense codes).
template <int M>
va_status launch_adc_screen(va_context* ctx, const AdcArgs& a, const uint32_t* packed, const float* scale) {
    constexpr uint32_t QP = 64 / M;
    const uint32_t groups = ((a.nq + 1) / 2 + QP - 1) / QP;
    const uint32_t rb = std::max<uint32_t>(
        1, uint32_t(std::min<uint64_t>((uint64_t(a.cols) + kAdcThreads - 1) / kAdcThreads,
                                       std::max<uint64_t>(1, 4096 * 256 / kAdcThreads / groups))));
    pq_adc_screen<M><<<dim3(rb, groups), dim3(kAdcThreads), 0, ctx->stream>>>(a, packed, scale);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// Whether the screened filter takes a search: the fast kernel's shapes, a grid within range.
bool adc_screen_ok(uint32_t Q, uint32_t M, uint32_t K, const uint8_t* codes) {
    if (K != 256 || !(M == 8 || M == 16 || M == 32 || M == 64) || (reinterpret_cast<uintptr_t>(codes) & 15) != 0)
        return false;
    return ((uint64_t(Q) + 1) / 2 + 64 / M - 1) / (64 / M) <= 65535;
}

// Query groups of QB (as many tables as fit in 160 KB of LDS, at most 16) on grid.y, in launches
// of at most 65535 groups.
template <bool FILTER>
va_status launch_adc(va_context* ctx, AdcArgs a) {
    if (a.nq == 0 || a.cols == 0) return VA_OK;
    const size_t per_q = size_t(a.M) * a.K * 4;
    const size_t lds_max = 160 * 1024;
    if (per_q > lds_max) return fail(ctx, VA_ERR_UNSUPPORTED, "PQ table of %zu bytes exceeds LDS", per_q);
    a.words = (a.M % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.codes) & 3) == 0);
    a.QB = uint32_t(std::min<size_t>({size_t(16), lds_max / per_q, size_t(a.nq)}));
    const bool fast = a.K == 256 && (a.M == 8 || a.M == 16 || a.M == 32 || a.M == 64) &&
                      (reinterpret_cast<uintptr_t>(a.codes) & 15) == 0;
    if (fast) a.QB = 64 / a.M;
    const uint64_t span = uint64_t(65535) * a.QB;
    if (a.nq > span) {
        AdcArgs b = a;
        for (uint64_t s0 = 0; s0 < a.nq; s0 += span) {
            b.nq = uint32_t(std::min<uint64_t>(span, a.nq - s0));
            if (a.qrow) b.qrow = a.qrow + s0;
            else b.q0 = a.q0 + uint32_t(s0);
            if (a.out_k) b.out_k = a.out_k + int64_t(s0) * a.ldo;
            if (a.out_f) b.out_f = a.out_f + int64_t(s0) * a.ldo;
            VA_CHECK_STATUS(launch_adc<FILTER>(ctx, b));
        }
        return VA_OK;
    }
    if (fast) {
        switch (a.M) {
            case 8: return launch_adc_fast<8, FILTER>(ctx, a);
            case 16: return launch_adc_fast<16, FILTER>(ctx, a);
            case 32: return launch_adc_fast<32, FILTER>(ctx, a);
            default: return launch_adc_fast<64, FILTER>(ctx, a);
        }
    }
    const uint32_t groups = (a.nq + a.QB - 1) / a.QB;
    // enough row blocks to fill the chip a few times over; each re-reads its group's tables
    uint32_t rb = std::max<uint32_t>(1, uint32_t(std::min<uint64_t>((uint64_t(a.cols) + 255) / 256,
                                                                     std::max<uint64_t>(1, 2048 / groups))));
    const size_t lds = size_t(a.QB) * per_q;
    auto kern = &pq_adc_kernel<FILTER>;
    if (lds > 65536)
        VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    kern<<<dim3(rb, groups), dim3(256), lds, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

struct AdcProducer final : KeyProducer {
    va_context* ctx;
    const uint8_t* codes;
    const float* tables;
    uint32_t Q, N, M, K;
    // fp16 pair tables and scales of the screened filter (nullptr: the fp32 filter)
    const uint32_t* packed = nullptr;
    const float* scale = nullptr;
    va_status fallback_pass(const FbArgs& a, int pass) override {
        return fb_launch_pass(ctx, FbAdc{codes, tables, N, M, K}, a, pass);
    }
    va_status dense(const uint32_t* qrow, uint32_t q0, uint32_t nq, uint32_t c0, uint32_t cols, uint32_t stride,
                    uint32_t* out_k, int64_t ldo) override {
        AdcArgs a;
        a.codes = codes;
        a.tables = tables;
        a.M = M;
        a.K = K;
        a.qrow = qrow;
        a.q0 = q0;
        a.nq = nq;
        a.c0 = c0;
        a.cols = cols;
        a.stride = stride;
        a.out_k = out_k;
        a.ldo = ldo;
        return launch_adc<false>(ctx, a);
    }
    va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) override {
        AdcArgs a;
        a.codes = codes;
        a.tables = tables;
        a.M = M;
        a.K = K;
        a.q0 = 0;
        a.nq = Q;
        a.c0 = 0;
        a.cols = N;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        if (packed) {
            switch (M) {
                case 8: return launch_adc_screen<8>(ctx, a, packed, scale);
                case 16: return launch_adc_screen<16>(ctx, a, packed, scale);
                case 32: return launch_adc_screen<32>(ctx, a, packed, scale);
                default: return launch_adc_screen<64>(ctx, a, packed, scale);
            }
        }
        return launch_adc<true>(ctx, a);
    }
};

__global__ __launch_bounds__(256) void sqrt_inplace(float* __restrict__ v, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) v[i] = sqrtf(v[i]);
}

struct Owned {
    std::vector<void*> p;
    ~Owned() {
        for (void* q : p) (void)hipFree(q);
    }
};
template <class T>
va_status alloc(va_context* ctx, Owned& own, size_t bytes, T** out) {
    void* q = nullptr;
    VA_CHECK_HIP(ctx, hipMalloc(&q, std::max<size_t>(bytes, 256)));
    own.p.push_back(q);
    *out = static_cast<T*>(q);
    return VA_OK;
}

uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace
}  // namespace va

#define VA_PQ_CHECK_SHAPE(ctx, D, M, K)                                                                       \
    do {                                                                                                      \
        VA_REQUIRE(ctx, (M) >= 1 && (D) >= 1 && (D) % (M) == 0, "Dimension must be divisible by M (D=%u, M=%u)", \
                   (D), (M));                                                                                 \
        VA_REQUIRE(ctx, (K) >= 1 && (K) <= 256, "K must be <= 256 for uint8 encoding, got %u", (K));           \
        VA_REQUIRE(ctx, (M) <= 65535, "at most 65535 subspaces, got %u", (M));                               \
    } while (0)

extern "C" {

va_status va_pq_train(va_context* ctx, const float* data, uint32_t count, uint32_t dim, uint32_t M, uint32_t K,
                      uint32_t iterations, float threshold, uint64_t seed, const float* initial_codebooks,
                      float* out_codebooks, uint32_t* out_iterations) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, data && out_codebooks, "va_pq_train: NULL pointer");
    VA_PQ_CHECK_SHAPE(ctx, dim, M, K);
    VA_REQUIRE(ctx, count >= 1, "va_pq_train: no training vectors");
    va::DeviceGuard g(ctx->device);
    const uint32_t N = count, D = dim, ds = dim / M;
    va::Owned own;
    uint8_t *codes, *col, *sorted;
    uint32_t *iota, *members, *first, *counts, *chunks, *chunk_end, *rows;
    float *partial, *movement, *mv;
    const uint64_t max_chunks = uint64_t(N) / va::kPQChunk + K;
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * M, &codes));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N), &col));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N), &sorted));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &iota));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &members));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(K) * 4, &first));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(K) * 4, &counts));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(K) * 4, &chunks));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(K) * 4, &chunk_end));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(M) * K * 4, &rows));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(max_chunks) * ds * 4, &partial));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(M) * K * 4, &movement));
    VA_CHECK_STATUS(va::alloc(ctx, own, 4, &mv));
    size_t sort_bytes = 0, scan_bytes = 0;
    VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(nullptr, sort_bytes, col, sorted, iota, members, N, 0, 8, ctx->stream));
    VA_CHECK_HIP(ctx, rocprim::inclusive_scan(nullptr, scan_bytes, chunks, chunk_end, K, rocprim::plus<uint32_t>(),
                                              ctx->stream));
    void* tmp;
    VA_CHECK_STATUS(va::alloc(ctx, own, std::max(sort_bytes, scan_bytes), &tmp));
    // initial codebooks: given, or codebook (m, k) = sub-vector m of a random training row
    // (initializeCodebooks, ProductQuantizationKernel.swift:548-572; rows from splitmix64(seed))
    std::vector<uint32_t> hrows(size_t(M) * K);
    if (initial_codebooks) {
        VA_CHECK_HIP(ctx, hipMemcpyAsync(out_codebooks, initial_codebooks, size_t(M) * K * ds * 4,
                                         hipMemcpyDeviceToDevice, ctx->stream));
    } else {
        uint64_t s = seed;
        for (auto& r : hrows) r = uint32_t((double(va::splitmix64(s) >> 11) * 0x1.0p-53) * double(N)) % N;
        VA_CHECK_HIP(ctx, hipMemcpyAsync(rows, hrows.data(), hrows.size() * 4, hipMemcpyHostToDevice, ctx->stream));
        va::pq_init<<<dim3(M * K), dim3(256), 0, ctx->stream>>>(data, D, M, K, rows, out_codebooks);
        VA_CHECK_LAUNCH(ctx);
    }
    const uint32_t nb = (N + 255) / 256;
    uint32_t it = 0;
    for (; it < iterations;) {
        va::pq_assign<<<dim3(nb, M), dim3(256), 0, ctx->stream>>>(data, N, D, M, K, out_codebooks, codes);
        VA_CHECK_LAUNCH(ctx);
        for (uint32_t m = 0; m < M; ++m) {
            va::pq_column<<<dim3(nb), dim3(256), 0, ctx->stream>>>(codes, N, M, m, col, iota);
            VA_CHECK_LAUNCH(ctx);
            VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(tmp, sort_bytes, col, sorted, iota, members, N, 0, 8, ctx->stream));
            va::pq_ranges<<<dim3((K + 255) / 256), dim3(256), 0, ctx->stream>>>(sorted, N, K, first, counts, chunks);
            VA_CHECK_LAUNCH(ctx);
            VA_CHECK_HIP(ctx, rocprim::inclusive_scan(tmp, scan_bytes, chunks, chunk_end, K, rocprim::plus<uint32_t>(),
                                                      ctx->stream));
            va::pq_chunk_sums<<<dim3(uint32_t(max_chunks)), dim3(256), 0, ctx->stream>>>(data, D, ds, m, K, members, first,
                                                                                        counts, chunk_end, partial);
            VA_CHECK_LAUNCH(ctx);
            va::pq_finalize<<<dim3((K + 63) / 64), dim3(64), 0, ctx->stream>>>(ds, m, K, counts, chunk_end, partial,
                                                                             out_codebooks, movement);
            VA_CHECK_LAUNCH(ctx);
        }
        va::pq_movement<<<dim3(1), dim3(64), 0, ctx->stream>>>(movement, M * K, mv);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_HIP(ctx, hipMemcpyAsync(ctx->host_word, mv, 4, hipMemcpyDeviceToHost, ctx->stream));
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        ++it;
        if (__builtin_bit_cast(float, ctx->host_word[0]) < threshold) break;
    }
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (out_iterations) *out_iterations = it;
    return VA_OK;
}

va_status va_pq_encode(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim, uint32_t M, uint32_t K,
                       const float* codebooks, uint8_t* codes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, x && codebooks && codes, "va_pq_encode: NULL pointer");
    VA_PQ_CHECK_SHAPE(ctx, dim, M, K);
    if (num_vectors == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    va::pq_assign<<<dim3((num_vectors + 255) / 256, M), dim3(256), 0, ctx->stream>>>(x, num_vectors, dim, M, K,
                                                                                       codebooks, codes);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_pq_distance_tables(va_context* ctx, const float* queries, uint32_t num_queries, uint32_t dim, uint32_t M,
                                uint32_t K, const float* codebooks, float* tables) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, queries && codebooks && tables, "va_pq_distance_tables: NULL pointer");
    VA_PQ_CHECK_SHAPE(ctx, dim, M, K);
    VA_REQUIRE(ctx, num_queries <= 65535, "va_pq_distance_tables: at most 65535 queries per call");
    if (num_queries == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    va::pq_tables<<<dim3((K + 255) / 256, M, num_queries), dim3(256), 0, ctx->stream>>>(queries, dim, M, K, codebooks,
                                                                                          tables);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_pq_adc_distances(va_context* ctx, const float* tables, uint32_t num_queries, const uint8_t* codes,
                              uint32_t num_vectors, uint32_t M, uint32_t K, float* out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, tables && codes && out, "va_pq_adc_distances: NULL pointer");
    VA_REQUIRE(ctx, M >= 1 && K >= 1 && K <= 256, "va_pq_adc_distances: bad M / K");
    if (num_queries == 0 || num_vectors == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    va::AdcArgs a;
    a.codes = codes;
    a.tables = tables;
    a.M = M;
    a.K = K;
    a.q0 = 0;
    a.nq = num_queries;
    a.c0 = 0;
    a.cols = num_vectors;
    a.out_f = out;
    a.ldo = num_vectors;
    return va::launch_adc<false>(ctx, a);
}

va_status va_pq_search(va_context* ctx, const float* queries, uint32_t num_queries, uint32_t dim, uint32_t M,
                       uint32_t K, const float* codebooks, const uint8_t* codes, uint32_t num_vectors, uint32_t k,
                       uint32_t* out_idx, float* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, queries && codebooks && codes && out_idx, "va_pq_search: NULL pointer");
    VA_PQ_CHECK_SHAPE(ctx, dim, M, K);
    VA_REQUIRE(ctx, k >= 1 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    if (num_queries == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    // the tables (and the screened filter's fp16 pair tables and scales) live in the context's
    // side buffer: the call returns without waiting for the scan
    const bool screen = va::adc_screen_ok(num_queries, M, K, codes);
    const size_t tbytes = (size_t(num_queries) * M * K * 4 + 255) & ~size_t(255);
    const size_t pbytes = screen ? (size_t(num_queries + 1) / 2 * M * K * 4 + 255) & ~size_t(255) : 0;
    const size_t sbytes = screen ? size_t(num_queries) * 4 : 0;
    void* side = nullptr;
    VA_CHECK_STATUS(va::side_reserve(ctx, tbytes + pbytes + sbytes, &side));
    float* tables = static_cast<float*>(side);
    uint32_t* packed = screen ? reinterpret_cast<uint32_t*>(static_cast<char*>(side) + tbytes) : nullptr;
    float* scale = screen ? reinterpret_cast<float*>(static_cast<char*>(side) + tbytes + pbytes) : nullptr;
    for (uint32_t q0 = 0; q0 < num_queries; q0 += 65535) {
        const uint32_t nq = std::min<uint32_t>(65535, num_queries - q0);
        VA_CHECK_STATUS(va_pq_distance_tables(ctx, queries + int64_t(q0) * dim, nq, dim, M, K, codebooks,
                                              tables + int64_t(q0) * M * K));
    }
    if (screen) {
        va::pq_pack_pairs<<<dim3((num_queries + 1) / 2), dim3(256), 0, ctx->stream>>>(tables, num_queries, M * K,
                                                                                        packed, scale);
        VA_CHECK_LAUNCH(ctx);
    }
    va::AdcProducer kp;
    kp.ctx = ctx;
    kp.codes = codes;
    kp.tables = tables;
    kp.packed = packed;
    kp.scale = scale;
    kp.Q = num_queries;
    kp.N = num_vectors;
    kp.M = M;
    kp.K = K;
    va::ScanOutputs o;
    o.idx = out_idx;
    o.f = out_dist;
    VA_CHECK_STATUS(va::exact_topk_scan(ctx, kp, num_queries, num_vectors, k, o));
    // findNearestNeighbors reports sqrt of the ADC sum (ProductQuantizationKernel.swift:531-537)
    if (out_dist) {
        const uint64_t n = uint64_t(num_queries) * k;
        va::sqrt_inplace<<<dim3(uint32_t((n + 255) / 256)), dim3(256), 0, ctx->stream>>>(out_dist, n);
        VA_CHECK_LAUNCH(ctx);
    }
    return VA_OK;
}

}  // extern "C"
