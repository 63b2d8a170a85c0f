// va_binary.hip — binary (sign-bit) quantization and Hamming scan on CDNA4.
//
//   pack : bit d = (x_d > 0), word w bit b = dimension 32w+b (binaryQuantize,
//          Metal/Shaders/QuantizationShaders.metal:132-160).  One wave per row; each lane reads
//          one float and __ballot turns 64 consecutive dimensions into two words, so every
//          load is a fully coalesced 256-byte wave access (the reference's shader has one
//          thread per vector striding through the row, and no bounds guard).
//   scan : Hamming distance sum(popcount(q ^ x)) with v_xor + v_bcnt (accumulating popcount)
//          on the VALU.  One database row per lane, held in VGPRs (128-bit loads); the query
//          words are wave-uniform and come through scalar loads, so each (query, row) pair
//          costs 2 VALU ops per 32-bit word.  Feeds the shared exact top-k driver with the
//          distance itself as the key (ties -> lower index, HammingDistanceKernel.swift:114-120).
#include <algorithm>

#include "va_internal.hpp"

namespace va {
namespace {

constexpr uint32_t kMaxWords = 32;  // register-resident rows up to D = 1024

__global__ __launch_bounds__(256) void pack_kernel(const float* __restrict__ x, uint32_t N, uint32_t D, uint32_t W,
                                                   uint32_t* __restrict__ codes) {
    const int lane = threadIdx.x & 63;
    const uint32_t waves = gridDim.x * 4;
    for (uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < N; r += waves) {
        const float* row = x + uint64_t(r) * D;
        uint32_t* out = codes + uint64_t(r) * W;
        for (uint32_t c = 0; c * 64 < D; ++c) {
            const uint32_t d = c * 64 + uint32_t(lane);
            const bool bit = (d < D) && (row[d] > 0.0f);
            const uint64_t m = __ballot(bit);
            if (lane == 0) {
                out[2 * c] = uint32_t(m);
                if (2 * c + 1 < W) out[2 * c + 1] = uint32_t(m >> 32);
            }
        }
    }
}

__global__ __launch_bounds__(256) void hamming_matrix_kernel(const uint32_t* __restrict__ q,
                                                             const uint32_t* __restrict__ x, uint32_t N, uint32_t W,
                                                             uint32_t* __restrict__ out) {
    const uint32_t qi = blockIdx.y;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= N) return;
    const uint32_t* qw = q + uint64_t(qi) * W;
    const uint32_t* xw = x + uint64_t(j) * W;
    uint32_t d = 0;
    for (uint32_t w = 0; w < W; ++w) d += __popc(qw[w] ^ xw[w]);
    out[uint64_t(qi) * N + j] = d;
}

struct HamArgs {
    const uint32_t* q = nullptr;
    const uint32_t* qrow = nullptr;  // optional query indirection
    uint32_t q0 = 0, nq = 0;
    const uint32_t* x = nullptr;
    uint32_t c0 = 0, cols = 0, stride = 1;  // rows c0 + j*stride, j < cols
    uint32_t W = 0;
    uint32_t* out_k = nullptr;
    int64_t ldo = 0;
    const uint32_t* thr = nullptr;
    uint32_t* cnt = nullptr;
    uint32_t* cand_key = nullptr;
    uint32_t* cand_id = nullptr;
    uint32_t cap = 0;
};

// wave-uniform word load through the scalar data cache (read-only constant address space)
__device__ __forceinline__ uint32_t uniform_load(const uint32_t* p) {
    return *(const __attribute__((address_space(4))) uint32_t*)(p);
}

// WC > 0: compile-time word count (fully unrolled; query words arrive in wide scalar loads);
// WC = 0: any W <= kMaxWords.
template <int WC, bool FILTER>
__global__ __launch_bounds__(256) void hamming_scan_kernel(HamArgs a) {
    constexpr uint32_t WR = WC > 0 ? uint32_t(WC) : kMaxWords;
    const uint32_t W = WC > 0 ? uint32_t(WC) : a.W;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    const bool valid = j < a.cols;
    const uint32_t row = a.c0 + (valid ? j : 0) * a.stride;
    // the row, word by word, in VGPRs (uint4 loads; rows are 16-byte aligned when W % 4 == 0)
    uint32_t xr[WR];
    const uint32_t* xp = a.x + uint64_t(row) * W;
    if ((W & 3) == 0) {
#pragma unroll
        for (uint32_t w = 0; w < WR; w += 4) {
            if (w < W) {
                const uint4 v = *reinterpret_cast<const uint4*>(xp + w);
                xr[w] = v.x;
                xr[w + 1] = v.y;
                xr[w + 2] = v.z;
                xr[w + 3] = v.w;
            }
        }
    } else {
#pragma unroll
        for (uint32_t w = 0; w < WR; ++w)
            if (w < W) xr[w] = xp[w];
    }
#pragma unroll 2
    for (uint32_t i = 0; i < a.nq; ++i) {
        const uint32_t qr = a.qrow ? uniform_load(a.qrow + i) : a.q0 + i;
        const uint32_t* qw = a.q + uint64_t(qr) * W;
        uint32_t d = 0;
#pragma unroll
        for (uint32_t w = 0; w < WR; ++w)
            if (w < W) d += __popc(xr[w] ^ uniform_load(qw + w));
        if (!valid) continue;
        if (FILTER) {
            const uint32_t qi = a.q0 + i;
            if (d <= uniform_load(a.thr + qi)) {
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_key[o] = d;
                    a.cand_id[o] = row;
                }
            }
        } else {
            a.out_k[int64_t(i) * a.ldo + j] = d;
        }
    }
}

// rows longer than kMaxWords words: the row is re-read from L1/L2 for every query
template <bool FILTER>
__global__ __launch_bounds__(256) void hamming_scan_wide_kernel(HamArgs a) {
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= a.cols) return;
    const uint32_t row = a.c0 + j * a.stride;
    const uint32_t* xp = a.x + uint64_t(row) * a.W;
    for (uint32_t i = 0; i < a.nq; ++i) {
        const uint32_t qr = a.qrow ? a.qrow[i] : a.q0 + i;
        const uint32_t* qw = a.q + uint64_t(qr) * a.W;
        uint32_t d = 0;
        for (uint32_t w = 0; w < a.W; ++w) d += __popc(xp[w] ^ qw[w]);
        if (FILTER) {
            const uint32_t qi = a.q0 + i;
            if (d <= a.thr[qi]) {
                const uint32_t pos = atomicAdd(a.cnt + qi, 1u);
                if (pos < a.cap) {
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_key[o] = d;
                    a.cand_id[o] = row;
                }
            }
        } else {
            a.out_k[int64_t(i) * a.ldo + j] = d;
        }
    }
}

va_status launch_ham(va_context* ctx, const HamArgs& a, bool filter) {
    if (a.nq == 0 || a.cols == 0) return VA_OK;
    const dim3 grid((a.cols + 255) / 256);
    const bool aligned = (a.W & 3) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
    if (a.W <= kMaxWords && (aligned || (a.W & 3) != 0)) {
#define VA_HAM_CASE(WC)                                                                       \
    if (filter)                                                                               \
        hamming_scan_kernel<WC, true><<<grid, dim3(256), 0, ctx->stream>>>(a);               \
    else                                                                                      \
        hamming_scan_kernel<WC, false><<<grid, dim3(256), 0, ctx->stream>>>(a);
        if (a.W == 8 && aligned) {
            VA_HAM_CASE(8)
        } else if (a.W == 16 && aligned) {
            VA_HAM_CASE(16)
        } else if (a.W == 24 && aligned) {
            VA_HAM_CASE(24)
        } else if (a.W == 32 && aligned) {
            VA_HAM_CASE(32)
        } else {
            VA_HAM_CASE(0)
        }
#undef VA_HAM_CASE
    } else {
        if (filter)
            hamming_scan_wide_kernel<true><<<grid, dim3(256), 0, ctx->stream>>>(a);
        else
            hamming_scan_wide_kernel<false><<<grid, dim3(256), 0, ctx->stream>>>(a);
    }
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

struct HamProducer final : KeyProducer {
    va_context* ctx;
    const uint32_t* q;
    const uint32_t* x;
    uint32_t Q, N, W;
    va_status dense(const uint32_t* qrow, uint32_t q0, uint32_t nq, uint32_t c0, uint32_t cols, uint32_t stride,
                    uint32_t* out_k, int64_t ldo) override {
        HamArgs a;
        a.q = q;
        a.qrow = qrow;
        a.q0 = q0;
        a.nq = nq;
        a.x = x;
        a.c0 = c0;
        a.cols = cols;
        a.stride = stride;
        a.W = W;
        a.out_k = out_k;
        a.ldo = ldo;
        return launch_ham(ctx, a, false);
    }
    va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) override {
        HamArgs a;
        a.q = q;
        a.q0 = 0;
        a.nq = Q;
        a.x = x;
        a.c0 = 0;
        a.cols = N;
        a.stride = 1;
        a.W = W;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        return launch_ham(ctx, a, true);
    }
};

}  // namespace
}  // namespace va

extern "C" {

va_status va_bq_pack(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim, uint32_t* codes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, x && codes, "va_bq_pack: NULL pointer");
    VA_REQUIRE(ctx, num_vectors > 0 && dim > 0, "Input vectors cannot be empty");
    va::DeviceGuard g(ctx->device);
    const uint32_t W = (dim + 31) / 32;
    const uint32_t blocks = std::min<uint32_t>((num_vectors + 3) / 4, 65536);
    va::pack_kernel<<<dim3(blocks), dim3(256), 0, ctx->stream>>>(x, num_vectors, dim, W, codes);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_hamming_matrix(va_context* ctx, const uint32_t* query_codes, const uint32_t* database_codes,
                            uint32_t num_queries, uint32_t num_database, uint32_t words, uint32_t* out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, query_codes && database_codes && out, "va_hamming_matrix: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0 && num_database > 0 && words > 0, "va_hamming_matrix: empty input");
    VA_REQUIRE(ctx, num_queries <= 65535, "va_hamming_matrix: at most 65535 queries per call");
    va::DeviceGuard g(ctx->device);
    va::hamming_matrix_kernel<<<dim3((num_database + 255) / 256, num_queries), dim3(256), 0, ctx->stream>>>(
        query_codes, database_codes, num_database, words, out);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_hamming_topk(va_context* ctx, const uint32_t* query_codes, const uint32_t* database_codes,
                          uint32_t num_queries, uint32_t num_database, uint32_t words, uint32_t k, uint32_t* out_idx,
                          uint32_t* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, query_codes && database_codes && out_idx, "va_hamming_topk: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0 && num_database > 0 && words > 0, "va_hamming_topk: empty input");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "k must be in [1, %u], got %u", VA_MAX_K, k);
    va::DeviceGuard g(ctx->device);
    va::HamProducer p;
    p.ctx = ctx;
    p.q = query_codes;
    p.x = database_codes;
    p.Q = num_queries;
    p.N = num_database;
    p.W = words;
    va::ScanOutputs o;
    o.idx = out_idx;
    o.key = out_dist;
    o.key_kind = 3;
    return va::exact_topk_scan(ctx, p, num_queries, num_database, k, o);
}

}  // extern "C"
