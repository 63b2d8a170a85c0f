// va_select.hip — exact row-wise top-k on 32-bit ordering keys.
//
// One workgroup per row:
//   1. radix select (4 x 8-bit LDS histograms) finds T, the k-th smallest key;
//   2. when more items share T than are needed, a second radix select over the ids of the
//      key == T items finds the cut id, so ties go to the lower index;
//   3. the exactly-k winners are gathered into LDS and bitonic-sorted by (key, id).
// The (distance, index) order is the reference's tie rule (Metal4Common.h:142-159,
// SearchAndRetrieval.metal:313-317); unlike topk_select_batch_kernel
// (SearchAndRetrieval.metal:88-156, value-only compares) the result is deterministic.
#include <algorithm>

#include "va_internal.hpp"

namespace va {
namespace {

constexpr int SEL_THREADS = 256;
constexpr uint32_t SEL_BUF = VA_MAX_K;  // winners buffer (k <= VA_MAX_K)

// Rows of up to kSelCache keys are first copied into LDS (one pass with many loads in flight);
// the radix passes then read LDS instead of re-reading the row from memory once per pass with
// one load in flight per thread, which left a short row's workgroup waiting on memory latency.
constexpr uint32_t kSelCache = 24576;  // 96 KiB

template <bool CACHED>
struct RowView {
    const uint32_t* keys;  // the row in memory, or its copy in LDS
    const uint32_t* ids;
    uint32_t n;
    __device__ uint32_t key(uint32_t i) const { return keys[i]; }
    __device__ uint32_t id(uint32_t i) const { return ids ? ids[i] : i; }
};

// Wave 0 scans the 256-bin histogram and finds the bin holding the `need`-th item.
// Writes digit, the count before it, and the bin count to shared memory.
__device__ void find_digit(const uint32_t* hist, uint32_t need, uint32_t* s_digit, uint32_t* s_before,
                           uint32_t* s_bin) {
    const int lane = threadIdx.x & 63;
    if (threadIdx.x >= 64) return;
    uint32_t c[4];
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c[i] = hist[lane * 4 + i];
        sum += c[i];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    uint32_t excl = incl - sum;
    if (excl < need && need <= incl) {
        uint32_t run = excl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (run < need && need <= run + c[i]) {
                *s_digit = uint32_t(lane * 4 + i);
                *s_before = run;
                *s_bin = c[i];
            }
            run += c[i];
        }
    }
}

// The bin of a histogram of nb <= 2048 bins holding the need-th item: each thread sums eight
// bins, a block-wide scan of the sums, then the thread whose range holds the item finds it.
__device__ void find_bin_wide(const uint32_t* hist, uint32_t nb, uint32_t need, uint32_t* s_digit,
                              uint32_t* s_before, uint32_t* s_bin) {
    __shared__ uint32_t wsum[SEL_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t c[8], sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t b = uint32_t(tid) * 8 + i;
        c[i] = b < nb ? hist[b] : 0u;
        sum += c[i];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint32_t base = 0;
    for (int i = 0; i < w; ++i) base += wsum[i];
    incl += base;
    const uint32_t excl = incl - sum;
    if (excl < need && need <= incl) {
        uint32_t run = excl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (run < need && need <= run + c[i]) {
                *s_digit = uint32_t(tid) * 8 + i;
                *s_before = run;
                *s_bin = c[i];
            }
            run += c[i];
        }
    }
}

// Adds this lane's item to the histogram when m.  Keys of one search crowd into few digits
// (the top bytes of nearby distances are equal; Hamming distances are below 1024), and 256
// threads incrementing one LDS bin serialise: when every active lane of the wave adds to the
// same bin, one lane adds the wave's count.
__device__ __forceinline__ void hist_add(uint32_t* hist, bool m, uint32_t d) {
    const uint32_t dd = m ? d : 0xFFFFFFFFu;
    const uint32_t first = __builtin_amdgcn_readfirstlane(dd);
    const uint64_t act = __ballot(1);
    if (__ballot(dd == first) == act) {
        if (first != 0xFFFFFFFFu && (threadIdx.x & 63) == uint32_t(__builtin_ctzll(act)))
            atomicAdd(&hist[first], uint32_t(__popcll(act)));
    } else if (m) {
        atomicAdd(&hist[d], 1u);
    }
}

// KTH: threshold mode only (a.out_kth set): no winners buffer, so a cached row of up to
// 16K keys leaves room for two workgroups per CU.
template <bool CACHED, bool KTH = false>
__global__ __launch_bounds__(SEL_THREADS) void select_kernel(SelectArgs a) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit, s_before, s_bin, s_cnt;
    __shared__ uint32_t okey[KTH ? 1 : SEL_BUF];
    __shared__ uint32_t oid[KTH ? 1 : SEL_BUF];
    __shared__ uint32_t whist[2048];     // one-pass histogram of keys below 2^11
    extern __shared__ uint32_t s_row[];  // CACHED: the row's keys

    const uint32_t row = blockIdx.x;
    if (a.rows_dev && row >= *a.rows_dev) return;  // past the device row count (uniform)
    const int tid = threadIdx.x;
    const uint32_t orow = a.row_map ? a.row_map[row] : row;

    RowView<CACHED> rv;
    rv.keys = a.keys + int64_t(row) * a.ld;
    rv.ids = a.ids ? a.ids + int64_t(row) * a.ld : nullptr;
    rv.n = a.n;
    if (a.counts) {
        const uint32_t c = a.counts[row];
        if (c > a.n || c < a.min_count) {
            // candidate list overflowed, or too short to be the whole top-k (a threshold below
            // the k-th key): listed for the exact fallback, which writes the row
            if (tid == 0 && a.overflow_count) {
                const uint32_t p = atomicAdd(a.overflow_count, 1u);
                a.overflow_rows[p] = row;
            }
            return;
        }
        rv.n = c;
    }
    const uint32_t n = rv.n;
    if (CACHED) {
        // eight independent loads per thread per round
        for (uint32_t i0 = 0; i0 < n; i0 += 8 * SEL_THREADS) {
            uint32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = i0 + uint32_t(j * SEL_THREADS + tid);
                v[j] = i < n ? rv.keys[i] : 0u;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = i0 + uint32_t(j * SEL_THREADS + tid);
                if (i < n) s_row[i] = v[j];
            }
        }
        rv.keys = s_row;
        __syncthreads();
    }
    const uint32_t K = a.k < n ? a.k : n;
    // f(key) over the row; rows read from memory load eight keys per thread before using them,
    // so a long row's pass is not one load latency per key
    auto for_keys = [&](auto&& f) {
        uint32_t i = uint32_t(tid);
        if (!CACHED)
            for (; i + 7u * SEL_THREADS < n; i += 8u * SEL_THREADS) {
                uint32_t v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = rv.key(i + uint32_t(j) * SEL_THREADS);
#pragma unroll
                for (int j = 0; j < 8; ++j) f(v[j]);
            }
        for (; i < n; i += SEL_THREADS) f(rv.key(i));
    };

    uint32_t T = 0xFFFFFFFFu, Tid = 0xFFFFFFFFu;
    bool take_all = (n <= a.k);
    if (!take_all) {
        // ---- phase 1: k-th smallest key ---------------------------------------------
        uint32_t prefix = 0, mask = 0, need = K;
        uint32_t eq = 0;
        int top = 24;  // first byte pass
        if (a.key_bits <= 11) {
            // small keys: one histogram over all key values
            const uint32_t nb = 1u << a.key_bits;
            for (uint32_t b = tid; b < nb; b += SEL_THREADS) whist[b] = 0;
            __syncthreads();
            // (a sentinel key, above every real one, lands in the top bin)
            for_keys([&](uint32_t k) { hist_add(whist, true, min(k, nb - 1u)); });
            __syncthreads();
            find_bin_wide(whist, nb, need, &s_digit, &s_before, &s_bin);
            __syncthreads();
            prefix = s_digit;
            mask = 0xFFFFFFFFu;
            need -= s_before;
            eq = s_bin;
            __syncthreads();
            top = -8;  // no byte passes left
        }
        for (int shift = top; shift >= 0; shift -= 8) {
            hist[tid] = 0;
            __syncthreads();
            for_keys([&](uint32_t k) { hist_add(hist, (k & mask) == prefix, (k >> shift) & 255u); });
            __syncthreads();
            find_digit(hist, need, &s_digit, &s_before, &s_bin);
            __syncthreads();
            prefix |= s_digit << shift;
            mask |= 255u << shift;
            need -= s_before;
            eq = s_bin;
            __syncthreads();
        }
        T = prefix;
        if (KTH || a.out_kth) {
            if (tid == 0) a.out_kth[orow] = T;
            return;
        }
        // ---- phase 2: among key == T take the `need` lowest ids ----------------------
        if (need < eq) {
            uint32_t ip = 0, im = 0, ineed = need;
            for (int shift = 24; shift >= 0; shift -= 8) {
                hist[tid] = 0;
                __syncthreads();
                for (uint32_t i = tid; i < n; i += SEL_THREADS) {
                    const bool t = rv.key(i) == T;
                    const uint32_t id = t ? rv.id(i) : 0u;
                    hist_add(hist, t && (id & im) == ip, (id >> shift) & 255u);
                }
                __syncthreads();
                find_digit(hist, ineed, &s_digit, &s_before, &s_bin);
                __syncthreads();
                ip |= s_digit << shift;
                im |= 255u << shift;
                ineed -= s_before;
                __syncthreads();
            }
            Tid = ip;
        }
    } else if (a.out_kth) {
        // fewer items than k: every key passes
        if (tid == 0) a.out_kth[orow] = 0xFFFFFFFFu;
        return;
    }

    // ---- phase 3: gather the winners and sort them by (key, id) -----------------------
    if constexpr (KTH) return;  // threshold launches always have out_kth (returned above)
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += SEL_THREADS) {
        const uint32_t k = rv.key(i);
        if (take_all || k < T || k == T) {
            const uint32_t id = rv.id(i);
            if (take_all || k < T || id <= Tid) {
                const uint32_t p = atomicAdd(&s_cnt, 1u);
                if (p < SEL_BUF) {
                    okey[p] = k;
                    oid[p] = id;
                }
            }
        }
    }
    __syncthreads();
    uint32_t cnt = s_cnt < SEL_BUF ? s_cnt : SEL_BUF;
    uint32_t P = 1;
    while (P < cnt) P <<= 1;
    for (uint32_t i = cnt + tid; i < P; i += SEL_THREADS) {
        okey[i] = 0xFFFFFFFFu;
        oid[i] = 0xFFFFFFFFu;
    }
    __syncthreads();
    for (uint32_t size = 2; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = tid; t < P / 2; t += SEL_THREADS) {
                const uint32_t i = 2 * t - (t & (stride - 1));
                const uint32_t j = i + stride;
                const bool asc = (i & size) == 0;
                const uint32_t ki = okey[i], kj = okey[j], ii = oid[i], ij = oid[j];
                const bool gt = (ki > kj) || (ki == kj && ii > ij);
                if (gt == asc) {
                    okey[i] = kj;
                    okey[j] = ki;
                    oid[i] = ij;
                    oid[j] = ii;
                }
            }
            __syncthreads();
        }
    }
    // ---- write k slots -----------------------------------------------------------------
    for (uint32_t r = tid; r < a.k; r += SEL_THREADS) {
        const int64_t o = int64_t(orow) * (a.out_ld ? a.out_ld : int64_t(a.k)) + r;
        const bool have = r < cnt && r < K && okey[r] != kAbsentKey;
        const uint32_t k = have ? okey[r] : 0xFFFFFFFFu;
        if (a.out_idx) a.out_idx[o] = have ? oid[r] + a.id_offset : kSentinel;
        if (a.out_key) a.out_key[o] = k;
        if (a.out_f) {
            float v;
            if (!have) v = (a.key_kind == 1) ? -__builtin_inff() : __builtin_inff();
            else v = (a.key_kind == 1) ? float_of_key_desc(k) : float_of_key(k);
            a.out_f[o] = v;
        }
        if (a.out_i32) a.out_i32[o] = have ? (a.key_kind == 3 ? int32_t(k) : i32_of_key(k)) : INT32_MAX;
    }
}

// float values -> ordering keys (dense matrices given to va_topk_select)
__global__ void keys_from_floats(const float* v, uint64_t n, int desc, uint32_t* out) {
    uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (; i < n; i += step) out[i] = desc ? key_of_float_desc(v[i]) : key_of_float(v[i]);
}

// two sorted k-lists per row -> 2k candidate (key, id) pairs; sentinels dropped
__global__ void merge_gather(const uint32_t* ai, const float* ad, const uint32_t* bi, const float* bd, uint32_t rows,
                             uint32_t k, uint32_t chunk_base, uint32_t* ckey, uint32_t* cid, uint32_t* ccnt) {
    const uint32_t row = blockIdx.x;
    __shared__ uint32_t s_n;
    if (threadIdx.x == 0) s_n = 0;
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < 2 * k; r += blockDim.x) {
        const bool from_a = r < k;
        const uint32_t j = from_a ? r : r - k;
        const uint32_t id = from_a ? ai[int64_t(row) * k + j] : bi[int64_t(row) * k + j];
        if (id == kSentinel) continue;
        const float d = from_a ? ad[int64_t(row) * k + j] : bd[int64_t(row) * k + j];
        const uint32_t p = atomicAdd(&s_n, 1u);
        ckey[int64_t(row) * 2 * k + p] = key_of_float(d);
        cid[int64_t(row) * 2 * k + p] = from_a ? id : id + chunk_base;
    }
    __syncthreads();
    if (threadIdx.x == 0) ccnt[row] = s_n;
}

}  // namespace

va_status launch_select(va_context* ctx, const SelectArgs& a) {
    if (a.rows == 0) return VA_OK;
    if (a.k > SEL_BUF) return fail(ctx, VA_ERR_INVALID_ARG, "k=%u exceeds the maximum %u", a.k, SEL_BUF);
    // Candidate lists are mostly far below their capacity, which sizes the LDS copy: past 8K
    // entries a large copy would leave one workgroup per CU, so such rows are read from memory
    // (L2-resident lists) by many workgroups at once instead.
    const bool cache = a.n <= kSelCache && !((a.counts || a.out_kth) && a.n > 8192);
    if (!cache && a.out_kth) {
        select_kernel<false, true><<<dim3(a.rows), dim3(SEL_THREADS), 0, ctx->stream>>>(a);
    } else if (cache) {
        const size_t lds = size_t(std::max<uint32_t>(a.n, 1)) * 4;
        auto kern = a.out_kth ? &select_kernel<true, true> : &select_kernel<true, false>;
        if (lds > 48 * 1024)
            VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
        kern<<<dim3(a.rows), dim3(SEL_THREADS), lds, ctx->stream>>>(a);
    } else {
        select_kernel<false><<<dim3(a.rows), dim3(SEL_THREADS), 0, ctx->stream>>>(a);
    }
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

}  // namespace va

extern "C" {

va_status va_topk_select(va_context* ctx, const float* values, uint32_t num_rows, uint32_t num_elements, uint32_t k,
                         va_select_mode mode, uint32_t* out_idx, float* out_values) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, values && out_idx, "va_topk_select: NULL pointer");
    VA_REQUIRE(ctx, num_rows > 0 && num_elements > 0, "va_topk_select: empty input");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "va_topk_select: k must be in [1, %u], got %u", VA_MAX_K, k);
    VA_REQUIRE(ctx, mode == VA_SELECT_MIN || mode == VA_SELECT_MAX, "va_topk_select: bad mode");
    va::DeviceGuard g(ctx->device);
    const uint64_t total = uint64_t(num_rows) * num_elements;
    va::Scratch s(ctx);
    VA_CHECK_STATUS(s.reserve(va::Scratch::round(total * 4)));
    uint32_t* keys = s.carve<uint32_t>(total);
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    va::keys_from_floats<<<dim3(uint32_t(blocks)), dim3(256), 0, ctx->stream>>>(values, total, mode == VA_SELECT_MAX,
                                                                                keys);
    VA_CHECK_LAUNCH(ctx);
    va::SelectArgs a;
    a.keys = keys;
    a.ld = num_elements;
    a.n = num_elements;
    a.rows = num_rows;
    a.k = k;
    a.out_idx = out_idx;
    a.out_f = out_values;
    a.key_kind = mode == VA_SELECT_MAX ? 1 : 0;
    return va::launch_select(ctx, a);
}

va_status va_topk_merge(va_context* ctx, const uint32_t* a_idx, const float* a_dist, const uint32_t* b_idx,
                        const float* b_dist, uint32_t num_rows, uint32_t k, uint32_t chunk_base, uint32_t* out_idx,
                        float* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, a_idx && a_dist && b_idx && b_dist && out_idx, "va_topk_merge: NULL pointer");
    VA_REQUIRE(ctx, num_rows > 0, "va_topk_merge: empty input");
    VA_REQUIRE(ctx, k > 0 && k <= VA_MAX_K, "va_topk_merge: k must be in [1, %u], got %u", VA_MAX_K, k);
    va::DeviceGuard g(ctx->device);
    const uint64_t cand = uint64_t(num_rows) * 2 * k;
    va::Scratch s(ctx);
    VA_CHECK_STATUS(s.reserve(va::Scratch::round(cand * 4) * 2 + va::Scratch::round(uint64_t(num_rows) * 4)));
    uint32_t* ckey = s.carve<uint32_t>(cand);
    uint32_t* cid = s.carve<uint32_t>(cand);
    uint32_t* ccnt = s.carve<uint32_t>(num_rows);
    va::merge_gather<<<dim3(num_rows), dim3(256), 0, ctx->stream>>>(a_idx, a_dist, b_idx, b_dist, num_rows, k,
                                                                     chunk_base, ckey, cid, ccnt);
    VA_CHECK_LAUNCH(ctx);
    va::SelectArgs a;
    a.keys = ckey;
    a.ids = cid;
    a.counts = ccnt;
    a.ld = 2 * k;
    a.n = 2 * k;
    a.rows = num_rows;
    a.k = k;
    a.out_idx = out_idx;
    a.out_f = out_dist;
    return va::launch_select(ctx, a);
}

}  // extern "C"
