// va_scan.hip — exact top-k scan driver shared by the fp32, int8 and binary search paths.
//
// The reference picks between a fused K<=8 shader and a two-pass path that materialises
// the Q x N distance matrix in 64 MB chunks (FusedL2TopKKernel.execute,
// Kernels/Metal4/FusedL2TopKKernel.swift:367-427, :765-1090).  Here every k takes one path
// and the full matrix is never stored:
//   1. sample:  dense keys of each query against S strided rows; tau_q = the r-th smallest
//               (r = k: an upper bound of the true k-th key, since the sample rows are real
//               rows and the filter pass computes bit-identical keys for them; r < k: a
//               tighter threshold that is checked in step 3, see sample_rank);
//   2. filter:  the scan kernel appends every key <= tau_q to the query's candidate list;
//   3. select:  exact (key, id) top-k of every candidate list that holds at least k keys
//               (then every key of the top-k is <= tau_q, so all of them are in the list);
//   4. overflow: rows whose list outgrew its capacity, or fell short of k, are recomputed
//               exactly by chunked dense keys + select + a final select over the per-chunk
//               winners.
#include <algorithm>
#include <cmath>
#include <vector>

#include "va_fallback.hpp"
#include "va_internal.hpp"

namespace va {

__global__ void mask_dense_kernel(uint32_t* keys, uint32_t cols, int64_t ld, uint32_t row0, uint32_t stride,
                                  const uint8_t* __restrict__ skip) {
    uint32_t* k = keys + int64_t(blockIdx.y) * ld;
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < cols; j += gridDim.x * 256)
        if (skip[row0 + uint64_t(j) * stride]) k[j] = kAbsentKey;
}

__global__ void mask_list_kernel(uint32_t* keys, uint32_t* keys2, const uint32_t* __restrict__ ids,
                                 const uint32_t* __restrict__ counts, uint32_t cap, int64_t ld,
                                 const uint8_t* __restrict__ skip, const uint32_t* __restrict__ id_map) {
    const uint32_t r = blockIdx.y;
    const uint32_t n = min(counts[r], cap);
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const int64_t o = int64_t(r) * ld + i;
        uint32_t id = ids[o];
        if (id != kSentinel && id_map) id = id_map[id];
        if (id != kSentinel && skip[id]) {
            keys[o] = kAbsentKey;
            if (keys2) keys2[o] = kAbsentKey;
        }
    }
}

va_status mask_dense_keys(va_context* ctx, uint32_t* keys, uint32_t rows, uint32_t cols, int64_t ld, uint32_t row0,
                          uint32_t stride, const uint8_t* skip) {
    if (!skip || rows == 0 || cols == 0) return VA_OK;
    const uint32_t bx = std::min<uint32_t>(64, (cols + 255) / 256);
    for (uint32_t r0 = 0; r0 < rows; r0 += 65535) {
        const uint32_t nr = std::min<uint32_t>(65535, rows - r0);
        mask_dense_kernel<<<dim3(bx, nr), dim3(256), 0, ctx->stream>>>(keys + int64_t(r0) * ld, cols, ld, row0, stride,
                                                                      skip);
        VA_CHECK_LAUNCH(ctx);
    }
    return VA_OK;
}

va_status mask_list_keys(va_context* ctx, uint32_t* keys, uint32_t* keys2, const uint32_t* ids, const uint32_t* counts,
                         uint32_t rows, uint32_t cap, int64_t ld, const uint8_t* skip, const uint32_t* id_map) {
    if (!skip || rows == 0 || cap == 0) return VA_OK;
    const uint32_t bx = std::min<uint32_t>(16, (cap + 255) / 256);
    for (uint32_t r0 = 0; r0 < rows; r0 += 65535) {
        const uint32_t nr = std::min<uint32_t>(65535, rows - r0);
        mask_list_kernel<<<dim3(bx, nr), dim3(256), 0, ctx->stream>>>(keys + int64_t(r0) * ld,
                                                                     keys2 ? keys2 + int64_t(r0) * ld : nullptr,
                                                                     ids + int64_t(r0) * ld, counts + r0, cap, ld, skip,
                                                                     id_map);
        VA_CHECK_LAUNCH(ctx);
    }
    return VA_OK;
}

bool fb_fits(const va_context* ctx, size_t need, uint32_t rows, uint32_t N, uint32_t k) {
    return fb_fits_in(ctx->fixed_scratch ? ctx->fixed_scratch_bytes : 0, need, rows, N, k);
}

size_t dense_budget(const va_context* ctx) {
    return dense_budget_for(ctx->fixed_scratch ? ctx->fixed_scratch_bytes : 0);
}

// (The screened scan took N/32 sample rows while its threshold was the sample's k-th bound; with
// the checked smaller rank N/64 is faster there too: configs[1] 3.98 -> 3.84 ms per search.)
ScanPlan plan_scan(const va_context* ctx, uint32_t Q, uint32_t N, uint32_t k) {
    return plan_scan_for(dense_budget(ctx), ctx->opt_sample_rows, ctx->opt_candidate_cap, Q, N, k);
}

va_status rescan_rows(va_context* ctx, KeyProducer& kp, uint32_t N, uint32_t k, const SelectArgs& base,
                      const uint32_t* rows_dev, uint32_t n_rows, const uint8_t* skip) {
    if (n_rows == 0) return VA_OK;
    // The row list is read back first: the arena below may be regrown (which frees it).
    std::vector<uint32_t> rows_host(n_rows);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(rows_host.data(), rows_dev, size_t(n_rows) * 4, hipMemcpyDeviceToHost,
                                     ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // rows are processed in batches of R; each batch scans the database in chunks of C rows
    // (a fixed scratch block halves R until the batch fits)
    const uint64_t budget = dense_budget(ctx);
    uint32_t R = std::min<uint32_t>(n_rows, 64), C = 0, nch = 0;
    size_t need = 0;
    for (;;) {
        C = uint32_t(std::max<uint64_t>(k, std::min<uint64_t>(N, budget / (uint64_t(R) * 4))));
        nch = (N + C - 1) / C;
        need = Scratch::round(uint64_t(n_rows) * 4) + Scratch::round(uint64_t(R) * C * 4) +
               Scratch::round(uint64_t(R) * nch * k * 4) * 2;
        if (!ctx->fixed_scratch || need <= ctx->fixed_scratch_bytes || R == 1) break;
        R = (R + 1) / 2;
    }
    Scratch f(ctx);
    VA_CHECK_STATUS(f.reserve(need));
    uint32_t* ovf_rows = f.carve<uint32_t>(n_rows);
    uint32_t* dkeys = f.carve<uint32_t>(uint64_t(R) * C);
    uint32_t* wkey = f.carve<uint32_t>(uint64_t(R) * nch * k);
    uint32_t* wid = f.carve<uint32_t>(uint64_t(R) * nch * k);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(ovf_rows, rows_host.data(), size_t(n_rows) * 4, hipMemcpyHostToDevice,
                                     ctx->stream));
    for (uint32_t r0 = 0; r0 < n_rows; r0 += R) {
        const uint32_t nr = std::min(R, n_rows - r0);
        const uint32_t* rows = ovf_rows + r0;
        for (uint32_t c = 0; c < nch; ++c) {
            const uint32_t c0 = c * C;
            const uint32_t cols = std::min(C, N - c0);
            VA_CHECK_STATUS(kp.dense(rows, 0, nr, c0, cols, 1, dkeys, C));
            VA_CHECK_STATUS(mask_dense_keys(ctx, dkeys, nr, cols, C, c0, 1, skip));
            SelectArgs a;
            a.keys = dkeys;
            a.ld = C;
            a.n = cols;
            a.rows = nr;
            a.k = k;
            a.id_offset = c0;
            a.out_ld = int64_t(nch) * k;
            a.out_idx = wid + int64_t(c) * k;
            a.out_key = wkey + int64_t(c) * k;
            VA_CHECK_STATUS(launch_select(ctx, a));
        }
        SelectArgs a = base;
        a.keys = wkey;
        a.ids = wid;
        a.counts = nullptr;
        a.ld = int64_t(nch) * k;
        a.n = nch * k;
        a.rows = nr;
        a.row_map = rows;
        a.overflow_count = nullptr;
        a.overflow_rows = nullptr;
        VA_CHECK_STATUS(launch_select(ctx, a));
    }
    // the host copy of the row list must outlive the upload above
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VA_OK;
}

// The order statistic of the sample that becomes a query's threshold (sample_rank_for): with
// r < k the filter keeps about r N / S rows instead of k N / S, and a query is short of k
// candidates exactly when r of its k nearest rows are in the sample (then the select lists it for
// the exact fallback).
uint32_t sample_rank(const va_context* ctx, uint32_t k, uint64_t S, uint32_t N, bool masked) {
    return sample_rank_for(ctx->opt_sample_rank, k, S, N, masked);
}

va_status exact_topk_scan(va_context* ctx, KeyProducer& kp, uint32_t Q, uint32_t N, uint32_t k,
                          const ScanOutputs& out) {
    SelectArgs base;
    base.k = k;
    base.out_idx = out.idx;
    base.out_f = out.f;
    base.out_i32 = out.i32;
    base.out_key = out.key;
    base.key_kind = out.key_kind;
    base.key_bits = kp.key_bits();

    // ---- plan ------------------------------------------------------------------------
    const ScanPlan plan = plan_scan(ctx, Q, N, k);
    const uint64_t S = plan.S;
    const bool direct = plan.direct;
    ScanPhaseMarks pm(ctx);
    ctx->last_scan = va_scan_timings{};
    VA_CHECK_STATUS(pm.mark(0));
    if (direct) {
        ctx->last_scan.scan_launches = 0;
        // small database: dense keys in query chunks + select
        const uint64_t per_q = uint64_t(N) * 4;
        uint32_t qc = uint32_t(std::max<uint64_t>(1, std::min<uint64_t>(Q, dense_budget(ctx) / per_q)));
        Scratch s(ctx);
        VA_CHECK_STATUS(s.reserve(Scratch::round(uint64_t(qc) * per_q)));
        uint32_t* keys = s.carve<uint32_t>(uint64_t(qc) * N);
        for (uint32_t q0 = 0; q0 < Q; q0 += qc) {
            const uint32_t nq = std::min(qc, Q - q0);
            VA_CHECK_STATUS(kp.dense(nullptr, q0, nq, 0, N, 1, keys, N));
            VA_CHECK_STATUS(mask_dense_keys(ctx, keys, nq, N, N, 0, 1, out.skip));
            ctx->last_scan.scan_launches++;
            SelectArgs a = base;
            a.keys = keys;
            a.ld = N;
            a.n = N;
            a.rows = nq;
            if (out.idx) a.out_idx = out.idx + int64_t(q0) * k;
            if (out.f) a.out_f = out.f + int64_t(q0) * k;
            if (out.i32) a.out_i32 = out.i32 + int64_t(q0) * k;
            if (out.key) a.out_key = out.key + int64_t(q0) * k;
            VA_CHECK_STATUS(launch_select(ctx, a));
        }
        return pm.finish(false, false);
    }
    const uint32_t stride = plan.stride;
    const uint64_t cap = plan.cap;
    const uint32_t rank = sample_rank(ctx, k, S, N, out.skip != nullptr);
    const uint32_t qs = plan.qs;

    Scratch s(ctx);
    size_t need = exact_scan_need(Q, plan);
    // overflowed rows are finished on the device (no read-back) when the fallback's buffers fit
    const bool device_fb = fb_fits(ctx, need, Q, N, k);
    if (device_fb) need += fb_bytes(Q, N, k);
    VA_CHECK_STATUS(s.reserve(need));
    uint32_t* thr = s.carve<uint32_t>(Q);
    uint32_t* cnt = s.carve<uint32_t>(Q);
    uint32_t* ovf_rows = s.carve<uint32_t>(Q);
    uint32_t* ckey = s.carve<uint32_t>(uint64_t(Q) * cap);
    uint32_t* cid = s.carve<uint32_t>(uint64_t(Q) * cap);
    uint32_t* ovf_cnt = s.carve<uint32_t>(64);
    uint32_t* skeys = s.carve<uint32_t>(uint64_t(qs) * S);
    FbArgs fb;
    if (device_fb) {
        fb = fb_carve(s, Q, N, k);
        fb.n_rows = ovf_cnt;
        fb.rows = ovf_rows;
        fb.skip = out.skip;
    }
    VA_CHECK_STATUS(s.verify(need));

    // ---- 1. sample thresholds -----------------------------------------------------------
    for (uint32_t q0 = 0; q0 < Q; q0 += qs) {
        const uint32_t nq = std::min(qs, Q - q0);
        VA_CHECK_STATUS(kp.dense(nullptr, q0, nq, 0, uint32_t(S), stride, skeys, int64_t(S)));
        VA_CHECK_STATUS(mask_dense_keys(ctx, skeys, nq, uint32_t(S), int64_t(S), 0, stride, out.skip));
        SelectArgs a;
        a.keys = skeys;
        a.ld = int64_t(S);
        a.n = uint32_t(S);
        a.rows = nq;
        a.k = rank;
        a.out_kth = thr + q0;
        a.key_bits = kp.key_bits();
        VA_CHECK_STATUS(launch_select(ctx, a));
    }
    // ---- 2. filter --------------------------------------------------------------------
    VA_CHECK_STATUS(fill_u32(ctx, cnt, Q, 0));
    VA_CHECK_STATUS(fill_u32(ctx, ovf_cnt, 1, 0));
    VA_CHECK_STATUS(pm.mark(1));
    VA_CHECK_STATUS(kp.filter(thr, cnt, ckey, cid, uint32_t(cap)));
    VA_CHECK_STATUS(pm.mark(2));
    VA_CHECK_STATUS(mask_list_keys(ctx, ckey, nullptr, cid, cnt, Q, uint32_t(cap), int64_t(cap), out.skip));
    ctx->last_scan.scan_launches = 1;
    ctx->last_scan.sample_rows = uint32_t(S);
    ctx->last_scan.candidate_cap = uint32_t(cap);
    // ---- 3. select ----------------------------------------------------------------------
    {
        SelectArgs a = base;
        a.keys = ckey;
        a.ids = cid;
        a.counts = cnt;
        a.ld = int64_t(cap);
        a.n = uint32_t(cap);
        a.rows = Q;
        a.overflow_count = ovf_cnt;
        a.overflow_rows = ovf_rows;
        a.min_count = rank < k ? k : 0;
        VA_CHECK_STATUS(launch_select(ctx, a));
    }
    if (device_fb) VA_CHECK_STATUS(pm.count_overflow(ovf_cnt));  // profiling only
    VA_CHECK_STATUS(pm.mark(3));
    if (device_fb) {
        // ---- 4. exact top-k of the overflowed rows, on the device ------------------------------
        VA_CHECK_STATUS(fb_run(ctx, kp, fb, base));
        return pm.finish(true, true);
    }
    VA_CHECK_HIP(ctx, hipMemcpyAsync(ctx->host_word, ovf_cnt, 4, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const uint32_t n_ovf = ctx->host_word[0];
    ctx->last_scan.overflow_rows = n_ovf;
    if (n_ovf == 0) return pm.finish(true, false);

    // ---- 4. exact chunked recomputation of overflowed rows ---------------------------------
    VA_CHECK_STATUS(rescan_rows(ctx, kp, N, k, base, ovf_rows, n_ovf, out.skip));
    return pm.finish(true, true);
}

}  // namespace va
