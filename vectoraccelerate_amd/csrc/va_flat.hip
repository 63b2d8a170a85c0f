// va_flat.hip — fp32 distance entry points and the fused flat top-k search.
#include <algorithm>
#include <vector>

#include "va_fallback.hpp"
#include "va_internal.hpp"

namespace va {
namespace {

// One wave64 per pair; float4 loads when the rows allow it.  HBM-bound.
// l2_distance / cosine_similarity (Metal/Shaders/DistanceShaders.metal:169-321) give one
// threadgroup per pair; a wave is enough on CDNA and keeps 4 pairs in flight per workgroup.
template <int COS>
__global__ __launch_bounds__(256) void pairs_kernel(const float* __restrict__ q, const float* __restrict__ t,
                                                    float* __restrict__ out, uint32_t P, uint32_t D, int flag,
                                                    int vec) {
    const uint32_t pair = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (pair >= P) return;
    const float* a = q + int64_t(pair) * D;
    const float* b = t + int64_t(pair) * D;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
    if (vec) {
        for (uint32_t i = uint32_t(lane) * 4; i < D; i += 256) {
            const float4 x = *reinterpret_cast<const float4*>(a + i);
            const float4 y = *reinterpret_cast<const float4*>(b + i);
            if (COS) {
                s0 = fmaf(x.x, y.x, s0); s0 = fmaf(x.y, y.y, s0); s0 = fmaf(x.z, y.z, s0); s0 = fmaf(x.w, y.w, s0);
                s1 = fmaf(x.x, x.x, s1); s1 = fmaf(x.y, x.y, s1); s1 = fmaf(x.z, x.z, s1); s1 = fmaf(x.w, x.w, s1);
                s2 = fmaf(y.x, y.x, s2); s2 = fmaf(y.y, y.y, s2); s2 = fmaf(y.z, y.z, s2); s2 = fmaf(y.w, y.w, s2);
            } else {
                const float d0 = x.x - y.x, d1 = x.y - y.y, d2 = x.z - y.z, d3 = x.w - y.w;
                s0 = fmaf(d0, d0, s0); s0 = fmaf(d1, d1, s0); s0 = fmaf(d2, d2, s0); s0 = fmaf(d3, d3, s0);
            }
        }
    } else {
        for (uint32_t i = uint32_t(lane); i < D; i += 64) {
            const float x = a[i], y = b[i];
            if (COS) {
                s0 = fmaf(x, y, s0);
                s1 = fmaf(x, x, s1);
                s2 = fmaf(y, y, s2);
            } else {
                const float d = x - y;
                s0 = fmaf(d, d, s0);
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        s0 += __shfl_xor(s0, off);
        if (COS) {
            s1 += __shfl_xor(s1, off);
            s2 += __shfl_xor(s2, off);
        }
    }
    if (lane != 0) return;
    if (COS) {
        // DistanceShaders.metal:300-319: sqrt(a)*sqrt(b), FLT_MIN floor, NaN-preserving clamp
        const float denom = sqrtf(s1) * sqrtf(s2);
        const float raw = (denom < 1.17549435e-38f) ? 0.0f : s0 / denom;
        const float sim = (raw != raw) ? raw : fminf(fmaxf(raw, -1.0f), 1.0f);
        out[pair] = flag ? 1.0f - sim : sim;
    } else {
        out[pair] = flag ? sqrtf(s0) : s0;
    }
}

bool rows_vec4(const void* p, uint32_t D) { return (D % 4 == 0) && ((reinterpret_cast<uintptr_t>(p) & 15) == 0); }

va_status launch_pairs(va_context* ctx, int cos, const float* q, const float* t, float* out, uint32_t P, uint32_t D,
                       int flag) {
    const int vec = rows_vec4(q, D) && rows_vec4(t, D);
    const uint32_t blocks = (P + 3) / 4;
    if (cos)
        pairs_kernel<1><<<dim3(blocks), dim3(256), 0, ctx->stream>>>(q, t, out, P, D, flag, vec);
    else
        pairs_kernel<0><<<dim3(blocks), dim3(256), 0, ctx->stream>>>(q, t, out, P, D, flag, vec);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status all_pairs(va_context* ctx, const char* fn, const float* q, const float* x, float* out, uint32_t Q,
                    uint32_t N, uint32_t D, DistOp op) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, q && x && out, "%s: NULL pointer", fn);
    VA_REQUIRE(ctx, Q > 0 && N > 0, "%s: empty input vectors", fn);
    VA_REQUIRE(ctx, D > 0, "%s: dimension must be positive", fn);
    DeviceGuard g(ctx->device);
    DistArgs a;
    a.q = q;
    a.ldq = D;
    a.x = x;
    a.ldx = D;
    a.Q = Q;
    a.N = N;
    a.D = D;
    a.op = op;
    a.out = OUT_VALUES;
    a.out_f = out;
    a.ldo = N;
    return launch_dist(ctx, a);
}

// fp32 distance keys for the exact scan driver
struct F32Producer final : KeyProducer {
    va_context* ctx;
    const float* q;
    const float* x;
    uint32_t Q, N, D;
    DistOp op;
    va_status fallback_pass(const FbArgs& a, int pass) override {
        return fb_launch_pass(ctx, FbF32{q, int64_t(D), x, int64_t(D), N, D, int(op)}, a, pass);
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
        a.op = op;
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
        a.op = op;
        a.out = OUT_FILTER;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_key = ckey;
        a.cand_id = cid;
        a.cap = cap;
        return launch_dist(ctx, a);
    }
};

}  // namespace

// Exact top-k of queries (device) against a device database: the screened path where it applies
// (over the fp16 shadow when one is given), else the fp32 scan.  Queued on the context's stream
// without a host synchronisation (overflowed queries are finished on the device), except with a
// fixed scratch block too small for the device fallback.
va_status flat_topk(va_context* ctx, DistOp op, const float* q, const float* x, uint32_t Q, uint32_t N, uint32_t D,
                    uint32_t k, uint32_t* out_idx, float* out_dist, const _Float16* shadow, const float* norms,
                    const uint8_t* skip, const float* errs) {
    F32Producer p;
    p.ctx = ctx;
    p.q = q;
    p.x = x;
    p.Q = Q;
    p.N = N;
    p.D = D;
    p.op = op;
    ScanOutputs o;
    o.idx = out_idx;
    o.f = out_dist;
    o.key_kind = 0;
    o.skip = skip;
    ScreenInput si;
    si.q = q;
    si.x = x;
    si.Q = Q;
    si.N = N;
    si.D = D;
    si.op = op;
    si.xh = shadow;
    si.xn = norms;
    si.xe = shadow ? errs : nullptr;
    if (screen_applies(ctx, si, k)) return screened_topk_scan(ctx, si, p, k, o);
    return exact_topk_scan(ctx, p, Q, N, k, o);
}

}  // namespace va

extern "C" {

va_status va_l2_pairs(va_context* ctx, const float* queries, const float* targets, float* out, uint32_t num_pairs,
                      uint32_t dim, int compute_sqrt) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, queries && targets && out, "va_l2_pairs: NULL pointer");
    VA_REQUIRE(ctx, num_pairs > 0 && dim > 0, "va_l2_pairs: empty input");
    va::DeviceGuard g(ctx->device);
    return va::launch_pairs(ctx, 0, queries, targets, out, num_pairs, dim, compute_sqrt != 0);
}

va_status va_cosine_pairs(va_context* ctx, const float* queries, const float* targets, float* out, uint32_t num_pairs,
                          uint32_t dim, int output_distance) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, queries && targets && out, "va_cosine_pairs: NULL pointer");
    VA_REQUIRE(ctx, num_pairs > 0 && dim > 0, "va_cosine_pairs: empty input");
    va::DeviceGuard g(ctx->device);
    return va::launch_pairs(ctx, 1, queries, targets, out, num_pairs, dim, output_distance != 0);
}

va_status va_l2_all_pairs(va_context* ctx, const float* queries, const float* database, float* out,
                          uint32_t num_queries, uint32_t num_database, uint32_t dim, int compute_sqrt) {
    return va::all_pairs(ctx, "va_l2_all_pairs", queries, database, out, num_queries, num_database, dim,
                         compute_sqrt ? va::OP_L2 : va::OP_L2SQ);
}

va_status va_cosine_all_pairs(va_context* ctx, const float* queries, const float* database, float* out,
                              uint32_t num_queries, uint32_t num_database, uint32_t dim, int output_distance) {
    return va::all_pairs(ctx, "va_cosine_all_pairs", queries, database, out, num_queries, num_database, dim,
                         output_distance ? va::OP_COS_DIST : va::OP_COS_SIM);
}

va_status va_dot_all_pairs(va_context* ctx, const float* queries, const float* database, float* out,
                           uint32_t num_queries, uint32_t num_database, uint32_t dim, int absolute_value) {
    return va::all_pairs(ctx, "va_dot_all_pairs", queries, database, out, num_queries, num_database, dim,
                         absolute_value ? va::OP_ABS_DOT : va::OP_DOT);
}

va_status va_fused_topk(va_context* ctx, va_metric metric, const float* queries, const float* database,
                        uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k, uint32_t* out_idx,
                        float* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    // FusedL2TopKParameters validation (Kernels/Metal4/FusedL2TopKKernel.swift:57-79), minus the
    // dimension <= 768 and k <= 128 limits of the reference shader
    VA_REQUIRE(ctx, queries && database && out_idx, "va_fused_topk: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "numQueries must be positive, got %u", num_queries);
    VA_REQUIRE(ctx, num_database > 0, "numDataset must be positive, got %u", num_database);
    VA_REQUIRE(ctx, dim > 0, "dimension must be positive, got %u", dim);
    VA_REQUIRE(ctx, k > 0, "k must be positive, got %u", k);
    VA_REQUIRE(ctx, k <= VA_MAX_K, "k %u exceeds maximum supported k %u", k, VA_MAX_K);
    VA_REQUIRE(ctx, metric >= VA_METRIC_L2SQ && metric <= VA_METRIC_L2, "va_fused_topk: unknown metric %d", int(metric));
    va::DeviceGuard g(ctx->device);
    return va::flat_topk(ctx, va::metric_op(metric), queries, database, num_queries, num_database, dim, k, out_idx,
                         out_dist);
}

va_status va_fused_topk_streamed(va_context* ctx, va_metric metric, const float* queries, const float* host_database,
                                 uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k,
                                 uint32_t chunk_rows, uint32_t* out_idx, float* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, queries && host_database && out_idx, "va_fused_topk_streamed: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "numQueries must be positive, got %u", num_queries);
    VA_REQUIRE(ctx, num_database > 0, "numDataset must be positive, got %u", num_database);
    VA_REQUIRE(ctx, dim > 0, "dimension must be positive, got %u", dim);
    VA_REQUIRE(ctx, k > 0, "k must be positive, got %u", k);
    VA_REQUIRE(ctx, k <= VA_MAX_K, "k %u exceeds maximum supported k %u", k, VA_MAX_K);
    VA_REQUIRE(ctx, metric >= VA_METRIC_L2SQ && metric <= VA_METRIC_L2, "va_fused_topk_streamed: unknown metric %d",
               int(metric));
    va::DeviceGuard g(ctx->device);
    const va::DistOp op = va::metric_op(metric);
    const uint64_t row_bytes = uint64_t(dim) * 4;
    // chunks of ~512 MiB by default (two are resident: the one being scanned and the next)
    uint64_t rows = chunk_rows ? chunk_rows : std::max<uint64_t>(1, (512ull << 20) / row_bytes);
    rows = std::min<uint64_t>(rows, num_database);
    const uint32_t C = uint32_t(rows);
    const uint32_t nch = uint32_t((uint64_t(num_database) + C - 1) / C);
    const uint64_t qk = uint64_t(num_queries) * k;

    // Buffers of this call (the scan and the merge use the context's scratch arena in turn, so the
    // running lists and the chunks cannot live there).
    struct Owned {
        std::vector<void*> p;
        std::vector<hipEvent_t> e;
        ~Owned() {
            for (void* q : p) (void)hipFree(q);
            for (hipEvent_t ev : e) (void)hipEventDestroy(ev);
        }
    } own;
    auto alloc = [&](size_t bytes, void** out) -> va_status {
        VA_CHECK_HIP(ctx, hipMalloc(out, bytes));
        own.p.push_back(*out);
        return VA_OK;
    };
    float* buf[2] = {nullptr, nullptr};
    uint32_t* run_idx[2];
    float* run_dist[2];
    uint32_t* ch_idx;
    float* ch_dist;
    for (int b = 0; b < (nch > 1 ? 2 : 1); ++b)
        VA_CHECK_STATUS(alloc(size_t(C) * row_bytes, reinterpret_cast<void**>(&buf[b])));
    for (int b = 0; b < 2; ++b) {
        VA_CHECK_STATUS(alloc(qk * 4, reinterpret_cast<void**>(&run_idx[b])));
        VA_CHECK_STATUS(alloc(qk * 4, reinterpret_cast<void**>(&run_dist[b])));
    }
    VA_CHECK_STATUS(alloc(qk * 4, reinterpret_cast<void**>(&ch_idx)));
    VA_CHECK_STATUS(alloc(qk * 4, reinterpret_cast<void**>(&ch_dist)));
    hipEvent_t up_ev[2], use_ev[2];
    for (int b = 0; b < 2; ++b) {
        VA_CHECK_HIP(ctx, hipEventCreateWithFlags(&up_ev[b], hipEventDisableTiming));
        own.e.push_back(up_ev[b]);
        VA_CHECK_HIP(ctx, hipEventCreateWithFlags(&use_ev[b], hipEventDisableTiming));
        own.e.push_back(use_ev[b]);
    }
    // uploads run on an auxiliary stream (after the work already queued on the context's stream)
    VA_CHECK_STATUS(va::aux_fork(ctx));
    hipStream_t cs = ctx->aux[0];
    auto upload = [&](uint32_t c) -> va_status {
        const uint64_t r0 = uint64_t(c) * C;
        const uint64_t n = std::min<uint64_t>(C, num_database - r0);
        VA_CHECK_HIP(ctx, hipMemcpyAsync(buf[c & 1], host_database + r0 * dim, size_t(n * row_bytes),
                                         hipMemcpyHostToDevice, cs));
        VA_CHECK_HIP(ctx, hipEventRecord(up_ev[c & 1], cs));
        return VA_OK;
    };
    VA_CHECK_STATUS(upload(0));
    if (nch > 1) VA_CHECK_STATUS(upload(1));
    int cur = 0;
    for (uint32_t c = 0; c < nch; ++c) {
        const int b = int(c & 1);
        const uint32_t r0 = c * C;
        const uint32_t n = std::min(C, num_database - r0);
        VA_CHECK_HIP(ctx, hipStreamWaitEvent(ctx->stream, up_ev[b], 0));
        // the scan synchronises the host, so the upload of chunk c+1 (queued before) overlaps it
        VA_CHECK_STATUS(va::flat_topk(ctx, op, queries, buf[b], num_queries, n, dim, k, c == 0 ? run_idx[0] : ch_idx,
                                      c == 0 ? run_dist[0] : ch_dist));
        VA_CHECK_HIP(ctx, hipEventRecord(use_ev[b], ctx->stream));
        if (c > 0) {
            VA_CHECK_STATUS(va_topk_merge(ctx, run_idx[cur], run_dist[cur], ch_idx, ch_dist, num_queries, k, r0,
                                          run_idx[cur ^ 1], run_dist[cur ^ 1]));
            cur ^= 1;
        }
        if (c + 2 < nch) {
            VA_CHECK_HIP(ctx, hipStreamWaitEvent(cs, use_ev[b], 0));
            VA_CHECK_STATUS(upload(c + 2));
        }
    }
    VA_CHECK_HIP(ctx, hipMemcpyAsync(out_idx, run_idx[cur], size_t(qk) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    if (out_dist)
        VA_CHECK_HIP(ctx, hipMemcpyAsync(out_dist, run_dist[cur], size_t(qk) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    // the buffers of this call are freed on return
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(cs));
    return VA_OK;
}

}  // extern "C"
