// va_context.hip — GPUContext (hipStream + scratch arena), buffers, status text.
//
// Replaces Metal4Context / GPUContext (Core/Metal4Context.swift:183-269, executeAndWait
// :342-410, getBuffer :471-488) and BufferPool tokens (Core/BufferPool.swift:89-200).
#include <cstdlib>
#include <cstring>

#include "va_internal.hpp"

namespace va {

va_status fail(va_context* ctx, va_status st, const char* fmt, ...) {
    if (ctx) {
        char buf[1024];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->last_error = buf;
    }
    return st;
}

va_status Scratch::reserve(size_t total) {
    if (ctx->fixed_scratch) {
        if (total <= ctx->fixed_scratch_bytes) return VA_OK;
        return fail(ctx, VA_ERR_INVALID_ARG,
                    "this search needs %zu bytes of scratch; the allocation-free entry point has %zu "
                    "(VA_NOALLOC_SCRATCH_BYTES): use va_fused_topk",
                    total, ctx->fixed_scratch_bytes);
    }
    if (total <= ctx->scratch_bytes) return VA_OK;
    // grow: wait for in-flight users of the old arena, then replace it
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->scratch) {
        VA_CHECK_HIP(ctx, hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
    }
    size_t want = total + total / 4;  // headroom to avoid regrowth on similar shapes
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        want = total;
        e = hipMalloc(&p, want);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(ctx, VA_ERR_OOM, "scratch allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
    }
    ctx->scratch = static_cast<char*>(p);
    ctx->scratch_bytes = want;
    return VA_OK;
}

va_context::ScanRecord* profile_record(va_context* ctx) {
    auto& r = ctx->rec[ctx->rec_next];
    if (!r.ev[0]) return nullptr;
    if (r.pending) profile_fold(ctx, r);
    ctx->rec_next = (ctx->rec_next + 1) % va_context::kScanRing;
    r.has_ovf = r.has_rerank = false;
    return &r;
}

void profile_fold(va_context* ctx, va_context::ScanRecord& r) {
    (void)ctx;
    r.pending = false;
    if (hipEventSynchronize(r.ev[r.light ? 2 : 4]) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    auto ms = [&](int a, int b) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, r.ev[a], r.ev[b]) != hipSuccess) {
            (void)hipGetLastError();
            return -1.0f;
        }
        return t;
    };
    va_scan_timings& t = r.t;
    if (r.light) {
        // the scan phase alone (events 1 and 2)
        t.scan_ms = ms(1, 2);
        t.total_ms = t.scan_ms;
        t.sample_ms = t.select_ms = t.fallback_ms = 0.0f;
    } else if (r.sampled) {
        t.total_ms = ms(0, 4);
        t.sample_ms = ms(0, 1);
        t.scan_ms = ms(1, 2);
        t.select_ms = ms(2, 3);
        t.fallback_ms = r.fallback ? ms(3, 4) : 0.0f;
    } else {
        t.total_ms = ms(0, 4);
        t.sample_ms = 0.0f;
        t.scan_ms = t.total_ms;
        t.select_ms = 0.0f;
        t.fallback_ms = 0.0f;
    }
    if (r.has_ovf) t.overflow_rows = r.host_word[0];
    if (r.has_rerank) t.rerank_rows = r.host_word[1];
    va_scan_timings& s = ctx->rec_sum;
    s.sample_ms += t.sample_ms;
    s.scan_ms += t.scan_ms;
    s.select_ms += t.select_ms;
    s.fallback_ms += t.fallback_ms;
    s.total_ms += t.total_ms;
    s.overflow_rows += t.overflow_rows;
    s.rerank_rows += t.rerank_rows;
    s.scan_launches += t.scan_launches;
    ctx->rec_count++;
}

__global__ __launch_bounds__(256) void sum_u32_kernel(const uint32_t* v, uint32_t n, uint32_t* out) {
    __shared__ uint32_t part[256];
    uint32_t s = 0;
    for (uint32_t i = threadIdx.x; i < n; i += 256) s += v[i];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (int(threadIdx.x) < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = part[0];
}

va_status sum_u32_into(va_context* ctx, const uint32_t* v, uint32_t n, uint32_t* out) {
    sum_u32_kernel<<<dim3(1), dim3(256), 0, ctx->stream>>>(v, n, out);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status side_reserve(va_context* ctx, size_t bytes, void** out) {
    if (bytes > ctx->side_bytes) {
        // grow: wait for in-flight readers of the old buffer, then replace it
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->side) {
            VA_CHECK_HIP(ctx, hipFree(ctx->side));
            ctx->side = nullptr;
            ctx->side_bytes = 0;
        }
        void* p = nullptr;
        const hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail(ctx, VA_ERR_OOM, "side buffer allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
        }
        ctx->side = static_cast<char*>(p);
        ctx->side_bytes = bytes;
    }
    *out = ctx->side;
    return VA_OK;
}

__global__ void fill_u32_kernel(uint32_t* p, uint64_t n, uint32_t v) {
    uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (; i < n; i += step) p[i] = v;
}

va_status fill_u32(va_context* ctx, uint32_t* p, uint64_t n, uint32_t v) {
    if (n == 0) return VA_OK;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    fill_u32_kernel<<<dim3(uint32_t(blocks)), dim3(256), 0, ctx->stream>>>(p, n, v);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status aux_fork(va_context* ctx, int n) {
    if (!ctx->fork_ev) {
        VA_CHECK_HIP(ctx, hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming));
        for (int i = 0; i < va_context::kAux; ++i) {
            // default priority, like the main stream
            VA_CHECK_HIP(ctx, hipStreamCreateWithFlags(&ctx->aux[i], hipStreamNonBlocking));
            VA_CHECK_HIP(ctx, hipEventCreateWithFlags(&ctx->join_ev[i], hipEventDisableTiming));
        }
    }
    VA_CHECK_HIP(ctx, hipEventRecord(ctx->fork_ev, ctx->stream));
    for (int i = 0; i < std::min(n, va_context::kAux); ++i)
        VA_CHECK_HIP(ctx, hipStreamWaitEvent(ctx->aux[i], ctx->fork_ev, 0));
    return VA_OK;
}

va_status aux_join(va_context* ctx, int n) {
    for (int i = 0; i < std::min(n, va_context::kAux); ++i) {
        VA_CHECK_HIP(ctx, hipEventRecord(ctx->join_ev[i], ctx->aux[i]));
        VA_CHECK_HIP(ctx, hipStreamWaitEvent(ctx->stream, ctx->join_ev[i], 0));
    }
    return VA_OK;
}

DistOp metric_op(va_metric m) {
    switch (m) {
        case VA_METRIC_L2SQ: return OP_L2SQ;
        case VA_METRIC_L2: return OP_L2;
        case VA_METRIC_COSINE: return OP_COS_DIST;
        case VA_METRIC_DOT:
        default: return OP_NEG_DOT;
    }
}

}  // namespace va

extern "C" {

int va_abi_version(void) { return VA_HIP_ABI_VERSION; }

const char* va_status_string(va_status s) {
    switch (s) {
        case VA_OK: return "ok";
        case VA_ERR_INVALID_ARG: return "invalid argument";
        case VA_ERR_DIMENSION_MISMATCH: return "dimension mismatch";
        case VA_ERR_OOM: return "device allocation failed";
        case VA_ERR_HIP: return "HIP runtime error";
        case VA_ERR_UNSUPPORTED: return "unsupported";
    }
    return "unknown status";
}

static va_status create_impl(int device, void* stream, va_context** out) {
    if (!out) return VA_ERR_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return VA_ERR_HIP;
    }
    if (device < 0 || device >= n) return VA_ERR_INVALID_ARG;
    va_context* ctx = new va_context();
    ctx->device = device;
    va::DeviceGuard g(device);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) ctx->num_cus = prop.multiProcessorCount;
    if (stream) {
        ctx->stream = static_cast<hipStream_t>(stream);
        ctx->owns_stream = false;
    } else {
        // default priority, non-blocking w.r.t. the legacy null stream
        if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
            delete ctx;
            return VA_ERR_HIP;
        }
        ctx->owns_stream = true;
    }
    void* hw = nullptr;
    if (hipHostMalloc(&hw, 64, hipHostMallocDefault) != hipSuccess) {
        if (ctx->owns_stream) (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return VA_ERR_OOM;
    }
    ctx->host_word = static_cast<uint32_t*>(hw);
    va::noalloc_setup_device(device);
    *out = ctx;
    return VA_OK;
}

va_status va_context_create(int device, va_context** out) { return create_impl(device, nullptr, out); }

va_status va_context_create_with_stream(int device, void* hip_stream, va_context** out) {
    if (!hip_stream) return VA_ERR_INVALID_ARG;
    return create_impl(device, hip_stream, out);
}

va_status va_context_destroy(va_context* ctx) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    {
        va::DeviceGuard g(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->scratch) (void)hipFree(ctx->scratch);
        if (ctx->side) (void)hipFree(ctx->side);
        if (ctx->host_word) (void)hipHostFree(ctx->host_word);
        for (auto& r : ctx->rec) {
            for (auto& e : r.ev)
                if (e) (void)hipEventDestroy(e);
            if (r.dev_word) (void)hipFree(r.dev_word);
            if (r.host_word) (void)hipHostFree(r.host_word);
        }
        for (int i = 0; i < va_context::kAux; ++i) {
            if (ctx->aux[i]) {
                (void)hipStreamSynchronize(ctx->aux[i]);
                (void)hipStreamDestroy(ctx->aux[i]);
            }
            if (ctx->join_ev[i]) (void)hipEventDestroy(ctx->join_ev[i]);
        }
        if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
        if (ctx->owns_stream) (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
    return VA_OK;
}

void* va_context_stream(va_context* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int va_context_device(const va_context* ctx) { return ctx ? ctx->device : -1; }

va_status va_context_synchronize(va_context* ctx) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    va::DeviceGuard g(ctx->device);
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VA_OK;
}

const char* va_last_error_message(const va_context* ctx) { return ctx ? ctx->last_error.c_str() : ""; }

va_status va_context_set_profiling(va_context* ctx, int enable) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, enable >= 0 && enable <= 2, "va_context_set_profiling: level %d (0, 1 or 2)", enable);
    va::DeviceGuard g(ctx->device);
    if (enable && !ctx->rec[0].ev[0]) {
        for (auto& r : ctx->rec) {
            for (auto& e : r.ev) VA_CHECK_HIP(ctx, hipEventCreate(&e));
            VA_CHECK_HIP(ctx, hipMalloc(&r.dev_word, 4));
            void* h = nullptr;
            VA_CHECK_HIP(ctx, hipHostMalloc(&h, 8, hipHostMallocDefault));
            r.host_word = static_cast<uint32_t*>(h);
        }
    }
    ctx->profiling = enable;
    return VA_OK;
}

static void fold_pending(va_context* ctx) {
    // oldest first, so the totals add up in enqueue order
    for (int i = 1; i <= va_context::kScanRing; ++i) {
        auto& r = ctx->rec[(ctx->rec_next + i - 1) % va_context::kScanRing];
        if (r.pending) va::profile_fold(ctx, r);
    }
}

va_status va_context_last_scan(va_context* ctx, va_scan_timings* out) {
    if (!ctx || !out) return VA_ERR_INVALID_ARG;
    va::DeviceGuard g(ctx->device);
    fold_pending(ctx);
    *out = ctx->rec_last >= 0 ? ctx->rec[ctx->rec_last].t : ctx->last_scan;
    return VA_OK;
}

va_status va_context_scan_totals(va_context* ctx, va_scan_timings* sum, uint32_t* count) {
    if (!ctx || !sum || !count) return VA_ERR_INVALID_ARG;
    va::DeviceGuard g(ctx->device);
    fold_pending(ctx);
    *sum = ctx->rec_sum;
    *count = ctx->rec_count;
    return VA_OK;
}

va_status va_context_reset_scan_totals(va_context* ctx) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    va::DeviceGuard g(ctx->device);
    fold_pending(ctx);
    ctx->rec_sum = va_scan_timings{};
    ctx->rec_count = 0;
    return VA_OK;
}

va_status va_context_set_option(va_context* ctx, va_option option, uint64_t value) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    switch (option) {
        case VA_OPT_CANDIDATE_CAP: ctx->opt_candidate_cap = value; return VA_OK;
        case VA_OPT_SAMPLE_ROWS: ctx->opt_sample_rows = value; return VA_OK;
        case VA_OPT_SAMPLE_RANK: ctx->opt_sample_rank = value; return VA_OK;
        case VA_OPT_SCREEN:
            VA_REQUIRE(ctx, value <= 2, "VA_OPT_SCREEN must be 0, 1 or 2, got %llu", (unsigned long long)value);
            ctx->opt_screen = uint32_t(value);
            return VA_OK;
    }
    return va::fail(ctx, VA_ERR_INVALID_ARG, "va_context_set_option: unknown option %d", int(option));
}

va_status va_buffer_alloc(va_context* ctx, size_t bytes, void** device_ptr) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, device_ptr != nullptr, "va_buffer_alloc: device_ptr is NULL");
    VA_REQUIRE(ctx, bytes > 0, "va_buffer_alloc: size must be positive");
    va::DeviceGuard g(ctx->device);
    *device_ptr = nullptr;
    hipError_t e = hipMalloc(device_ptr, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return va::fail(ctx, VA_ERR_OOM, "va_buffer_alloc: %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    return VA_OK;
}

va_status va_buffer_free(va_context* ctx, void* device_ptr) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    if (!device_ptr) return VA_OK;
    va::DeviceGuard g(ctx->device);
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    VA_CHECK_HIP(ctx, hipFree(device_ptr));
    return VA_OK;
}

va_status va_buffer_upload(va_context* ctx, void* dst_device, const void* src_host, size_t bytes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, dst_device && src_host, "va_buffer_upload: NULL pointer");
    if (bytes == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(dst_device, src_host, bytes, hipMemcpyHostToDevice, ctx->stream));
    return VA_OK;
}

va_status va_buffer_download(va_context* ctx, void* dst_host, const void* src_device, size_t bytes) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, dst_host && src_device, "va_buffer_download: NULL pointer");
    if (bytes == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(dst_host, src_device, bytes, hipMemcpyDeviceToHost, ctx->stream));
    return VA_OK;
}

}  // extern "C"
