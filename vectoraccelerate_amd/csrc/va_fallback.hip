// va_fallback.hip — the device-side overflow fallback's clear kernel and driver (the passes are
// templates over the key producers, instantiated beside each producer).
#include "va_fallback.hpp"

namespace va {

__global__ __launch_bounds__(256) void fb_init_kernel(FbArgs a) {
    const uint32_t n = fb_count(a);
    if (n == 0) return;
    const uint64_t step = uint64_t(gridDim.x) * 256;
    const uint64_t i0 = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    for (uint64_t i = i0; i < uint64_t(n) * 2048; i += step) a.hist[i] = 0;
    for (uint64_t i = i0; i < uint64_t(n) * kFbTieBins; i += step) a.tidh[i] = 0;
    for (uint64_t i = i0; i < uint64_t(n) * 8; i += step) a.st[i] = 0;
    for (uint64_t i = i0; i < n; i += step) a.cnt[i] = 0;
    if (i0 < 8) a.done[i0] = 0;
}

va_status fb_init(va_context* ctx, const FbArgs& a) {
    fb_init_kernel<<<dim3(256), dim3(256), 0, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status fb_passes(va_context* ctx, KeyProducer& kp, const FbArgs& a) {
    VA_CHECK_STATUS(fb_init(ctx, a));
    for (int pass = 0; pass < kFbPasses; ++pass) VA_CHECK_STATUS(kp.fallback_pass(a, pass));
    return VA_OK;
}

va_status fb_run(va_context* ctx, KeyProducer& kp, const FbArgs& a, const SelectArgs& base) {
    VA_CHECK_STATUS(fb_passes(ctx, kp, a));
    return fb_select(ctx, a, base, kp.key_bits());
}

va_status fb_select(va_context* ctx, const FbArgs& a, const SelectArgs& base, uint32_t key_bits) {
    SelectArgs s = base;
    s.keys = a.lkey;
    s.ids = a.lid;
    s.counts = a.cnt;
    s.ld = a.cap;
    s.n = a.cap;
    s.rows = a.rmax;
    s.rows_dev = a.n_rows;
    s.row_map = a.rows;
    s.overflow_count = nullptr;
    s.overflow_rows = nullptr;
    s.key_bits = key_bits;
    return launch_select(ctx, s);
}

}  // namespace va
