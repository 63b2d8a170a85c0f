// va_probe.hip — the matrix-core, LDS and HBM ceilings of the board, measured (no reference
// counterpart).
//
// The roofline fractions of the scans are quoted against MI355X's published dense peaks; this
// probe measures what the board sustains for each MFMA instruction the scans use, so that a
// fraction can also be read against the measured ceiling.  Every SIMD runs two waves of
// back-to-back MFMAs of one instruction on register operands (eight independent accumulators per
// wave, no memory traffic), with random or constant operands (the matrix cores draw more power,
// and the clock drops further, on random bits).  Lane 0 of each workgroup's first wave reads the
// shader clock counter and the constant-rate wall clock at the start and end, which gives the
// engine clock during the run.
#include "va_internal.hpp"

namespace va {
namespace {

typedef _Float16 pr_h8 __attribute__((ext_vector_type(8)));
typedef float pr_f16 __attribute__((ext_vector_type(16)));
typedef int pr_i4 __attribute__((ext_vector_type(4)));
typedef int pr_i8 __attribute__((ext_vector_type(8)));
typedef int pr_i16 __attribute__((ext_vector_type(16)));

constexpr int kAcc = 8;

__device__ inline uint32_t pr_next(uint32_t& s) {
    s = s * 1664525u + 1013904223u;
    return s;
}

// clocks[0] += shader clock ticks, clocks[1] += wall clock ticks (per workgroup)
__device__ inline void pr_clock_begin(uint64_t& c0, uint64_t& w0) {
    c0 = __builtin_amdgcn_s_memtime();
    w0 = __builtin_amdgcn_s_memrealtime();
}
__device__ inline void pr_clock_end(uint64_t c0, uint64_t w0, unsigned long long* clocks) {
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), w1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        atomicAdd(clocks, (unsigned long long)(c1 - c0));
        atomicAdd(clocks + 1, (unsigned long long)(w1 - w0));
    }
}

template <int KIND>
__global__ __launch_bounds__(256) void mfma_probe_kernel(uint32_t iters, int rnd, float* sink,
                                                         unsigned long long* clocks) {
    uint32_t s = (blockIdx.x * 256u + threadIdx.x) * 2654435761u + 12345u;
    uint64_t c0, w0;
    float z = 0.0f;
    if constexpr (KIND == VA_PROBE_FP32) {
        float a[4], b[4];
        for (int i = 0; i < 4; ++i) {
            a[i] = rnd ? float(int(pr_next(s) >> 16) - 32768) * 0x1p-15f : 0.5f;
            b[i] = rnd ? float(int(pr_next(s) >> 16) - 32768) * 0x1p-15f : 0.25f;
        }
        pr_f16 acc[kAcc];
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
        pr_clock_begin(c0, w0);
        for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < kAcc; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j & 3], b[(j >> 2) & 3], acc[j], 0, 0, 0);
        }
        pr_clock_end(c0, w0, clocks);
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) z += acc[j][v];
    } else if constexpr (KIND == VA_PROBE_FP16) {
        pr_h8 a[4], b[4];
        for (int i = 0; i < 4; ++i)
            for (int e = 0; e < 8; ++e) {
                a[i][e] = rnd ? _Float16(float(int(pr_next(s) >> 16) - 32768) * 0x1p-15f) : _Float16(0.5f);
                b[i][e] = rnd ? _Float16(float(int(pr_next(s) >> 16) - 32768) * 0x1p-15f) : _Float16(0.25f);
            }
        pr_f16 acc[kAcc];
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
        pr_clock_begin(c0, w0);
        for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < kAcc; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j & 3], b[(j >> 2) & 3], acc[j], 0, 0, 0);
        }
        pr_clock_end(c0, w0, clocks);
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) z += acc[j][v];
    } else if constexpr (KIND == VA_PROBE_INT8) {
        pr_i4 a[4], b[4];
        for (int i = 0; i < 4; ++i)
            for (int e = 0; e < 4; ++e) {
                a[i][e] = rnd ? int(pr_next(s)) : 0x01010101;
                b[i][e] = rnd ? int(pr_next(s)) : 0x01010101;
            }
        pr_i16 acc[kAcc];
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) acc[j][v] = 0;
        pr_clock_begin(c0, w0);
        for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < kAcc; ++j)
                acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j & 3], b[(j >> 2) & 3], acc[j], 0, 0, 0);
        }
        pr_clock_end(c0, w0, clocks);
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) z += float(acc[j][v]);
    } else if constexpr (KIND == VA_PROBE_LDS) {
        // 8 KiB of LDS per wave (the workgroup's 32 KiB), each lane's 16 bytes at lane * 16 of a
        // 1 KiB row: consecutive lanes on consecutive banks.  The reads are asm volatile so that
        // the loop is not folded away; their results are xor-ed so that they stay live.
        __shared__ __attribute__((aligned(16))) uint32_t buf[8192];
        for (int i = threadIdx.x; i < 8192; i += 256) buf[i] = rnd ? pr_next(s) : 0x3F800000u;
        __syncthreads();
        const uint32_t addr = uint32_t(reinterpret_cast<uintptr_t>(buf)) + uint32_t(threadIdx.x & 63) * 16u +
                              uint32_t(threadIdx.x >> 6) * 8192u;
        pr_i4 x = {0, 0, 0, 0};
        pr_clock_begin(c0, w0);
        for (uint32_t it = 0; it < iters; ++it) {
            pr_i4 v0, v1, v2, v3, v4, v5, v6, v7;
            asm volatile(
                "ds_read_b128 %0, %8 offset:0\n\tds_read_b128 %1, %8 offset:1024\n\t"
                "ds_read_b128 %2, %8 offset:2048\n\tds_read_b128 %3, %8 offset:3072\n\t"
                "ds_read_b128 %4, %8 offset:4096\n\tds_read_b128 %5, %8 offset:5120\n\t"
                "ds_read_b128 %6, %8 offset:6144\n\tds_read_b128 %7, %8 offset:7168\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
                : "v"(addr));
            x ^= v0 ^ v1 ^ v2 ^ v3 ^ v4 ^ v5 ^ v6 ^ v7;
        }
        pr_clock_end(c0, w0, clocks);
        z = float(x[0] ^ x[1] ^ x[2] ^ x[3]);
    } else {
        // fp4 (e2m1) operands of the scaled 32x32x64 MFMA, unit scales (format 4 = fp4 on both sides)
        pr_i8 a[4], b[4];
        for (int i = 0; i < 4; ++i)
            for (int e = 0; e < 8; ++e) {
                a[i][e] = e < 4 ? (rnd ? int(pr_next(s)) : 0x22222222) : 0;
                b[i][e] = e < 4 ? (rnd ? int(pr_next(s)) : 0x22222222) : 0;
            }
        pr_f16 acc[kAcc];
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
        pr_clock_begin(c0, w0);
        for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < kAcc; ++j)
                acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[j & 3], b[(j >> 2) & 3], acc[j], 4, 4, 0,
                                                                         127, 0, 127);
        }
        pr_clock_end(c0, w0, clocks);
        for (int j = 0; j < kAcc; ++j)
            for (int v = 0; v < 16; ++v) z += acc[j][v];
    }
    if (z == 1234.5f) sink[0] = z;  // keeps the accumulators live; never true in practice
}

// HBM read bandwidth: each workgroup streams contiguous 32 KiB blocks (eight 16-byte loads per
// thread in flight, a wave reading 1 KiB of contiguous bytes per load; sixteen per thread and
// grid-strided loads measured slower), the blocks spread over the workgroups; the words are
// xor-folded so the loads stay live.  The buffer (4 GiB in the bench) is
// far larger than the L2s and the last-level cache, so the bytes come from HBM.
__global__ __launch_bounds__(256) void hbm_probe_kernel(const pr_i4* __restrict__ p, uint64_t n16, float* sink,
                                                        unsigned long long* clocks) {
    uint64_t c0, w0;
    pr_clock_begin(c0, w0);
    constexpr uint64_t kBlock = 256 * 8;  // 16-byte words per block
    const uint64_t nb = n16 / kBlock;
    pr_i4 x = {0, 0, 0, 0};
    for (uint64_t b = blockIdx.x; b < nb; b += gridDim.x) {
        const pr_i4* q = p + b * kBlock + threadIdx.x;
        pr_i4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = q[u * 256];
#pragma unroll
        for (int u = 0; u < 8; ++u) x ^= v[u];
    }
    pr_clock_end(c0, w0, clocks);
    if ((x[0] ^ x[1] ^ x[2] ^ x[3]) == 0x7F123456) sink[0] = 1.0f;  // keeps the loads live
}

// dense operations of one MFMA of the kind (2 per multiply-add)
double ops_per_mfma(int kind) {
    switch (kind) {
        case VA_PROBE_FP32: return 2.0 * 32 * 32 * 2;
        case VA_PROBE_FP16: return 2.0 * 32 * 32 * 16;
        case VA_PROBE_INT8: return 2.0 * 32 * 32 * 32;
        case VA_PROBE_LDS: return 1024.0;  // bytes of one wave's ds_read_b128
        default: return 2.0 * 32 * 32 * 64;
    }
}

}  // namespace
}  // namespace va

extern "C" va_status va_probe_mfma(va_context* ctx, va_probe_kind kind, int random_operands, uint32_t iterations,
                                   va_probe_result* out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, out != nullptr, "va_probe_mfma: NULL output");
    VA_REQUIRE(ctx, kind >= VA_PROBE_FP32 && kind <= VA_PROBE_HBM, "va_probe_mfma: unknown kind %d", int(kind));
    VA_REQUIRE(ctx, kind != VA_PROBE_HBM || (iterations >= 256 && iterations <= 65536),
               "va_probe_mfma: the HBM kind reads `iterations` MiB, 256 .. 65536");
    VA_REQUIRE(ctx, iterations >= 1 && iterations <= (1u << 24), "va_probe_mfma: iterations %u out of range",
               iterations);
    va::DeviceGuard g(ctx->device);
    int wall_khz = 0;
    VA_CHECK_HIP(ctx, hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, ctx->device));
    struct Tmp {
        void* p = nullptr;
        hipEvent_t e[2] = {nullptr, nullptr};
        ~Tmp() {
            if (p) (void)hipFree(p);
            for (hipEvent_t x : e)
                if (x) (void)hipEventDestroy(x);
        }
    } t;
    // the HBM kind's buffer follows the 256-byte clock block
    const uint64_t hbm_bytes = kind == VA_PROBE_HBM ? uint64_t(iterations) << 20 : 0;
    VA_CHECK_HIP(ctx, hipMalloc(&t.p, 256 + hbm_bytes));
    if (hbm_bytes) VA_CHECK_HIP(ctx, hipMemsetAsync(static_cast<char*>(t.p) + 256, random_operands ? 0x5A : 0, hbm_bytes, ctx->stream));
    VA_CHECK_HIP(ctx, hipEventCreate(&t.e[0]));
    VA_CHECK_HIP(ctx, hipEventCreate(&t.e[1]));
    auto* clocks = static_cast<unsigned long long*>(t.p);
    float* sink = reinterpret_cast<float*>(clocks + 2);
    VA_CHECK_STATUS(va::fill_u32(ctx, reinterpret_cast<uint32_t*>(clocks), 4, 0));
    // two waves per SIMD: two 4-wave workgroups per CU
    const uint32_t grid = uint32_t(ctx->num_cus) * 2u;
    auto launch = [&]() -> va_status {
        switch (kind) {
            case VA_PROBE_FP32:
                va::mfma_probe_kernel<VA_PROBE_FP32><<<grid, 256, 0, ctx->stream>>>(iterations, random_operands, sink,
                                                                                    clocks);
                break;
            case VA_PROBE_FP16:
                va::mfma_probe_kernel<VA_PROBE_FP16><<<grid, 256, 0, ctx->stream>>>(iterations, random_operands, sink,
                                                                                    clocks);
                break;
            case VA_PROBE_INT8:
                va::mfma_probe_kernel<VA_PROBE_INT8><<<grid, 256, 0, ctx->stream>>>(iterations, random_operands, sink,
                                                                                    clocks);
                break;
            case VA_PROBE_LDS:
                va::mfma_probe_kernel<VA_PROBE_LDS><<<grid, 256, 0, ctx->stream>>>(iterations, random_operands, sink,
                                                                                   clocks);
                break;
            case VA_PROBE_HBM:
                // eight 4-wave workgroups per CU
                va::hbm_probe_kernel<<<grid * 4, 256, 0, ctx->stream>>>(
                    reinterpret_cast<const va::pr_i4*>(static_cast<char*>(t.p) + 256), hbm_bytes / 16, sink, clocks);
                break;
            default:
                va::mfma_probe_kernel<VA_PROBE_FP4><<<grid, 256, 0, ctx->stream>>>(iterations, random_operands, sink,
                                                                                   clocks);
        }
        VA_CHECK_LAUNCH(ctx);
        return VA_OK;
    };
    VA_CHECK_STATUS(launch());  // warm-up (clocks ramp, code object loaded)
    VA_CHECK_STATUS(va::fill_u32(ctx, reinterpret_cast<uint32_t*>(clocks), 4, 0));
    VA_CHECK_HIP(ctx, hipEventRecord(t.e[0], ctx->stream));
    VA_CHECK_STATUS(launch());
    VA_CHECK_HIP(ctx, hipEventRecord(t.e[1], ctx->stream));
    unsigned long long h[2] = {0, 0};
    VA_CHECK_HIP(ctx, hipMemcpyAsync(h, clocks, 16, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    float ms = 0.0f;
    VA_CHECK_HIP(ctx, hipEventElapsedTime(&ms, t.e[0], t.e[1]));
    out->ms = ms;
    out->ops = kind == VA_PROBE_HBM ? double(hbm_bytes)
                                    : double(grid) * 4.0 * double(iterations) * va::kAcc * va::ops_per_mfma(int(kind));
    out->ops_per_second = ms > 0 ? out->ops / (double(ms) * 1e-3) : 0.0;
    out->engine_mhz = h[1] ? double(h[0]) / double(h[1]) * double(wall_khz) * 1e-3 : 0.0;
    return VA_OK;
}
