// va_noalloc.hip — the allocation-free flat top-k entry point (va_fused_topk_noalloc).
//
// Callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc) get the same search as va_fused_topk with every scratch
// buffer — thresholds, candidate lists, counters, the dense sample keys, the rerank lists — taken
// from one fixed device array per GPU instead of the context's growable arena.  The array lives
// in the code object (each device the library runs on holds its own copy until the process
// ends).  Its device address is resolved once per device with hipGetSymbolAddress while a
// context is created on that device; the host never passes the array's name itself to a kernel.
//
// Every call on a device shares that device's array and leaves its contents behind: counters
// are cleared by each call before use, and two calls that overlap on one device (different
// contexts, different streams) race on the array.
#include <mutex>

#include "va_internal.hpp"

namespace va {
namespace {

static_assert(VA_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size is a multiple of the carve alignment");

// The fixed scratch block.  In host code this name is a host-side stand-in, not a device address:
// only the per-device pointer from hipGetSymbolAddress below is used.
static __device__ __align__(256) char scratch[VA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
struct DeviceScratch {
    bool done = false;
    char* ptr = nullptr;
    hipError_t err = hipSuccess;
};
DeviceScratch g_scratch[kMaxDevices];
std::mutex g_mu;

}  // namespace

void noalloc_setup_device(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceScratch& d = g_scratch[device];
    if (d.done) return;
    void* p = nullptr;
    d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (d.err != hipSuccess) {
        (void)hipGetLastError();
        p = nullptr;
    }
    d.ptr = static_cast<char*>(p);
    d.done = true;
}

}  // namespace va

extern "C" va_status va_fused_topk_noalloc(va_context* ctx, va_metric metric, const float* queries,
                                           const float* database, uint32_t num_queries, uint32_t num_database,
                                           uint32_t dim, uint32_t k, uint32_t* out_idx, float* out_dist) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    // the same validation as va_fused_topk
    VA_REQUIRE(ctx, queries && database && out_idx, "va_fused_topk_noalloc: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "numQueries must be positive, got %u", num_queries);
    VA_REQUIRE(ctx, num_database > 0, "numDataset must be positive, got %u", num_database);
    VA_REQUIRE(ctx, dim > 0, "dimension must be positive, got %u", dim);
    VA_REQUIRE(ctx, k > 0, "k must be positive, got %u", k);
    VA_REQUIRE(ctx, k <= VA_MAX_K, "k %u exceeds maximum supported k %u", k, VA_MAX_K);
    VA_REQUIRE(ctx, metric >= VA_METRIC_L2SQ && metric <= VA_METRIC_L2, "va_fused_topk_noalloc: unknown metric %d",
               int(metric));
    const int dev = ctx->device;
    char* ptr = nullptr;
    hipError_t err = hipErrorInvalidDevice;
    if (dev >= 0 && dev < va::kMaxDevices) {
        std::lock_guard<std::mutex> lock(va::g_mu);
        ptr = va::g_scratch[dev].done ? va::g_scratch[dev].ptr : nullptr;
        err = va::g_scratch[dev].err;
    }
    if (!ptr)
        return va::fail(ctx, VA_ERR_HIP, "va_fused_topk_noalloc: no scratch block on device %d (%s)", dev,
                        hipGetErrorString(err));
    va::DeviceGuard g(dev);
    // route the scan's scratch to the fixed block for the duration of this call
    struct FixedScratch {
        va_context* c;
        FixedScratch(va_context* cc, char* p) : c(cc) {
            c->fixed_scratch = p;
            c->fixed_scratch_bytes = VA_NOALLOC_SCRATCH_BYTES;
        }
        ~FixedScratch() {
            c->fixed_scratch = nullptr;
            c->fixed_scratch_bytes = 0;
        }
    } fixed(ctx, ptr);
    return va::flat_topk(ctx, va::metric_op(metric), queries, database, num_queries, num_database, dim, k, out_idx,
                         out_dist);
}
