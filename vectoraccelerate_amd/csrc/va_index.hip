// va_index.hip — a native flat index with stable handles (AcceleratedVectorIndex's storage,
// handle table and search, Index/AcceleratedVectorIndex.swift:481-1265;
// Index/Internal/HandleAllocator.swift:39-242).
//
// Storage per slot, on the device: the fp32 row, its fp16 shadow (rows rounded to fp16 at insert
// time plus fp32 squared norms; the screening scan reads it instead of converting the fp32 rows on
// every search), a deletion byte and the slot's stable id.  Handles are stable ids handed out in
// insertion order; a removed handle's slot stays in place (the deletion byte excludes it from every
// search) until compact() moves the live rows down, keeping their order.
//
// Search returns the k nearest live rows by (distance, slot): deleted rows are excluded inside the
// scan (their keys become absent before every selection), so k is not widened by the number of
// deletions and no result is short while live rows remain.  Filtered search fetches the best
// not-yet-examined rows round after round (rows already examined are excluded the same way), so
// the accepted results are exactly the k nearest rows that pass the filter, in order, however
// many rows it rejects.
#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <vector>

#include "va_internal.hpp"

struct va_index {
    int device = 0;
    uint32_t dim = 0;
    uint32_t pitch = 0;      // halves per shadow row (0: no shadow, dim % 4 != 0)
    uint64_t capacity = 0;   // slots allocated
    uint32_t slots = 0;      // slots in use, deleted included
    uint32_t deleted = 0;
    float* rows = nullptr;          // [capacity x dim]
    _Float16* shadow = nullptr;     // [capacity x pitch]
    float* norms = nullptr;         // [capacity]
    float* errs = nullptr;          // [capacity] upper bound of |fp16(x) - x| (the shadow's rounding)
    uint8_t* skip = nullptr;        // [capacity] 1 = deleted
    uint8_t* seen = nullptr;        // [capacity] filtered search: deleted or already examined
    uint32_t* slot_stable = nullptr;  // [capacity] stable id of each slot
    std::vector<uint32_t> stable_to_slot;  // kTombstone for removed ids
    std::vector<uint32_t> slot_to_stable;
    // IVF (IndexConfiguration.ivf): inverted lists over the slots, built when the index is trained
    // and kept current by insert (new slots appended to their nearest lists) and compact (lists
    // rebuilt from the trained centroids); deleted slots stay in the lists and are excluded by the
    // deletion mask inside the scan
    uint32_t nlist = 0;           // 0: flat index
    uint32_t nprobe = 0;
    uint32_t routing = 0;         // routingThreshold: fewer live vectors than this search flat
    float* centroids = nullptr;   // [nlist x dim] once trained
    va_ivf* ivf = nullptr;        // lists over slots [0, slots); nullptr while untrained or empty
};

namespace va {
namespace {

constexpr uint32_t kTombstone = 0xFFFFFFFFu;

__global__ void iota_kernel(uint32_t* out, uint32_t n, uint32_t first) {
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) out[i] = first + i;
}

__global__ void scatter_byte_kernel(uint8_t* dst, const uint32_t* idx, uint32_t n, uint8_t v) {
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) dst[idx[i]] = v;
}

__global__ void fill_byte_kernel(uint8_t* dst, uint64_t n, uint8_t v) {
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) dst[i] = v;
}

// results: slot ids -> stable ids (sentinels stay)
__global__ void slots_to_handles_kernel(uint32_t* idx, uint64_t n, const uint32_t* __restrict__ slot_stable) {
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) {
        const uint32_t s = idx[i];
        if (s != kSentinel) idx[i] = slot_stable[s];
    }
}

// compaction: row keep[j] -> slot j of the new arrays (one workgroup per kept row)
__global__ void gather_rows_kernel(const float* __restrict__ rows, const _Float16* __restrict__ shadow,
                                   const float* __restrict__ norms, const float* __restrict__ errs,
                                   const uint32_t* __restrict__ slot_stable, const uint32_t* __restrict__ keep,
                                   uint32_t n, uint32_t dim, uint32_t pitch, float* __restrict__ rows2,
                                   _Float16* __restrict__ shadow2, float* __restrict__ norms2, float* __restrict__ errs2,
                                   uint32_t* __restrict__ slot_stable2) {
    const uint32_t j = blockIdx.x;
    if (j >= n) return;
    const uint32_t s = keep[j];
    for (uint32_t d = threadIdx.x; d < dim; d += 256) rows2[uint64_t(j) * dim + d] = rows[uint64_t(s) * dim + d];
    if (pitch)
        for (uint32_t d = threadIdx.x; d < pitch; d += 256) shadow2[uint64_t(j) * pitch + d] = shadow[uint64_t(s) * pitch + d];
    if (threadIdx.x == 0) {
        if (pitch) {
            norms2[j] = norms[s];
            errs2[j] = errs[s];
        }
        slot_stable2[j] = slot_stable[s];
    }
}

uint32_t grid_for(uint64_t n) { return uint32_t(std::max<uint64_t>(1, std::min<uint64_t>((n + 255) / 256, 4096))); }

struct DevBuffers {
    float* rows = nullptr;
    _Float16* shadow = nullptr;
    float* norms = nullptr;
    float* errs = nullptr;
    uint8_t* skip = nullptr;
    uint8_t* seen = nullptr;
    uint32_t* slot_stable = nullptr;
    void release() {
        (void)hipFree(rows);
        (void)hipFree(shadow);
        (void)hipFree(norms);
        (void)hipFree(errs);
        (void)hipFree(skip);
        (void)hipFree(seen);
        (void)hipFree(slot_stable);
        *this = DevBuffers{};
    }
};

va_status alloc_buffers(va_context* ctx, uint64_t cap, uint32_t dim, uint32_t pitch, DevBuffers& b) {
    auto get = [&](void** p, size_t bytes) -> bool {
        if (hipMalloc(p, std::max<size_t>(bytes, 256)) == hipSuccess) return true;
        (void)hipGetLastError();
        return false;
    };
    bool ok = get(reinterpret_cast<void**>(&b.rows), cap * dim * 4) && get(reinterpret_cast<void**>(&b.skip), cap) &&
              get(reinterpret_cast<void**>(&b.seen), cap) && get(reinterpret_cast<void**>(&b.slot_stable), cap * 4);
    if (ok && pitch)
        ok = get(reinterpret_cast<void**>(&b.shadow), cap * pitch * 2) && get(reinterpret_cast<void**>(&b.norms), cap * 4) &&
             get(reinterpret_cast<void**>(&b.errs), cap * 4);
    if (!ok) {
        b.release();
        return fail(ctx, VA_ERR_OOM, "index storage of %llu slots x %u dimensions: device allocation failed",
                    (unsigned long long)cap, dim);
    }
    return VA_OK;
}

DevBuffers current(const va_index* ix) {
    DevBuffers b;
    b.rows = ix->rows;
    b.shadow = ix->shadow;
    b.norms = ix->norms;
    b.errs = ix->errs;
    b.skip = ix->skip;
    b.seen = ix->seen;
    b.slot_stable = ix->slot_stable;
    return b;
}

void install(va_index* ix, const DevBuffers& b, uint64_t cap) {
    ix->rows = b.rows;
    ix->shadow = b.shadow;
    ix->norms = b.norms;
    ix->errs = b.errs;
    ix->skip = b.skip;
    ix->seen = b.seen;
    ix->slot_stable = b.slot_stable;
    ix->capacity = cap;
}

// grow to hold `need` slots (doubling); the old contents move over
va_status reserve_slots(va_context* ctx, va_index* ix, uint64_t need) {
    if (need <= ix->capacity) return VA_OK;
    const uint64_t cap = std::max<uint64_t>(need, ix->capacity * 2);
    DevBuffers nb;
    VA_CHECK_STATUS(alloc_buffers(ctx, cap, ix->dim, ix->pitch, nb));
    const uint64_t n = ix->slots;
    if (n) {
        VA_CHECK_HIP(ctx, hipMemcpyAsync(nb.rows, ix->rows, n * ix->dim * 4, hipMemcpyDeviceToDevice, ctx->stream));
        VA_CHECK_HIP(ctx, hipMemcpyAsync(nb.skip, ix->skip, n, hipMemcpyDeviceToDevice, ctx->stream));
        VA_CHECK_HIP(ctx, hipMemcpyAsync(nb.slot_stable, ix->slot_stable, n * 4, hipMemcpyDeviceToDevice, ctx->stream));
        if (ix->pitch) {
            VA_CHECK_HIP(ctx, hipMemcpyAsync(nb.shadow, ix->shadow, n * ix->pitch * 2, hipMemcpyDeviceToDevice,
                                             ctx->stream));
            VA_CHECK_HIP(ctx, hipMemcpyAsync(nb.norms, ix->norms, n * 4, hipMemcpyDeviceToDevice, ctx->stream));
            VA_CHECK_HIP(ctx, hipMemcpyAsync(nb.errs, ix->errs, n * 4, hipMemcpyDeviceToDevice, ctx->stream));
        }
    }
    // the old buffers are freed once the copies (and any search still reading them) are done
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    DevBuffers old = current(ix);
    old.release();
    install(ix, nb, cap);
    return VA_OK;
}

// device copy of a host list of slots (staged through the context's scratch arena), then
// dst[slot] = v for each; synchronises so the host list may go away
va_status set_bytes(va_context* ctx, uint8_t* dst, const std::vector<uint32_t>& slots, uint8_t v) {
    if (slots.empty()) return VA_OK;
    Scratch s(ctx);
    VA_CHECK_STATUS(s.reserve(Scratch::round(slots.size() * 4)));
    uint32_t* d = s.carve<uint32_t>(slots.size());
    VA_CHECK_HIP(ctx, hipMemcpyAsync(d, slots.data(), slots.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    scatter_byte_kernel<<<dim3(grid_for(slots.size())), dim3(256), 0, ctx->stream>>>(dst, d, uint32_t(slots.size()), v);
    VA_CHECK_LAUNCH(ctx);
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VA_OK;
}

// (Re)builds the inverted lists over every slot from the trained centroids (none while empty).
va_status rebuild_lists(va_context* ctx, va_index* ix) {
    if (ix->ivf) {
        (void)va_ivf_destroy(ix->ivf);
        ix->ivf = nullptr;
    }
    if (!ix->centroids || ix->slots == 0) return VA_OK;
    return va_ivf_build(ctx, ix->centroids, ix->nlist, ix->rows, ix->slots, ix->dim, &ix->ivf);
}

// Whether a search goes to the inverted lists (AcceleratedVectorIndex.search routing,
// Index/AcceleratedVectorIndex.swift:911-926): trained, and not below the routing threshold.
bool ivf_route(const va_index* ix) {
    const uint32_t live = ix->slots - ix->deleted;
    return ix->ivf != nullptr && !(ix->routing > 0 && live < ix->routing);
}

va_status check_ctx(va_context* ctx, const va_index* ix, const char* fn) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, ix != nullptr, "%s: NULL index", fn);
    VA_REQUIRE(ctx, ix->device == ctx->device, "%s: the index lives on device %d, the context on %d", fn, ix->device,
               ctx->device);
    return VA_OK;
}

}  // namespace
}  // namespace va

extern "C" {

va_status va_index_create(va_context* ctx, uint32_t dim, uint32_t capacity, va_index** out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, out != nullptr, "va_index_create: NULL output");
    *out = nullptr;
    VA_REQUIRE(ctx, dim > 0, "dimension must be positive, got %u", dim);
    VA_REQUIRE(ctx, capacity > 0, "capacity must be positive, got %u", capacity);
    va::DeviceGuard g(ctx->device);
    va_index* ix = new va_index();
    ix->device = ctx->device;
    ix->dim = dim;
    ix->pitch = dim % 4 == 0 ? va::shadow_pitch(dim) : 0;
    va::DevBuffers b;
    const va_status st = va::alloc_buffers(ctx, capacity, dim, ix->pitch, b);
    if (st != VA_OK) {
        delete ix;
        return st;
    }
    va::install(ix, b, capacity);
    *out = ix;
    return VA_OK;
}

va_status va_index_destroy(va_index* index) {
    if (!index) return VA_ERR_INVALID_ARG;
    va::DeviceGuard g(index->device);
    (void)hipDeviceSynchronize();
    va::DevBuffers b = va::current(index);
    b.release();
    if (index->ivf) (void)va_ivf_destroy(index->ivf);
    if (index->centroids) (void)hipFree(index->centroids);
    delete index;
    return VA_OK;
}

va_status va_index_create_ivf(va_context* ctx, uint32_t dim, uint32_t capacity, uint32_t nlist, uint32_t nprobe,
                              uint32_t routing_threshold, va_index** out) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    VA_REQUIRE(ctx, out != nullptr, "va_index_create_ivf: NULL output");
    *out = nullptr;
    VA_REQUIRE(ctx, nlist >= 1 && nprobe >= 1 && nprobe <= nlist, "invalid IVF parameters nlist=%u nprobe=%u", nlist,
               nprobe);
    VA_REQUIRE(ctx, dim <= 4096, "dimension must be 1-4096, got %u", dim);
    va_index* ix = nullptr;
    VA_CHECK_STATUS(va_index_create(ctx, dim, capacity, &ix));
    ix->nlist = nlist;
    ix->nprobe = nprobe;
    ix->routing = routing_threshold;
    *out = ix;
    return VA_OK;
}

va_status va_index_train(va_context* ctx, va_index* index, const float* centroids, uint64_t seed) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_train"));
    if (index->nlist == 0) return VA_OK;  // a flat index has nothing to train (train(), :405-407)
    va::DeviceGuard g(ctx->device);
    const uint32_t C = index->nlist, D = index->dim;
    struct Tmp {
        void* p[2] = {};
        ~Tmp() {
            for (void* q : p)
                if (q) (void)hipFree(q);
        }
    } t;
    float* cen = nullptr;
    VA_CHECK_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&cen), uint64_t(C) * D * 4));
    t.p[0] = cen;
    if (centroids) {
        VA_CHECK_HIP(ctx, hipMemcpyAsync(cen, centroids, uint64_t(C) * D * 4, hipMemcpyDeviceToDevice, ctx->stream));
    } else {
        // k-means over the live vectors (IVFStructure.train, Index/Internal/IVFStructure.swift:202-259:
        // k-means++ seeding, at most 25 Lloyd iterations, convergence threshold 0.001)
        const uint32_t live = index->slots - index->deleted;
        VA_REQUIRE(ctx, live > 0, "Cannot train IVF index with no vectors");
        VA_REQUIRE(ctx, live >= C, "Need at least %u vectors for %u clusters, got %u", C, C, live);
        // retraining replaces the old lists (not rebuilt by the compaction below)
        if (index->ivf) (void)va_ivf_destroy(index->ivf);
        index->ivf = nullptr;
        if (index->centroids) (void)hipFree(index->centroids);
        index->centroids = nullptr;
        VA_CHECK_STATUS(va_index_compact(ctx, index));  // the live rows are then slots [0, live)
        float* init = nullptr;
        VA_CHECK_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&init), uint64_t(C) * D * 4 + uint64_t(live) * 4));
        t.p[1] = init;
        uint32_t* assign = reinterpret_cast<uint32_t*>(init + uint64_t(C) * D);
        VA_CHECK_STATUS(va_kmeans_plusplus(ctx, index->rows, live, D, C, seed, init, nullptr));
        VA_CHECK_STATUS(va_kmeans_fit(ctx, index->rows, live, D, C, init, 25, 0.001f, cen, assign, nullptr, nullptr,
                                      nullptr));
    }
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (index->centroids) (void)hipFree(index->centroids);
    index->centroids = cen;
    t.p[0] = nullptr;
    // the lists over every slot (IVFStructure.train clears them; AcceleratedVectorIndex.train
    // reassigns every vector, :438-446)
    return va::rebuild_lists(ctx, index);
}

va_status va_index_insert(va_context* ctx, va_index* index, const float* vectors, uint32_t num_vectors,
                          uint32_t* out_handles) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_insert"));
    VA_REQUIRE(ctx, vectors != nullptr || num_vectors == 0, "va_index_insert: NULL vectors");
    if (num_vectors == 0) return VA_OK;
    VA_REQUIRE(ctx, uint64_t(index->slots) + num_vectors < 0xFFFFFFFFull &&
                        uint64_t(index->stable_to_slot.size()) + num_vectors < 0xFFFFFFFFull,
               "va_index_insert: too many vectors");
    va::DeviceGuard g(ctx->device);
    VA_CHECK_STATUS(va::reserve_slots(ctx, index, uint64_t(index->slots) + num_vectors));
    const uint32_t s0 = index->slots, n = num_vectors, dim = index->dim;
    const uint32_t first = uint32_t(index->stable_to_slot.size());
    VA_CHECK_HIP(ctx, hipMemcpyAsync(index->rows + uint64_t(s0) * dim, vectors, uint64_t(n) * dim * 4,
                                     hipMemcpyDeviceToDevice, ctx->stream));
    if (index->pitch)
        VA_CHECK_STATUS(va::build_shadow(ctx, index->rows + uint64_t(s0) * dim, n, dim,
                                         index->shadow + uint64_t(s0) * index->pitch, index->norms + s0, nullptr,
                                         index->errs + s0));
    va::fill_byte_kernel<<<dim3(va::grid_for(n)), dim3(256), 0, ctx->stream>>>(index->skip + s0, n, 0);
    VA_CHECK_LAUNCH(ctx);
    va::iota_kernel<<<dim3(va::grid_for(n)), dim3(256), 0, ctx->stream>>>(index->slot_stable + s0, n, first);
    VA_CHECK_LAUNCH(ctx);
    for (uint32_t i = 0; i < n; ++i) {
        index->stable_to_slot.push_back(s0 + i);
        index->slot_to_stable.push_back(first + i);
        if (out_handles) out_handles[i] = first + i;
    }
    index->slots += n;
    // a trained IVF index: the new slots go to the end of their nearest lists
    // (IVFStructure.assignToCluster, Index/Internal/IVFStructure.swift:280-287)
    if (index->ivf) return va_ivf_add(ctx, index->ivf, index->rows + uint64_t(s0) * dim, n, dim, s0);
    if (index->centroids) return va::rebuild_lists(ctx, index);
    return VA_OK;
}

va_status va_index_remove(va_context* ctx, va_index* index, const uint32_t* handles, uint32_t num_handles,
                          uint32_t* out_removed) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_remove"));
    VA_REQUIRE(ctx, handles != nullptr || num_handles == 0, "va_index_remove: NULL handles");
    va::DeviceGuard g(ctx->device);
    std::vector<uint32_t> slots;
    for (uint32_t i = 0; i < num_handles; ++i) {
        const uint32_t h = handles[i];
        if (h >= index->stable_to_slot.size()) continue;
        const uint32_t s = index->stable_to_slot[h];
        if (s == va::kTombstone) continue;
        index->stable_to_slot[h] = va::kTombstone;
        index->slot_to_stable[s] = va::kTombstone;
        slots.push_back(s);
    }
    index->deleted += uint32_t(slots.size());
    if (out_removed) *out_removed = uint32_t(slots.size());
    return va::set_bytes(ctx, index->skip, slots, 1);
}

va_status va_index_compact(va_context* ctx, va_index* index) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_compact"));
    if (index->deleted == 0) return VA_OK;
    va::DeviceGuard g(ctx->device);
    std::vector<uint32_t> keep;
    keep.reserve(index->slots - index->deleted);
    for (uint32_t s = 0; s < index->slots; ++s)
        if (index->slot_to_stable[s] != va::kTombstone) keep.push_back(s);
    const uint32_t n = uint32_t(keep.size());
    va::DevBuffers nb;
    VA_CHECK_STATUS(va::alloc_buffers(ctx, index->capacity, index->dim, index->pitch, nb));
    if (n) {
        va::Scratch sc(ctx);
        va_status st = sc.reserve(va::Scratch::round(uint64_t(n) * 4));
        if (st != VA_OK) {
            nb.release();
            return st;
        }
        uint32_t* dkeep = sc.carve<uint32_t>(n);
        VA_CHECK_HIP(ctx, hipMemcpyAsync(dkeep, keep.data(), uint64_t(n) * 4, hipMemcpyHostToDevice, ctx->stream));
        va::gather_rows_kernel<<<dim3(n), dim3(256), 0, ctx->stream>>>(index->rows, index->shadow, index->norms,
                                                                      index->errs, index->slot_stable, dkeep, n,
                                                                      index->dim, index->pitch, nb.rows, nb.shadow,
                                                                      nb.norms, nb.errs,
                                                                      nb.slot_stable);
        VA_CHECK_LAUNCH(ctx);
    }
    va::fill_byte_kernel<<<dim3(va::grid_for(index->capacity)), dim3(256), 0, ctx->stream>>>(nb.skip, index->capacity, 0);
    VA_CHECK_LAUNCH(ctx);
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    va::DevBuffers old = va::current(index);
    old.release();
    va::install(index, nb, index->capacity);
    std::vector<uint32_t> s2h(n);
    for (uint32_t j = 0; j < n; ++j) {
        const uint32_t h = index->slot_to_stable[keep[j]];
        s2h[j] = h;
        index->stable_to_slot[h] = j;
    }
    index->slot_to_stable.swap(s2h);
    index->slots = n;
    index->deleted = 0;
    // the lists name slots, which moved: rebuilt from the trained centroids
    return va::rebuild_lists(ctx, index);
}

va_status va_index_get_info(const va_index* index, va_index_info* out) {
    if (!index || !out) return VA_ERR_INVALID_ARG;
    out->count = index->slots - index->deleted;
    out->deleted = index->deleted;
    out->slots = index->slots;
    out->dimension = index->dim;
    out->capacity = index->capacity;
    out->rows = index->rows;
    out->next_handle = uint32_t(index->stable_to_slot.size());
    out->nlist = index->nlist;
    out->nprobe = index->nprobe;
    out->routing_threshold = index->routing;
    out->trained = index->centroids != nullptr;
    out->ivf_routed = va::ivf_route(index);
    out->centroids = index->centroids;
    out->lists = index->ivf;
    return VA_OK;
}

int va_index_contains(const va_index* index, uint32_t handle) {
    return index && handle < index->stable_to_slot.size() && index->stable_to_slot[handle] != va::kTombstone;
}

va_status va_index_get_vector(va_context* ctx, const va_index* index, uint32_t handle, float* out) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_get_vector"));
    VA_REQUIRE(ctx, out != nullptr, "va_index_get_vector: NULL output");
    VA_REQUIRE(ctx, va_index_contains(index, handle), "invalid handle %u", handle);
    va::DeviceGuard g(ctx->device);
    const uint32_t s = index->stable_to_slot[handle];
    VA_CHECK_HIP(ctx, hipMemcpyAsync(out, index->rows + uint64_t(s) * index->dim, uint64_t(index->dim) * 4,
                                     hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VA_OK;
}

va_status va_index_search(va_context* ctx, const va_index* index, va_metric metric, const float* queries,
                          uint32_t num_queries, uint32_t k, uint32_t* out_handles, float* out_dist) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_search"));
    VA_REQUIRE(ctx, queries && out_handles, "va_index_search: NULL pointer");
    VA_REQUIRE(ctx, num_queries > 0, "numQueries must be positive, got %u", num_queries);
    VA_REQUIRE(ctx, k > 0, "k must be positive, got %u", k);
    VA_REQUIRE(ctx, k <= VA_MAX_K, "k %u exceeds maximum supported k %u", k, VA_MAX_K);
    VA_REQUIRE(ctx, metric >= VA_METRIC_L2SQ && metric <= VA_METRIC_L2, "va_index_search: unknown metric %d",
               int(metric));
    va::DeviceGuard g(ctx->device);
    const uint64_t total = uint64_t(num_queries) * k;
    if (index->slots == index->deleted) {
        // nothing live: every result slot is missing
        VA_CHECK_STATUS(va::fill_u32(ctx, out_handles, total, va::kSentinel));
        if (out_dist) VA_CHECK_STATUS(va::fill_u32(ctx, reinterpret_cast<uint32_t*>(out_dist), total, 0x7F800000u));
        return VA_OK;
    }
    if (va::ivf_route(index)) {
        // searchIVF / searchIVFBatch (Index/AcceleratedVectorIndex.swift:1378-1481): the nprobe
        // nearest lists, deleted slots excluded inside the scan (no over-fetch)
        VA_REQUIRE(ctx, metric == VA_METRIC_L2SQ, "an IVF index searches by L2^2 only (metric %d)", int(metric));
        VA_CHECK_STATUS(va::ivf_search_masked(ctx, index->ivf, queries, num_queries, index->nprobe, k, out_handles,
                                              out_dist, index->deleted ? index->skip : nullptr));
    } else {
        VA_CHECK_STATUS(va::flat_topk(ctx, va::metric_op(metric), queries, index->rows, num_queries, index->slots,
                                      index->dim, k, out_handles, out_dist, index->pitch ? index->shadow : nullptr,
                                      index->pitch ? index->norms : nullptr, index->deleted ? index->skip : nullptr,
                                      index->pitch ? index->errs : nullptr));
    }
    va::slots_to_handles_kernel<<<dim3(va::grid_for(total)), dim3(256), 0, ctx->stream>>>(out_handles, total,
                                                                                         index->slot_stable);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status va_index_search_filtered(va_context* ctx, va_index* index, va_metric metric, const float* query, uint32_t k,
                                   va_index_filter filter, void* user, uint32_t* out_handles, float* out_dist,
                                   uint32_t* out_count, uint32_t* out_examined) {
    VA_CHECK_STATUS(va::check_ctx(ctx, index, "va_index_search_filtered"));
    VA_REQUIRE(ctx, query && out_handles && out_count, "va_index_search_filtered: NULL pointer");
    VA_REQUIRE(ctx, k > 0, "k must be positive, got %u", k);
    VA_REQUIRE(ctx, metric >= VA_METRIC_L2SQ && metric <= VA_METRIC_L2,
               "va_index_search_filtered: unknown metric %d", int(metric));
    va::DeviceGuard g(ctx->device);
    *out_count = 0;
    if (out_examined) *out_examined = 0;
    const uint32_t live = index->slots - index->deleted;
    if (live == 0) return VA_OK;
    const bool ivf = va::ivf_route(index);
    VA_REQUIRE(ctx, !ivf || metric == VA_METRIC_L2SQ, "an IVF index searches by L2^2 only (metric %d)", int(metric));
    // seen = deleted rows, then also every row a round has examined
    VA_CHECK_HIP(ctx, hipMemcpyAsync(index->seen, index->skip, index->slots, hipMemcpyDeviceToDevice, ctx->stream));
    // one round's results (device, then host)
    struct DevTmp {
        void* p[3] = {};
        ~DevTmp() {
            for (void* q : p)
                if (q) (void)hipFree(q);
        }
    } rb;
    VA_CHECK_HIP(ctx, hipMalloc(&rb.p[0], uint64_t(VA_MAX_K) * 4));
    VA_CHECK_HIP(ctx, hipMalloc(&rb.p[1], uint64_t(VA_MAX_K) * 4));
    uint32_t* d_idx = static_cast<uint32_t*>(rb.p[0]);
    float* d_dist = static_cast<float*>(rb.p[1]);
    std::vector<uint32_t> h_idx(VA_MAX_K), slots;
    std::vector<float> h_dist(VA_MAX_K);
    uint32_t examined = 0, accepted = 0;
    auto take = [&](uint32_t sl, float dist) {
        ++examined;
        const uint32_t h = index->slot_to_stable[sl];
        if (accepted < k && (!filter || filter(h, user))) {
            out_handles[accepted] = h;
            if (out_dist) out_dist[accepted] = dist;
            ++accepted;
        }
    };
    // round sizes: twice k (the reference's first over-fetch), doubling, at most VA_MAX_K
    uint32_t fetch = std::min<uint32_t>(std::max<uint32_t>(2 * k, 16), VA_MAX_K);
    bool sorted_pass = false;
    while (accepted < k && examined < live) {
        if (sorted_pass) break;
        const uint32_t f = std::min(fetch, live - examined);
        if (ivf)
            VA_CHECK_STATUS(va::ivf_search_masked(ctx, index->ivf, query, 1, index->nprobe, f, d_idx, d_dist,
                                                  index->seen));
        else
            VA_CHECK_STATUS(va::flat_topk(ctx, va::metric_op(metric), query, index->rows, 1, index->slots, index->dim,
                                          f, d_idx, d_dist, index->pitch ? index->shadow : nullptr,
                                          index->pitch ? index->norms : nullptr, index->seen,
                                          index->pitch ? index->errs : nullptr));
        VA_CHECK_HIP(ctx, hipMemcpyAsync(h_idx.data(), d_idx, uint64_t(f) * 4, hipMemcpyDeviceToHost, ctx->stream));
        VA_CHECK_HIP(ctx, hipMemcpyAsync(h_dist.data(), d_dist, uint64_t(f) * 4, hipMemcpyDeviceToHost, ctx->stream));
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        slots.clear();
        for (uint32_t i = 0; i < f; ++i) {
            const uint32_t sl = h_idx[i];
            if (sl == va::kSentinel) break;
            slots.push_back(sl);
            take(sl, h_dist[i]);
        }
        if (slots.empty()) break;
        if (ivf && slots.size() < f) break;  // the probed lists hold no more live rows
        VA_CHECK_STATUS(va::set_bytes(ctx, index->seen, slots, 1));
        // a round of VA_MAX_K rows did not find k: the rest in one sorted pass (below)
        sorted_pass = !ivf && fetch == VA_MAX_K;
        fetch = std::min<uint32_t>(fetch * 2, VA_MAX_K);
    }
    if (sorted_pass && accepted < k && examined < live) {
        // Every row's key (the fp32 scan's arithmetic, so the same keys the rounds saw), the rows
        // already examined or deleted made absent, a stable device sort by key (ties stay in slot
        // order), then the sorted rows filtered on the host in batches until k pass.
        const uint32_t N = index->slots;
        const uint64_t n4 = (uint64_t(N) + 63) & ~uint64_t(63);  // 256-byte aligned sub-buffers
        size_t tmp_bytes = 0;
        uint32_t* null_u32 = nullptr;
        VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(nullptr, tmp_bytes, null_u32, null_u32, null_u32, null_u32, N, 0, 32,
                                                    ctx->stream));
        VA_CHECK_HIP(ctx, hipMalloc(&rb.p[2], n4 * 4 * 4 + tmp_bytes));
        uint32_t* keys = static_cast<uint32_t*>(rb.p[2]);
        uint32_t* keys2 = keys + n4;
        uint32_t* ids = keys2 + n4;
        uint32_t* ids2 = ids + n4;
        void* tmp = ids2 + n4;
        va::DistArgs a;
        a.q = query;
        a.ldq = index->dim;
        a.x = index->rows;
        a.ldx = index->dim;
        a.Q = 1;
        a.N = N;
        a.D = index->dim;
        a.op = va::metric_op(metric);
        a.out = va::OUT_KEYS;
        a.out_k = keys;
        a.ldo = N;
        VA_CHECK_STATUS(va::launch_dist(ctx, a));
        VA_CHECK_STATUS(va::mask_dense_keys(ctx, keys, 1, N, N, 0, 1, index->seen));
        va::iota_kernel<<<dim3(va::grid_for(N)), dim3(256), 0, ctx->stream>>>(ids, N, 0);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(tmp, tmp_bytes, keys, keys2, ids, ids2, N, 0, 32, ctx->stream));
        constexpr uint32_t kBatch = 65536;
        std::vector<uint32_t> hk(kBatch), hs(kBatch);
        for (uint32_t off = 0; off < N && accepted < k; off += kBatch) {
            const uint32_t n = std::min(kBatch, N - off);
            VA_CHECK_HIP(ctx, hipMemcpyAsync(hk.data(), keys2 + off, uint64_t(n) * 4, hipMemcpyDeviceToHost, ctx->stream));
            VA_CHECK_HIP(ctx, hipMemcpyAsync(hs.data(), ids2 + off, uint64_t(n) * 4, hipMemcpyDeviceToHost, ctx->stream));
            VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
            bool rest_absent = false;
            for (uint32_t i = 0; i < n && accepted < k; ++i) {
                if (hk[i] == va::kAbsentKey) {
                    rest_absent = true;  // examined or deleted: everything after it too
                    break;
                }
                take(hs[i], va::float_of_key(hk[i]));
            }
            if (rest_absent) break;
        }
    }
    *out_count = accepted;
    if (out_examined) *out_examined = examined;
    return VA_OK;
}

}  // extern "C"
