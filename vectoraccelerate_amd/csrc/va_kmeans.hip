// va_kmeans.hip — Lloyd k-means and k-means++ seeding on the device: the IVF build's
// centroid training.
//
// va_kmeans_fit replaces KMeansPipeline.fit (Index/Kernels/Clustering/KMeansPipeline.swift:102-270)
// with its kernels: assignment (kmeans_assign_points, Metal/Shaders/ClusteringShaders.metal:16-120),
// update (kmeans_update_accumulate / kmeans_update_normalize, ClusteringShaders.metal:492-613),
// empty-cluster repair (KMeansUpdateKernel.handleEmptyClusters, KMeansUpdateKernel.swift:228-283)
// and the convergence test (KMeansConvergenceKernel.checkConvergence / computeInertia,
// KMeansConvergenceKernel.swift:76-183).  Per iteration, in the reference's order:
//   1. every point goes to its nearest centroid (squared L2, ties to the lower centroid), on the
//      fp32 MFMA distance kernel with an argmin epilogue; its distance is then recomputed in
//      difference form against that centroid (the reference's form, more accurate than the
//      expanded one);
//   2. a centroid becomes the mean of its points (sum times 1/count); an empty one stays;
//   3. the empty clusters, in index order, take the points farthest from their centroids
//      (ties to the lower point, each point once) with count 1;
//   4. converged when the largest centroid movement (L2) is below the threshold.
// The reference sums with float atomics, in an order that varies from run to run; here the
// points are grouped by cluster with a stable radix sort and summed in a fixed order (chunks of
// 256 points in point order, then the chunk sums in order), so every run gives the same bits.
//
// va_kmeans_plusplus replaces KMeansPlusPlusKernel.selectCentroids (KMeansPlusPlusKernel.swift:94-203)
// with compute_min_distances (ClusteringShaders.metal:419-447): D^2 sampling with the running
// minimum squared distance kept on the device, the cumulative weights as a double prefix sum and
// the pick as a binary search, so the k steps run without a host round trip.  The reference
// draws from the system generator; here the uniform draws come from splitmix64(seed).
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "va_internal.hpp"

namespace va {
namespace {

constexpr uint32_t kChunk = 256;  // points per partial centroid sum

__global__ __launch_bounds__(256) void fill_u64(unsigned long long* p, uint64_t n, unsigned long long v) {
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) p[i] = v;
}

// packed (key of |x - c|^2, centroid) -> assignment, L2 distance, sort value (point id)
__global__ __launch_bounds__(256) void unpack_assign(const unsigned long long* __restrict__ best, uint32_t N,
                                                     uint32_t* __restrict__ assign, float* __restrict__ dist,
                                                     uint32_t* __restrict__ sort_vals) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N) return;
    const unsigned long long b = best[i];
    if (b == ~0ull) {  // no finite distance: centroid 0 at infinity, as the reference leaves it
        assign[i] = 0;
        dist[i] = __builtin_inff();
    } else {
        assign[i] = uint32_t(b);
        dist[i] = sqrtf(float_of_key(uint32_t(b >> 32)));
    }
    sort_vals[i] = i;
}

// The assignment's distance again in difference form, sqrt(sum_d (x_d - c_d)^2), one wave per
// point with a fixed reduction order: error ~D 2^-24 |x - c|^2 instead of the expanded form's
// ~D 2^-24 (|x|^2 + |c|^2), so the empty-cluster repair ranks points by accurate distances.
__global__ __launch_bounds__(256) void refine_dist(const float* __restrict__ x, uint32_t N, uint32_t D,
                                                   const float* __restrict__ cen, const uint32_t* __restrict__ assign,
                                                   float* __restrict__ dist) {
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t i = blockIdx.x * 4 + (threadIdx.x >> 6); i < N; i += gridDim.x * 4) {
        if (dist[i] == __builtin_inff()) continue;  // no finite distance: left as infinity
        const float* xi = x + int64_t(i) * D;
        const float* ci = cen + int64_t(assign[i]) * D;
        float s = 0.0f;
        for (uint32_t d = lane; d < D; d += 64) {
            const float diff = xi[d] - ci[d];
            s = __builtin_fmaf(diff, diff, s);
        }
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) s += __shfl_xor(s, m);
        if (lane == 0) dist[i] = sqrtf(s);
    }
}

// first position of each cluster in the sorted assignments and its size
__global__ __launch_bounds__(256) void cluster_ranges(const uint32_t* __restrict__ sorted_assign, uint32_t N,
                                                      uint32_t C, uint32_t* __restrict__ first,
                                                      uint32_t* __restrict__ counts, uint32_t* __restrict__ chunks,
                                                      uint32_t* __restrict__ n_empty) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    auto lower = [&](uint32_t v) {
        uint32_t lo = 0, hi = N;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (sorted_assign[mid] < v) lo = mid + 1;
            else hi = mid;
        }
        return lo;
    };
    const uint32_t a = lower(c), b = lower(c + 1);
    first[c] = a;
    counts[c] = b - a;
    chunks[c] = (b - a + kChunk - 1) / kChunk;
    if (b == a) atomicAdd(n_empty, 1u);
}

// Centroid sums in a fixed order: a cluster's points (in point order) form chunks of kChunk;
// each chunk is summed in order in fp32 by one workgroup, then a cluster's chunk sums are added
// in chunk order and multiplied by 1/count (kmeans_update_normalize).  Chunking spreads a large
// cluster over many workgroups; the order never depends on scheduling.
// workgroup b -> (cluster, chunk): chunk_end is the inclusive scan of chunks per cluster
__global__ __launch_bounds__(256) void chunk_sums(const float* __restrict__ x, uint32_t D, uint32_t C,
                                                  const uint32_t* __restrict__ members,
                                                  const uint32_t* __restrict__ first,
                                                  const uint32_t* __restrict__ counts,
                                                  const uint32_t* __restrict__ chunk_end,
                                                  float* __restrict__ partial) {
    __shared__ uint32_t rows[kChunk];
    const uint32_t b = blockIdx.x;
    if (b >= chunk_end[C - 1]) return;
    uint32_t lo = 0, hi = C - 1;  // first cluster whose chunk_end exceeds b
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (chunk_end[mid] > b) hi = mid;
        else lo = mid + 1;
    }
    const uint32_t c = lo, n = counts[c];
    const uint32_t nch = (n + kChunk - 1) / kChunk;
    const uint32_t t = b - (chunk_end[c] - nch);
    const uint32_t p0 = first[c] + t * kChunk;
    const uint32_t m = min(kChunk, n - t * kChunk);
    if (threadIdx.x < m) rows[threadIdx.x] = members[p0 + threadIdx.x];
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < D; d += 256) {
        float s = 0.0f;
#pragma unroll 8
        for (uint32_t i = 0; i < m; ++i) s += x[int64_t(rows[i]) * D + d];
        partial[int64_t(b) * D + d] = s;
    }
}

// one workgroup per cluster: its chunk sums in chunk order, times 1/count; an empty cluster keeps
// its previous centroid
__global__ __launch_bounds__(256) void cluster_means(uint32_t D, const uint32_t* __restrict__ counts,
                                                     const uint32_t* __restrict__ chunk_end,
                                                     const float* __restrict__ partial,
                                                     const float* __restrict__ old_c, float* __restrict__ new_c) {
    const uint32_t c = blockIdx.x;
    const uint32_t n = counts[c];
    float* out = new_c + int64_t(c) * D;
    if (n == 0) {
        for (uint32_t d = threadIdx.x; d < D; d += 256) out[d] = old_c[int64_t(c) * D + d];
        return;
    }
    const uint32_t nch = (n + kChunk - 1) / kChunk, b0 = chunk_end[c] - nch;
    const float inv = 1.0f / float(n);
    for (uint32_t d = threadIdx.x; d < D; d += 256) {
        float s = 0.0f;
        for (uint32_t t = 0; t < nch; ++t) s += partial[int64_t(b0 + t) * D + d];
        out[d] = s * inv;
    }
}

// empty cluster ids in index order (one workgroup: a running offset over 256-wide chunks)
__global__ __launch_bounds__(256) void list_empty(const uint32_t* __restrict__ counts, uint32_t C,
                                                  uint32_t* __restrict__ empty_ids) {
    __shared__ uint32_t wsum[4];
    __shared__ uint32_t base;
    if (threadIdx.x == 0) base = 0;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t c0 = 0; c0 < C; c0 += 256) {
        const uint32_t c = c0 + threadIdx.x;
        const bool e = c < C && counts[c] == 0;
        const unsigned long long m = __ballot(e);
        if (lane == 0) wsum[wave] = uint32_t(__popcll(m));
        __syncthreads();
        uint32_t off = base;
        for (uint32_t w = 0; w < wave; ++w) off += wsum[w];
        if (e) empty_ids[off + uint32_t(__popcll(m & ((1ull << lane) - 1)))] = c;
        __syncthreads();
        if (threadIdx.x == 0) base += wsum[0] + wsum[1] + wsum[2] + wsum[3];
        __syncthreads();
    }
}

// distances as descending sort keys; NaN sorts last (the reference's `>` never takes it)
__global__ __launch_bounds__(256) void desc_keys(const float* __restrict__ dist, uint32_t N, uint32_t* __restrict__ keys) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < N) keys[i] = dist[i] != dist[i] ? 0xFFFFFFFFu : key_of_float_desc(dist[i]);
}

// empty cluster j takes the j-th farthest point (order[j]); a NaN distance is never taken
__global__ __launch_bounds__(256) void repair_empty(const float* __restrict__ x, uint32_t D,
                                                    const uint32_t* __restrict__ empty_ids,
                                                    const uint32_t* __restrict__ order,
                                                    const float* __restrict__ dist,
                                                    float* __restrict__ centroids, uint32_t* __restrict__ counts) {
    const uint32_t j = blockIdx.x;
    const uint32_t c = empty_ids[j], p = order[j];
    if (dist[p] != dist[p]) return;
    for (uint32_t d = threadIdx.x; d < D; d += 256) centroids[int64_t(c) * D + d] = x[int64_t(p) * D + d];
    if (threadIdx.x == 0) counts[c] = 1;
}

// movement of each centroid; the largest goes to max_bits (non-negative floats order as their bits)
__global__ __launch_bounds__(256) void centroid_movement(const float* __restrict__ old_c, const float* __restrict__ new_c,
                                                         uint32_t D, uint32_t* __restrict__ max_bits) {
    __shared__ float part[256];
    const uint32_t c = blockIdx.x;
    float s = 0.0f;
    for (uint32_t d = threadIdx.x; d < D; d += 256) {
        const float diff = new_c[int64_t(c) * D + d] - old_c[int64_t(c) * D + d];
        s += diff * diff;
    }
    part[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (int(threadIdx.x) < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicMax(max_bits, __builtin_bit_cast(uint32_t, sqrtf(part[0])));
}

// inertia: fixed per-workgroup partial sums in double, then one thread adds them in order
__global__ __launch_bounds__(256) void sum_partials(const float* __restrict__ v, uint32_t N, double* __restrict__ part) {
    __shared__ double s[256];
    double a = 0.0;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < N; i += gridDim.x * 256) a += double(v[i]);
    s[threadIdx.x] = a;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (int(threadIdx.x) < w) s[threadIdx.x] += s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = s[0];
}
__global__ void sum_final(const double* __restrict__ part, uint32_t n, double* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double a = 0.0;
    for (uint32_t i = 0; i < n; ++i) a += part[i];
    *out = a;
}

// ---- k-means++ -------------------------------------------------------------------------

// running minimum of |x - c|^2 against the newest centroid, and the sampling weight (0 once the
// point is a centroid).  One wave per point: lane l sums (x_d - c_d)^2 over d = l, l + 64, ...
// with fused multiply-adds, then the 64 partials combine by a butterfly (xor 32, 16, ..., 1).
__global__ __launch_bounds__(256) void pp_update(const float* __restrict__ x, uint32_t N, uint32_t D,
                                                 const float* __restrict__ c, const uint8_t* __restrict__ sel,
                                                 float* __restrict__ mind, double* __restrict__ w, int first) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= N) return;
    const float* xi = x + int64_t(i) * D;
    float s = 0.0f;
#pragma unroll 4
    for (uint32_t d = lane; d < D; d += 64) {
        const float diff = xi[d] - c[d];
        s = __builtin_fmaf(diff, diff, s);
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) s += __shfl_xor(s, m);
    if (lane == 0) {
        const float m = first ? s : fminf(mind[i], s);
        mind[i] = m;
        w[i] = sel[i] ? 0.0 : double(m);
    }
}

// pick step j: the first unselected point whose cumulative weight reaches u * total (the first
// unselected point when the total is 0), then copy it into centroid j
__global__ __launch_bounds__(256) void pp_pick(const float* __restrict__ x, uint32_t N, uint32_t D,
                                               const double* __restrict__ cum, const double* __restrict__ u,
                                               uint32_t j, uint8_t* __restrict__ sel, uint32_t* __restrict__ idx,
                                               float* __restrict__ centroids) {
    __shared__ uint32_t pick;
    if (threadIdx.x == 0) {
        uint32_t p = 0;
        if (j == 0) {
            p = uint32_t(u[0] * double(N));
            if (p >= N) p = N - 1;
        } else {
            const double total = cum[N - 1];
            if (total > 0.0) {
                const double thr = u[j] * total;
                uint32_t lo = 0, hi = N - 1;  // cum[N-1] = total > thr, so the answer exists
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (cum[mid] >= thr) hi = mid;
                    else lo = mid + 1;
                }
                p = lo;
                while (p < N && sel[p]) ++p;  // weights of selected points are 0: cum stays >= thr
                if (p >= N) p = lo;
            } else {
                while (p < N && sel[p]) ++p;
                if (p >= N) p = 0;
            }
        }
        sel[p] = 1;
        idx[j] = p;
        pick = p;
    }
    __syncthreads();
    const uint32_t p = pick;
    for (uint32_t d = threadIdx.x; d < D; d += 256) centroids[int64_t(j) * D + d] = x[int64_t(p) * D + d];
}

__global__ __launch_bounds__(256) void fill_iota(uint32_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = i;
}

__global__ __launch_bounds__(256) void fill_u8(uint8_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
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

va_status assign_points(va_context* ctx, const float* x, const float* cen, uint32_t N, uint32_t C, uint32_t D,
                        unsigned long long* best, uint32_t* assign, float* dist, uint32_t* sort_vals) {
    const uint32_t nb = (N + 255) / 256;
    fill_u64<<<dim3(std::min<uint32_t>(nb, 4096)), dim3(256), 0, ctx->stream>>>(best, N, ~0ull);
    VA_CHECK_LAUNCH(ctx);
    DistArgs a;
    a.q = x;
    a.ldq = D;
    a.x = cen;
    a.ldx = D;
    a.Q = N;
    a.N = C;
    a.D = D;
    a.op = OP_L2SQ;
    a.out = OUT_ARGMIN;
    a.best = best;
    VA_CHECK_STATUS(launch_dist(ctx, a));
    unpack_assign<<<dim3(nb), dim3(256), 0, ctx->stream>>>(best, N, assign, dist, sort_vals);
    VA_CHECK_LAUNCH(ctx);
    refine_dist<<<dim3(std::min<uint32_t>((N + 3) / 4, 8192)), dim3(256), 0, ctx->stream>>>(x, N, D, cen, assign, dist);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// packed minimum -> nearest centroid (0 when no distance is finite, as the reference's search
// from bestIdx = 0 leaves it)
__global__ __launch_bounds__(256) void unpack_nearest(const unsigned long long* __restrict__ best, uint32_t N,
                                                      uint32_t* __restrict__ assign) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < N) assign[i] = best[i] == ~0ull ? 0u : uint32_t(best[i]);
}

// offsets[c] = first position of cluster c in the sorted assignments, offsets[C] = N
__global__ __launch_bounds__(256) void csr_offsets(const uint32_t* __restrict__ sorted_assign, uint32_t N, uint32_t C,
                                                   uint32_t* __restrict__ offsets) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c > C) return;
    uint32_t lo = 0, hi = N;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (sorted_assign[mid] < c) lo = mid + 1;
        else hi = mid;
    }
    offsets[c] = lo;
}

}  // namespace

va_status nearest_centroids(va_context* ctx, const float* x, const float* cen, uint32_t N, uint32_t C, uint32_t D,
                            unsigned long long* best, uint32_t* assign) {
    const uint32_t nb = (N + 255) / 256;
    fill_u64<<<dim3(std::min<uint32_t>(nb, 4096)), dim3(256), 0, ctx->stream>>>(best, N, ~0ull);
    VA_CHECK_LAUNCH(ctx);
    DistArgs a;
    a.q = x;
    a.ldq = D;
    a.x = cen;
    a.ldx = D;
    a.Q = N;
    a.N = C;
    a.D = D;
    a.op = OP_L2SQ;
    a.out = OUT_ARGMIN;
    a.best = best;
    VA_CHECK_STATUS(launch_dist(ctx, a));
    unpack_nearest<<<dim3(nb), dim3(256), 0, ctx->stream>>>(best, N, assign);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status csr_from_assignments(va_context* ctx, const uint32_t* assign, uint32_t N, uint32_t C, uint32_t* ids,
                               uint32_t* offsets) {
    Owned own;
    uint32_t *iota, *sorted;
    VA_CHECK_STATUS(alloc(ctx, own, size_t(N) * 4, &iota));
    VA_CHECK_STATUS(alloc(ctx, own, size_t(N) * 4, &sorted));
    int bits = 1;
    while (bits < 32 && (1ull << bits) < C) ++bits;
    size_t tmp_bytes = 0;
    VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(nullptr, tmp_bytes, assign, sorted, iota, ids, N, 0, bits, ctx->stream));
    void* tmp;
    VA_CHECK_STATUS(alloc(ctx, own, tmp_bytes, &tmp));
    fill_iota<<<dim3((N + 255) / 256), dim3(256), 0, ctx->stream>>>(iota, N);
    VA_CHECK_LAUNCH(ctx);
    VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(tmp, tmp_bytes, assign, sorted, iota, ids, N, 0, bits, ctx->stream));
    csr_offsets<<<dim3((C + 1 + 255) / 256), dim3(256), 0, ctx->stream>>>(sorted, N, C, offsets);
    VA_CHECK_LAUNCH(ctx);
    // the temporaries are freed on return: finish the work that reads them first
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VA_OK;
}

}  // namespace va

extern "C" {

va_status va_kmeans_plusplus(va_context* ctx, const float* vectors, uint32_t num_vectors, uint32_t dim, uint32_t k,
                             uint64_t seed, float* out_centroids, uint32_t* out_indices) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    // KMeansPlusPlusKernel.selectCentroids' checks (KMeansPlusPlusKernel.swift:100-107)
    VA_REQUIRE(ctx, vectors && out_centroids, "va_kmeans_plusplus: NULL pointer");
    VA_REQUIRE(ctx, k > 0, "k must be positive");
    VA_REQUIRE(ctx, num_vectors >= k, "Not enough vectors (%u) for %u clusters", num_vectors, k);
    VA_REQUIRE(ctx, dim > 0, "dimension must be positive");
    va::DeviceGuard g(ctx->device);
    const uint32_t N = num_vectors, D = dim;
    va::Owned own;
    float* mind;
    double *w, *cum, *u;
    uint8_t* sel;
    uint32_t* idx;
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &mind));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 8, &w));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 8, &cum));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(k) * 8, &u));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N), &sel));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(k) * 4, &idx));
    size_t scan_bytes = 0;
    VA_CHECK_HIP(ctx, rocprim::inclusive_scan(nullptr, scan_bytes, w, cum, N, rocprim::plus<double>(), ctx->stream));
    void* scan_tmp;
    VA_CHECK_STATUS(va::alloc(ctx, own, scan_bytes, &scan_tmp));
    std::vector<double> hu(k);
    uint64_t s = seed;
    for (uint32_t j = 0; j < k; ++j) hu[j] = double(va::splitmix64(s) >> 11) * 0x1.0p-53;
    VA_CHECK_HIP(ctx, hipMemcpyAsync(u, hu.data(), size_t(k) * 8, hipMemcpyHostToDevice, ctx->stream));
    const uint32_t nb = (N + 255) / 256;
    va::fill_u8<<<dim3(nb), dim3(256), 0, ctx->stream>>>(sel, N);
    VA_CHECK_LAUNCH(ctx);
    va::pp_pick<<<dim3(1), dim3(256), 0, ctx->stream>>>(vectors, N, D, cum, u, 0, sel, idx, out_centroids);
    VA_CHECK_LAUNCH(ctx);
    for (uint32_t j = 1; j < k; ++j) {
        va::pp_update<<<dim3((N + 3) / 4), dim3(256), 0, ctx->stream>>>(vectors, N, D, out_centroids + int64_t(j - 1) * D, sel,
                                                               mind, w, j == 1);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_HIP(ctx, rocprim::inclusive_scan(scan_tmp, scan_bytes, w, cum, N, rocprim::plus<double>(), ctx->stream));
        va::pp_pick<<<dim3(1), dim3(256), 0, ctx->stream>>>(vectors, N, D, cum, u, j, sel, idx, out_centroids);
        VA_CHECK_LAUNCH(ctx);
    }
    if (out_indices)
        VA_CHECK_HIP(ctx, hipMemcpyAsync(out_indices, idx, size_t(k) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));  // the host draws outlive the upload
    return VA_OK;
}

va_status va_kmeans_fit(va_context* ctx, const float* vectors, uint32_t num_vectors, uint32_t dim,
                        uint32_t num_clusters, const float* initial_centroids, uint32_t max_iterations,
                        float convergence_threshold, float* out_centroids, uint32_t* out_assignments,
                        float* out_distances, uint32_t* out_counts, va_kmeans_info* out_info) {
    if (!ctx) return VA_ERR_INVALID_ARG;
    // KMeansPipeline.fit's checks (KMeansPipeline.swift:106-118, 137-141)
    VA_REQUIRE(ctx, vectors && initial_centroids && out_centroids && out_assignments, "va_kmeans_fit: NULL pointer");
    VA_REQUIRE(ctx, num_vectors > 0, "Vectors cannot be empty");
    VA_REQUIRE(ctx, dim > 0, "dimension must be positive");
    VA_REQUIRE(ctx, num_clusters > 0 && num_clusters <= num_vectors,
               "numClusters must be in [1, numVectors], got %u for %u vectors", num_clusters, num_vectors);
    va::DeviceGuard g(ctx->device);
    const uint32_t N = num_vectors, D = dim, C = num_clusters;
    int bits = 1;
    while (bits < 32 && (1ull << bits) < C) ++bits;

    va::Owned own;
    unsigned long long* best;
    uint32_t *assign, *sort_vals, *sorted_keys, *members, *first, *counts, *flags, *keys, *empty_ids, *chunks,
        *chunk_end;
    float *dist, *cur, *next;
    double* partials;
    const uint32_t nparts = std::min<uint32_t>(1024, (N + 255) / 256);
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 8, &best));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &assign));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &dist));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &sort_vals));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &sorted_keys));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &members));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(N) * 4, &keys));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * 4, &first));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * 4, &counts));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * 4, &empty_ids));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * 4, &chunks));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * 4, &chunk_end));
    // sum over clusters of ceil(count / kChunk) <= N / kChunk + C
    const uint64_t max_chunks = uint64_t(N) / va::kChunk + C;
    float* partial;
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(max_chunks) * D * 4, &partial));
    VA_CHECK_STATUS(va::alloc(ctx, own, 64, &flags));  // [0] empty clusters, [1] largest movement (bits)
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * D * 4, &cur));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(C) * D * 4, &next));
    VA_CHECK_STATUS(va::alloc(ctx, own, size_t(nparts + 1) * 8, &partials));
    size_t sort_bytes = 0, sort_bytes32 = 0;
    VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(nullptr, sort_bytes, assign, sorted_keys, sort_vals, members, N, 0,
                                                bits, ctx->stream));
    VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(nullptr, sort_bytes32, keys, sorted_keys, sort_vals, members, N, 0,
                                                32, ctx->stream));
    size_t scan_bytes = 0;
    VA_CHECK_HIP(ctx, rocprim::inclusive_scan(nullptr, scan_bytes, chunks, chunk_end, C, rocprim::plus<uint32_t>(),
                                              ctx->stream));
    sort_bytes = std::max(std::max(sort_bytes, sort_bytes32), scan_bytes);
    void* sort_tmp;
    VA_CHECK_STATUS(va::alloc(ctx, own, sort_bytes, &sort_tmp));
    VA_CHECK_HIP(ctx, hipMemcpyAsync(cur, initial_centroids, size_t(C) * D * 4, hipMemcpyDeviceToDevice, ctx->stream));

    const uint32_t nb = (N + 255) / 256, cb = (C + 255) / 256;
    uint32_t it = 0;
    bool converged = false;
    float max_move = 0.0f;
    auto group = [&]() -> va_status {
        // points grouped by cluster, in point order inside each (the sort is stable)
        VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(sort_tmp, sort_bytes, assign, sorted_keys, sort_vals, members, N,
                                                    0, bits, ctx->stream));
        VA_CHECK_STATUS(va::fill_u32(ctx, flags, 2, 0));
        va::cluster_ranges<<<dim3(cb), dim3(256), 0, ctx->stream>>>(sorted_keys, N, C, first, counts, chunks, flags);
        VA_CHECK_LAUNCH(ctx);
        return VA_OK;
    };
    while (it < max_iterations && !converged) {
        VA_CHECK_STATUS(va::assign_points(ctx, vectors, cur, N, C, D, best, assign, dist, sort_vals));
        VA_CHECK_STATUS(group());
        VA_CHECK_HIP(ctx, rocprim::inclusive_scan(sort_tmp, scan_bytes, chunks, chunk_end, C,
                                                  rocprim::plus<uint32_t>(), ctx->stream));
        va::chunk_sums<<<dim3(uint32_t(max_chunks)), dim3(256), 0, ctx->stream>>>(vectors, D, C, members, first, counts,
                                                                                  chunk_end, partial);
        VA_CHECK_LAUNCH(ctx);
        va::cluster_means<<<dim3(C), dim3(256), 0, ctx->stream>>>(D, counts, chunk_end, partial, cur, next);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_HIP(ctx, hipMemcpyAsync(ctx->host_word, flags, 4, hipMemcpyDeviceToHost, ctx->stream));
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        const uint32_t n_empty = ctx->host_word[0];
        if (n_empty > 0) {
            // the farthest points first, ties to the lower point (stable sort of descending keys)
            va::list_empty<<<dim3(1), dim3(256), 0, ctx->stream>>>(counts, C, empty_ids);
            VA_CHECK_LAUNCH(ctx);
            va::desc_keys<<<dim3(nb), dim3(256), 0, ctx->stream>>>(dist, N, keys);
            VA_CHECK_LAUNCH(ctx);
            VA_CHECK_HIP(ctx, rocprim::radix_sort_pairs(sort_tmp, sort_bytes, keys, sorted_keys, sort_vals, members, N,
                                                        0, 32, ctx->stream));
            va::repair_empty<<<dim3(n_empty), dim3(256), 0, ctx->stream>>>(vectors, D, empty_ids, members, dist, next,
                                                                           counts);
            VA_CHECK_LAUNCH(ctx);
        }
        va::centroid_movement<<<dim3(C), dim3(256), 0, ctx->stream>>>(cur, next, D, flags + 1);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_HIP(ctx, hipMemcpyAsync(ctx->host_word + 1, flags + 1, 4, hipMemcpyDeviceToHost, ctx->stream));
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        max_move = __builtin_bit_cast(float, ctx->host_word[1]);
        converged = max_move < convergence_threshold;
        std::swap(cur, next);
        ++it;
    }
    if (it == 0) {
        // no iteration (max_iterations == 0): assignment and counts for the initial centroids
        VA_CHECK_STATUS(va::assign_points(ctx, vectors, cur, N, C, D, best, assign, dist, sort_vals));
        VA_CHECK_STATUS(group());
    }
    va::sum_partials<<<dim3(nparts), dim3(256), 0, ctx->stream>>>(dist, N, partials);
    VA_CHECK_LAUNCH(ctx);
    va::sum_final<<<dim3(1), dim3(64), 0, ctx->stream>>>(partials, nparts, partials + nparts);
    VA_CHECK_LAUNCH(ctx);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(out_centroids, cur, size_t(C) * D * 4, hipMemcpyDeviceToDevice, ctx->stream));
    VA_CHECK_HIP(ctx, hipMemcpyAsync(out_assignments, assign, size_t(N) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    if (out_distances)
        VA_CHECK_HIP(ctx, hipMemcpyAsync(out_distances, dist, size_t(N) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    if (out_counts)
        VA_CHECK_HIP(ctx, hipMemcpyAsync(out_counts, counts, size_t(C) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    double* host_inertia = reinterpret_cast<double*>(ctx->host_word + 2);
    VA_CHECK_HIP(ctx, hipMemcpyAsync(host_inertia, partials + nparts, 8, hipMemcpyDeviceToHost, ctx->stream));
    VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (out_info) {
        out_info->iterations = it;
        out_info->converged = converged ? 1 : 0;
        out_info->inertia = *host_inertia;
        out_info->max_movement = max_move;
    }
    return VA_OK;
}

}  // extern "C"
