/*
 * vectoraccelerate.hpp — header-only C++17 host mirror of the reference's Swift classes over the
 * C ABI of libva_hip.so (va_hip.h).  Link with -lva_hip; no HIP headers are needed: device
 * memory is allocated and copied through va_buffer_*.
 *
 * Mirrors (paths relative to the reference's Sources/VectorAccelerate/):
 *   Context                    Metal4Context / GPUContext (Core/Metal4Context.swift:183-269)
 *   DeviceBuffer<T>            BufferToken / getBuffer (Core/Metal4Context.swift:471-488)
 *   VectorError                VectorError / IndexError (invalidInput, dimensionMismatch, ...)
 *   FusedL2TopKKernel          Kernels/Metal4/FusedL2TopKKernel.swift (findNearestNeighbors, encode)
 *   TopKSelectionKernel        Kernels/Metal4/TopKSelectionKernel.swift
 *   ScalarQuantizationKernel   Kernels/Metal4/ScalarQuantizationKernel.swift (per-dimension int8)
 *   BinaryQuantizationKernel   Kernels/Metal4/BinaryQuantizationKernel.swift + HammingDistanceKernel.swift
 *   IVFIndex                   Index/Kernels/IVF/IVFSearchPipeline.swift + Index/Internal/IVFStructure.swift
 *   AcceleratedVectorIndex     Index/AcceleratedVectorIndex.swift (flat: handles, removal, compaction, filters)
 *   MetalComputeProvider       Integration/MetalComputeProvider.swift (batchDistance, findNearest)
 *   KMeansPipeline             Index/Kernels/Clustering/KMeansPipeline.swift
 *   ProductQuantizationKernel  Kernels/Metal4/ProductQuantizationKernel.swift
 * Every call checks the status and throws VectorError with the library's message.
 */
#ifndef VECTORACCELERATE_HPP
#define VECTORACCELERATE_HPP

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "va_hip.h"

namespace vectoraccelerate {

class VectorError : public std::runtime_error {
   public:
    VectorError(va_status st, const std::string& msg) : std::runtime_error(msg), status(st) {}
    va_status status;
    // VectorError / IndexError case of the status (invalidInput, dimensionMismatch, ...)
    const char* kind() const {
        switch (status) {
            case VA_ERR_INVALID_ARG: return "invalidInput";
            case VA_ERR_DIMENSION_MISMATCH: return "dimensionMismatch";
            case VA_ERR_OOM: return "bufferAllocationFailed";
            case VA_ERR_UNSUPPORTED: return "unsupported";
            default: return "computeFailed";
        }
    }
};

class Context {
   public:
    explicit Context(int device = 0) {
        va_status st = va_context_create(device, &h_);
        if (st != VA_OK) throw VectorError(st, std::string("va_context_create: ") + va_status_string(st));
    }
    ~Context() {
        if (h_) va_context_destroy(h_);
    }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    va_context* handle() const { return h_; }
    void check(va_status st, const char* what) const {
        if (st != VA_OK) throw VectorError(st, std::string(what) + ": " + va_last_error_message(h_));
    }
    // executeAndWait's wait
    void synchronize() const { check(va_context_synchronize(h_), "va_context_synchronize"); }
    void setOption(va_option o, uint64_t v) const { check(va_context_set_option(h_, o, v), "va_context_set_option"); }

   private:
    va_context* h_ = nullptr;
};

// Device array of n elements owned by a context.
template <class T>
class DeviceBuffer {
   public:
    DeviceBuffer() = default;
    DeviceBuffer(const Context& ctx, size_t n) : ctx_(&ctx), n_(n) {
        void* p = nullptr;
        ctx.check(va_buffer_alloc(ctx.handle(), n * sizeof(T), &p), "va_buffer_alloc");
        p_ = static_cast<T*>(p);
    }
    DeviceBuffer(const Context& ctx, const std::vector<T>& host) : DeviceBuffer(ctx, host.size()) { upload(host); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer(DeviceBuffer&& o) noexcept { *this = std::move(o); }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            release();
            ctx_ = o.ctx_;
            p_ = o.p_;
            n_ = o.n_;
            o.p_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    T* data() const { return p_; }
    size_t size() const { return n_; }
    void upload(const std::vector<T>& host) {
        if (host.size() != n_) throw VectorError(VA_ERR_INVALID_ARG, "upload: size mismatch");
        ctx_->check(va_buffer_upload(ctx_->handle(), p_, host.data(), n_ * sizeof(T)), "va_buffer_upload");
        ctx_->synchronize();
    }
    std::vector<T> download() const {
        std::vector<T> host(n_);
        ctx_->check(va_buffer_download(ctx_->handle(), host.data(), p_, n_ * sizeof(T)), "va_buffer_download");
        ctx_->synchronize();
        return host;
    }

   private:
    void release() {
        if (p_ && ctx_) va_buffer_free(ctx_->handle(), p_);
        p_ = nullptr;
    }
    const Context* ctx_ = nullptr;
    T* p_ = nullptr;
    size_t n_ = 0;
};

// Row-major [rows x dim] host matrix.
struct Matrix {
    std::vector<float> data;
    uint32_t rows = 0, dim = 0;
};

// Metal4FusedL2TopKResult / IVFSearchResult: idx[numQueries x k] (VA_SENTINEL_INDEX = empty).
struct SearchResult {
    std::vector<uint32_t> indices;
    std::vector<float> distances;
    uint32_t numQueries = 0, k = 0;
    std::vector<std::pair<uint32_t, float>> results(uint32_t q) const {
        std::vector<std::pair<uint32_t, float>> r;
        for (uint32_t j = 0; j < k; ++j)
            if (indices[size_t(q) * k + j] != VA_SENTINEL_INDEX)
                r.emplace_back(indices[size_t(q) * k + j], distances[size_t(q) * k + j]);
        return r;
    }
};

class FusedL2TopKKernel {
   public:
    explicit FusedL2TopKKernel(const Context& c) : ctx_(c) {}
    // encode tier: device inputs and outputs
    void encode(va_metric metric, const float* q, const float* x, uint32_t Q, uint32_t N, uint32_t D, uint32_t k,
                uint32_t* idx, float* dist) const {
        ctx_.check(va_fused_topk(ctx_.handle(), metric, q, x, Q, N, D, k, idx, dist), "va_fused_topk");
    }
    SearchResult findNearestNeighbors(const Matrix& queries, const Matrix& dataset, uint32_t k,
                                      va_metric metric = VA_METRIC_L2SQ) const {
        if (queries.dim != dataset.dim) throw VectorError(VA_ERR_DIMENSION_MISMATCH, "query / dataset dimension");
        DeviceBuffer<float> q(ctx_, queries.data), x(ctx_, dataset.data);
        DeviceBuffer<uint32_t> idx(ctx_, size_t(queries.rows) * k);
        DeviceBuffer<float> dist(ctx_, size_t(queries.rows) * k);
        encode(metric, q.data(), x.data(), queries.rows, dataset.rows, dataset.dim, k, idx.data(), dist.data());
        return SearchResult{idx.download(), dist.download(), queries.rows, k};
    }

   private:
    const Context& ctx_;
};

// MetalComputeProvider (Integration/MetalComputeProvider.swift:119-269): the VectorCore façade.
// batchDistance: euclidean -> L2 distance, cosine -> 1 - similarity, dotProduct -> raw dot;
// findNearest: the min(k, count) nearest (index, distance) pairs, nearest first (dotProduct:
// largest dot first, raw dot reported); with dotProductAsDistance (VectorCore's
// DotProductDistance through the BatchKernelProvider conformance) -dot, ascending.
// Manhattan / chebyshev have no GPU kernel here and are not offered.
class MetalComputeProvider {
   public:
    enum class Metric { euclidean, cosine, dotProduct };
    explicit MetalComputeProvider(const Context& c) : ctx_(c) {}

    std::vector<float> batchDistance(const std::vector<float>& query, const Matrix& candidates, Metric metric,
                                     bool dotProductAsDistance = false) const {
        if (candidates.rows == 0) return {};
        Matrix q{query, 1, uint32_t(query.size())};
        std::vector<float> row = distanceMatrix(q, candidates, metric);
        if (metric == Metric::dotProduct && dotProductAsDistance)
            for (float& v : row) v = -v;
        return row;
    }
    // queries x candidates, row-major
    std::vector<float> distanceMatrix(const Matrix& queries, const Matrix& candidates, Metric metric) const {
        if (queries.rows == 0 || candidates.rows == 0) return {};
        check_dims(queries, candidates);
        DeviceBuffer<float> q(ctx_, queries.data), x(ctx_, candidates.data);
        DeviceBuffer<float> out(ctx_, size_t(queries.rows) * candidates.rows);
        const uint32_t Q = queries.rows, N = candidates.rows, D = queries.dim;
        va_status st = metric == Metric::euclidean ? va_l2_all_pairs(ctx_.handle(), q.data(), x.data(), out.data(), Q, N, D, 1)
                       : metric == Metric::cosine ? va_cosine_all_pairs(ctx_.handle(), q.data(), x.data(), out.data(), Q, N, D, 1)
                                                  : va_dot_all_pairs(ctx_.handle(), q.data(), x.data(), out.data(), Q, N, D, 0);
        ctx_.check(st, "MetalComputeProvider.distanceMatrix");
        return out.download();
    }
    std::vector<std::pair<uint32_t, float>> findNearest(const std::vector<float>& query, const Matrix& candidates,
                                                        uint32_t k, Metric metric,
                                                        bool dotProductAsDistance = false) const {
        Matrix q{query, 1, uint32_t(query.size())};
        auto all = findNearestBatch(q, candidates, k, metric, dotProductAsDistance);
        return all.empty() ? std::vector<std::pair<uint32_t, float>>{} : all[0];
    }
    std::vector<std::vector<std::pair<uint32_t, float>>> findNearestBatch(const Matrix& queries,
                                                                         const Matrix& candidates, uint32_t k,
                                                                         Metric metric,
                                                                         bool dotProductAsDistance = false) const {
        std::vector<std::vector<std::pair<uint32_t, float>>> out(queries.rows);
        if (k == 0 || candidates.rows == 0 || queries.rows == 0) return out;
        check_dims(queries, candidates);
        const uint32_t kk = std::min<uint32_t>(std::min<uint32_t>(k, candidates.rows), VA_MAX_K);
        const va_metric vm = metric == Metric::euclidean ? VA_METRIC_L2
                             : metric == Metric::cosine  ? VA_METRIC_COSINE
                                                         : VA_METRIC_DOT;
        SearchResult r = FusedL2TopKKernel(ctx_).findNearestNeighbors(queries, candidates, kk, vm);
        const bool raw_dot = metric == Metric::dotProduct && !dotProductAsDistance;
        for (uint32_t i = 0; i < queries.rows; ++i)
            for (auto& p : r.results(i)) out[i].emplace_back(p.first, raw_dot ? -p.second : p.second);
        return out;
    }

   private:
    static void check_dims(const Matrix& a, const Matrix& b) {
        if (a.dim != b.dim)
            throw VectorError(VA_ERR_INVALID_ARG,
                              "All candidates must match the query dimension (" + std::to_string(a.dim) + ")");
    }
    const Context& ctx_;
};

// IndexConfiguration.ivf(dimension:nlist:nprobe:capacity:routingThreshold) (Index/Types/IndexConfiguration.swift)
struct IVFConfiguration {
    uint32_t nlist = 0, nprobe = 0, routingThreshold = 0;
};

// AcceleratedVectorIndex over va_index_* (Index/AcceleratedVectorIndex.swift:406-1481): stable
// handles in insertion order, removal, compaction, plain and filtered search; with an
// IVFConfiguration, train() and IVF routing (searchIVF / searchIVFBatch) once trained.
class AcceleratedVectorIndex {
   public:
    AcceleratedVectorIndex(const Context& c, uint32_t dim, uint32_t capacity = 10000, va_metric metric = VA_METRIC_L2SQ)
        : ctx_(c), metric_(metric) {
        ctx_.check(va_index_create(ctx_.handle(), dim, capacity, &h_), "va_index_create");
    }
    // IVF index (L2^2): flat until trained
    AcceleratedVectorIndex(const Context& c, uint32_t dim, const IVFConfiguration& ivf, uint32_t capacity = 100000)
        : ctx_(c), metric_(VA_METRIC_L2SQ) {
        ctx_.check(va_index_create_ivf(ctx_.handle(), dim, capacity, ivf.nlist, ivf.nprobe, ivf.routingThreshold, &h_),
                   "va_index_create_ivf");
    }
    // train(): device k-means over the live vectors (seeded by `seed`), then the lists
    void train(uint64_t seed = 0x5EED) { ctx_.check(va_index_train(ctx_.handle(), h_, nullptr, seed), "va_index_train"); }
    // train with given centroids (host, [nlist x dim])
    void train(const std::vector<float>& centroids) {
        DeviceBuffer<float> c(ctx_, centroids);
        ctx_.check(va_index_train(ctx_.handle(), h_, c.data(), 0), "va_index_train");
    }
    bool isTrained() const { return info().trained != 0; }
    // the inverted lists (offsets[nlist + 1], slots in list order); empty while untrained
    std::pair<std::vector<uint32_t>, std::vector<uint32_t>> lists() const {
        const va_index_info i = info();
        std::pair<std::vector<uint32_t>, std::vector<uint32_t>> r;
        if (!i.lists) return r;
        r.first.resize(size_t(i.nlist) + 1);
        r.second.resize(i.slots);
        ctx_.check(va_ivf_get_lists(ctx_.handle(), i.lists, r.first.data(), r.second.data()), "va_ivf_get_lists");
        return r;
    }
    ~AcceleratedVectorIndex() {
        if (h_) va_index_destroy(h_);
    }
    AcceleratedVectorIndex(const AcceleratedVectorIndex&) = delete;
    AcceleratedVectorIndex& operator=(const AcceleratedVectorIndex&) = delete;
    va_index* handle() const { return h_; }
    // insert(contentsOf:): host rows -> their handles
    std::vector<uint32_t> insert(const Matrix& vectors) {
        std::vector<uint32_t> hs(vectors.rows);
        if (vectors.rows == 0) return hs;
        DeviceBuffer<float> d(ctx_, vectors.data);
        ctx_.check(va_index_insert(ctx_.handle(), h_, d.data(), vectors.rows, hs.data()), "va_index_insert");
        ctx_.synchronize();  // the staging buffer is released on return
        return hs;
    }
    uint32_t remove(const std::vector<uint32_t>& handles) {
        uint32_t n = 0;
        ctx_.check(va_index_remove(ctx_.handle(), h_, handles.data(), uint32_t(handles.size()), &n), "va_index_remove");
        return n;
    }
    void compact() { ctx_.check(va_index_compact(ctx_.handle(), h_), "va_index_compact"); }
    va_index_info info() const {
        va_index_info i{};
        ctx_.check(va_index_get_info(h_, &i), "va_index_get_info");
        return i;
    }
    uint32_t count() const { return info().count; }
    bool contains(uint32_t handle) const { return va_index_contains(h_, handle) != 0; }
    std::vector<float> vector(uint32_t handle) const {
        std::vector<float> v(info().dimension);
        ctx_.check(va_index_get_vector(ctx_.handle(), h_, handle, v.data()), "va_index_get_vector");
        return v;
    }
    // search(queries:k:): handles in SearchResult::indices (VA_SENTINEL_INDEX past the live count)
    SearchResult search(const Matrix& queries, uint32_t k) const {
        DeviceBuffer<float> q(ctx_, queries.data);
        DeviceBuffer<uint32_t> idx(ctx_, size_t(queries.rows) * k);
        DeviceBuffer<float> dist(ctx_, size_t(queries.rows) * k);
        ctx_.check(va_index_search(ctx_.handle(), h_, metric_, q.data(), queries.rows, k, idx.data(), dist.data()),
                   "va_index_search");
        return SearchResult{idx.download(), dist.download(), queries.rows, k};
    }
    // search(query:k:filter:): the k nearest vectors the filter accepts, nearest first
    template <class Filter>
    std::vector<std::pair<uint32_t, float>> search(const std::vector<float>& query, uint32_t k, Filter filter) const {
        DeviceBuffer<float> q(ctx_, query);
        std::vector<uint32_t> hs(k);
        std::vector<float> ds(k);
        uint32_t n = 0;
        auto tramp = [](uint32_t h, void* user) -> int { return (*static_cast<Filter*>(user))(h) ? 1 : 0; };
        ctx_.check(va_index_search_filtered(ctx_.handle(), h_, metric_, q.data(), k, tramp, &filter, hs.data(),
                                            ds.data(), &n, nullptr),
                   "va_index_search_filtered");
        std::vector<std::pair<uint32_t, float>> r;
        for (uint32_t i = 0; i < n; ++i) r.emplace_back(hs[i], ds[i]);
        return r;
    }

   private:
    const Context& ctx_;
    va_metric metric_;
    va_index* h_ = nullptr;
};

class TopKSelectionKernel {
   public:
    explicit TopKSelectionKernel(const Context& c) : ctx_(c) {}
    SearchResult select(const std::vector<float>& values, uint32_t rows, uint32_t n, uint32_t k,
                        va_select_mode mode = VA_SELECT_MIN) const {
        DeviceBuffer<float> v(ctx_, values);
        DeviceBuffer<uint32_t> idx(ctx_, size_t(rows) * k);
        DeviceBuffer<float> out(ctx_, size_t(rows) * k);
        ctx_.check(va_topk_select(ctx_.handle(), v.data(), rows, n, k, mode, idx.data(), out.data()), "va_topk_select");
        return SearchResult{idx.download(), out.download(), rows, k};
    }

   private:
    const Context& ctx_;
};

// Per-dimension int8 scalar quantization and the int8 dot-product top-k scan.
class ScalarQuantizationKernel {
   public:
    explicit ScalarQuantizationKernel(const Context& c) : ctx_(c) {}
    struct Params {
        DeviceBuffer<float> min, max, scale;
        DeviceBuffer<int32_t> zeroPoint;
    };
    Params computeParameters(const DeviceBuffer<float>& x, uint32_t N, uint32_t D) const {
        Params p{DeviceBuffer<float>(ctx_, D), DeviceBuffer<float>(ctx_, D), DeviceBuffer<float>(ctx_, D),
                 DeviceBuffer<int32_t>(ctx_, D)};
        ctx_.check(va_sq_params_per_dim(ctx_.handle(), x.data(), N, D, p.min.data(), p.max.data(), p.scale.data(),
                                        p.zeroPoint.data()),
                   "va_sq_params_per_dim");
        return p;
    }
    DeviceBuffer<int8_t> quantize(const DeviceBuffer<float>& x, uint64_t N, uint32_t D, const Params& p) const {
        DeviceBuffer<int8_t> codes(ctx_, size_t(N) * D);
        ctx_.check(va_sq_quantize_i8(ctx_.handle(), x.data(), N, D, p.scale.data(), p.zeroPoint.data(), codes.data()),
                   "va_sq_quantize_i8");
        return codes;
    }
    // top-k by largest int8 dot product: (ids, dots)
    std::pair<std::vector<uint32_t>, std::vector<int32_t>> scan(const DeviceBuffer<int8_t>& q, const DeviceBuffer<int8_t>& x,
                                                                uint32_t Q, uint32_t N, uint32_t D, uint32_t k) const {
        DeviceBuffer<uint32_t> idx(ctx_, size_t(Q) * k);
        DeviceBuffer<int32_t> dot(ctx_, size_t(Q) * k);
        ctx_.check(va_i8_scan_topk(ctx_.handle(), q.data(), x.data(), Q, N, D, k, idx.data(), dot.data()),
                   "va_i8_scan_topk");
        return {idx.download(), dot.download()};
    }

   private:
    const Context& ctx_;
};

// Binary codes (bit d = x_d > 0, LSB first) and the Hamming top-k.
class BinaryQuantizationKernel {
   public:
    explicit BinaryQuantizationKernel(const Context& c) : ctx_(c) {}
    static uint32_t words(uint32_t D) { return (D + 31) / 32; }
    DeviceBuffer<uint32_t> quantize(const DeviceBuffer<float>& x, uint32_t N, uint32_t D) const {
        DeviceBuffer<uint32_t> codes(ctx_, size_t(N) * words(D));
        ctx_.check(va_bq_pack(ctx_.handle(), x.data(), N, D, codes.data()), "va_bq_pack");
        return codes;
    }
    std::pair<std::vector<uint32_t>, std::vector<uint32_t>> hammingTopK(const DeviceBuffer<uint32_t>& q,
                                                                      const DeviceBuffer<uint32_t>& x, uint32_t Q,
                                                                      uint32_t N, uint32_t W, uint32_t k) const {
        DeviceBuffer<uint32_t> idx(ctx_, size_t(Q) * k), dist(ctx_, size_t(Q) * k);
        ctx_.check(va_hamming_topk(ctx_.handle(), q.data(), x.data(), Q, N, W, k, idx.data(), dist.data()),
                   "va_hamming_topk");
        return {idx.download(), dist.download()};
    }

   private:
    const Context& ctx_;
};

// IVF-Flat (L2^2): build from centroids, add rows, probe + list scan.
class IVFIndex {
   public:
    IVFIndex(const Context& c, const DeviceBuffer<float>& centroids, uint32_t C, const DeviceBuffer<float>& x, uint32_t N,
             uint32_t D, uint32_t nprobe)
        : ctx_(c), D_(D), N_(N), nprobe_(nprobe) {
        ctx_.check(va_ivf_build(c.handle(), centroids.data(), C, x.data(), N, D, &h_), "va_ivf_build");
    }
    ~IVFIndex() {
        if (h_) va_ivf_destroy(h_);
    }
    IVFIndex(const IVFIndex&) = delete;
    IVFIndex& operator=(const IVFIndex&) = delete;
    void add(const DeviceBuffer<float>& x, uint32_t n) {
        ctx_.check(va_ivf_add(ctx_.handle(), h_, x.data(), n, D_, N_), "va_ivf_add");
        N_ += n;
    }
    SearchResult search(const DeviceBuffer<float>& q, uint32_t Q, uint32_t k) const {
        DeviceBuffer<uint32_t> idx(ctx_, size_t(Q) * k);
        DeviceBuffer<float> dist(ctx_, size_t(Q) * k);
        ctx_.check(va_ivf_search(ctx_.handle(), h_, q.data(), Q, nprobe_, k, idx.data(), dist.data()), "va_ivf_search");
        return SearchResult{idx.download(), dist.download(), Q, k};
    }
    uint32_t count() const { return N_; }

   private:
    const Context& ctx_;
    va_ivf* h_ = nullptr;
    uint32_t D_, N_, nprobe_;
};

// Lloyd k-means (KMeansConfiguration defaults: 100 iterations, threshold 1e-4).
class KMeansPipeline {
   public:
    struct Result {
        std::vector<float> centroids;
        std::vector<uint32_t> assignments, clusterCounts;
        va_kmeans_info info{};
    };
    KMeansPipeline(const Context& c, uint32_t numClusters, uint32_t maxIterations = 100,
                   float convergenceThreshold = 1e-4f, uint64_t seed = 0x5EED)
        : ctx_(c), C_(numClusters), iters_(maxIterations), thr_(convergenceThreshold), seed_(seed) {}
    // initialCentroids empty: k-means++ seeding
    Result fit(const DeviceBuffer<float>& x, uint32_t N, uint32_t D, const std::vector<float>& initialCentroids = {}) const {
        DeviceBuffer<float> init(ctx_, size_t(C_) * D);
        if (initialCentroids.empty())
            ctx_.check(va_kmeans_plusplus(ctx_.handle(), x.data(), N, D, C_, seed_, init.data(), nullptr),
                       "va_kmeans_plusplus");
        else
            init.upload(initialCentroids);
        DeviceBuffer<float> cen(ctx_, size_t(C_) * D);
        DeviceBuffer<uint32_t> assign(ctx_, N), counts(ctx_, C_);
        Result r;
        ctx_.check(va_kmeans_fit(ctx_.handle(), x.data(), N, D, C_, init.data(), iters_, thr_, cen.data(), assign.data(),
                                 nullptr, counts.data(), &r.info),
                   "va_kmeans_fit");
        r.centroids = cen.download();
        r.assignments = assign.download();
        r.clusterCounts = counts.download();
        return r;
    }

   private:
    const Context& ctx_;
    uint32_t C_, iters_;
    float thr_;
    uint64_t seed_;
};

// Product quantization (Metal4PQConfig defaults: M 8, K 256, 25 iterations, threshold 0.001).
class ProductQuantizationKernel {
   public:
    struct Config {
        uint32_t dimension, M = 8, K = 256, trainIterations = 25;
        float convergenceThreshold = 0.001f;
    };
    ProductQuantizationKernel(const Context& c, Config cfg) : ctx_(c), cfg_(cfg) {
        if (cfg.M == 0 || cfg.dimension % cfg.M != 0)
            throw VectorError(VA_ERR_INVALID_ARG, "Dimension must be divisible by M");
        if (cfg.K == 0 || cfg.K > 256) throw VectorError(VA_ERR_INVALID_ARG, "K must be <= 256 for uint8 encoding");
    }
    DeviceBuffer<float> train(const DeviceBuffer<float>& x, uint32_t N, uint64_t seed = 0x5EED) const {
        DeviceBuffer<float> cb(ctx_, size_t(cfg_.M) * cfg_.K * (cfg_.dimension / cfg_.M));
        uint32_t it = 0;
        ctx_.check(va_pq_train(ctx_.handle(), x.data(), N, cfg_.dimension, cfg_.M, cfg_.K, cfg_.trainIterations,
                               cfg_.convergenceThreshold, seed, nullptr, cb.data(), &it),
                   "va_pq_train");
        return cb;
    }
    DeviceBuffer<uint8_t> encode(const DeviceBuffer<float>& x, uint32_t N, const DeviceBuffer<float>& cb) const {
        DeviceBuffer<uint8_t> codes(ctx_, size_t(N) * cfg_.M);
        ctx_.check(va_pq_encode(ctx_.handle(), x.data(), N, cfg_.dimension, cfg_.M, cfg_.K, cb.data(), codes.data()),
                   "va_pq_encode");
        return codes;
    }
    SearchResult search(const DeviceBuffer<float>& q, uint32_t Q, const DeviceBuffer<float>& cb,
                        const DeviceBuffer<uint8_t>& codes, uint32_t N, uint32_t k) const {
        DeviceBuffer<uint32_t> idx(ctx_, size_t(Q) * k);
        DeviceBuffer<float> dist(ctx_, size_t(Q) * k);
        ctx_.check(va_pq_search(ctx_.handle(), q.data(), Q, cfg_.dimension, cfg_.M, cfg_.K, cb.data(), codes.data(), N,
                                k, idx.data(), dist.data()),
                   "va_pq_search");
        return SearchResult{idx.download(), dist.download(), Q, k};
    }

   private:
    const Context& ctx_;
    Config cfg_;
};

}  // namespace vectoraccelerate

#endif /* VECTORACCELERATE_HPP */
