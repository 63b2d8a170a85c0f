// C++ host-mirror check (include/vectoraccelerate.hpp): runs each class on inputs read from a
// directory and writes the outputs there as raw little-endian arrays; tests/test_gpu_cpp.py
// compares them with the CPU oracle.  Usage: va_example DIR Q N D C k nprobe
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

#include "vectoraccelerate.hpp"

namespace va = vectoraccelerate;

template <class T>
static std::vector<T> load(const std::string& path, size_t n) {
    std::vector<T> v(n);
    std::ifstream f(path, std::ios::binary);
    if (!f.read(reinterpret_cast<char*>(v.data()), std::streamsize(n * sizeof(T)))) {
        std::fprintf(stderr, "cannot read %s\n", path.c_str());
        std::exit(2);
    }
    return v;
}

template <class T>
static void save(const std::string& path, const std::vector<T>& v) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), std::streamsize(v.size() * sizeof(T)));
}

int main(int argc, char** argv) {
    if (argc != 8) {
        std::fprintf(stderr, "usage: %s DIR Q N D C k nprobe\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const uint32_t Q = std::atoi(argv[2]), N = std::atoi(argv[3]), D = std::atoi(argv[4]), C = std::atoi(argv[5]),
                   k = std::atoi(argv[6]), nprobe = std::atoi(argv[7]);
    try {
        va::Context ctx(0);
        va::Matrix q{load<float>(dir + "/q.bin", size_t(Q) * D), Q, D};
        va::Matrix x{load<float>(dir + "/x.bin", size_t(N) * D), N, D};
        std::vector<float> cen = load<float>(dir + "/c.bin", size_t(C) * D);

        va::FusedL2TopKKernel topk(ctx);
        va::SearchResult l2 = topk.findNearestNeighbors(q, x, k, VA_METRIC_L2SQ);
        save(dir + "/l2_idx.bin", l2.indices);
        save(dir + "/l2_dist.bin", l2.distances);
        va::SearchResult cs = topk.findNearestNeighbors(q, x, k, VA_METRIC_COSINE);
        save(dir + "/cos_idx.bin", cs.indices);

        va::DeviceBuffer<float> xd(ctx, x.data), qd(ctx, q.data), cd(ctx, cen);
        const uint32_t half = N / 2;
        std::vector<float> first(x.data.begin(), x.data.begin() + size_t(half) * D);
        std::vector<float> rest(x.data.begin() + size_t(half) * D, x.data.end());
        va::DeviceBuffer<float> x0(ctx, first), x1(ctx, rest);
        va::IVFIndex ivf(ctx, cd, C, x0, half, D, nprobe);
        ivf.add(x1, N - half);
        va::SearchResult iv = ivf.search(qd, Q, k);
        save(dir + "/ivf_idx.bin", iv.indices);

        va::KMeansPipeline km(ctx, C, 5, 0.0f);
        va::KMeansPipeline::Result kr = km.fit(xd, N, D, cen);
        save(dir + "/km_cen.bin", kr.centroids);
        save(dir + "/km_assign.bin", kr.assignments);

        va::ProductQuantizationKernel pq(ctx, {D, 4, 16, 5, 0.0f});
        va::DeviceBuffer<float> cb = pq.train(xd, N, 11);
        va::DeviceBuffer<uint8_t> codes = pq.encode(xd, N, cb);
        va::SearchResult pr = pq.search(qd, Q, cb, codes, N, k);
        save(dir + "/pq_cb.bin", cb.download());
        save(dir + "/pq_codes.bin", codes.download());
        save(dir + "/pq_idx.bin", pr.indices);

        // MetalComputeProvider: distances of query 0 and the nearest candidates of every query
        va::MetalComputeProvider prov(ctx);
        std::vector<float> q0(q.data.begin(), q.data.begin() + D);
        save(dir + "/prov_l2.bin", prov.batchDistance(q0, x, va::MetalComputeProvider::Metric::euclidean));
        save(dir + "/prov_cos.bin", prov.batchDistance(q0, x, va::MetalComputeProvider::Metric::cosine));
        save(dir + "/prov_dot.bin", prov.batchDistance(q0, x, va::MetalComputeProvider::Metric::dotProduct));
        std::vector<uint32_t> nn;
        std::vector<float> nd;
        for (auto m : {va::MetalComputeProvider::Metric::euclidean, va::MetalComputeProvider::Metric::cosine,
                       va::MetalComputeProvider::Metric::dotProduct})
            for (auto& row : prov.findNearestBatch(q, x, k, m))
                for (auto& p : row) {
                    nn.push_back(p.first);
                    nd.push_back(p.second);
                }
        save(dir + "/prov_nn_idx.bin", nn);
        save(dir + "/prov_nn_dist.bin", nd);

        // AcceleratedVectorIndex: handles, removal of every 7th vector, search, filtered search
        va::AcceleratedVectorIndex index(ctx, D, 16);
        std::vector<uint32_t> hs = index.insert(x);
        std::vector<uint32_t> gone;
        for (uint32_t i = 0; i < N; i += 7) gone.push_back(hs[i]);
        const uint32_t removed = index.remove(gone);
        va::SearchResult ir = index.search(q, k);
        save(dir + "/index_idx.bin", ir.indices);
        auto odd = [](uint32_t h) { return (h & 1u) == 1u; };
        std::vector<uint32_t> fi;
        for (auto& p : index.search(q0, k, odd)) fi.push_back(p.first);
        save(dir + "/index_filtered_idx.bin", fi);
        index.compact();
        std::ofstream(dir + "/index_counts.txt") << removed << " " << index.count() << " " << index.contains(hs[0])
                                                 << " " << index.contains(hs[1]);

        // AcceleratedVectorIndex (IVF): half the vectors, train with the given centroids, the other
        // half joins the lists, every 5th vector removed, then batch search through the lists
        va::AcceleratedVectorIndex ivx(ctx, D, va::IVFConfiguration{C, nprobe, 0}, 64);
        va::Matrix xa{first, half, D}, xb{rest, N - half, D};
        ivx.insert(xa);
        ivx.train(cen);
        ivx.insert(xb);
        std::vector<uint32_t> gone5;
        for (uint32_t i = 0; i < N; i += 5) gone5.push_back(i);
        ivx.remove(gone5);
        va::SearchResult vr = ivx.search(q, k);
        save(dir + "/ivx_idx.bin", vr.indices);
        save(dir + "/ivx_dist.bin", vr.distances);
        auto lists = ivx.lists();
        save(dir + "/ivx_off.bin", lists.first);
        save(dir + "/ivx_ids.bin", lists.second);
        std::ofstream(dir + "/ivx_state.txt") << ivx.isTrained() << " " << ivx.info().ivf_routed << " " << ivx.count();

        std::string kind = "none";
        try {
            topk.findNearestNeighbors(q, x, 0);
        } catch (const va::VectorError& e) {
            kind = e.kind();
        }
        std::ofstream(dir + "/error_kind.txt") << kind;
    } catch (const va::VectorError& e) {
        std::fprintf(stderr, "VectorError(%s): %s\n", e.kind(), e.what());
        return 1;
    }
    std::printf("va_example: ok\n");
    return 0;
}
