/*
 * va_oracle.h — CPU oracle for the flat/IVF search path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker, never the product: only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it.  The product
 * path (libva_hip.so) never links, calls or falls back to it.
 *
 * It restates, in plain C, the CPU semantics of gifton/VectorAccelerate 0.5.0
 * (Swift + Metal; the reference cannot be built on Linux, so there is no
 * oracle/_ref build).  Each function cites the reference file:line it follows.
 *
 * Conventions shared with the GPU library:
 *   - missing results: index 0xFFFFFFFF, distance +inf (int paths: INT32_MAX / 0xFFFFFFFF);
 *   - top-K order: (distance ascending, index ascending) everywhere
 *     (Metal4Common.h:142-159, AdvancedTopK.metal:48-52);
 *   - a NaN distance orders after +inf (it is treated as the largest key).
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   fp distances        closed forms + numpy/scipy float64 on small inputs + reference KATs
 *   top-K               numpy lexsort on small inputs + reference KATs
 *   int8 params/codes   closed form on hand-made inputs + numpy re-derivation
 *   int8 top-K          numpy int64 matmul + lexsort
 *   binary pack/hamming reference KATs (packBinary, hamming 0/4/2) + numpy unpackbits
 *   IVF                 brute-force numpy re-derivation on small inputs
 */
#ifndef VA_ORACLE_H
#define VA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* metric codes (same values as VA_METRIC_* in include/va_hip.h) */
enum {
    VO_METRIC_L2SQ = 0,   /* sum (q-x)^2                                     */
    VO_METRIC_COSINE = 1, /* 1 - clamp(dot / (|q||x|)), 0 similarity if |q||x| < FLT_MIN */
    VO_METRIC_DOT = 2,    /* -dot  (ascending order = maximum inner product) */
    VO_METRIC_L2 = 3      /* sqrt(sum (q-x)^2)                               */
};

int vo_version(void);
int vo_num_threads(void);

/* ---- distances ---------------------------------------------------------- */
/* 1:1 pairs, L2DistanceKernel / l2_distance (DistanceShaders.metal:169-226). */
void vo_l2_pairs(const float* q, const float* t, int64_t P, int64_t D, int compute_sqrt, float* out);
/* 1:1 pairs, cosine_similarity (DistanceShaders.metal:239-321). */
void vo_cosine_pairs(const float* q, const float* t, int64_t P, int64_t D, int output_distance, float* out);
/* All-pairs matrices, out[Q x N] row-major.
 *   kind 0: L2^2, 1: L2, 2: cosine similarity, 3: cosine distance, 4: dot, 5: |dot|.
 * l2_distance_kernel (L2Distance.metal:34-91), dot_product_kernel (DotProduct.metal:29-96),
 * AccelerateFallback.batchCosineSimilarity (AccelerateFallback.swift:209-237). */
void vo_distance_matrix(int kind, const float* q, const float* x, int64_t Q, int64_t N, int64_t D, float* out);
/* Single (query, row) distance in double, metric as VO_METRIC_*. */
double vo_distance(int metric, const float* q, const float* x, int64_t D);

/* ---- top-K -------------------------------------------------------------- */
/* Row-wise top-k of a value matrix (TopKSelectionKernel, SearchAndRetrieval.metal:88-156),
 * with the (value, index) tie rule.  mode 0 = minimum, 1 = maximum (value desc, index asc).
 * Missing slots (k > N) get index 0xFFFFFFFF and value +inf (min) / -inf (max). */
void vo_topk_rows(const float* in, int64_t Q, int64_t N, int64_t k, int mode, uint32_t* idx, float* val);
/* Flat exact top-k: CPUTopK.search (CPU/CPUTopK.swift:34-84) generalised to the three
 * metrics.  accum_double=1 accumulates in double (the parity oracle); 0 accumulates in
 * float with eight partial sums like vDSP_distancesq / vDSP_dotpr (the CPU baseline port). */
void vo_flat_topk(int metric, const float* q, const float* x, int64_t Q, int64_t N, int64_t D,
                  int64_t k, int accum_double, uint32_t* idx, float* dist);
/* Merge two sorted top-k lists; b indices are offset by chunk_base
 * (merge_topk_sorted_kernel, SearchAndRetrieval.metal:320-385). */
void vo_topk_merge(const uint32_t* a_idx, const float* a_d, const uint32_t* b_idx, const float* b_d,
                   int64_t Q, int64_t k, uint32_t chunk_base, uint32_t* out_idx, float* out_d);

/* ---- scalar int8 quantization ------------------------------------------- */
/* Per-dimension affine parameters over a row-major [N x D] matrix.
 *   mn/mx = per-dimension min/max; scale = max((mx-mn)/255, 1e-8)
 *   (ScalarQuantizationKernel.swift:496-520, asymmetric branch);
 *   zp = -128 - round_half_away(mn/scale) as int32, so that codes span [-128, 127]
 *   (the reference's Int8(clamping:) zero point saturates: with a range of 255 steps an Int8
 *   zero point cannot place min at -128 for every data range). */
void vo_sq_params_per_dim(const float* x, int64_t N, int64_t D, float* mn, float* mx, float* scale, int32_t* zp);
/* q = clamp(rint(x/scale + zp), -128, 127); |scale| < 1e-9 -> clamp(zp)
 * (quantize_int8_kernel, DataTransformations.metal:174-201), per dimension d = i % D. */
/* The global (one scale for all values) int8 parameters of ScalarQuantizationKernel.quantize:
 * computeQuantizationParams, Kernels/Metal4/ScalarQuantizationKernel.swift:496-520 (int8 branch;
 * symmetric: zero_point 0; asymmetric: the saturating Int8 zero point). */
void vo_sq_global_params(const float* x, int64_t n, int asymmetric, float* scale, int32_t* zero_point);
void vo_sq_quantize(const float* x, int64_t N, int64_t D, const float* scale, const int32_t* zp, int8_t* codes);
/* x = (q - zp) * scale (dequantize_int8_kernel, DataTransformations.metal:203-221). */
void vo_sq_dequantize(const int8_t* codes, int64_t N, int64_t D, const float* scale, const int32_t* zp, float* out);
/* Exact int32 dot of int8 codes; distance = -dot; top-k by (distance, index). */
void vo_i8_topk(const int8_t* qc, const int8_t* xc, int64_t Q, int64_t N, int64_t D, int64_t k,
                uint32_t* idx, int32_t* dist);
void vo_i8_dot_matrix(const int8_t* qc, const int8_t* xc, int64_t Q, int64_t N, int64_t D, int32_t* out);

/* ---- binary quantization ------------------------------------------------ */
/* bit d = (x_d > 0.0f), word w bit b = dimension 32w+b (binaryQuantize,
 * QuantizationShaders.metal:132-160; Metal4BinaryVector, BinaryQuantizationKernel.swift:23-75). */
void vo_bq_pack(const float* x, int64_t N, int64_t D, uint32_t* codes);
/* sum popcount(q ^ x) (Metal4BinaryVector.hammingDistance, BinaryQuantizationKernel.swift:65-74). */
void vo_hamming_matrix(const uint32_t* q, const uint32_t* x, int64_t Q, int64_t N, int64_t W, uint32_t* out);
/* top-k of Hamming distances, stable (ties -> lower index)
 * (Metal4HammingResult.nearestNeighbors, HammingDistanceKernel.swift:114-120). */
void vo_hamming_topk(const uint32_t* q, const uint32_t* x, int64_t Q, int64_t N, int64_t W, int64_t k,
                     uint32_t* idx, uint32_t* dist);

/* ---- IVF ------------------------------------------------------------------ */
/* Nearest centroid by L2^2, strict < so ties go to the lowest centroid id
 * (IVFStructure.findNearestCentroid, IVFStructure.swift:292-307). */
void vo_ivf_assign(const float* x, int64_t N, const float* c, int64_t C, int64_t D, int32_t* list);
/* CSR in centroid order, entries in insertion (row) order (IVFStructure.swift:370-381).
 * offsets[C+1], ids[N]. */
void vo_ivf_csr(const int32_t* list, int64_t N, int64_t C, uint32_t* offsets, uint32_t* ids);
/* Coarse probe: nprobe nearest centroids by (L2^2, id) (IVFCoarseQuantizerKernel.swift:133-174). */
void vo_ivf_probe(const float* q, int64_t Q, const float* c, int64_t C, int64_t D, int64_t nprobe, uint32_t* probes);
/* List scan over given probes + exact top-k by (L2^2, id) over the original row ids
 * (ivf_list_search, IVFListSearch.metal:247-338; exact for every k). */
void vo_ivf_scan(const float* q, int64_t Q, const float* x, int64_t D, const uint32_t* offsets, const uint32_t* ids,
                 int64_t C, const uint32_t* probes, int64_t nprobe, int64_t k, uint32_t* idx, float* dist);

/* ---- k-means (IVF centroid training) ------------------------------------------ */
/* Lloyd k-means (KMeansPipeline.fit, Index/Kernels/Clustering/KMeansPipeline.swift:102-270):
 * assignment = argmin_c sum_d (x_d - c_d)^2 in float, d in order, strict < (lowest centroid
 * wins ties), distance = sqrt (kmeans_assign_points, ClusteringShaders.metal:16-120);
 * centroid = (float sum) * (1/count), the sum taken over chunks of 256 of its points in point
 * order, chunk sums added in order (the reference's float atomics fix no order), empty keeps the old one
 * (kmeans_update_normalize, ClusteringShaders.metal:585-613); each empty cluster, in index
 * order, takes the unused point of largest distance, first index on ties, count = 1
 * (KMeansUpdateKernel.handleEmptyClusters, KMeansUpdateKernel.swift:228-283); converged when
 * max_c sqrt(sum_d (new - old)^2) < threshold (KMeansConvergenceKernel.swift:76-127); inertia =
 * float sum of the distances in point order (KMeansConvergenceKernel.swift:176-182).
 * info_u32 = {iterations, converged}; info_f = {inertia, max_movement}. */
void vo_kmeans_fit(const float* x, int64_t N, int64_t D, int64_t C, const float* init, int64_t max_iter,
                   float threshold, float* centroids, uint32_t* assign, float* dist, uint32_t* counts,
                   uint32_t* info_u32, float* info_f);
/* k-means++ seeding (KMeansPlusPlusKernel.selectCentroids, KMeansPlusPlusKernel.swift:94-203):
 * u_j = (splitmix64(seed) >> 11) * 2^-53 for j = 0..k-1; first = floor(u_0 * N); then
 * min squared distance (compute_min_distances, ClusteringShaders.metal:419-447; summed as 64
 * strided fmaf partials combined pairwise, the device's order),
 * total = double sum over unselected points, pick the first unselected i whose cumulative
 * double sum reaches u_j * total (the first unselected point when total is 0). */
/* One k-means update given an assignment (and the distances handleEmptyClusters ranks by):
 * the update step of vo_kmeans_fit (KMeansUpdateKernel, ClusteringShaders.metal:490-613;
 * KMeansUpdateKernel.swift:228-283).  out_centroids [C x D], counts [C]. */
void vo_kmeans_update(const float* x, int64_t N, int64_t D, int64_t C, const uint32_t* assign, const float* dist,
                      const float* old_centroids, float* out_centroids, uint32_t* counts);
void vo_kmeans_plusplus(const float* x, int64_t N, int64_t D, int64_t k, uint64_t seed, uint32_t* idx);

/* ---- product quantization --------------------------------------------------- */
/* |v - c|^2 over n values in calculate_l2_sq_dist's order (ProductQuantization.metal:30-58):
 * four lanes fmaf over the float4 blocks, ((x + y) + z) + w, then the tail one by one. */
float vo_pq_sub_l2sq(const float* v, const float* c, int64_t n);
/* codes[n*M + m] = argmin_k (strict <) (pq_assignment_or_encoding, ProductQuantization.metal:61-101). */
void vo_pq_encode(const float* x, int64_t N, int64_t D, int64_t M, int64_t K, const float* cb, uint8_t* codes);
/* tables[q][m][k] (pq_precompute_distance_table, ProductQuantization.metal:191-213). */
void vo_pq_tables(const float* q, int64_t Q, int64_t D, int64_t M, int64_t K, const float* cb, float* tables);
/* out[q][n] = sum_m tables[q][m][code] in m order (pq_compute_distances_adc, :215-254). */
void vo_pq_adc(const float* tables, int64_t Q, const uint8_t* codes, int64_t N, int64_t M, int64_t K, float* out);
/* top-k by (ADC sum, row id), distances sqrt(sum) (findNearestNeighbors,
 * ProductQuantizationKernel.swift:504-540, with a deterministic tie rule). */
void vo_pq_search(const float* q, int64_t Q, int64_t D, int64_t M, int64_t K, const float* cb, const uint8_t* codes,
                  int64_t N, int64_t k, uint32_t* idx, float* dist);
/* Lloyd training from cb (updated in place), ProductQuantizationKernel.train (:260-369):
 * assignment, then per (m, k) the mean of its members (sums over chunks of 256 members in point
 * order, chunk sums added in order; the reference's float atomics fix no order), empty keeps its
 * value; movement_sq = sum_d (old - new)^2; stop after the round where
 * sqrt(sum movement_sq / (M K)) < threshold.  Returns the rounds run. */
int64_t vo_pq_train(const float* x, int64_t N, int64_t D, int64_t M, int64_t K, int64_t iterations, float threshold,
                    float* cb);

#ifdef __cplusplus
}
#endif
#endif
