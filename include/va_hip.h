/*
 * va_hip.h — C ABI of the MI355X (gfx950) flat/IVF vector-search library (libva_hip.so).
 *
 * This is the drop-in boundary that replaces gifton/VectorAccelerate's Metal path.
 * Every entry point names the reference interface it replaces
 * (paths relative to the reference's Sources/VectorAccelerate/).
 *
 * Conventions
 *  - Plain C: opaque handles, device pointers, sizes, int status.  No C++/torch types.
 *  - All compute entry points take DEVICE pointers (caller-owned, the reference's
 *    encode(into:) tier, KernelProtocol.swift:42-63) and enqueue on the context's
 *    stream.  They return once the work is enqueued unless stated otherwise; call
 *    va_context_synchronize() before reading results on the host (the reference's
 *    executeAndWait, Core/Metal4Context.swift:342-410).  The top-k searches
 *    (va_fused_topk, va_i8_scan_topk, va_hamming_topk, va_pq_search, va_ivf_search,
 *    va_ivf_scan, va_index_search) never wait on the host: queries whose candidate list
 *    overflows are
 *    finished on the device by a fallback whose launches exit at once when nothing
 *    overflowed, so searches can be queued back to back on one stream.  A call that has to
 *    grow the context's scratch arena waits for the stream once, before the growth.
 *  - A context is externally synchronised: one caller at a time per context (the
 *    reference's actor contract).  Different contexts may be used concurrently.
 *  - Missing results use index VA_SENTINEL_INDEX (0xFFFFFFFF) and distance +inf
 *    (int32 paths: INT32_MAX; Hamming: 0xFFFFFFFF), as FusedL2TopKKernel.swift:166 and
 *    IVFKernels.swift:269-287 skip them.
 *  - Top-K order everywhere: (distance ascending, index ascending); MAX mode orders
 *    (value descending, index ascending).  NaN orders after every number.
 *  - Row-major matrices; counts are uint32 (indices must fit below 0xFFFFFFFF).
 */
#ifndef VA_HIP_H
#define VA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VA_HIP_ABI_VERSION 5
#define VA_SENTINEL_INDEX 0xFFFFFFFFu
/* largest k accepted by the top-K entry points */
#define VA_MAX_K 1024u

/* Status codes.  Mirror VectorError / IndexError (VectorCore; Index/Types/IndexError.swift):
 * INVALID_ARG ~ invalidInput, DIMENSION_MISMATCH ~ dimensionMismatch,
 * OOM ~ bufferAllocationFailed, HIP ~ computeFailed. */
typedef enum {
    VA_OK = 0,
    VA_ERR_INVALID_ARG = 1,
    VA_ERR_DIMENSION_MISMATCH = 2,
    VA_ERR_OOM = 3,
    VA_ERR_HIP = 4,
    VA_ERR_UNSUPPORTED = 5
} va_status;

/* Distance metrics.  L2SQ is the index's native distance (FlatIndexSearchTests.swift:577-595);
 * COSINE = 1 - similarity (MetalComputeProvider.swift:136); DOT = -dot (maximum inner product
 * as an ascending distance, MetalComputeProvider.swift:221-225); L2 = sqrt(L2SQ). */
typedef enum { VA_METRIC_L2SQ = 0, VA_METRIC_COSINE = 1, VA_METRIC_DOT = 2, VA_METRIC_L2 = 3 } va_metric;

/* Metal4SelectionMode (Kernels/Metal4/TopKSelectionKernel.swift:23-29) */
typedef enum { VA_SELECT_MIN = 0, VA_SELECT_MAX = 1 } va_select_mode;

typedef struct va_context va_context;
typedef struct va_ivf va_ivf;

int va_abi_version(void);
const char* va_status_string(va_status status);

/* ---- context: replaces Metal4Context / GPUContext (VectorAccelerate.swift:254;
 *      Core/Metal4Context.swift:183-269) ------------------------------------- */
/* Create a context on HIP device `device` with its own stream. */
va_status va_context_create(int device, va_context** out);
/* Create a context that enqueues on a caller-owned hipStream_t (passed as void*). */
va_status va_context_create_with_stream(int device, void* hip_stream, va_context** out);
va_status va_context_destroy(va_context* ctx);
/* The hipStream_t the context enqueues on. */
void* va_context_stream(va_context* ctx);
int va_context_device(const va_context* ctx);
/* executeAndWait: block until all work enqueued on the context has finished. */
va_status va_context_synchronize(va_context* ctx);
/* Text of the last error on this context ("" when none). */
const char* va_last_error_message(const va_context* ctx);

/* Tuning overrides of the exact top-k scan (0 restores the automatic choice).  They play the
 * role of Metal4FusedL2Config's maxDistanceMatrixBytes / enableChunkedFallback
 * (Kernels/Metal4/FusedL2TopKKernel.swift:91-136): CANDIDATE_CAP bounds the per-query
 * candidate list (rows that overflow it take the exact chunked path), SAMPLE_ROWS sets the
 * size of the threshold sample (>= num_database forces the dense path).  SCREEN selects the
 * filtering scan of va_fused_topk: 0 = automatic (fp16 screening pass with an exact fp32
 * rerank wherever it applies), 1 = never screen (fp32 scan only), 2 = screen whenever the
 * metric and layout allow it.  Screening changes no result: the ids and distances are the
 * fp32 scan's, bit for bit.  SAMPLE_RANK sets which order statistic of the sample becomes a
 * query's filter threshold: rank k always leaves at least k candidates; a smaller rank r
 * filters far fewer rows, and a query left with fewer than k candidates takes the exact
 * fallback, so results do not change.  0 = automatic: the smallest r for which, with the
 * sample drawn at random, the chance that r of the k nearest rows fall in it (which is what
 * leaves fewer than k candidates) is below 1e-4; r = k when a deletion mask is in use.
 * Values >= k give rank k. */
typedef enum {
    VA_OPT_CANDIDATE_CAP = 1,
    VA_OPT_SAMPLE_ROWS = 2,
    VA_OPT_SCREEN = 3,
    VA_OPT_SAMPLE_RANK = 4
} va_option;
va_status va_context_set_option(va_context* ctx, va_option option, uint64_t value);

/* Phase timings of the top-k scans, from hipEvents on the context stream.  Replaces
 * Metal4Configuration.enableProfiling + GPUTimingInfo (Core/Metal4Context.swift:17,48-64,389-404)
 * and IVFPhaseTimings (Index/Kernels/IVF/IVFKernels.swift:295).  With profiling on, a scan
 * records its events (and copies its overflow / rerank counts) without waiting; the events are
 * read when va_context_last_scan or va_context_scan_totals is called, or when the record is
 * reused 16 scans later.  va_context_set_profiling: enable 0 off, 1 every phase (five events, the
 * counts), 2 the scan phase alone (its two events, no counts: scan_ms is set, the other phase
 * times and counts read 0), for timing loops that should carry as little as possible. */
typedef struct {
    float sample_ms;        /* threshold sample: dense keys + k-th selection          */
    float scan_ms;          /* the filtering scan kernel (the dominant kernel)         */
    float select_ms;        /* candidate-list selection                               */
    float fallback_ms;      /* exact recomputation of overflowed rows (0 when none)   */
    float total_ms;         /* whole scan                                             */
    uint32_t sample_rows;   /* 0 when the dense path ran                              */
    uint32_t candidate_cap; /* per-query candidate capacity                            */
    uint32_t overflow_rows; /* queries that took the exact chunked path               */
    uint32_t scan_launches; /* number of scan-kernel launches timed in scan_ms        */
    uint32_t screened;      /* fp16 screening scan of an fp32 search: 0 none, 1 over   
                             * converted fp32 rows (flat) or the IVF list shadow, 2 over
                             * the native index's fp16 shadow (screen16_kernel)        */
    uint32_t rerank_rows;   /* screened search: rows re-scored exactly, all queries   */
} va_scan_timings;
va_status va_context_set_profiling(va_context* ctx, int enable);
/* The last profiled scan (waits for its events). */
va_status va_context_last_scan(va_context* ctx, va_scan_timings* out);
/* Phase times and counts summed over the profiled scans since the last reset (waits for their
 * events); *count = the number of scans.  No reference counterpart: averaging a timed loop
 * without reading events inside it. */
va_status va_context_scan_totals(va_context* ctx, va_scan_timings* sum, uint32_t* count);
va_status va_context_reset_scan_totals(va_context* ctx);

/* ---- buffers: replace getBuffer / BufferToken (Core/Metal4Context.swift:471-488;
 *      Core/BufferPool.swift:89-200) ------------------------------------------ */
va_status va_buffer_alloc(va_context* ctx, size_t bytes, void** device_ptr);
va_status va_buffer_free(va_context* ctx, void* device_ptr);
/* Stream-ordered copies.  Host memory must stay valid until the context is synchronised. */
va_status va_buffer_upload(va_context* ctx, void* dst_device, const void* src_host, size_t bytes);
va_status va_buffer_download(va_context* ctx, void* dst_host, const void* src_device, size_t bytes);

/* ---- distances ---------------------------------------------------------------- */
/* 1:1 pairs: out[i] = |q_i - t_i|^2 (sqrt when compute_sqrt).
 * Replaces L2DistanceKernel.encode (Kernels/Metal4/L2DistanceKernel.swift:49-86). */
va_status va_l2_pairs(va_context* ctx, const float* queries, const float* targets, float* out,
                      uint32_t num_pairs, uint32_t dim, int compute_sqrt);
/* 1:1 pairs: cosine similarity (or 1 - similarity when output_distance).
 * Replaces CosineSimilarityKernel.encode (Kernels/Metal4/CosineSimilarityKernel.swift:50-87). */
va_status va_cosine_pairs(va_context* ctx, const float* queries, const float* targets, float* out,
                          uint32_t num_pairs, uint32_t dim, int output_distance);
/* All pairs out[Q x N] = L2^2 (or L2).  Replaces the l2_distance_kernel dispatch of
 * FusedL2TopKKernel.encodeAllPairsL2 (Kernels/Metal4/FusedL2TopKKernel.swift:1111-1150). */
va_status va_l2_all_pairs(va_context* ctx, const float* queries, const float* database, float* out,
                          uint32_t num_queries, uint32_t num_database, uint32_t dim, int compute_sqrt);
/* All pairs cosine similarity (or 1 - s).  All-pairs form of CosineSimilarityKernel
 * (orphaned cosine_similarity_general_kernel, Metal/Shaders/CosineSimilarity.metal:42-565). */
va_status va_cosine_all_pairs(va_context* ctx, const float* queries, const float* database, float* out,
                              uint32_t num_queries, uint32_t num_database, uint32_t dim, int output_distance);
/* All pairs dot (|dot| when absolute_value).  Replaces DotProductKernel.encode/execute
 * (Kernels/Metal4/DotProductKernel.swift:216-305; DotProductParameters :25-96). */
va_status va_dot_all_pairs(va_context* ctx, const float* queries, const float* database, float* out,
                           uint32_t num_queries, uint32_t num_database, uint32_t dim, int absolute_value);

/* ---- top-K -------------------------------------------------------------------- */
/* Fused distance + exact top-k (the Q x N matrix is never materialised).
 * Replaces FusedL2TopKKernel.execute (Kernels/Metal4/FusedL2TopKKernel.swift:367-427) without
 * its K <= 128 / D <= 768 limits; FusedTopKKernel is its alias (VectorAccelerate.swift:288).
 * out_idx[Q x k], out_dist[Q x k] (out_dist may be NULL: includeDistances = false).
 * Returns once enqueued (no host read-back). */
va_status va_fused_topk(va_context* ctx, va_metric metric, const float* queries, const float* database,
                        uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k,
                        uint32_t* out_idx, float* out_dist);
/* The same search over a database in HOST memory (larger than HBM, or not resident): the
 * database is streamed in chunks of chunk_rows rows (0 = ~512 MiB) through two device buffers,
 * uploads on an auxiliary stream overlapping the scan of the previous chunk, and the per-chunk
 * top-k lists are merged into a running top-k (ids offset by each chunk's first row).  Results
 * equal va_fused_topk's on the same database.  host_database should be pinned (hipHostMalloc /
 * torch pin_memory) for the uploads to overlap; queries and outputs are device pointers.
 * Synchronous (returns when the outputs are complete).  Replaces FusedL2TopKKernel's chunked
 * fallback with a running GPU merge (Kernels/Metal4/FusedL2TopKKernel.swift:765-931), which on
 * Apple's unified memory reads the dataset buffer in place. */
va_status va_fused_topk_streamed(va_context* ctx, va_metric metric, const float* queries, const float* host_database,
                                 uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k,
                                 uint32_t chunk_rows, uint32_t* out_idx, float* out_dist);
/* Size of the fixed device scratch block of va_fused_topk_noalloc (one block per GPU). */
#define VA_NOALLOC_SCRATCH_BYTES (64u << 20)
/* va_fused_topk without device allocation.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as va_fused_topk, but every
 * scratch buffer comes from a fixed block of VA_NOALLOC_SCRATCH_BYTES
 * that each GPU holds until the process ends (about 128 queries x 1M rows at k = 100 fit).
 * A search that needs more fails with VA_ERR_INVALID_ARG before any work is enqueued, and the
 * message gives the size it needs.  Every call on one GPU shares that GPU's block and leaves its
 * contents behind (each call clears what it needs cleared): calls that overlap on one GPU, from
 * different contexts or streams, race.  Returns once enqueued when the device-side overflow
 * fallback's buffers fit in the block too; otherwise it reads the overflow count back (one
 * synchronisation) and finishes overflowed queries from the host. */
va_status va_fused_topk_noalloc(va_context* ctx, va_metric metric, const float* queries, const float* database,
                                uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k,
                                uint32_t* out_idx, float* out_dist);
/* Row-wise top-k of a value matrix values[Q x N] (sorted output).
 * Replaces TopKSelectionKernel.encode/execute (Kernels/Metal4/TopKSelectionKernel.swift:228-368). */
va_status va_topk_select(va_context* ctx, const float* values, uint32_t num_rows, uint32_t num_elements,
                         uint32_t k, va_select_mode mode, uint32_t* out_idx, float* out_values);
/* Merge two sorted top-k lists per row; b's indices are offset by chunk_base.
 * Replaces TopKMergeKernel / merge_topk_sorted_kernel (Metal/Shaders/SearchAndRetrieval.metal:320-385). */
va_status va_topk_merge(va_context* ctx, const uint32_t* a_idx, const float* a_dist, const uint32_t* b_idx,
                        const float* b_dist, uint32_t num_rows, uint32_t k, uint32_t chunk_base,
                        uint32_t* out_idx, float* out_dist);

/* ---- scalar int8 quantization --------------------------------------------------- */
/* Per-dimension affine parameters of x[N x D]: min, max, scale = max((max-min)/255, 1e-8),
 * zero_point = -128 - round(min/scale) (int32).  Replaces ScalarQuantizationKernel's
 * computeQuantizationParams (Kernels/Metal4/ScalarQuantizationKernel.swift:496-520) per dimension. */
va_status va_sq_params_per_dim(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim,
                               float* out_min, float* out_max, float* out_scale, int32_t* out_zero_point);
/* codes[i,d] = clamp(rint(x[i,d]/scale[d] + zp[d]), -128, 127).
 * Replaces quantize_int8_kernel (Metal/Shaders/DataTransformations.metal:174-201) via
 * ScalarQuantizationKernel.encodeQuantize (ScalarQuantizationKernel.swift:214-252). */
va_status va_sq_quantize_i8(va_context* ctx, const float* x, uint64_t num_vectors, uint32_t dim,
                            const float* scale, const int32_t* zero_point, int8_t* codes);
/* x[i,d] = (codes[i,d] - zp[d]) * scale[d].  Replaces dequantize_int8_kernel
 * (DataTransformations.metal:203-221). */
va_status va_sq_dequantize_i8(va_context* ctx, const int8_t* codes, uint64_t num_vectors, uint32_t dim,
                              const float* scale, const int32_t* zero_point, float* out);
/* int8 scan: distance = -sum(qc * xc) accumulated in int32, exact top-k.
 * No reference counterpart (the reference has no int8-domain distance); defined by the
 * scalar-int8 quantize-and-scan search path.  out_dist may be NULL.  dim is at most
 * VA_I8_MAX_DIM: the dot of two code vectors then lies in [-16256 dim, 16384 dim], inside int32. */
#define VA_I8_MAX_DIM 131071u
va_status va_i8_scan_topk(va_context* ctx, const int8_t* query_codes, const int8_t* database_codes,
                          uint32_t num_queries, uint32_t num_database, uint32_t dim, uint32_t k,
                          uint32_t* out_idx, int32_t* out_dist);

/* ---- binary quantization -------------------------------------------------------- */
/* codes[N x ceil(D/32)]: bit d = (x_d > 0), LSB-first.  Replaces binaryQuantize
 * (Metal/Shaders/QuantizationShaders.metal:132-160; BinaryQuantizationKernel.swift:335-401). */
va_status va_bq_pack(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim, uint32_t* codes);
/* Hamming matrix out[Q x N] (uint32).  Replaces hamming_distance_batch
 * (Metal/Shaders/HammingDistance.metal:28-127; HammingDistanceKernel.swift:313-363) and the
 * 1 x N binaryHammingDistance (QuantizationShaders.metal:163-187). */
va_status va_hamming_matrix(va_context* ctx, const uint32_t* query_codes, const uint32_t* database_codes,
                            uint32_t num_queries, uint32_t num_database, uint32_t words, uint32_t* out);
/* Hamming scan + exact top-k, ties to the lower index (Metal4HammingResult.nearestNeighbors,
 * HammingDistanceKernel.swift:114-120).  out_dist may be NULL. */
va_status va_hamming_topk(va_context* ctx, const uint32_t* query_codes, const uint32_t* database_codes,
                          uint32_t num_queries, uint32_t num_database, uint32_t words, uint32_t k,
                          uint32_t* out_idx, uint32_t* out_dist);

/* ---- IVF-Flat (L2^2) -------------------------------------------------------------- */
/* Build an IVF index: assign every row of x to its nearest centroid (ties to the lower id,
 * IVFStructure.findNearestCentroid, Index/Internal/IVFStructure.swift:292-307) and lay the
 * lists out in device CSR order with insertion order inside each list
 * (IVFStructure.prepareGPUStructure, IVFStructure.swift:347-467).  The index copies what it
 * needs; x and centroids may be freed afterwards.  For dim % 4 == 0 it also keeps an fp16 copy
 * of the list vectors (2 bytes per value + 8 per row), the input of the screened list scan.
 * Synchronises the context. */
va_status va_ivf_build(va_context* ctx, const float* centroids, uint32_t num_centroids, const float* x,
                       uint32_t num_vectors, uint32_t dim, va_ivf** out);
va_status va_ivf_destroy(va_ivf* ivf);
/* Add rows to a built index without rebuilding it: each row of x [num_vectors x dim] goes to the
 * end of its nearest list (ties -> lower id), with id first_id + row; the lists stay in CSR order
 * with insertion order inside each list, as a rebuild over all rows would lay them out
 * (IVFStructure.assignToCluster, Index/Internal/IVFStructure.swift:280-287, then
 * prepareGPUStructure).  Moves the existing list data once (no distance work for it).
 * Synchronises the context. */
va_status va_ivf_add(va_context* ctx, va_ivf* ivf, const float* x, uint32_t num_vectors, uint32_t dim,
                     uint32_t first_id);
/* Copy the CSR structure to the host: offsets[C+1], ids[N] (row ids in list order). */
va_status va_ivf_get_lists(va_context* ctx, const va_ivf* ivf, uint32_t* host_offsets, uint32_t* host_ids);
/* Coarse quantizer: probes[Q x nprobe] = the nprobe nearest centroids by (L2^2, id).
 * Replaces IVFCoarseQuantizerKernel.findNearestCentroids (IVFCoarseQuantizerKernel.swift:133-174). */
va_status va_ivf_probe(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                       uint32_t nprobe, uint32_t* probes);
/* List scan over given probes + exact top-k over original row ids (L2^2).
 * Replaces IVFListSearchKernel / ivf_list_search (Metal/Shaders/IVFListSearch.metal:199-339).
 * With the index's fp16 copy (and 16-byte aligned queries) the lists are screened on the fp16
 * MFMA and the rows that can reach the top-k re-scored in fp32: the ids and distances are those
 * of the fp32 list scan, bit for bit; VA_OPT_SCREEN = 1 runs the fp32 list scan alone. */
va_status va_ivf_scan(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                      const uint32_t* probes, uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist);
/* Full IVF search = probe + scan.  Replaces IVFSearchPipeline.search
 * (Index/Kernels/IVF/IVFSearchPipeline.swift:197-568). */
va_status va_ivf_search(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                        uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist);

/* ---- index with stable handles: replaces AcceleratedVectorIndex's flat storage, handle table
 *      and search (Index/AcceleratedVectorIndex.swift:481-1265; Index/Internal/HandleAllocator.swift:39-242)
 * The index keeps every row on the device in slots, with an fp16 shadow of each row (rounded at
 * insert time; the screening scan reads it, results are the fp32 scan's) when dim % 4 == 0.
 * Handles are stable ids in insertion order (VectorHandle.stableID); removing one leaves its
 * slot excluded from every search until va_index_compact moves the live rows down (handles keep
 * their ids).  An index is used through one context at a time (the actor contract). */
typedef struct va_index va_index;
typedef struct {
    uint32_t count;        /* live vectors */
    uint32_t deleted;      /* removed, not yet compacted */
    uint32_t slots;        /* count + deleted */
    uint32_t dimension;
    uint64_t capacity;     /* slots allocated */
    const float* rows;     /* device, [slots x dimension]; valid until the next insert or compact */
    uint32_t next_handle;  /* the id the next inserted vector gets */
    uint32_t nlist;        /* IVF lists (0: flat index) */
    uint32_t nprobe;       /* IVF lists probed per query */
    uint32_t routing_threshold; /* IVF: fewer live vectors than this are searched flat (0: never) */
    uint32_t trained;      /* IVF: 1 once centroids are installed */
    uint32_t ivf_routed;   /* 1 when va_index_search currently goes to the inverted lists */
    const float* centroids; /* IVF: device, [nlist x dimension] once trained (until the next train) */
    const va_ivf* lists;   /* IVF: the inverted lists over the slots (row id = slot; NULL while
                            * untrained or empty), for va_ivf_get_lists / va_ivf_probe; valid
                            * until the next insert, compact or train */
} va_index_info;
/* Returns nonzero to accept a result (IndexFilter, Index/AcceleratedVectorIndex.swift:1188-1265). */
typedef int (*va_index_filter)(uint32_t handle, void* user);
va_status va_index_create(va_context* ctx, uint32_t dim, uint32_t capacity, va_index** out);
/* An IVF index (IndexConfiguration.ivf(dimension:nlist:nprobe:capacity:routingThreshold),
 * Index/Types/IndexConfiguration.swift): flat until trained; once trained, va_index_search probes
 * the nprobe nearest of nlist lists, unless fewer than routing_threshold (> 0) vectors are live
 * (AcceleratedVectorIndex.search routing, Index/AcceleratedVectorIndex.swift:911-926).  L2^2 only.
 * 1 <= nprobe <= nlist. */
va_status va_index_create_ivf(va_context* ctx, uint32_t dim, uint32_t capacity, uint32_t nlist, uint32_t nprobe,
                              uint32_t routing_threshold, va_index** out);
/* Train an IVF index (train(), Index/AcceleratedVectorIndex.swift:406-446): with centroids
 * (device, [nlist x dim]) installs them; with NULL runs k-means on the device over the live
 * vectors (compacting the index first; k-means++ seeding from splitmix64(seed), at most 25 Lloyd
 * iterations, threshold 0.001, as IVFStructure.train, Index/Internal/IVFStructure.swift:202-259).
 * Then every vector is assigned to its nearest list (device CSR); later inserts join their
 * nearest lists and compact() rebuilds the lists, so the index never needs retraining to stay
 * searchable.  Removed vectors stay in the lists and are excluded inside every scan, so k is
 * never widened by deletions.  A flat index: no-op.  Synchronises. */
va_status va_index_train(va_context* ctx, va_index* index, const float* centroids, uint64_t seed);
va_status va_index_destroy(va_index* index);
/* Append num_vectors device rows; out_handles (host, may be NULL) gets their handles.  Grows the
 * storage by doubling (synchronising the context then).  insert(_:) / insert(contentsOf:),
 * AcceleratedVectorIndex.swift:481-700. */
va_status va_index_insert(va_context* ctx, va_index* index, const float* vectors, uint32_t num_vectors,
                          uint32_t* out_handles);
/* Remove host-listed handles; unknown or already removed ones are skipped.  *out_removed (may be
 * NULL) = how many were removed.  Synchronises.  remove(_:), AcceleratedVectorIndex.swift:771-833. */
va_status va_index_remove(va_context* ctx, va_index* index, const uint32_t* handles, uint32_t num_handles,
                          uint32_t* out_removed);
/* Drop removed slots, keeping the live rows' order and handles.  Synchronises.
 * compact(), AcceleratedVectorIndex.swift:834-893. */
va_status va_index_compact(va_context* ctx, va_index* index);
va_status va_index_get_info(const va_index* index, va_index_info* out);
/* 1 when the handle names a live vector (contains(_:)). */
int va_index_contains(const va_index* index, uint32_t handle);
/* Copy a live vector to host memory out[dim] (synchronous; vector(for:)). */
va_status va_index_get_vector(va_context* ctx, const va_index* index, uint32_t handle, float* out);
/* Exact top-k over the live vectors for each device query: out_handles / out_dist [Q x k]
 * (device), ordered by (distance, slot); slots past the number of live vectors hold
 * VA_SENTINEL_INDEX / +inf.  k <= VA_MAX_K whatever the number of removed vectors.
 * searchUnfiltered / searchBatchGPU, AcceleratedVectorIndex.swift:1103-1186, 1278-1374.
 * A trained IVF index (see va_index_train) returns the exact top-k over the live vectors of each
 * query's nprobe nearest lists instead (searchIVF / searchIVFBatch, :1378-1481), L2^2 only. */
va_status va_index_search(va_context* ctx, const va_index* index, va_metric metric, const float* queries,
                          uint32_t num_queries, uint32_t k, uint32_t* out_handles, float* out_dist);
/* The k nearest live vectors that pass filter (NULL: all), for one device query: round after
 * round the nearest not yet examined vectors are fetched and filtered on the host, so results
 * are exact however many the filter rejects.  out_handles / out_dist are host arrays of k;
 * *out_count results were found; *out_examined (may be NULL) vectors were examined.
 * searchFiltered, AcceleratedVectorIndex.swift:1188-1265.  Cost: rounds of 2k, 4k, ... up to
 * VA_MAX_K rows (one scan each); if the filter has still not accepted k, one scan computes the
 * distances of every row, a device sort orders the unexamined ones by (distance, slot), and they
 * are filtered in that order in host batches of 64K rows: at most log2(VA_MAX_K / 16) + 2 scans
 * and one sort whatever the filter rejects.  A trained IVF index filters its lists' rows the
 * same way, round after round (each round an IVF search excluding the rows already examined),
 * until k pass or the probed lists are exhausted (searchIVF with a filter, :1378-1431, which
 * over-fetches 3k instead). */
va_status va_index_search_filtered(va_context* ctx, va_index* index, va_metric metric, const float* query, uint32_t k,
                                   va_index_filter filter, void* user, uint32_t* out_handles, float* out_dist,
                                   uint32_t* out_count, uint32_t* out_examined);

/* ---- k-means (IVF centroid training) ------------------------------------------------ */
typedef struct {
    uint32_t iterations;  /* Lloyd iterations run */
    int32_t converged;    /* 1 when the last iteration's largest centroid movement < threshold */
    double inertia;       /* sum over points of the L2 distance to the assigned centroid */
    float max_movement;   /* largest centroid movement (L2) of the last iteration */
} va_kmeans_info;
/* Lloyd k-means from initial centroids [num_clusters x dim].  Replaces KMeansPipeline.fit
 * (Index/Kernels/Clustering/KMeansPipeline.swift:102-270): per iteration, assignment to the
 * nearest centroid (L2^2, ties to the lower id; distance = L2), centroid = mean of its points
 * (sum * (1/count)), empty clusters keep their centroid and are then re-seeded, in index
 * order, with the points farthest from their centroids (KMeansUpdateKernel.handleEmptyClusters,
 * KMeansUpdateKernel.swift:228-283); stops after max_iterations or when the largest movement
 * is below convergence_threshold (KMeansConvergenceKernel.swift:76-127).  out_assignments and
 * out_distances [num_vectors] are the last iteration's assignment; out_counts [num_clusters]
 * the updated sizes (1 for a re-seeded cluster).  out_distances, out_counts and out_info may be
 * NULL.  Deterministic: the same inputs give the same bits.  Synchronises the context. */
va_status va_kmeans_fit(va_context* ctx, const float* vectors, uint32_t num_vectors, uint32_t dim,
                        uint32_t num_clusters, const float* initial_centroids, uint32_t max_iterations,
                        float convergence_threshold, float* out_centroids, uint32_t* out_assignments,
                        float* out_distances, uint32_t* out_counts, va_kmeans_info* out_info);
/* k-means++ seeding: k rows of vectors chosen by D^2 sampling, copied to out_centroids
 * [k x dim], their row ids to out_indices [k] (may be NULL).  Replaces
 * KMeansPlusPlusKernel.selectCentroids (KMeansPlusPlusKernel.swift:94-203); the uniform draws
 * come from splitmix64(seed) instead of the system generator.  Synchronises the context. */
va_status va_kmeans_plusplus(va_context* ctx, const float* vectors, uint32_t num_vectors, uint32_t dim, uint32_t k,
                             uint64_t seed, float* out_centroids, uint32_t* out_indices);

/* ---- product quantization (ADC) --------------------------------------------------- */
/* Layout: codebooks [M x K x (dim / M)] fp32, codes [N x M] bytes, tables [Q x M x K] fp32.
 * dim % M == 0 and K <= 256 (Metal4PQConfig, Kernels/Metal4/ProductQuantizationKernel.swift:23-60).
 * Sub-vector distances use the reference shader's order (calculate_l2_sq_dist,
 * Metal/Shaders/ProductQuantization.metal:30-58), so codes and tables are reproducible. */
/* Lloyd training of the M codebooks (ProductQuantizationKernel.train, :260-369): up to
 * `iterations` rounds of assignment (nearest centroid, lowest k on ties) and update (mean of
 * the members; an empty centroid keeps its value); stops after the round whose movement
 * sqrt(sum of squared moves / (M K)) is below threshold.  Initial codebooks: initial_codebooks
 * when not NULL, else sub-vectors of training rows drawn by splitmix64(seed)
 * (initializeCodebooks, :548-572).  *out_iterations = rounds run (may be NULL).  Synchronises. */
va_status va_pq_train(va_context* ctx, const float* data, uint32_t count, uint32_t dim, uint32_t M, uint32_t K,
                      uint32_t iterations, float threshold, uint64_t seed, const float* initial_codebooks,
                      float* out_codebooks, uint32_t* out_iterations);
/* codes[n * M + m] = nearest centroid of sub-vector m (pq_assignment_or_encoding, :61-101;
 * ProductQuantizationKernel.encode, :372-406). */
va_status va_pq_encode(va_context* ctx, const float* x, uint32_t num_vectors, uint32_t dim, uint32_t M, uint32_t K,
                       const float* codebooks, uint8_t* codes);
/* tables[q][m][k] = |q_m - c_mk|^2 (pq_precompute_distance_table, :191-213). */
va_status va_pq_distance_tables(va_context* ctx, const float* queries, uint32_t num_queries, uint32_t dim, uint32_t M,
                                uint32_t K, const float* codebooks, float* tables);
/* out[q * N + n] = sum_m tables[q][m][codes[n][m]], added in m order (pq_compute_distances_adc,
 * :215-254; computeDistances, :409-478). */
va_status va_pq_adc_distances(va_context* ctx, const float* tables, uint32_t num_queries, const uint8_t* codes,
                              uint32_t num_vectors, uint32_t M, uint32_t K, float* out);
/* Exact ADC top-k: tables, then the k smallest ADC sums per query by (sum, row id), reported as
 * sqrt(sum) (findNearestNeighbors, :504-540, batched over queries).  out_dist may be NULL. */
va_status va_pq_search(va_context* ctx, const float* queries, uint32_t num_queries, uint32_t dim, uint32_t M,
                       uint32_t K, const float* codebooks, const uint8_t* codes, uint32_t num_vectors, uint32_t k,
                       uint32_t* out_idx, float* out_dist);

/* ---- measurement: the matrix-core ceiling of the board (and its LDS read bandwidth) -------------
 * No reference counterpart (the reference publishes no hardware peaks).  Every SIMD runs two waves
 * of back-to-back MFMAs of one instruction on register operands (no memory traffic), random or
 * constant (the clock falls further on random bits), `iterations` rounds of 8 MFMAs per wave,
 * after one untimed warm-up launch.  Reports the dense rate sustained (2 operations per
 * multiply-add), the launch time from events on the context stream, and the engine clock during
 * the launch (the shader clock counter over the constant-rate wall clock).  Synchronises. */
typedef enum {
    VA_PROBE_FP32 = 0, /* v_mfma_f32_32x32x2_f32: the fp32 distance GEMM */
    VA_PROBE_FP16 = 1, /* v_mfma_f32_32x32x16_f16: the fp16 screens */
    VA_PROBE_INT8 = 2, /* v_mfma_i32_32x32x32_i8: the int8 scan */
    VA_PROBE_FP4 = 3,  /* v_mfma_scale_f32_32x32x64_f8f6f4 on fp4 operands: the Hamming scan */
    VA_PROBE_LDS = 4,  /* ds_read_b128 of 1 KiB per wave, bank-conflict free, 8 per round (no MFMA):
                        * the LDS read bandwidth the scans' fragment reads draw on; ops = bytes */
    VA_PROBE_HBM = 5   /* a streaming read of `iterations` MiB (256 .. 65536) of device memory, 16-byte
                        * loads, a wave reading 1 KiB contiguous per load: the HBM read bandwidth the
                        * HBM-bound scans draw on; ops = bytes */
} va_probe_kind;
typedef struct {
    double ops_per_second; /* dense operations per second sustained */
    double engine_mhz;     /* mean engine clock over the timed launch */
    double ms;             /* timed launch */
    double ops;            /* operations in the timed launch */
} va_probe_result;
va_status va_probe_mfma(va_context* ctx, va_probe_kind kind, int random_operands, uint32_t iterations,
                        va_probe_result* out);

#ifdef __cplusplus
}
#endif
#endif /* VA_HIP_H */
