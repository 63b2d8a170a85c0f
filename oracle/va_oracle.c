/*
 * va_oracle.c — CPU oracle for the flat/IVF search path (TEST INFRASTRUCTURE ONLY).
 *
 * Plain C restatement of gifton/VectorAccelerate 0.5.0's CPU semantics for the
 * search hot path.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load this library; the product (libva_hip.so) never does.  Citations are
 * paths inside the reference tree (Sources/VectorAccelerate/...).
 *
 * Built with -ffp-contract=off so float expressions round exactly as written
 * (the int8 quantizer must match the GPU bit for bit).
 */
#include "va_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define VO_SENTINEL 0xFFFFFFFFu

int vo_version(void) { return 1; }

int vo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* ordering helpers: (key, index) with NaN after +inf                        */
/* ------------------------------------------------------------------------ */

/* returns 1 when (a, ai) orders strictly before (b, bi) in ascending order */
static inline int before_d(double a, uint32_t ai, double b, uint32_t bi) {
    int an = isnan(a), bn = isnan(b);
    if (an || bn) {
        if (an && bn) return ai < bi;
        return bn; /* non-NaN before NaN */
    }
    if (a < b) return 1;
    if (a > b) return 0;
    return ai < bi;
}

typedef struct {
    double key;
    uint32_t idx;
} vo_item;

/* bounded max-heap of the k best items under before_d (CPU/CPUTopK.swift:48-76, 89-112) */
typedef struct {
    vo_item* a;
    int64_t n, cap;
} vo_heap;

static void heap_sift_down(vo_heap* h, int64_t i) {
    for (;;) {
        int64_t l = 2 * i + 1, r = l + 1, m = i;
        if (l < h->n && before_d(h->a[m].key, h->a[m].idx, h->a[l].key, h->a[l].idx)) m = l;
        if (r < h->n && before_d(h->a[m].key, h->a[m].idx, h->a[r].key, h->a[r].idx)) m = r;
        if (m == i) return;
        vo_item t = h->a[i];
        h->a[i] = h->a[m];
        h->a[m] = t;
        i = m;
    }
}

static void heap_sift_up(vo_heap* h, int64_t i) {
    while (i > 0) {
        int64_t p = (i - 1) / 2;
        if (!before_d(h->a[p].key, h->a[p].idx, h->a[i].key, h->a[i].idx)) return;
        vo_item t = h->a[i];
        h->a[i] = h->a[p];
        h->a[p] = t;
        i = p;
    }
}

static inline void heap_push(vo_heap* h, double key, uint32_t idx) {
    if (h->cap == 0) return;
    if (h->n < h->cap) {
        h->a[h->n].key = key;
        h->a[h->n].idx = idx;
        heap_sift_up(h, h->n);
        h->n++;
    } else if (before_d(key, idx, h->a[0].key, h->a[0].idx)) {
        h->a[0].key = key;
        h->a[0].idx = idx;
        heap_sift_down(h, 0);
    }
}

static int cmp_item(const void* pa, const void* pb) {
    const vo_item* a = (const vo_item*)pa;
    const vo_item* b = (const vo_item*)pb;
    if (before_d(a->key, a->idx, b->key, b->idx)) return -1;
    if (before_d(b->key, b->idx, a->key, a->idx)) return 1;
    return 0;
}

/* sort the heap ascending and emit k slots, padding with sentinels */
static void heap_emit(vo_heap* h, int64_t k, uint32_t* idx, float* dist, float pad) {
    qsort(h->a, (size_t)h->n, sizeof(vo_item), cmp_item);
    for (int64_t i = 0; i < k; i++) {
        if (i < h->n) {
            idx[i] = h->a[i].idx;
            if (dist) dist[i] = (float)h->a[i].key;
        } else {
            idx[i] = VO_SENTINEL;
            if (dist) dist[i] = pad;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* distances                                                                 */
/* ------------------------------------------------------------------------ */

static inline void dots_d(const float* a, const float* b, int64_t D, double* ab, double* aa, double* bb) {
    double s_ab = 0, s_aa = 0, s_bb = 0;
    for (int64_t i = 0; i < D; i++) {
        double x = a[i], y = b[i];
        s_ab += x * y;
        s_aa += x * x;
        s_bb += y * y;
    }
    *ab = s_ab;
    *aa = s_aa;
    *bb = s_bb;
}

static inline double l2sq_d(const float* a, const float* b, int64_t D) {
    double s = 0;
    for (int64_t i = 0; i < D; i++) {
        double d = (double)a[i] - (double)b[i];
        s += d * d;
    }
    return s;
}

/* Cosine similarity rule of cosine_similarity (DistanceShaders.metal:300-319):
 * s = ab / (sqrt(aa)*sqrt(bb)); 0 when the denominator is below FLT_MIN;
 * finite values clamped to [-1, 1], NaN propagated. */
static inline double cosine_sim_rule(double ab, double aa, double bb) {
    double denom = sqrt(aa) * sqrt(bb);
    double raw = (denom < (double)FLT_MIN) ? 0.0 : ab / denom;
    if (isnan(raw)) return raw;
    if (raw < -1.0) raw = -1.0;
    if (raw > 1.0) raw = 1.0;
    return raw;
}

double vo_distance(int metric, const float* q, const float* x, int64_t D) {
    double ab, aa, bb;
    switch (metric) {
        case VO_METRIC_L2SQ:
            return l2sq_d(q, x, D);
        case VO_METRIC_L2:
            return sqrt(l2sq_d(q, x, D));
        case VO_METRIC_COSINE:
            dots_d(q, x, D, &ab, &aa, &bb);
            return 1.0 - cosine_sim_rule(ab, aa, bb);
        case VO_METRIC_DOT:
        default:
            dots_d(q, x, D, &ab, &aa, &bb);
            return -ab;
    }
}

void vo_l2_pairs(const float* q, const float* t, int64_t P, int64_t D, int compute_sqrt, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < P; p++) {
        double s = l2sq_d(q + p * D, t + p * D, D);
        out[p] = (float)(compute_sqrt ? sqrt(s) : s);
    }
}

void vo_cosine_pairs(const float* q, const float* t, int64_t P, int64_t D, int output_distance, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < P; p++) {
        double ab, aa, bb;
        dots_d(q + p * D, t + p * D, D, &ab, &aa, &bb);
        double s = cosine_sim_rule(ab, aa, bb);
        out[p] = (float)(output_distance ? 1.0 - s : s);
    }
}

void vo_distance_matrix(int kind, const float* q, const float* x, int64_t Q, int64_t N, int64_t D, float* out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < Q; i++) {
        const float* qi = q + i * D;
        for (int64_t j = 0; j < N; j++) {
            const float* xj = x + j * D;
            double v, ab, aa, bb;
            switch (kind) {
                case 0: v = l2sq_d(qi, xj, D); break;
                case 1: v = sqrt(l2sq_d(qi, xj, D)); break;
                case 2: dots_d(qi, xj, D, &ab, &aa, &bb); v = cosine_sim_rule(ab, aa, bb); break;
                case 3: dots_d(qi, xj, D, &ab, &aa, &bb); v = 1.0 - cosine_sim_rule(ab, aa, bb); break;
                case 4: dots_d(qi, xj, D, &ab, &aa, &bb); v = ab; break;
                default: dots_d(qi, xj, D, &ab, &aa, &bb); v = fabs(ab); break;
            }
            out[i * N + j] = (float)v;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* top-K                                                                     */
/* ------------------------------------------------------------------------ */

void vo_topk_rows(const float* in, int64_t Q, int64_t N, int64_t k, int mode, uint32_t* idx, float* val) {
#pragma omp parallel
    {
        vo_heap h;
        h.cap = k < N ? k : N;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(h.cap > 0 ? h.cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < Q; i++) {
            h.n = 0;
            const float* row = in + i * N;
            for (int64_t j = 0; j < N; j++) {
                double v = row[j];
                heap_push(&h, mode ? -v : v, (uint32_t)j);
            }
            heap_emit(&h, k, idx + i * k, val + i * k, INFINITY);
            if (mode) {
                for (int64_t r = 0; r < k; r++) val[i * k + r] = -val[i * k + r];
            }
        }
        free(h.a);
    }
}

/* float accumulation with eight partial sums (vDSP-style baseline port) */
static inline float l2sq_f(const float* a, const float* b, int64_t D) {
    float acc[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= D; i += 16) {
        for (int j = 0; j < 16; j++) {
            float d = a[i + j] - b[i + j];
            acc[j] = fmaf(d, d, acc[j]);
        }
    }
    for (; i < D; i++) {
        float d = a[i] - b[i];
        acc[0] = fmaf(d, d, acc[0]);
    }
    float s = 0;
    for (int j = 0; j < 16; j++) s += acc[j];
    return s;
}

static inline void dots_f(const float* a, const float* b, int64_t D, float* ab, float* bb) {
    float s1[16] = {0}, s2[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= D; i += 16) {
        for (int j = 0; j < 16; j++) {
            s1[j] = fmaf(a[i + j], b[i + j], s1[j]);
            s2[j] = fmaf(b[i + j], b[i + j], s2[j]);
        }
    }
    for (; i < D; i++) {
        s1[0] = fmaf(a[i], b[i], s1[0]);
        s2[0] = fmaf(b[i], b[i], s2[0]);
    }
    float r1 = 0, r2 = 0;
    for (int j = 0; j < 16; j++) {
        r1 += s1[j];
        r2 += s2[j];
    }
    *ab = r1;
    *bb = r2;
}

void vo_flat_topk(int metric, const float* q, const float* x, int64_t Q, int64_t N, int64_t D, int64_t k,
                  int accum_double, uint32_t* idx, float* dist) {
#pragma omp parallel
    {
        vo_heap h;
        h.cap = k < N ? k : N;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(h.cap > 0 ? h.cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < Q; i++) {
            h.n = 0;
            const float* qi = q + i * D;
            float qq_f = 0;
            if (!accum_double && metric == VO_METRIC_COSINE) {
                float unused;
                dots_f(qi, qi, D, &unused, &qq_f);
            }
            for (int64_t j = 0; j < N; j++) {
                const float* xj = x + j * D;
                double v;
                if (accum_double) {
                    v = vo_distance(metric, qi, xj, D);
                } else if (metric == VO_METRIC_L2SQ || metric == VO_METRIC_L2) {
                    float s = l2sq_f(qi, xj, D);
                    v = metric == VO_METRIC_L2 ? sqrtf(s) : s;
                } else {
                    float ab, bb;
                    dots_f(qi, xj, D, &ab, &bb);
                    if (metric == VO_METRIC_COSINE)
                        v = 1.0 - cosine_sim_rule(ab, qq_f, bb);
                    else
                        v = -(double)ab;
                }
                heap_push(&h, v, (uint32_t)j);
            }
            heap_emit(&h, k, idx + i * k, dist + i * k, INFINITY);
        }
        free(h.a);
    }
}

void vo_topk_merge(const uint32_t* a_idx, const float* a_d, const uint32_t* b_idx, const float* b_d, int64_t Q,
                   int64_t k, uint32_t chunk_base, uint32_t* out_idx, float* out_d) {
    for (int64_t i = 0; i < Q; i++) {
        const uint32_t* ai = a_idx + i * k;
        const float* ad = a_d + i * k;
        const uint32_t* bi = b_idx + i * k;
        const float* bd = b_d + i * k;
        int64_t x = 0, y = 0;
        for (int64_t r = 0; r < k; r++) {
            uint32_t bidx = (y < k && bi[y] != VO_SENTINEL) ? bi[y] + chunk_base : VO_SENTINEL;
            int take_a;
            if (x >= k || ai[x] == VO_SENTINEL)
                take_a = 0;
            else if (y >= k || bi[y] == VO_SENTINEL)
                take_a = 1;
            else
                take_a = !before_d(bd[y], bidx, ad[x], ai[x]);
            if (take_a && x < k && ai[x] != VO_SENTINEL) {
                out_idx[i * k + r] = ai[x];
                out_d[i * k + r] = ad[x];
                x++;
            } else if (y < k && bi[y] != VO_SENTINEL) {
                out_idx[i * k + r] = bidx;
                out_d[i * k + r] = bd[y];
                y++;
            } else {
                out_idx[i * k + r] = VO_SENTINEL;
                out_d[i * k + r] = INFINITY;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* scalar int8                                                               */
/* ------------------------------------------------------------------------ */

void vo_sq_params_per_dim(const float* x, int64_t N, int64_t D, float* mn, float* mx, float* scale, int32_t* zp) {
    for (int64_t d = 0; d < D; d++) {
        mn[d] = INFINITY;
        mx[d] = -INFINITY;
    }
    for (int64_t i = 0; i < N; i++) {
        const float* r = x + i * D;
        for (int64_t d = 0; d < D; d++) {
            if (r[d] < mn[d]) mn[d] = r[d];
            if (r[d] > mx[d]) mx[d] = r[d];
        }
    }
    for (int64_t d = 0; d < D; d++) {
        if (N == 0 || mn[d] > mx[d]) { /* no rows, or only NaN values in this dimension */
            mn[d] = 0.0f;
            mx[d] = 0.0f;
        }
        /* ScalarQuantizationKernel.swift:513-518: scale = max(range / 255, 1e-8) */
        float range = mx[d] - mn[d];
        float s = range / 255.0f;
        if (!(s > 1e-8f)) s = 1e-8f;
        scale[d] = s;
        /* Swift round() is round-half-away-from-zero, which C roundf() also is */
        float r = roundf(mn[d] / s);
        zp[d] = -128 - (int32_t)r;
    }
}

static inline int8_t quantize_one(float v, float s, int32_t z) {
    /* DataTransformations.metal:188-200 */
    if (fabsf(s) < 1e-9f) {
        int32_t c = z < -128 ? -128 : (z > 127 ? 127 : z);
        return (int8_t)c;
    }
    float scaled = v / s + (float)z;
    float r = rintf(scaled);
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    if (isnan(r)) r = 0.0f; /* NaN input: int8(NaN) is undefined in MSL; both sides pin it to 0 */
    return (int8_t)r;
}

/* computeQuantizationParams (Kernels/Metal4/ScalarQuantizationKernel.swift:496-520), int8 branch,
 * over all n values: symmetric scale = max(max(|min|, |max|) / 127, 1e-8), no zero point;
 * asymmetric scale = max((max - min) / 255, 1e-8), zero point = Int8(clamping: Int(-round(min /
 * scale))) with Swift's round (half away from zero, as C roundf) and a saturating conversion. */
void vo_sq_global_params(const float* x, int64_t n, int asymmetric, float* scale, int32_t* zero_point) {
    float mn = 0.0f, mx = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        if (i == 0 || x[i] < mn) mn = x[i];
        if (i == 0 || x[i] > mx) mx = x[i];
    }
    if (asymmetric) {
        float range = mx - mn;
        float s = range / 255.0f;
        s = s > 1e-8f ? s : 1e-8f;
        float r = -roundf(mn / s);
        int32_t z = r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int32_t)r);
        *scale = s;
        *zero_point = z;
    } else {
        float amin = fabsf(mn), amax = fabsf(mx);
        float absmax = amin > amax ? amin : amax;
        float s = absmax / 127.0f;
        *scale = s > 1e-8f ? s : 1e-8f;
        *zero_point = 0;
    }
}

void vo_sq_quantize(const float* x, int64_t N, int64_t D, const float* scale, const int32_t* zp, int8_t* codes) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; i++) {
        for (int64_t d = 0; d < D; d++) codes[i * D + d] = quantize_one(x[i * D + d], scale[d], zp[d]);
    }
}

void vo_sq_dequantize(const int8_t* codes, int64_t N, int64_t D, const float* scale, const int32_t* zp, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; i++) {
        for (int64_t d = 0; d < D; d++)
            out[i * D + d] = ((float)codes[i * D + d] - (float)zp[d]) * scale[d];
    }
}

static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int64_t D) {
    int32_t s = 0;
    for (int64_t i = 0; i < D; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

void vo_i8_dot_matrix(const int8_t* qc, const int8_t* xc, int64_t Q, int64_t N, int64_t D, int32_t* out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < Q; i++)
        for (int64_t j = 0; j < N; j++) out[i * N + j] = dot_i8(qc + i * D, xc + j * D, D);
}

void vo_i8_topk(const int8_t* qc, const int8_t* xc, int64_t Q, int64_t N, int64_t D, int64_t k, uint32_t* idx,
                int32_t* dist) {
#pragma omp parallel
    {
        vo_heap h;
        h.cap = k < N ? k : N;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(h.cap > 0 ? h.cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < Q; i++) {
            h.n = 0;
            for (int64_t j = 0; j < N; j++) heap_push(&h, -(double)dot_i8(qc + i * D, xc + j * D, D), (uint32_t)j);
            qsort(h.a, (size_t)h.n, sizeof(vo_item), cmp_item);
            for (int64_t r = 0; r < k; r++) {
                if (r < h.n) {
                    idx[i * k + r] = h.a[r].idx;
                    dist[i * k + r] = (int32_t)h.a[r].key;
                } else {
                    idx[i * k + r] = VO_SENTINEL;
                    dist[i * k + r] = INT32_MAX;
                }
            }
        }
        free(h.a);
    }
}

/* ------------------------------------------------------------------------ */
/* binary                                                                    */
/* ------------------------------------------------------------------------ */

void vo_bq_pack(const float* x, int64_t N, int64_t D, uint32_t* codes) {
    int64_t W = (D + 31) / 32;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; i++) {
        for (int64_t w = 0; w < W; w++) {
            uint32_t word = 0;
            for (int64_t b = 0; b < 32 && w * 32 + b < D; b++) {
                if (x[i * D + w * 32 + b] > 0.0f) word |= (1u << b);
            }
            codes[i * W + w] = word;
        }
    }
}

static inline uint32_t hamming(const uint32_t* a, const uint32_t* b, int64_t W) {
    uint32_t s = 0;
    for (int64_t w = 0; w < W; w++) s += (uint32_t)__builtin_popcount(a[w] ^ b[w]);
    return s;
}

void vo_hamming_matrix(const uint32_t* q, const uint32_t* x, int64_t Q, int64_t N, int64_t W, uint32_t* out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < Q; i++)
        for (int64_t j = 0; j < N; j++) out[i * N + j] = hamming(q + i * W, x + j * W, W);
}

void vo_hamming_topk(const uint32_t* q, const uint32_t* x, int64_t Q, int64_t N, int64_t W, int64_t k,
                     uint32_t* idx, uint32_t* dist) {
#pragma omp parallel
    {
        vo_heap h;
        h.cap = k < N ? k : N;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(h.cap > 0 ? h.cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < Q; i++) {
            h.n = 0;
            for (int64_t j = 0; j < N; j++) heap_push(&h, (double)hamming(q + i * W, x + j * W, W), (uint32_t)j);
            qsort(h.a, (size_t)h.n, sizeof(vo_item), cmp_item);
            for (int64_t r = 0; r < k; r++) {
                if (r < h.n) {
                    idx[i * k + r] = h.a[r].idx;
                    dist[i * k + r] = (uint32_t)h.a[r].key;
                } else {
                    idx[i * k + r] = VO_SENTINEL;
                    dist[i * k + r] = VO_SENTINEL;
                }
            }
        }
        free(h.a);
    }
}

/* ------------------------------------------------------------------------ */
/* IVF                                                                       */
/* ------------------------------------------------------------------------ */

void vo_ivf_assign(const float* x, int64_t N, const float* c, int64_t C, int64_t D, int32_t* list) {
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < N; i++) {
        int32_t best = 0;
        double bd = INFINITY;
        for (int64_t j = 0; j < C; j++) {
            double d = l2sq_d(x + i * D, c + j * D, D);
            if (d < bd) {
                bd = d;
                best = (int32_t)j;
            }
        }
        list[i] = best;
    }
}

void vo_ivf_csr(const int32_t* list, int64_t N, int64_t C, uint32_t* offsets, uint32_t* ids) {
    for (int64_t j = 0; j <= C; j++) offsets[j] = 0;
    for (int64_t i = 0; i < N; i++) offsets[list[i] + 1]++;
    for (int64_t j = 0; j < C; j++) offsets[j + 1] += offsets[j];
    uint32_t* fill = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(C > 0 ? C : 1));
    for (int64_t j = 0; j < C; j++) fill[j] = offsets[j];
    for (int64_t i = 0; i < N; i++) ids[fill[list[i]]++] = (uint32_t)i;
    free(fill);
}

void vo_ivf_probe(const float* q, int64_t Q, const float* c, int64_t C, int64_t D, int64_t nprobe,
                  uint32_t* probes) {
#pragma omp parallel
    {
        vo_heap h;
        h.cap = nprobe < C ? nprobe : C;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(h.cap > 0 ? h.cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < Q; i++) {
            h.n = 0;
            for (int64_t j = 0; j < C; j++) heap_push(&h, l2sq_d(q + i * D, c + j * D, D), (uint32_t)j);
            heap_emit(&h, nprobe, probes + i * nprobe, NULL, 0.0f);
        }
        free(h.a);
    }
}

void vo_ivf_scan(const float* q, int64_t Q, const float* x, int64_t D, const uint32_t* offsets, const uint32_t* ids,
                 int64_t C, const uint32_t* probes, int64_t nprobe, int64_t k, uint32_t* idx, float* dist) {
#pragma omp parallel
    {
        vo_heap h;
        h.cap = k;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(k > 0 ? k : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < Q; i++) {
            h.n = 0;
            for (int64_t p = 0; p < nprobe; p++) {
                uint32_t list = probes[i * nprobe + p];
                if (list == VO_SENTINEL || (int64_t)list >= C) continue;
                for (uint32_t e = offsets[list]; e < offsets[list + 1]; e++) {
                    uint32_t row = ids[e];
                    heap_push(&h, l2sq_d(q + i * D, x + (int64_t)row * D, D), row);
                }
            }
            heap_emit(&h, k, idx + i * k, dist + i * k, INFINITY);
        }
        free(h.a);
    }
}

/* ------------------------------------------------------------------------ */
/* k-means                                                                   */
/* ------------------------------------------------------------------------ */

/* kmeans_assign_points (ClusteringShaders.metal:16-120): float difference form, strict < */
static void km_assign(const float* x, int64_t N, int64_t D, const float* c, int64_t C, uint32_t* assign,
                      float* dist) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        float best = INFINITY;
        uint32_t bi = 0;
        for (int64_t j = 0; j < C; ++j) {
            float s = 0.0f;
            for (int64_t d = 0; d < D; ++d) {
                float diff = x[i * D + d] - c[j * D + d];
                s += diff * diff;
            }
            if (s < best) {
                best = s;
                bi = (uint32_t)j;
            }
        }
        assign[i] = bi;
        dist[i] = sqrtf(best);
    }
}

/* KMeansPipeline's update (KMeansUpdateKernel, ClusteringShaders.metal:490-613) given an
 * assignment: a cluster's points in point order form chunks of 256; each chunk is summed in
 * order, the chunk sums are added in order, times 1/count; an empty cluster keeps its centroid;
 * then handleEmptyClusters (KMeansUpdateKernel.swift:228-283): empty clusters in index order take
 * the unused point of largest distance (`>` from -1, so the first index on ties and never a NaN). */
static void km_update(const float* x, int64_t N, int64_t D, int64_t C, const uint32_t* assign, const float* dist,
                      const float* cur, float* nxt, uint32_t* counts) {
    float* sums = (float*)calloc((size_t)(C * D), sizeof(float));
    float* chunk = (float*)calloc((size_t)(C * D), sizeof(float));
    uint32_t* seen = (uint32_t*)calloc((size_t)C, sizeof(uint32_t));
    unsigned char* used = (unsigned char*)calloc((size_t)N, 1);
    memset(counts, 0, sizeof(uint32_t) * C);
    for (int64_t i = 0; i < N; ++i) counts[assign[i]]++;
    for (int64_t i = 0; i < N; ++i) {
        uint32_t a = assign[i];
        for (int64_t d = 0; d < D; ++d) chunk[a * D + d] += x[i * D + d];
        if (++seen[a] % 256 == 0 || seen[a] == counts[a]) {
            for (int64_t d = 0; d < D; ++d) {
                sums[a * D + d] += chunk[a * D + d];
                chunk[a * D + d] = 0.0f;
            }
        }
    }
    for (int64_t c = 0; c < C; ++c) {
        if (counts[c] > 0) {
            float inv = 1.0f / (float)counts[c];
            for (int64_t d = 0; d < D; ++d) nxt[c * D + d] = sums[c * D + d] * inv;
        } else {
            for (int64_t d = 0; d < D; ++d) nxt[c * D + d] = cur[c * D + d];
        }
    }
    for (int64_t c = 0; c < C; ++c) {
        if (counts[c] != 0) continue;
        float md = -1.0f;
        int64_t bv = -1;
        for (int64_t i = 0; i < N; ++i)
            if (!used[i] && dist[i] > md) {
                md = dist[i];
                bv = i;
            }
        if (bv >= 0) {
            used[bv] = 1;
            memcpy(nxt + c * D, x + bv * D, sizeof(float) * D);
            counts[c] = 1;
        }
    }
    free(sums);
    free(chunk);
    free(seen);
    free(used);
}

void vo_kmeans_update(const float* x, int64_t N, int64_t D, int64_t C, const uint32_t* assign, const float* dist,
                      const float* old_centroids, float* out_centroids, uint32_t* counts) {
    km_update(x, N, D, C, assign, dist, old_centroids, out_centroids, counts);
}

void vo_kmeans_fit(const float* x, int64_t N, int64_t D, int64_t C, const float* init, int64_t max_iter,
                   float threshold, float* centroids, uint32_t* assign, float* dist, uint32_t* counts,
                   uint32_t* info_u32, float* info_f) {
    float* cur = (float*)malloc(sizeof(float) * C * D);
    float* nxt = (float*)malloc(sizeof(float) * C * D);
    memcpy(cur, init, sizeof(float) * C * D);
    int64_t it = 0;
    int converged = 0;
    float max_move = 0.0f;
    while (it < max_iter && !converged) {
        km_assign(x, N, D, cur, C, assign, dist);
        km_update(x, N, D, C, assign, dist, cur, nxt, counts);
        /* checkConvergence: max over centroids of sqrt(sum (new - old)^2) */
        max_move = 0.0f;
        for (int64_t c = 0; c < C; ++c) {
            float s = 0.0f;
            for (int64_t d = 0; d < D; ++d) {
                float diff = nxt[c * D + d] - cur[c * D + d];
                s += diff * diff;
            }
            float m = sqrtf(s);
            if (m > max_move) max_move = m;
        }
        converged = max_move < threshold;
        float* t = cur;
        cur = nxt;
        nxt = t;
        ++it;
    }
    if (it == 0) {
        km_assign(x, N, D, cur, C, assign, dist);
        memset(counts, 0, sizeof(uint32_t) * C);
        for (int64_t i = 0; i < N; ++i) counts[assign[i]]++;
    }
    float inertia = 0.0f;
    for (int64_t i = 0; i < N; ++i) inertia += dist[i];
    memcpy(centroids, cur, sizeof(float) * C * D);
    info_u32[0] = (uint32_t)it;
    info_u32[1] = (uint32_t)converged;
    info_f[0] = inertia;
    info_f[1] = max_move;
    free(cur);
    free(nxt);
}

static uint64_t vo_splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void vo_kmeans_plusplus(const float* x, int64_t N, int64_t D, int64_t k, uint64_t seed, uint32_t* idx) {
    float* mind = (float*)malloc(sizeof(float) * N);
    unsigned char* sel = (unsigned char*)calloc((size_t)N, 1);
    uint64_t s = seed;
    double u0 = (double)(vo_splitmix64(&s) >> 11) * 0x1.0p-53;
    int64_t first = (int64_t)(u0 * (double)N);
    if (first >= N) first = N - 1;
    idx[0] = (uint32_t)first;
    sel[first] = 1;
    for (int64_t i = 0; i < N; ++i) mind[i] = INFINITY;
    for (int64_t j = 1; j < k; ++j) {
        const float* c = x + (int64_t)idx[j - 1] * D;
        /* compute_min_distances over all chosen centroids = running min against the newest;
         * the sum of squares in a fixed order: 64 partials (d = l, l + 64, ... with fmaf), then
         * combined pairwise at strides 32, 16, ..., 1 */
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < N; ++i) {
            float part[64];
            for (int l = 0; l < 64; ++l) {
                float t = 0.0f;
                for (int64_t d = l; d < D; d += 64) {
                    float diff = x[i * D + d] - c[d];
                    t = fmaf(diff, diff, t);
                }
                part[l] = t;
            }
            for (int m = 32; m > 0; m >>= 1)
                for (int l = 0; l < m; ++l) part[l] = part[l] + part[l + m];
            if (part[0] < mind[i]) mind[i] = part[0];
        }
        double u = (double)(vo_splitmix64(&s) >> 11) * 0x1.0p-53;
        double total = 0.0;
        for (int64_t i = 0; i < N; ++i)
            if (!sel[i]) total += (double)mind[i];
        int64_t next = 0;
        if (total > 0.0) {
            double thr = u * total, cum = 0.0;
            for (int64_t i = 0; i < N; ++i) {
                if (sel[i]) continue;
                cum += (double)mind[i];
                if (cum >= thr) {
                    next = i;
                    break;
                }
            }
        } else {
            for (int64_t i = 0; i < N; ++i)
                if (!sel[i]) {
                    next = i;
                    break;
                }
        }
        idx[j] = (uint32_t)next;
        sel[next] = 1;
    }
    free(mind);
    free(sel);
}

/* ------------------------------------------------------------------------ */
/* product quantization                                                      */
/* ------------------------------------------------------------------------ */

float vo_pq_sub_l2sq(const float* v, const float* c, int64_t n) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int64_t n4 = n / 4;
    for (int64_t d = 0; d < n4; ++d) {
        float e0 = v[4 * d] - c[4 * d], e1 = v[4 * d + 1] - c[4 * d + 1];
        float e2 = v[4 * d + 2] - c[4 * d + 2], e3 = v[4 * d + 3] - c[4 * d + 3];
        a0 = fmaf(e0, e0, a0);
        a1 = fmaf(e1, e1, a1);
        a2 = fmaf(e2, e2, a2);
        a3 = fmaf(e3, e3, a3);
    }
    float s = ((a0 + a1) + a2) + a3;
    for (int64_t d = n4 * 4; d < n; ++d) {
        float e = v[d] - c[d];
        s += e * e;
    }
    return s;
}

void vo_pq_encode(const float* x, int64_t N, int64_t D, int64_t M, int64_t K, const float* cb, uint8_t* codes) {
    int64_t ds = D / M;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) {
            float best = INFINITY;
            int64_t bk = 0;
            for (int64_t k = 0; k < K; ++k) {
                float d = vo_pq_sub_l2sq(x + n * D + m * ds, cb + (m * K + k) * ds, ds);
                if (d < best) {
                    best = d;
                    bk = k;
                }
            }
            codes[n * M + m] = (uint8_t)bk;
        }
}

void vo_pq_tables(const float* q, int64_t Q, int64_t D, int64_t M, int64_t K, const float* cb, float* tables) {
    int64_t ds = D / M;
    for (int64_t i = 0; i < Q; ++i)
        for (int64_t m = 0; m < M; ++m)
            for (int64_t k = 0; k < K; ++k)
                tables[(i * M + m) * K + k] = vo_pq_sub_l2sq(q + i * D + m * ds, cb + (m * K + k) * ds, ds);
}

void vo_pq_adc(const float* tables, int64_t Q, const uint8_t* codes, int64_t N, int64_t M, int64_t K, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < Q; ++i)
        for (int64_t n = 0; n < N; ++n) {
            float s = 0.0f;
            for (int64_t m = 0; m < M; ++m) s += tables[(i * M + m) * K + codes[n * M + m]];
            out[i * N + n] = s;
        }
}

void vo_pq_search(const float* q, int64_t Q, int64_t D, int64_t M, int64_t K, const float* cb, const uint8_t* codes,
                  int64_t N, int64_t k, uint32_t* idx, float* dist) {
    float* tables = (float*)malloc(sizeof(float) * Q * M * K);
    vo_pq_tables(q, Q, D, M, K, cb, tables);
#pragma omp parallel for schedule(dynamic)
    for (int64_t i = 0; i < Q; ++i) {
        vo_heap h;
        h.a = (vo_item*)malloc(sizeof(vo_item) * (size_t)(k > 0 ? k : 1));
        h.n = 0;
        h.cap = k;
        const float* t = tables + i * M * K;
        for (int64_t n = 0; n < N; ++n) {
            float s = 0.0f;
            for (int64_t m = 0; m < M; ++m) s += t[m * K + codes[n * M + m]];
            heap_push(&h, (double)s, (uint32_t)n);
        }
        heap_emit(&h, k, idx + i * k, dist + i * k, INFINITY);
        for (int64_t j = 0; j < k; ++j) dist[i * k + j] = sqrtf(dist[i * k + j]);
        free(h.a);
    }
    free(tables);
}

int64_t vo_pq_train(const float* x, int64_t N, int64_t D, int64_t M, int64_t K, int64_t iterations, float threshold,
                    float* cb) {
    int64_t ds = D / M;
    uint8_t* codes = (uint8_t*)malloc((size_t)(N * M));
    float* sums = (float*)malloc(sizeof(float) * M * K * ds);
    float* chunk = (float*)malloc(sizeof(float) * M * K * ds);
    uint32_t* counts = (uint32_t*)malloc(sizeof(uint32_t) * M * K);
    uint32_t* seen = (uint32_t*)malloc(sizeof(uint32_t) * M * K);
    float* mv = (float*)malloc(sizeof(float) * M * K);
    int64_t it = 0;
    while (it < iterations) {
        vo_pq_encode(x, N, D, M, K, cb, codes);
        memset(sums, 0, sizeof(float) * M * K * ds);
        memset(chunk, 0, sizeof(float) * M * K * ds);
        memset(counts, 0, sizeof(uint32_t) * M * K);
        memset(seen, 0, sizeof(uint32_t) * M * K);
        for (int64_t n = 0; n < N; ++n)
            for (int64_t m = 0; m < M; ++m) counts[m * K + codes[n * M + m]]++;
        for (int64_t n = 0; n < N; ++n)
            for (int64_t m = 0; m < M; ++m) {
                int64_t c = m * K + codes[n * M + m];
                for (int64_t d = 0; d < ds; ++d) chunk[c * ds + d] += x[n * D + m * ds + d];
                if (++seen[c] % 256 == 0 || seen[c] == counts[c])
                    for (int64_t d = 0; d < ds; ++d) {
                        sums[c * ds + d] += chunk[c * ds + d];
                        chunk[c * ds + d] = 0.0f;
                    }
            }
        for (int64_t c = 0; c < M * K; ++c) {
            float mvs = 0.0f;
            if (counts[c] > 0) {
                float inv = 1.0f / (float)counts[c];
                for (int64_t d = 0; d < ds; ++d) {
                    float nv = sums[c * ds + d] * inv, ov = cb[c * ds + d];
                    cb[c * ds + d] = nv;
                    float diff = ov - nv;
                    mvs += diff * diff;
                }
            }
            mv[c] = mvs;
        }
        float total = 0.0f;
        for (int64_t c = 0; c < M * K; ++c) total += mv[c];
        ++it;
        if (sqrtf(total / (float)(M * K)) < threshold) break;
    }
    free(codes);
    free(sums);
    free(chunk);
    free(counts);
    free(seen);
    free(mv);
    return it;
}
