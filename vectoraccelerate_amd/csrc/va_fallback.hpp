// va_fallback.hpp — exact top-k of the rows whose candidate list overflowed, enqueued without
// reading the overflow count back to the host.
//
// A scan that selects from per-query candidate lists lists the queries whose list outgrew its
// capacity (a device count and a device list of query ids).  The fallback finds their exact
// top-k in a fixed number of launches whose work follows that device count; with no overflowed
// query every workgroup exits at once.  Each pass recomputes the keys of (overflowed query,
// database row) pairs with the producer's own arithmetic — bit-identical to its scan:
//   pass 0 .. 2  histograms of key bits 31:21, 20:10 and 9:0 of the keys in the bucket chosen so
//                far: after pass 2 the k-th smallest key K and how many keys equal to K the
//                top-k takes ("need") are known;
//   pass 3       collects every (key, id) with key <= K, and a histogram of the ids of the ties;
//   pass 4       (rows whose ties overflowed the list) collects key < K, and the ties whose id is
//                below the first id-histogram edge that holds `need` of them;
//   then the selection kernel orders each row's list by (key, id) and writes the top-k.
// Between passes the last workgroup to finish (a completion ticket, no waiting) turns the
// histograms into the next pass's bucket.  Work items are 32 queries x 32 database rows in the
// 32x32 MFMA output layout: lane (l, h) holds query slot l % 32 and rows 8j + 4h + e.
#pragma once

#include <algorithm>

#include "va_distop.hpp"
#include "va_internal.hpp"

namespace va {

struct FbArgs {
    const uint32_t* n_rows = nullptr;  // device: how many queries overflowed
    const uint32_t* rows = nullptr;    // device: their query ids
    uint32_t rmax = 0;                 // slots the buffers hold (a host bound on the count)
    uint32_t N = 0, k = 0;
    uint32_t ishift = 0;               // tie-id histogram bin = id >> ishift (ids below N: bins < 4096)
    uint32_t cap = 0;                  // list capacity per slot: k + min(2^ishift, rows), rounded up
    uint32_t* hist = nullptr;          // [rmax][2048] key histogram (cleared after each use)
    uint32_t* tidh = nullptr;          // [rmax][4096] tie-id histogram
    uint32_t* st = nullptr;            // [rmax][8] bucket state (see FbState)
    uint32_t* cnt = nullptr;           // [rmax] list lengths
    uint32_t* lkey = nullptr;          // [rmax][cap]
    uint32_t* lid = nullptr;           // [rmax][cap]
    uint32_t* done = nullptr;          // [8] completion tickets, one per pass
    uint32_t grid = kFbGrid;           // workgroups per pass (fewer for a few rows: each launch that
                                       // finds nothing overflowed still costs its dispatch)
    const uint8_t* skip = nullptr;     // excluded rows: their keys are kAbsentKey
};
enum FbState : int { FB_PREFIX = 0, FB_NEED = 1, FB_K = 2, FB_EDGE = 3, FB_OVF = 4 };
static_assert(kFbKeyBins == 2048, "the passes' key histograms have 2048 bins");
// (the pass count, grid, bins and buffer sizes: fb_geometry / fb_bytes in va_plan.hpp)

inline FbArgs fb_carve(Scratch& s, uint32_t rmax, uint32_t N, uint32_t k, uint32_t rows = 0) {
    FbArgs a;
    a.rmax = rmax;
    a.N = N;
    a.k = k;
    fb_geometry(N, k, a.ishift, a.cap, rows);
    a.hist = s.carve<uint32_t>(uint64_t(rmax) * kFbKeyBins);
    a.tidh = s.carve<uint32_t>(uint64_t(rmax) * kFbTieBins);
    a.st = s.carve<uint32_t>(uint64_t(rmax) * 8);
    a.cnt = s.carve<uint32_t>(rmax);
    a.lkey = s.carve<uint32_t>(uint64_t(rmax) * a.cap);
    a.lid = s.carve<uint32_t>(uint64_t(rmax) * a.cap);
    a.done = s.carve<uint32_t>(8);
    a.grid = rmax <= 64 ? 256u : kFbGrid;
    return a;
}

// ---- device key producers ----------------------------------------------------------------------
// keys16: the lane's 16 keys of query slot s0 + l (rows[]: query ids, slots >= n are padding)
// against database rows r0 + 8j + 4h + e.  Every lane of the wave calls it.

typedef float fb_f32x16 __attribute__((ext_vector_type(16)));
typedef float fb_f32x4 __attribute__((ext_vector_type(4)));

// fp32 distances exactly as the distance GEMM forms them: v_mfma_f32_32x32x2_f32 over 16-value
// stages, step e of each 8-value group pairing d = 8g + e (lane half 0) with 8g + 4 + e (half 1);
// squared norms as per-half fmaf chains over the same values, the halves then added; values
// past D are zeros.  The per-element sequence is the GEMM's, so the keys are bit-identical.
// qp: the query of column l % 32 (nullptr: zeros); xp: the database row of row l % 32 (nullptr:
// zeros).  keys[4j + e] = key of (column l % 32, row 8j + 4h + e), h = l / 32.
// VEC: D % 4 == 0 and 16-byte aligned rows (one 16-byte load per value group).  The loads of
// stage s + 1 are issued before stage s computes (two register sets); exactly ceil(D / 16)
// stages run, as in the GEMM (a further all-zero stage could turn a -0 dot into +0).
template <bool VEC>
__device__ inline void f32_block_keys(const float* qp, const float* xp, uint32_t D, int op, int lane,
                                      uint32_t* keys) {
    const int hh = lane >> 5;
    auto load4 = [&](const float* p, uint32_t d) {
        fb_f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (p && d < D) {
            if (VEC) {
                v = *reinterpret_cast<const fb_f32x4*>(p + d);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d + e < D) v[e] = p[d + e];
            }
        }
        return v;
    };
    fb_f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    float qss = 0.0f, xss = 0.0f;
    fb_f32x4 xa[2], qa[2], xb[2], qb[2];
    auto ld = [&](uint32_t d0, fb_f32x4(&xv)[2], fb_f32x4(&qv)[2]) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t d = d0 + 8 * g + 4 * hh;
            xv[g] = load4(xp, d);
            qv[g] = load4(qp, d);
        }
    };
    auto cmp = [&](const fb_f32x4(&xv)[2], const fb_f32x4(&qv)[2]) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int e = 0; e < 4; ++e) qss = fmaf(qv[g][e], qv[g][e], qss);
#pragma unroll
            for (int e = 0; e < 4; ++e) xss = fmaf(xv[g][e], xv[g][e], xss);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[g][e], qv[g][e], acc, 0, 0, 0);
        }
    };
    const uint32_t ns = (D + 15) / 16;
    ld(0, xa, qa);
    for (uint32_t s = 0; s < ns; s += 2) {
        ld(16 * (s + 1), xb, qb);  // past D: zeros, not computed
        cmp(xa, qa);
        if (s + 1 >= ns) break;
        ld(16 * (s + 2), xa, qa);
        cmp(xb, qb);
    }
    const float qq = qss + __shfl_xor(qss, 32);
    const float xt = xss + __shfl_xor(xss, 32);  // |x|^2 of row l % 32
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float xx = __shfl(xt, 8 * j + 4 * hh + e);
            keys[4 * j + e] = key_of_float(apply_op(op, acc[4 * j + e], qq, xx));
        }
}

// ---- the same keys on the VALU, one (query, row) pair per lane --------------------------------
// Every element of v_mfma_f32_32x32x2_f32 and v_mfma_f32_16x16x4_f32 is formed by sequential
// fmas in k order: d = fma(a_k1, b_k1, fma(a_k0, b_k0, c)) (measured on gfx950, bit for bit
// against a correctly rounded fmaf on 1M cases: wide exponent ranges, cancellation, fp32
// subnormal inputs and products, signed zeros, inf and NaN).  So the keys of the MFMA kernels
// are reproduced exactly by a per-lane fmaf chain in the same element order, with every zero
// step the kernels run (a zero fma turns a -0 into +0).  The query is wave-uniform (scalar
// loads), each lane streams its own row (nullptr: a lane with no row, whose key is unused).

// x[d .. d + 3] with zeros past D (VEC: D % 4 == 0 and 16-byte aligned rows)
template <bool VEC>
__device__ __forceinline__ fb_f32x4 valu_load4(const float* p, uint32_t d, uint32_t D) {
    fb_f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p && d < D) {
        if (VEC) {
            v = *reinterpret_cast<const fb_f32x4*>(p + d);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (d + e < D) v[e] = p[d + e];
        }
    }
    return v;
}

// The chains consume a row in groups of 32 values (elements 32j .. 32j + 31, zeros past D):
// xv[i] / qv[i] hold elements 32j + 4i .. + 3 of the row and of the query.

// The distance GEMM's key (f32_block_keys): ceil(D / 16) stages of 16; in stage s, for g < 2 and
// e < 4, the pair (16s + 8g + e, 16s + 8g + 4 + e); the squared norms as the two half-chains
// (elements 8g + e and 8g + 4 + e of every stage), added.
struct GemmChain {
    float acc = 0.0f, xs0 = 0.0f, xs1 = 0.0f, qs0 = 0.0f, qs1 = 0.0f;
    __device__ __forceinline__ void stage(const fb_f32x4 (&xv)[8], const fb_f32x4 (&qv)[8], int h) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = xv[4 * h + 2 * g][e], b = xv[4 * h + 2 * g + 1][e];
                const float qa = qv[4 * h + 2 * g][e], qb = qv[4 * h + 2 * g + 1][e];
                qs0 = fmaf(qa, qa, qs0);
                qs1 = fmaf(qb, qb, qs1);
                xs0 = fmaf(a, a, xs0);
                xs1 = fmaf(b, b, xs1);
                acc = fmaf(a, qa, acc);
                acc = fmaf(b, qb, acc);
            }
        }
    }
    // group j of a row of D values (the GEMM runs exactly ceil(D / 16) stages)
    __device__ __forceinline__ void group(const fb_f32x4 (&xv)[8], const fb_f32x4 (&qv)[8], uint32_t j, uint32_t D) {
        stage(xv, qv, 0);
        if (32 * j + 16 < D) stage(xv, qv, 1);
    }
    __device__ __forceinline__ uint32_t key(int op) const {
        return key_of_float(apply_op(op, acc, qs0 + qs1, xs0 + xs1));
    }
};

// ivf_small_kernel's key (small_keys32): ceil(D / 32) * 2 chunks of 16 (whole groups); in chunk c,
// for e < 4 and g < 4, element 16c + 4g + e; the squared norms as four chains (g), combined
// (x0 + x1) + (x2 + x3); L2^2 = |q|^2 + |x|^2 - 2 dot clamped at 0.
struct SmallChain {
    float acc = 0.0f;
    float xs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, qs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    __device__ __forceinline__ void group(const fb_f32x4 (&xv)[8], const fb_f32x4 (&qv)[8]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    qs[g] = fmaf(qv[4 * h + g][e], qv[4 * h + g][e], qs[g]);
                    xs[g] = fmaf(xv[4 * h + g][e], xv[4 * h + g][e], xs[g]);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int g = 0; g < 4; ++g) acc = fmaf(xv[4 * h + g][e], qv[4 * h + g][e], acc);
        }
    }
    __device__ __forceinline__ uint32_t key() const {
        const float qsum = (qs[0] + qs[1]) + (qs[2] + qs[3]);
        const float xx = (xs[0] + xs[1]) + (xs[2] + xs[3]);
        float d = qsum + xx - 2.0f * acc;
        d = (d < 0.0f) ? 0.0f : d;
        return key_of_float(d);
    }
};

// Scores up to 8 NRG rows (lane l < 8 NRG: row id rid_of(l), valid_of(l)) against one
// wave-uniform query with a VALU chain per lane.  The rows move in coalesced groups of 32 values:
// load instruction i of a group brings rows 8i .. 8i + 7 (lane L: row 8i + L / 8, 16-byte chunk
// L % 8, whole 128-byte lines), the wave's LDS slot (8 KiB, chunk c of row r at c ^ ((r >> 1) & 7):
// conflict-free reads) turns them into rows, and lane l reads its own row's 32 values (lanes past
// 8 NRG read slot entries no row filled; their chains are discarded).  Groups j + 1 .. j + R are in
// flight (registers) while group j computes (R groups in all).  feed(j, xv, qv) runs the lane's
// chain on group j.  Fewer row groups per wave (NRG < 8) spread a few rows over more waves, each
// streaming less, with more groups in flight.  Needs D % 4 == 0 and 16-byte aligned rows and query.
template <int R = 2, int NRG = 8, class Feed>
__device__ inline void rows_through_lds(const float* q, const float* x, const uint32_t (&rid)[NRG],
                                        const bool (&rvalid)[NRG], uint32_t D, fb_f32x4* slot, Feed&& feed) {
    static_assert(NRG >= 1 && NRG <= 8, "row groups of 8 rows in a 64-row slot");
    const int lane = threadIdx.x & 63;
    const int ck = lane & 7;
    const uint32_t ng = (D + 31) / 32;
    fb_f32x4 g[R][NRG];
    auto load = [&](uint32_t j, fb_f32x4(&gr)[NRG]) {
        const uint32_t d = 32 * j + 4 * uint32_t(ck);
#pragma unroll
        for (int i = 0; i < NRG; ++i)
            gr[i] = valu_load4<true>(rvalid[i] ? x + int64_t(rid[i]) * D : nullptr, d, D);
    };
    auto stash = [&](const fb_f32x4(&gr)[NRG]) {
#pragma unroll
        for (int i = 0; i < NRG; ++i) {
            const int r = 8 * i + (lane >> 3);
            slot[r * 8 + (ck ^ ((r >> 1) & 7))] = gr[i];
        }
    };
    auto run = [&](uint32_t j) {
        fb_f32x4 xv[8], qv[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            xv[m] = slot[lane * 8 + (m ^ ((lane >> 1) & 7))];
            qv[m] = valu_load4<true>(q, 32 * j + 4 * m, D);  // (wave-uniform: scalar loads)
        }
        feed(j, xv, qv);
    };
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (uint32_t(r) < ng) load(uint32_t(r), g[r]);
    for (uint32_t j = 0; j < ng; j += R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (j + r >= ng) break;
            stash(g[r]);
            if (j + r + R < ng) load(j + r + R, g[r]);
            run(j + r);
        }
    }
}

struct FbF32 {
    const float* q;
    int64_t ldq;
    const float* x;
    int64_t ldx;
    uint32_t N, D;
    int op;
    __device__ void keys16(const uint32_t* rows, uint32_t s0, uint32_t n, uint32_t r0, int lane, uint32_t* keys) const {
        const int l32 = lane & 31;
        const float* qp = (s0 + l32 < n) ? q + int64_t(rows[s0 + l32]) * ldq : nullptr;
        const float* xp = (r0 + l32 < N) ? x + int64_t(r0 + l32) * ldx : nullptr;
        f32_block_keys<false>(qp, xp, D, op, lane, keys);
    }
};

// int8 codes: key of -sum(q * x), exact in int32 (any order)
struct FbI8 {
    const int8_t* q;
    int64_t ldq;
    const int8_t* x;
    int64_t ldx;
    uint32_t N, D;
    __device__ void keys16(const uint32_t* rows, uint32_t s0, uint32_t n, uint32_t r0, int lane, uint32_t* keys) const {
        const int l32 = lane & 31, hh = lane >> 5;
        const bool qv = s0 + l32 < n;
        const int8_t* qp = qv ? q + int64_t(rows[s0 + l32]) * ldq : nullptr;
#pragma unroll 1
        for (int t = 0; t < 16; ++t) {
            const uint32_t r = r0 + 8 * (t >> 2) + 4 * hh + (t & 3);
            int32_t dot = 0;
            if (qv && r < N) {
                const int8_t* xp = x + int64_t(r) * ldx;
                for (uint32_t d = 0; d < D; ++d) dot += int32_t(qp[d]) * int32_t(xp[d]);
            }
            keys[t] = key_of_i32(-dot);
        }
    }
};

// packed binary codes: Hamming distance (the key itself)
struct FbHam {
    const uint32_t* q;
    const uint32_t* x;
    uint32_t N, W;
    __device__ void keys16(const uint32_t* rows, uint32_t s0, uint32_t n, uint32_t r0, int lane, uint32_t* keys) const {
        const int l32 = lane & 31, hh = lane >> 5;
        const bool qv = s0 + l32 < n;
        const uint32_t* qp = qv ? q + int64_t(rows[s0 + l32]) * W : nullptr;
#pragma unroll 1
        for (int t = 0; t < 16; ++t) {
            const uint32_t r = r0 + 8 * (t >> 2) + 4 * hh + (t & 3);
            uint32_t d = 0;
            if (qv && r < N) {
                const uint32_t* xp = x + int64_t(r) * W;
                for (uint32_t w = 0; w < W; ++w) d += __popc(qp[w] ^ xp[w]);
            }
            keys[t] = d;
        }
    }
};

// PQ asymmetric distances: the tables of the query summed over the subspaces in order from 0.0f
// (the order of the ADC scan), as a float key
struct FbAdc {
    const uint8_t* codes;
    const float* tables;  // [query][M][K]
    uint32_t N, M, K;
    __device__ void keys16(const uint32_t* rows, uint32_t s0, uint32_t n, uint32_t r0, int lane, uint32_t* keys) const {
        const int l32 = lane & 31, hh = lane >> 5;
        const bool qv = s0 + l32 < n;
        const float* t = qv ? tables + int64_t(rows[s0 + l32]) * M * K : nullptr;
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = r0 + 8 * (i >> 2) + 4 * hh + (i & 3);
            float s = 0.0f;
            if (qv && r < N) {
                const uint8_t* c = codes + int64_t(r) * M;
                for (uint32_t m = 0; m < M; ++m) s += t[m * K + c[m]];
            }
            keys[i] = key_of_float(s);
        }
    }
};

// ---- kernels ------------------------------------------------------------------------------------

__device__ inline uint32_t fb_count(const FbArgs& a) {
    const uint32_t n = *a.n_rows;
    return n < a.rmax ? n : a.rmax;
}

// Block-wide search of a histogram: the bin b holding the need-th item (1-based) and the count
// of the bins before it.  256 threads; bins is a multiple of 256.
__device__ inline void fb_find_bin(const uint32_t* h, uint32_t bins, uint32_t need, uint32_t* sh, uint32_t& bin,
                                   uint32_t& before) {
    const uint32_t per = bins / 256, t = threadIdx.x;
    uint32_t part = 0;
    for (uint32_t i = 0; i < per; ++i) part += h[t * per + i];
    sh[t] = part;
    __syncthreads();
    if (t == 0) {
        uint32_t run = 0, b = bins - 1, bef = 0;
        bool found = false;
        for (uint32_t u = 0; u < 256 && !found; ++u) {
            if (run + sh[u] >= need) {
                uint32_t r2 = run;
                for (uint32_t i = 0; i < per; ++i) {
                    const uint32_t c = h[u * per + i];
                    if (r2 + c >= need) {
                        b = u * per + i;
                        bef = r2;
                        found = true;
                        break;
                    }
                    r2 += c;
                }
            }
            run += sh[u];
        }
        if (!found) bef = run - h[bins - 1];  // fewer items than need: the last bin
        sh[256] = b;
        sh[257] = bef;
    }
    __syncthreads();
    bin = sh[256];
    before = sh[257];
    __syncthreads();
}

// The last workgroup of a pass: the histograms of every slot -> the next pass's state.
__device__ inline void fb_resolve(const FbArgs& a, int pass, uint32_t n) {
    __shared__ uint32_t sh[258];
    for (uint32_t s = 0; s < n; ++s) {
        uint32_t* st = a.st + int64_t(s) * 8;
        uint32_t* h = a.hist + int64_t(s) * 2048;
        if (pass <= 2) {
            const uint32_t bins = pass == 2 ? 1024u : 2048u;
            const uint32_t need = pass == 0 ? a.k : st[FB_NEED];
            uint32_t b, before;
            fb_find_bin(h, bins, need, sh, b, before);
            for (uint32_t i = threadIdx.x; i < 2048; i += 256) h[i] = 0;  // ready for the next pass
            if (threadIdx.x == 0) {
                st[FB_NEED] = need - before;
                if (pass == 0) st[FB_PREFIX] = b;
                else if (pass == 1) st[FB_PREFIX] = (st[FB_PREFIX] << 11) | b;
                else st[FB_K] = (st[FB_PREFIX] << 10) | b;
            }
        } else if (pass == 3) {
            if (a.cnt[s] > a.cap) {
                // too many ties for the list: keep those below the id edge that holds `need`
                uint32_t b, before;
                fb_find_bin(a.tidh + int64_t(s) * kFbTieBins, kFbTieBins, st[FB_NEED], sh, b, before);
                if (threadIdx.x == 0) {
                    const uint64_t edge = uint64_t(b + 1) << a.ishift;
                    st[FB_EDGE] = edge > 0xFFFFFFFFull ? 0xFFFFFFFFu : uint32_t(edge);
                    st[FB_OVF] = 1;
                    a.cnt[s] = 0;
                }
            } else if (threadIdx.x == 0) {
                st[FB_OVF] = 0;
            }
        }
        __syncthreads();
    }
}

// Adds c to bin b of slot s's histogram, combining runs of one bin within the lane.
struct FbRun {
    uint32_t* h;
    uint32_t bin = 0xFFFFFFFFu, c = 0;
    __device__ void add(uint32_t b) {
        if (b == bin) {
            ++c;
            return;
        }
        flush();
        bin = b;
        c = 1;
    }
    __device__ void flush() {
        if (c) atomicAdd(h + bin, c);
        c = 0;
    }
};

// One slot's state for a pass (read once per work item).
struct FbSlot {
    uint32_t s, prefix, K, edge;
    FbRun run;
};
// false: the slot takes no part in this pass (pass 4 runs only for rows whose ties overflowed)
__device__ inline bool fb_slot_begin(const FbArgs& a, int pass, uint32_t s, FbSlot& sl) {
    const uint32_t* st = a.st + int64_t(s) * 8;
    if (pass == 4 && !st[FB_OVF]) return false;
    sl.s = s;
    sl.prefix = pass >= 1 ? st[FB_PREFIX] : 0u;
    sl.K = pass >= 3 ? st[FB_K] : 0u;
    sl.edge = pass == 4 ? st[FB_EDGE] : 0u;
    sl.run = FbRun{a.hist + int64_t(s) * 2048};
    return true;
}
// The pass's action for one (key, id) of the slot.
__device__ inline void fb_consume(const FbArgs& a, int pass, FbSlot& sl, uint32_t key, uint32_t id) {
    if (pass == 0) {
        sl.run.add(key >> 21);
    } else if (pass == 1) {
        if ((key >> 21) == sl.prefix) sl.run.add((key >> 10) & 2047u);
    } else if (pass == 2) {
        if ((key >> 10) == sl.prefix) sl.run.add(key & 1023u);
    } else if (key < sl.K || (key == sl.K && (pass == 3 || id < sl.edge))) {
        const uint32_t pos = atomicAdd(a.cnt + sl.s, 1u);
        if (pos < a.cap) {
            a.lkey[int64_t(sl.s) * a.cap + pos] = key;
            a.lid[int64_t(sl.s) * a.cap + pos] = id;
        }
        if (pass == 3 && key == sl.K) {
            const uint32_t bin = id >> a.ishift;  // below kFbTieBins for ids below N (clamped regardless)
            atomicAdd(a.tidh + int64_t(sl.s) * kFbTieBins + (bin < kFbTieBins ? bin : kFbTieBins - 1), 1u);
        }
    }
}
// End of a pass kernel (every thread of every workgroup): the last workgroup to finish (a
// completion ticket, nobody waits) resolves the pass.
__device__ inline void fb_pass_done(const FbArgs& a, int pass, uint32_t n) {
    __shared__ uint32_t s_last;
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        s_last = atomicAdd(a.done + pass, 1u) == gridDim.x - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    fb_resolve(a, pass, n);
}

template <class P>
__global__ __launch_bounds__(256) void fb_pass_kernel(P p, FbArgs a, int pass) {
    const uint32_t n = fb_count(a);
    if (n == 0) return;  // nothing overflowed: every workgroup leaves at once
    const int lane = threadIdx.x & 63, l32 = lane & 31, hh = lane >> 5;
    const uint32_t ngr = (n + 31) / 32, ntl = (a.N + 31) / 32;
    const uint64_t items = uint64_t(ngr) * ntl;
    const uint32_t nw = gridDim.x * 4;
    for (uint64_t it = blockIdx.x * 4 + (threadIdx.x >> 6); it < items; it += nw) {
        const uint32_t g = uint32_t(it / ntl), t = uint32_t(it % ntl);
        const uint32_t s = g * 32 + l32;
        uint32_t keys[16];
        p.keys16(a.rows, g * 32, n, t * 32, lane, keys);
        FbSlot sl;
        if (s >= n || !fb_slot_begin(a, pass, s, sl)) continue;
#pragma unroll 1
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = t * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
            if (r >= a.N) continue;
            fb_consume(a, pass, sl, (a.skip && a.skip[r]) ? kAbsentKey : keys[i], r);
        }
        sl.run.flush();
    }
    fb_pass_done(a, pass, n);
}

__global__ __launch_bounds__(256) void fb_init_kernel(FbArgs a);

template <class P>
va_status fb_launch_pass(va_context* ctx, const P& p, const FbArgs& a, int pass) {
    fb_pass_kernel<P><<<dim3(a.grid), dim3(256), 0, ctx->stream>>>(p, a, pass);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// Enqueues the whole fallback (clear, five passes, selection) for the producer's keys; base
// carries the outputs and the key kind of the scan's selection.
va_status fb_run(va_context* ctx, KeyProducer& kp, const FbArgs& a, const SelectArgs& base);
// fb_run without the selection: the clear and the passes, which write only a's buffers (a caller
// may run them on another stream and select after joining it).
va_status fb_passes(va_context* ctx, KeyProducer& kp, const FbArgs& a);
// The clear before the first pass and the selection after the last, for callers with their own
// pass kernels (the IVF list scan).
va_status fb_init(va_context* ctx, const FbArgs& a);
va_status fb_select(va_context* ctx, const FbArgs& a, const SelectArgs& base, uint32_t key_bits);

}  // namespace va
