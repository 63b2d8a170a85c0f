// va_screen.hip — fp32 flat top-k with an fp16 screening pass on v_mfma_f32_32x32x16_f16.
//
// The fp32 filtering scan (va_dist.hip) runs at the fp32 MFMA rate.  This path finds the same
// top-k with the expensive pass at the fp16 MFMA rate, and returns exactly what the fp32 scan
// returns (same ids, same fp32 distances, bit for bit):
//
//   1. prep:    queries -> fp16, each scaled by a power of two (exact) so its largest entry
//               sits in [2^14, 2^15); fp32 |q|^2 on the side;
//   2. sample:  screened keys of every query against S strided rows; a screened key is an
//               interval [lo, hi] that provably contains the fp32 scan's key s for that pair;
//               tau_q = k-th smallest hi, so the true k-th key s_k <= tau_q.  With a checked
//               rank r < k (step 5 verifies the threshold, so any tau_q is safe) the sample
//               keeps only the smallest approximate hi of each 32-row group and tau_q is the
//               r-th smallest of those;
//   3. screen:  the full pass appends (hi, lo, id) for every pair with lo <= tau_q (every row
//               with s <= s_k is among them);
//   4. bound:   U_q = k-th smallest hi among the candidates (>= s_k again);
//   5. compact: the rows with lo <= U_q (a superset of the fp32 top-k, ~k + a thin band);
//   6. rerank:  the fp32 distance kernel (the same kernel, k order and epilogue as the fp32
//               scan, so the same bits) computes the exact keys of those rows;
//   7. select:  exact (key, id) top-k.  Lists that overflow take the exact chunked path.
//
// The interval comes from a bound on |s_fp16 - s_fp32| (below): rounding each entry to fp16
// (relative 2^-11, absolute 2^-25 for subnormals; the query's scale makes the query side
// relative only), the fp32 accumulation of the exact fp16 products in the MFMA (n * 2^-23 for
// n terms, whatever the adder's order or rounding), the fp32 scan's own accumulation error
// (2D terms), the norms computed in two different orders, and the rounding of the key
// formula.  Anything non-finite (an entry beyond the fp16 range, NaN, inf) makes the pair's
// interval (-inf, NaN-key], so such rows always reach the exact rerank.
//
// Scan kernel: 256 queries x 256 rows per workgroup, 4 waves of 128 x 128 (4 x 4 MFMA blocks,
// 256 accumulators per lane), 64 d-values per LDS stage, two stages in LDS.  Database rows are
// read as fp32 (buffer loads, 16 B per lane, 4 rows x 256 B per wave-wide load), converted to
// fp16 in registers and written to LDS; the fp16 queries go global -> LDS by direct loads.
// One workgroup per CU (130 KiB of LDS).
#include <cfloat>
#include <cmath>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "va_fallback.hpp"
#include "va_internal.hpp"
#include "va_screen_bound.hpp"

namespace va {
namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

namespace scr {
constexpr int TQ = 256;              // queries per workgroup tile
constexpr int TN = 256;              // database rows per workgroup tile
constexpr int KC = 64;               // d-values per LDS stage
constexpr int ROWB = KC * 2;         // bytes per LDS row (fp16)
constexpr int QBYTES = TQ * ROWB;    // 32 KiB of queries per stage
constexpr int XBYTES = TN * ROWB;    // 32 KiB of rows per stage
constexpr int QDMA = QBYTES / 1024 / 4;   // 1 KiB direct loads per wave per stage (8)
constexpr int XLD = TN * KC / 4 / 256;    // float4 row loads per thread per stage (16)
constexpr int PF_OPS = 2;                 // one-dword L2 prefetches per wave per stage (64 rows x 2 lines)
constexpr int PF_AHEAD = 3;               // stages between a row prefetch and the compute
constexpr int DP_ALIGN = KC;              // fp16 query rows are padded to a multiple of KC
}  // namespace scr

// SCREEN_GMIN: per query, the smallest approximate upper bound of each 32-row group (the sample of
// a search whose threshold is checked afterwards, where any threshold is safe)
enum ScreenMode : int { SCREEN_KEYS = 0, SCREEN_FILTER = 1, SCREEN_GMIN = 2 };
// below this many queries a search over the fp16 shadow takes screen16_small_kernel (a 256-query
// tile of screen16_kernel would be mostly padding)
constexpr uint32_t kSmallBatch = 192;
// screen16_small_kernel serves at most this many queries: above it a query tile of
// screen16_kernel (MFMA-bound) costs less than the small kernel's query-register traffic
// (measured at 1M x 768: 64 queries 0.63 ms small, ~0.41 ms in one 256-query screen16 tile)
constexpr uint32_t kSmallBatchMax = 32;

struct ScreenArgs {
    const float* x = nullptr;     // database rows, row j at x + j * ldx
    int64_t ldx = 0;
    uint32_t N = 0, D = 0, Dp = 0, Q = 0;
    const _Float16* qh = nullptr;  // [Q x Dp] scaled fp16 queries
    const float4* qinfo = nullptr; // {|q|^2, |q|, 2^-scale, c0q}
    int op = OP_L2SQ;
    float c1 = 0, cn = 0, c0x = 0, kabs = 0;  // bound coefficients (see screen_bounds)
    // SCREEN_KEYS: out_dot[q * ldo + j] = fp16 dot of query q and row j; out_xx[j] = |x_j|^2
    // SCREEN_GMIN: out_dot[q * ldo + g] (as keys) = smallest approximate upper bound of the rows
    // 32g .. 32g + 31 (ldo = 8 x the row tiles; groups past N hold the key of +inf)
    float* out_dot = nullptr;
    float* out_xx = nullptr;
    int64_t ldo = 0;
    // SCREEN_FILTER: append (dot, |x|^2, id) of every pair that passes the pre-test of thr[q]
    const uint32_t* thr = nullptr;
    uint32_t* cnt = nullptr;
    float* cand_dot = nullptr;
    float* cand_xx = nullptr;
    uint32_t* cand_id = nullptr;
    uint32_t cap = 0;
    uint32_t id_base = 0;
    // fp16 shadow of the database (screen16_kernel): row j at xh + j * Dp, |x_j|^2 at xn[j]
    const _Float16* xh = nullptr;
    const float* xn = nullptr;
    // screen16_small_kernel: row j of the scan is shadow row j * xstride (the threshold sample)
    uint32_t xstride = 1;
    // screen16_kernel: the pre-test constants of each query, {A, B, C, 2^-scale} (pretest_kernel)
    const float4* ptc = nullptr;
    // the candidates' intervals with measured rounding errors (screen_bounds_m) when both are
    // set: qerr[q] >= |fp16 image of q - q| (unscaled), xe[id] >= |fp16(x_id) - x_id|
    const float* qerr = nullptr;
    const float* xe = nullptr;
    float vcn = 0, vgd = 0, vg2d = 0;  // make_bound_v's coefficients
};

// ---- bound of the screened key (va_screen_bound.hpp) --------------------------------------------
static_assert(int(SOP_L2SQ) == int(OP_L2SQ) && int(SOP_L2) == int(OP_L2) && int(SOP_COS_DIST) == int(OP_COS_DIST) &&
                  int(SOP_NEG_DOT) == int(OP_NEG_DOT),
              "screen ops are distance ops");
__device__ __forceinline__ ScreenBound bound_of(const ScreenArgs& a) { return ScreenBound{a.op, a.c1, a.cn, a.c0x, a.kabs}; }
__device__ __forceinline__ void screen_keys(const ScreenArgs& a, float dot, float qq, float nq, float xx, float nx,
                                            float c0q, uint32_t& klo, uint32_t& khi) {
    screen_keys(bound_of(a), dot, qq, nq, xx, nx, c0q, klo, khi);
}
__device__ __forceinline__ PreTest pretest_consts(const ScreenArgs& a, float4 info, uint32_t thr_key) {
    return pretest_consts(bound_of(a), info.x, info.y, info.z, info.w, thr_key);
}

// The pre-test constants of every query, once per search (they depend on the query and its
// threshold only; computing them per tile cost each wave a division and the op's branch per
// query block): ptc[q] = {A, B, C, 2^-scale}.
__global__ __launch_bounds__(256) void pretest_kernel(ScreenArgs a, uint32_t Q, float4* __restrict__ ptc) {
    const uint32_t q = blockIdx.x * 256 + threadIdx.x;
    if (q >= Q) return;
    const float4 inf = a.qinfo[q];
    const PreTest p = pretest_consts(a, inf, a.thr[q]);
    ptc[q] = float4{p.A, p.B, p.C, inf.z};
}

// ---- query preparation: one wave per query ------------------------------------------------
// With vec (D % 4 == 0, 16-byte aligned rows) and Dp <= 2048 the row is read once, as float4s
// all in flight together, and converted from registers.  zero0[0 .. n0) and zero1[0 .. n1) are
// cleared on the side (the scan's counters), so that no separate fill launch is needed.
constexpr uint32_t kPrepRegDp = 2048;
__global__ __launch_bounds__(256) void screen_prep_kernel(const float* __restrict__ q, int64_t ldq, uint32_t Q,
                                                          uint32_t D, uint32_t Dp, _Float16* __restrict__ qh,
                                                          float4* __restrict__ qinfo, float c0, float* __restrict__ qerr,
                                                          int vec, uint32_t* __restrict__ zero0, uint32_t n0,
                                                          uint32_t* __restrict__ zero1, uint32_t n1) {
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n0; i += gridDim.x * 256) zero0[i] = 0u;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n1; i += gridDim.x * 256) zero1[i] = 0u;
    const uint32_t qi = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (qi >= Q) return;
    const float* row = q + int64_t(qi) * ldq;
    _Float16* out = qh + int64_t(qi) * Dp;
    float m = 0.0f, ss = 0.0f;
    bool bad = false;
    if (vec && Dp <= kPrepRegDp) {
        constexpr int NV = kPrepRegDp / 256;
        f32x4v v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t d = 256u * uint32_t(i) + 4u * uint32_t(lane);
            v[i] = d < D ? *reinterpret_cast<const f32x4v*>(row + d) : f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bad |= !(fabsf(v[i][e]) <= FLT_MAX);
                m = fmaxf(m, fabsf(v[i][e]));
                ss = fmaf(v[i][e], v[i][e], ss);
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            m = fmaxf(m, __shfl_xor(m, off));
            ss += __shfl_xor(ss, off);
            bad |= __shfl_xor(int(bad), off) != 0;
        }
        const int sc = query_scale_exponent(m, bad);
        const float scale = ldexpf(1.0f, sc);
        float es = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t d = 256u * uint32_t(i) + 4u * uint32_t(lane);
            if (d >= Dp) break;
            const f32x4v sv = v[i] * scale;  // (zero past D)
            const h4v h = __builtin_convertvector(sv, h4v);
            *reinterpret_cast<h4v*>(out + d) = h;
            const f32x4v ev = __builtin_convertvector(h, f32x4v) - sv;
#pragma unroll
            for (int e = 0; e < 4; ++e) es = fmaf(ev[e], ev[e], es);
        }
        if (qerr) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) es += __shfl_xor(es, off);
        }
        if (lane == 0) {
            const float inv = ldexpf(1.0f, -sc);
            qinfo[qi] = make_float4(ss, sqrtf(ss), inv, c0 * 0x1p-25f * inv);
            if (qerr) qerr[qi] = err_norm_up(es, D) * inv;
        }
        return;
    }
    for (uint32_t d = lane; d < D; d += 64) {
        const float v = row[d];
        bad |= !(fabsf(v) <= FLT_MAX);
        m = fmaxf(m, fabsf(v));
        ss = fmaf(v, v, ss);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        ss += __shfl_xor(ss, off);
        bad |= __shfl_xor(int(bad), off) != 0;
    }
    // scale 2^sc puts the largest entry in [2^14, 2^15): products and sums stay far from fp16
    // and fp32 overflow, and subnormal rounding on the query side is 2^-39 of its largest entry.
    // At most 2^40, so that the scan's pre-test constants stay finite.
    const int sc = query_scale_exponent(m, bad);
    const float scale = ldexpf(1.0f, sc);
    float es = 0.0f;  // squared norm of the rounding error of the scaled query (differences exact)
    for (uint32_t d = lane; d < Dp; d += 64) {
        const float v = d < D ? row[d] * scale : 0.0f;
        const _Float16 h = _Float16(v);
        out[d] = h;
        const float e = float(h) - v;
        es = fmaf(e, e, es);
    }
    if (qerr) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) es += __shfl_xor(es, off);
    }
    if (lane == 0) {
        const float inv = ldexpf(1.0f, -sc);
        qinfo[qi] = make_float4(ss, sqrtf(ss), inv, c0 * 0x1p-25f * inv);
        if (qerr) qerr[qi] = err_norm_up(es, D) * inv;
    }
}

// ---- the filter epilogue of both screening scans ---------------------------------------------
// acc[m][n] holds the 32 x 32 block (rows wn*128 + 32m .., queries wq*128 + 32n ..) of the tile's
// fp16 dots (queries scaled by 2^scale); xxs/xxp/nxp are the tile's row norms (xxp/nxp NaN for
// flagged rows); dump is 32 KiB of LDS private to the wave.
__device__ __forceinline__ void filter_epilogue(const ScreenArgs& a, f32x16 (&acc)[4][4], const float4 (&qinf)[4],
                                                const uint32_t (&qthr)[4], f32x4v* dump, const float* xxs,
                                                const float* xxp, const float* nxp, uint32_t qs, uint32_t rs,
                                                uint32_t qc, uint32_t rc, int wq, int wn, int lane) {
    const int l32 = lane & 31, hh = lane >> 5;
    // The accumulators leave the AGPRs only through LDS stores (two query blocks at a time,
    // 32 KiB per wave of the free LDS), so they are never copied to VGPRs wholesale.  Per
    // query block the pre-test over the lane's 64 values (read back from LDS) builds a bit
    // mask without branches; one atomic per lane reserves list space; the appends of a pair
    // of blocks run after both atomics are issued, so the round trips overlap.
    uint64_t valid = 0;  // rows of the tile (the last tile is partial)
#pragma unroll
    for (int t = 0; t < 64; ++t) {
        const int r = wn * 128 + 32 * (t >> 4) + 8 * ((t >> 2) & 3) + 4 * hh + (t & 3);
        valid |= uint64_t(uint32_t(r) < rc) << t;
    }
    auto dump_half = [&](auto HC) {
        constexpr int h = decltype(HC)::value;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    f32x4v v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[m][2 * h + b][4 * j + e];
                    dump[(16 * b + 4 * m + j) * 64 + lane] = v;
                }
    };
    // Quick rejection: the pre-test's right-hand side A|x|^2 + B|x| + C over the lane's 64 rows is
    // bounded below by its value at the corner of their (|x|^2, |x|) box that A's and B's signs
    // select (fp32 fma is monotone in each argument for a multiplier of fixed sign), so a lane
    // whose largest value is below that bound passes nothing.  Flagged (NaN) rows disable it.
    float bxlo = INFINITY, bxhi = -INFINITY, bnlo = INFINITY, bnhi = -INFINITY;
    bool bflag = false;
#pragma unroll 1
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = wn * 128 + 32 * m + 8 * j + 4 * hh;
            const f32x4v xx = *reinterpret_cast<const f32x4v*>(xxp + r);
            const f32x4v nx = *reinterpret_cast<const f32x4v*>(nxp + r);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bflag |= !(xx[e] == xx[e]) || !(nx[e] == nx[e]);
                bxlo = fminf(bxlo, xx[e]);
                bxhi = fmaxf(bxhi, xx[e]);
                bnlo = fminf(bnlo, nx[e]);
                bnhi = fmaxf(bnhi, nx[e]);
            }
        }
    auto test_block = [&](int n) -> uint64_t {
        const PreTest pt = pretest_consts(a, qinf[n], qthr[n]);
        const f32x4v* src = dump + 16 * (n & 1) * 64 + lane;
        if (!bflag) {
            const float lo = fmaf(pt.A, pt.A >= 0.0f ? bxlo : bxhi, fmaf(pt.B, pt.B >= 0.0f ? bnlo : bnhi, pt.C));
            float mx = -INFINITY;
#pragma unroll 4
            for (int i = 0; i < 16; ++i) {
                const f32x4v v = src[i * 64];
                mx = fmaxf(mx, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
            }
            if (mx < lo) return 0;
            asm volatile("" ::: "memory");  // the full test re-reads the values
        }
        uint64_t mk = 0;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = wn * 128 + 32 * m + 8 * j + 4 * hh;
                const f32x4v xx = *reinterpret_cast<const f32x4v*>(xxp + r);
                const f32x4v nx = *reinterpret_cast<const f32x4v*>(nxp + r);
                const f32x4v v = src[(4 * m + j) * 64];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float rhs = fmaf(pt.A, xx[e], fmaf(pt.B, nx[e], pt.C));
                    mk |= uint64_t(!(v[e] < rhs)) << (16 * m + 4 * j + e);
                }
            }
        return (uint32_t(wq * 128 + 32 * n + l32) < qc) ? (mk & valid) : 0;
    };
    // lanes l and l + 32 hold the same query (the two row halves of each 8-row group): one
    // atomic reserves the pair's passes, and the second lane takes the places after the first's
    auto reserve = [&](int n, uint64_t mk) -> uint32_t {
        const uint32_t qi = qs + uint32_t(wq * 128 + 32 * n + l32);
        const uint32_t c = uint32_t(__popcll(mk));
        const uint32_t other = uint32_t(__shfl_xor(int(c), 32));
        uint32_t base = 0;
        if (hh == 0 && c + other) base = atomicAdd(a.cnt + qi, c + other);
        base = uint32_t(__shfl(int(base), l32));
        return hh ? base + other : base;
    };
    auto append = [&](int n, uint64_t mk, uint32_t pos) {
        const uint32_t qi = qs + uint32_t(wq * 128 + 32 * n + l32);
        const float inv = qinf[n].z;
        const float* src = reinterpret_cast<const float*>(dump + 16 * (n & 1) * 64 + lane);
        for (uint32_t i = pos; mk && i < a.cap; ++i) {
            const int t = __builtin_ctzll(mk);
            mk &= mk - 1;
            const int r = wn * 128 + 32 * (t >> 4) + 8 * ((t >> 2) & 3) + 4 * hh + (t & 3);
            const float v = src[(t >> 2) * 256 + (t & 3)];
            const int64_t o = int64_t(qi) * a.cap + i;
            a.cand_dot[o] = v * inv;
            a.cand_xx[o] = xxs[r];
            a.cand_id[o] = a.id_base + rs + uint32_t(r);
        }
    };
    dump_half(std::integral_constant<int, 0>());
    {
        const uint64_t m0 = test_block(0);
        const uint32_t p0 = reserve(0, m0);
        const uint64_t m1 = test_block(1);
        const uint32_t p1 = reserve(1, m1);
        append(0, m0, p0);
        append(1, m1, p1);
    }
    dump_half(std::integral_constant<int, 1>());
    {
        const uint64_t m2 = test_block(2);
        const uint32_t p2 = reserve(2, m2);
        const uint64_t m3 = test_block(3);
        const uint32_t p3 = reserve(3, m3);
        append(2, m2, p2);
        append(3, m3, p3);
    }
}

// ---- the screening scan -----------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256, 1) void screen_kernel(ScreenArgs a) {
    using namespace scr;
    // LDS: two query stages and two row stages (separate objects, so the compiler sees that the
    // conversion's writes to one row slot never alias the fragment reads of the other), the
    // landing area of the L2 prefetches, and the row norms.  After the main loop the four
    // stage slots hold the epilogue's accumulator dumps.
    __shared__ __attribute__((aligned(1024))) char qslot0[QBYTES];
    __shared__ __attribute__((aligned(1024))) char qslot1[QBYTES];
    __shared__ __attribute__((aligned(1024))) char xslot0[XBYTES];
    __shared__ __attribute__((aligned(1024))) char xslot1[XBYTES];
    __shared__ __attribute__((aligned(1024))) char pf_sink[4 * PF_OPS * 256];
    __shared__ __attribute__((aligned(16))) float norms[3 * TN];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave & 1;   // query half of the tile
    const int wn = wave >> 1;  // row half of the tile
    const int l32 = lane & 31;
    const int hh = lane >> 5;

    // XCD-aware order (as in the fp32 scan): XCD x takes row tiles x, x+8, ... and runs every
    // query block of a tile back to back
    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t xcd = blockIdx.x % kXcds, seq = blockIdx.x / kXcds;
    const uint32_t qb = seq % nqb;
    const uint32_t tb = (seq / nqb) * kXcds + xcd;
    if (tb * uint32_t(TN) >= a.N) return;  // padding workgroup
    const uint32_t qs = qb * TQ, rs = tb * TN;
    const uint32_t qc = min(uint32_t(TQ), a.Q - qs);
    const uint32_t rc = min(uint32_t(TN), a.N - rs);
    const uint32_t nst = a.Dp / KC;

    // query direct loads: wave w fills 1 KiB groups g = w + 4i, rows 8g .. 8g+7; lane L loads
    // row 8g + L/8 at physical chunk L%8 = logical chunk (L%8) ^ ((row >> 1) & 7).  Rows past qc
    // read past the descriptor and land as zeros.
    const dma_rsrc qres = make_dma_rsrc(a.qh + int64_t(qs) * a.Dp, qc * a.Dp * 2u);
    uint32_t qoff[QDMA];
#pragma unroll
    for (int i = 0; i < QDMA; ++i) {
        const int row = 8 * (wave + 4 * i) + (lane >> 3);
        const int c = (lane & 7) ^ ((row >> 1) & 7);
        qoff[i] = uint32_t(row) * a.Dp * 2u + 16u * uint32_t(c);
    }
    // row loads: lane L of wave w reads rows 64w + 4i + L/16 (i < 16), d-values 4(L%16) .. +3 of
    // the stage.  The descriptor ends at the tile's last valid byte, so rows past rc read zeros;
    // d-values past D are skipped explicitly (they would alias the next row).
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a.x + int64_t(rs) * a.ldx), 0, int((uint64_t(rc - 1) * a.ldx + a.D) * 4), 0x00020000);
    const uint32_t xcol = 4u * uint32_t(lane & 15);
    const uint32_t xbase = (uint32_t(64 * wave) + uint32_t(lane >> 4)) * uint32_t(a.ldx) * 4u + xcol * 4u;
    const uint32_t xstep = 4u * uint32_t(a.ldx) * 4u;
    // LDS byte offsets of this lane's converted values: row r = 64w + 4i + L/16, logical chunk
    // (L%16)/2, half L%2; physical chunk = logical ^ ((r >> 1) & 7)
    const int wc = (lane & 15) >> 1;
    const int wr0 = 64 * wave + (lane >> 4);
    auto xw_off = [&](int i) -> uint32_t {
        const int r = wr0 + 4 * i;
        return uint32_t(r * ROWB + 16 * (wc ^ ((r >> 1) & 7)) + 8 * (lane & 1));
    };
    // fragment offsets: rows 32-aligned + l32, so the swizzle is (l32 >> 1) & 7 for both operands
    const int swz = (l32 >> 1) & 7;
    const uint32_t a_off = uint32_t((wn * 128 + l32) * ROWB);
    const uint32_t b_off = uint32_t((wq * 128 + l32) * ROWB);

    // the lane's four queries (one per 32-query block): their data is loaded before the main loop
    // so that the epilogue does not wait for it
    float4 qinf[4];
    uint32_t qthr[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        const uint32_t qi = qs + min(uint32_t(wq * 128 + 32 * n + l32), qc - 1);
        qinf[n] = a.qinfo[qi];
        qthr[n] = MODE == SCREEN_FILTER ? a.thr[qi] : 0u;
    }

    f32x4v st[XLD];
    float xs[XLD];
#pragma unroll
    for (int i = 0; i < XLD; ++i) xs[i] = 0.0f;
    f32x16 acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[m][n][v] = 0.0f;

    auto slot_ptr = [&](int slot) -> char* { return slot ? xslot1 : xslot0; };

    auto issue_q = [&](uint32_t s, int qslot) {
        const uint32_t d0 = s * KC;
        const bool ok = d0 < a.Dp;
#pragma unroll
        for (int i = 0; i < QDMA; ++i) {
            const int grp = wave + 4 * i;
            lds_dma16(qres, ok ? qoff[i] + d0 * 2u : kDmaSkip, lds_addr_of((qslot ? qslot1 : qslot0) + grp * 1024));
        }
    };
    auto convert_row = [&](int slot, int i) {
        const f32x4v v = st[i];
        xs[i] = fmaf(v[0], v[0], xs[i]);
        xs[i] = fmaf(v[1], v[1], xs[i]);
        xs[i] = fmaf(v[2], v[2], xs[i]);
        xs[i] = fmaf(v[3], v[3], xs[i]);
        const h4v h = __builtin_convertvector(v, h4v);
        *reinterpret_cast<h4v*>(slot_ptr(slot) + xw_off(i)) = h;
    };
    auto convert_x = [&](int slot) {
#pragma unroll
        for (int i = 0; i < XLD; ++i) convert_row(slot, i);
    };
    auto load_row = [&](uint32_t coff, int i) {
        const uint32_t off = xbase + uint32_t(i) * xstep + coff;
        st[i] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(xres, int(off), 0, 0));
    };
    auto col_off = [&](uint32_t s) -> uint32_t {
        const uint32_t d0 = s * KC;
        uint32_t coff = d0 + xcol < a.D ? d0 * 4u : 0x80000000u;
        asm volatile("" : "+v"(coff));
        return coff;
    };
    // d-values past D: an offset of 2^31 + (< 2^31) lies past the descriptor and reads zeros
    // (the select is hidden from the optimizer, which would otherwise branch around each load)
    auto load_x = [&](uint32_t s) {
        const uint32_t coff = col_off(s);
#pragma unroll
        for (int i = 0; i < XLD; ++i) load_row(coff, i);
    };
    // L2 prefetch of this wave's rows of stage s: one dword per 128-byte line (rows 64w + 32i +
    // L/2, line L%2 of the row's 256 bytes), landing in a per-wave sink of the LDS.  Invisible
    // to the compiler's wait counts, like the query loads.
    const uint32_t pf_base = (uint32_t(64 * wave) + uint32_t(lane >> 1)) * uint32_t(a.ldx) * 4u + 128u * uint32_t(lane & 1);
    const dma_rsrc pres = make_dma_rsrc(a.x + int64_t(rs) * a.ldx, uint32_t((uint64_t(rc - 1) * a.ldx + a.D) * 4));
    auto prefetch = [&](uint32_t s) {
        const uint32_t d0 = s * KC;
        const bool ok = d0 + 32u * uint32_t(lane & 1) < a.D;
#pragma unroll
        for (int i = 0; i < PF_OPS; ++i) {
            const uint32_t off = ok ? pf_base + uint32_t(i) * 32u * uint32_t(a.ldx) * 4u + d0 * 4u : kDmaSkip;
            lds_dma4(pres, off, lds_addr_of(pf_sink + (wave * PF_OPS + i) * 256));
        }
    };
    h8v av[4], bv[4];
    auto frags = [&](int slot, int t) {
        const char* base = slot_ptr(slot);
        const char* qbase = slot ? qslot1 : qslot0;
        const uint32_t ko = 16u * uint32_t((2 * t + hh) ^ swz);
#pragma unroll
        for (int m = 0; m < 4; ++m) av[m] = *reinterpret_cast<const h8v*>(base + a_off + m * 32 * ROWB + ko);
#pragma unroll
        for (int n = 0; n < 4; ++n) bv[n] = *reinterpret_cast<const h8v*>(qbase + b_off + n * 32 * ROWB + ko);
    };
    auto mma = [&]() {
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int n = 0; n < 4; ++n)
                acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[m], bv[n], acc[m][n], 0, 0, 0);
    };

    // prologue: query stage 0 and row stage 0 in slot 0, row stage 1 in registers, rows of stages
    // 1 .. PF_AHEAD-1 prefetched
    issue_q(0, 0);
    load_x(0);
    convert_x(0);
    load_x(1);
#pragma unroll
    for (uint32_t p = 1; p < PF_AHEAD; ++p) prefetch(p);
    wait_vmcnt<XLD + PF_OPS * (PF_AHEAD - 1)>();  // the query loads (older than the rest)
    __syncthreads();
    // Stage s computes from slot s&1.  At its start the rows of stage s+1 (loaded during stage
    // s-1) are complete (only younger prefetches may be in flight); it issues the query loads of
    // stage s+1 into the other query slot and converts stage s+1's rows into the other row slot
    // (both last read in stage s-1, before the previous barrier), loads stage s+2's rows and
    // prefetches stage s+PF_AHEAD's, interleaved with the MFMAs of its first k-step: one wave per
    // SIMD, so VALU work not hidden under MFMAs leaves the matrix unit idle.  Before its closing
    // barrier (which publishes stage s+1) it waits for its query loads only.  Past the last stage
    // the loads skip (zeros).  Scheduling barriers keep each stage's work inside its stage.
    auto stage = [&](uint32_t s, auto cur) {
        constexpr int C = decltype(cur)::value;
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<PF_OPS * (PF_AHEAD - 2)>();
        issue_q(s + 1, C ^ 1);
        frags(C, 0);
        __builtin_amdgcn_sched_barrier(0);
        // k-step 0: each MFMA is followed by the conversion of one row of stage s+1 and the load
        // of the same row of stage s+2 into the registers just freed
        const uint32_t coff = col_off(s + 2);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[i >> 2][i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i >> 2], bv[i & 3], acc[i >> 2][i & 3], 0, 0, 0);
            convert_row(C ^ 1, i);
            load_row(coff, i);
            __builtin_amdgcn_sched_barrier(0);
        }
        prefetch(s + PF_AHEAD);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 1; t < KC / 16; ++t) {
            frags(C, t);
            mma();
        }
        wait_vmcnt<XLD + PF_OPS>();  // younger than the query loads: stage s+2's rows and prefetch
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };
    uint32_t s = 0;
    for (; s + 1 < nst; s += 2) {
        stage(s, std::integral_constant<int, 0>());
        stage(s + 1, std::integral_constant<int, 1>());
    }
    if (s < nst) stage(s, std::integral_constant<int, 0>());
    // loads issued past the last stage (zeros) land in LDS the epilogue reuses
    wait_vmcnt<0>();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

    // squared norms of the tile's rows: the 16 lanes of a row hold 4 columns each; summed across
    // them with DPP (quad xor 1, quad xor 2, mirror within 8, mirror within 16: every lane ends
    // with the total, in one fixed order).  The pre-test copies flag (NaN) rows whose fp16 image
    // may hold an infinity (|x| near 65504 or more) and, for cosine, rows too small for the linear
    // form; their |x| is the hardware square root (the pre-test's 2^-18 margin covers its ulp).
    float* xxs = norms;
    float* xxp = norms + TN;
    float* nxp = norms + 2 * TN;
    const float tiny = a.op == OP_COS_DIST ? 8.0f * a.c0x : 0.0f;
    auto dpp_add = [](float v, auto CTRL) -> float {
        constexpr int ctrl = decltype(CTRL)::value;
        return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
    };
#pragma unroll
    for (int i = 0; i < XLD; ++i) {
        float t = xs[i];
        t = dpp_add(t, std::integral_constant<int, 0xB1>());   // quad_perm [1,0,3,2]
        t = dpp_add(t, std::integral_constant<int, 0x4E>());   // quad_perm [2,3,0,1]
        t = dpp_add(t, std::integral_constant<int, 0x141>());  // row_half_mirror
        t = dpp_add(t, std::integral_constant<int, 0x140>());  // row_mirror
        if ((lane & 15) == 0) {
            const int r = wr0 + 4 * i;
            const float nx = __builtin_amdgcn_sqrtf(t);
            xxs[r] = t;
            const bool flag = !(t < 4.29e9f) || nx < tiny;
            xxp[r] = flag ? __builtin_nanf("") : t;
            nxp[r] = flag ? __builtin_nanf("") : nx;
        }
    }
    __syncthreads();

    if constexpr (MODE == SCREEN_GMIN) {
        // v = alpha acc + beta approximates the pair's upper bound hi (the interval's error term
        // without its small absolute part, no clamp): alpha = an * ra(row), beta = b + bb * rb(row)
        //   cosine:  1 - dot / (|q||x|) + E      an = -2^-sc / |q|, ra = 1/|x|, b = 1 + E
        //   L2^2:    |q|^2 + |x|^2 - 2 dot + E   an = -2^(1-sc), b = (1+c)|q|^2, bb = 1+c, rb = |x|^2
        //   -dot:    -dot + c1 |q||x|            an = -2^-sc, bb = c1 |q|, rb = |x|
        // (L2 takes the square root of the group's smallest L2^2 value.)  Only a checked
        // threshold is taken from these values, so they need not bound anything.
        const float cE = (a.c1 + a.cn) * (1.0f + 0x1p-20f);
        uint32_t* outk = reinterpret_cast<uint32_t*>(a.out_dot);
        const bool cosine = a.op == OP_COS_DIST, ndot = a.op == OP_NEG_DOT;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const float4 inf = qinf[n];  // {|q|^2, |q|, 2^-scale, c0q}
            const float an = cosine ? -inf.z / inf.y : ndot ? -inf.z : -2.0f * inf.z;
            const float b = cosine ? 1.0f + cE : ndot ? 0.0f : (1.0f + cE) * inf.x;
            const float bb = cosine ? 0.0f : ndot ? a.c1 * inf.y : 1.0f + cE;
            uint32_t g[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                float mn = INFINITY;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r0 = wn * 128 + 32 * m + 8 * j + 4 * hh;
                    const f32x4v xx = *reinterpret_cast<const f32x4v*>(xxs + r0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float ra = cosine ? __builtin_amdgcn_rsqf(xx[e]) : 1.0f;
                        const float rb = ndot ? __builtin_amdgcn_sqrtf(xx[e]) : xx[e];
                        const float v = fmaf(an * ra, acc[m][n][4 * j + e], fmaf(bb, rb, b));
                        mn = uint32_t(r0 + e) < rc ? fminf(mn, v) : mn;
                    }
                }
                mn = fminf(mn, __shfl_xor(mn, 32));
                if (a.op == OP_L2) mn = __builtin_amdgcn_sqrtf(fmaxf(mn, 0.0f));
                g[m] = key_of_float(mn);
            }
            const uint32_t ql = uint32_t(wq * 128 + 32 * n + l32);
            if (hh == 0 && ql < qc)
                *reinterpret_cast<uint4*>(outk + int64_t(qs + ql) * a.ldo + tb * 8 + wn * 4) =
                    make_uint4(g[0], g[1], g[2], g[3]);
        }
        return;
    } else if constexpr (MODE == SCREEN_KEYS) {
        // dense fp16 dots (the bounds are computed by screen_bound_kernel) and the row norms
        if (qb == 0 && wave == 0)
            for (uint32_t r = uint32_t(lane); r < rc; r += 64) a.out_xx[rs + r] = xxs[r];
        // Each query block leaves through the wave's free LDS slot (32 queries x 128 rows, rows
        // padded to 129 words) and is stored one output row at a time with the lanes on
        // consecutive database rows: 256-byte stores instead of scattered words.
        float* stg = reinterpret_cast<float*>(wave == 0 ? qslot0 : wave == 1 ? qslot1 : wave == 2 ? xslot0 : xslot1);
        static_assert(XBYTES >= 32 * 129 * 4 && QBYTES >= 32 * 129 * 4, "key staging: 16.5 KiB per wave");
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const float inv = qinf[n].z;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        stg[l32 * 129 + 32 * m + 8 * j + 4 * hh + e] = acc[m][n][4 * j + e] * inv;
            __syncthreads();
            const uint32_t r0 = uint32_t(wn * 128 + lane);
            for (int q = 0; q < 32; ++q) {
                const uint32_t ql = uint32_t(wq * 128 + 32 * n + q);
                if (ql >= qc) break;
                float* o = a.out_dot + int64_t(qs + ql) * a.ldo + rs;
                if (r0 < rc) o[r0] = stg[q * 129 + lane];
                if (r0 + 64 < rc) o[r0 + 64] = stg[q * 129 + 64 + lane];
            }
            __syncthreads();  // the block is stored before the next one overwrites it
        }
        return;
    } else {
        // The accumulators leave through LDS, 32 KiB per wave (one of the four stage slots).
        static_assert(XBYTES >= 2 * 64 * 64 * 4 && QBYTES >= 2 * 64 * 64 * 4, "dump: 32 KiB per wave");
        f32x4v* dump = reinterpret_cast<f32x4v*>(wave == 0 ? qslot0 : wave == 1 ? qslot1 : wave == 2 ? xslot0 : xslot1);
        filter_epilogue(a, acc, qinf, qthr, dump, xxs, xxp, nxp, qs, rs, qc, rc, wq, wn, lane);
    }
}

// ---- the screening scan over an fp16 shadow of the database ---------------------------------------
// 256 queries x 256 rows per workgroup as screen_kernel's filter mode, but the rows come already
// rounded to fp16 (the same RNE rounding) with their squared norms, so both operands move
// global -> LDS by direct loads and the main loop is MFMAs, fragment reads and loads only.
// Sixteen waves of 64 queries x 64 rows (2 x 2 MFMA blocks, 64 accumulators: four waves per
// SIMD, so one wave's fragment waits and barrier are covered by the others' MFMAs; one wave per
// SIMD with 128 x 128 tiles ran the same loop 10-25 % slower).  64 d-values per stage, two
// stages in LDS (128 KiB); the fragments of k-step g+1 are read while the 4 MFMAs of k-step g
// run, and the stage barrier sits inside the last k-step of a stage, after its fragments are in
// registers (a bare s_barrier: the direct loads of the next stage stay in flight across it).
namespace s16 {
constexpr int TQ = 256, KC = 64;  // (TQ: the default query tile)
constexpr int ROWB = KC * 2;              // bytes per LDS row
// the wave layout of the launch: waves per workgroup, 32-query and 32-row blocks per wave
constexpr int kWaves = 16, kQueryBlocks = 2, kRowBlocks = 2;
// A workgroup of WAVES waves, each (32 NQB queries) x (32 MB rows), over a tile of TQ queries x
// TN rows; a stage holds 64 d-values of both (queries, then rows), two stages in LDS.
template <int WAVES, int NQB, int MB, int TQ_ = TQ>
struct Shape {
    static constexpr int TQ = TQ_;
    static constexpr int WQ = 32 * NQB, WN = 32 * MB;  // a wave's queries x rows
    static constexpr int QW = TQ / WQ;                 // waves along the queries
    static constexpr int TN = WN * (WAVES / QW);
    static constexpr int OPQ = TQ * ROWB, OPX = TN * ROWB;
    static constexpr int STAGE = OPQ + OPX;
    static constexpr int LDS = 2 * STAGE;
    // 1 KiB direct-load groups (8 rows) per stage: GQ of queries, GX of rows; a wave loads up to
    // LPW of each, LMIN loads in all at least
    static constexpr int GQ = OPQ / 1024, GX = OPX / 1024;
    static constexpr int LPW = ((GQ > GX ? GQ : GX) + WAVES - 1) / WAVES, LMIN = GQ / WAVES + GX / WAVES;
    static_assert(QW * WQ == TQ && WAVES % QW == 0 && TN % 8 == 0, "wave layout");
    static_assert(64 * WAVES >= TN && 64 * WAVES >= TQ, "one thread per row and query");
    static_assert(WAVES * 4096 <= STAGE, "the epilogue's dump fits in one stage slot");
};
}  // namespace s16

// WAVES waves of (32 NQB queries) x (32 MB rows) over tiles of TQ_ queries: four waves per SIMD
// at 16 waves.  MODE SCREEN_FILTER: the screen's pre-tested appends; SCREEN_GMIN: the threshold
// sample's group minima (screen_kernel's SCREEN_GMIN values) over shadow rows j * xstride.
template <int WAVES, int NQB, int MB, int TQ_ = s16::TQ, int MODE = SCREEN_FILTER>
__global__ __launch_bounds__(64 * WAVES, 16 / WAVES) void screen16_kernel(ScreenArgs a) {
    using namespace s16;
    using Sh = Shape<WAVES, NQB, MB, TQ_>;
    constexpr int TQ = Sh::TQ;
    static_assert(MODE == SCREEN_FILTER || MODE == SCREEN_GMIN, "filter or group-minimum epilogue");
    static_assert(MODE != SCREEN_GMIN || (Sh::TN == scr::TN && 32 * MB * (WAVES / Sh::QW) == scr::TN),
                  "the group layout of screen_kernel's SCREEN_GMIN output");
    // rows of the scan: shadow rows j * xs (the sample's stride; 1 for the screen)
    const uint32_t xs = MODE == SCREEN_GMIN ? a.xstride : 1u;
    constexpr int WQ = Sh::WQ, WN = Sh::WN, QW = Sh::QW, TN = Sh::TN;
    constexpr int OPQ = Sh::OPQ, STAGE = Sh::STAGE, GQ = Sh::GQ, GX = Sh::GX, LPW = Sh::LPW;
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    __shared__ __attribute__((aligned(16))) float norms[3 * TN];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave % QW, wn = wave / QW, l32 = lane & 31, hh = lane >> 5;
    // Persistent: the workgroup takes the tiles T = blockIdx.x, blockIdx.x + gridDim.x, ... in
    // screen_kernel's XCD-aware order (gridDim.x is a multiple of the XCD count, so all of a
    // workgroup's tiles run on its XCD).  The next tile's first stage is loaded during this tile's
    // epilogue, into stage slot 0 (the epilogue's LDS dump uses slot 1 only), so after the first
    // tile no workgroup waits for a prologue load with its matrix cores idle.
    const uint32_t nqb = (a.Q + TQ - 1) / TQ;
    const uint32_t ntb = (a.N + TN - 1) / TN;
    const uint32_t total = nqb * ((ntb + kXcds - 1) / kXcds) * kXcds;
    auto tile_of = [&](uint32_t T, uint32_t& qb, uint32_t& tb) {
        const uint32_t xcd = T % kXcds, seq = T / kXcds;
        qb = seq % nqb;
        tb = (seq / nqb) * kXcds + xcd;
    };
    // the first tile at or after T (in steps of gridDim.x) that holds rows
    auto next_tile = [&](uint32_t T) {
        for (; T < total; T += gridDim.x) {
            uint32_t qb, tb;
            tile_of(T, qb, tb);
            if (tb * uint32_t(TN) < a.N) return T;
        }
        return total;
    };
    const uint32_t nst = a.Dp / KC;

    // Direct loads: wave w fills 1 KiB groups g = w + WAVES i (rows 8g .. 8g+7) of each operand;
    // lane L loads row 8g + L/8 at physical chunk L%8 = logical chunk (L%8) ^ ((row >> 1) & 7).
    // Rows past qc / rc read past their descriptor and land as zeros.
    auto tile_rsrc = [&](uint32_t T, dma_rsrc& qr, dma_rsrc& xr) {
        uint32_t qb, tb;
        tile_of(T, qb, tb);
        const uint32_t q0 = qb * TQ, r0 = tb * TN;
        qr = make_dma_rsrc(a.qh + int64_t(q0) * a.Dp, min(uint32_t(TQ), a.Q - q0) * a.Dp * 2u);
        xr = make_dma_rsrc(a.xh + int64_t(r0) * xs * a.Dp, ((min(uint32_t(TN), a.N - r0) - 1u) * xs + 1u) * a.Dp * 2u);
    };
    uint32_t off[LPW], offx[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const int row = 8 * (wave + WAVES * i) + (lane >> 3);
        const uint32_t ch = 16u * uint32_t((lane & 7) ^ ((row >> 1) & 7));
        off[i] = uint32_t(row) * a.Dp * 2u + ch;
        offx[i] = uint32_t(row) * xs * a.Dp * 2u + ch;
    }
    const uint32_t lds0 = lds_addr_of(lds);
    auto issue_with = [&](const dma_rsrc& qr, const dma_rsrc& xr, uint32_t s) {
        const uint32_t d0 = s * KC;
        const bool ok = d0 < a.Dp;
        const uint32_t sb = lds0 + (s & 1u) * uint32_t(STAGE);
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int g = wave + WAVES * i;  // wave-uniform; compile-time true when the waves' LPW loads
                                             // cover exactly the operand's groups
            if (GQ == LPW * WAVES || g < GQ) lds_dma16(qr, ok ? off[i] + d0 * 2u : kDmaSkip, sb + uint32_t(g) * 1024u);
            if (GX == LPW * WAVES || g < GX)
                lds_dma16(xr, ok ? offx[i] + d0 * 2u : kDmaSkip, sb + uint32_t(OPQ + g * 1024));
        }
    };
    // fragment rows start at multiples of 32, so the chunk swizzle is (l32 >> 1) & 7 for both
    const int swz = (l32 >> 1) & 7;
    const uint32_t a_off = uint32_t(OPQ + (wn * WN + l32) * ROWB);
    const uint32_t b_off = uint32_t((wq * WQ + l32) * ROWB);

    f32x16 acc[MB][NQB];
    h8v fa[2][MB], fb[2][NQB];
    auto read_frags = [&](int buf, uint32_t slot, int t) {
        const char* base = lds + slot * STAGE;
        const uint32_t ko = 16u * uint32_t((2 * t + hh) ^ swz);
#pragma unroll
        for (int m = 0; m < MB; ++m) fa[buf][m] = *reinterpret_cast<const h8v*>(base + a_off + m * 32 * ROWB + ko);
#pragma unroll
        for (int n = 0; n < NQB; ++n) fb[buf][n] = *reinterpret_cast<const h8v*>(base + b_off + n * 32 * ROWB + ko);
    };
    auto mma = [&](int buf) {
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int n = 0; n < NQB; ++n)
                acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[buf][m], fb[buf][n], acc[m][n], 0, 0, 0);
    };
    // the MB + NQB fragment reads of the next k-step go between the MB NQB MFMAs
    auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < MB * NQB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < MB + NQB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    };
    // workgroup barrier without the release fence of __syncthreads (which would also wait for
    // the direct loads in flight); this wave's LDS reads are complete before it
    auto barrier = [&]() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    float* xxs = norms;
    float* xxp = norms + TN;
    float* nxp = norms + 2 * TN;
    // uniform: kept in a scalar register across the tile loop
    const float tiny = __builtin_bit_cast(
        float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, a.op == OP_COS_DIST ? 8.0f * a.c0x : 0.0f)));
    __shared__ float4 gbox[TN / 4];
    __shared__ float4 ptl[TQ];  // {A, B, C, 2^-scale} of the tile's queries
    auto row_of = [&](int t) { return wn * WN + 32 * (t >> 4) + 8 * ((t >> 2) & 3) + 4 * hh + (t & 3); };
    using Mask = std::conditional_t<(16 * MB > 32), uint64_t, uint32_t>;  // bit t: value t of a block
    // the epilogue's LDS: one 32-row block of a query block (16 values a lane) per wave, in stage
    // slot 1
    f32x4v* dump = reinterpret_cast<f32x4v*>(lds + STAGE + wave * 4096) + lane;  // [c][lane], c < 4

    uint32_t T = next_tile(blockIdx.x);
    if (T >= total) return;
    dma_rsrc qres, xres;
    tile_rsrc(T, qres, xres);
    issue_with(qres, xres, 0);  // later tiles: stage 0 is loaded during the previous epilogue
    while (T < total) {
        uint32_t qb, tb;
        tile_of(T, qb, tb);
        const uint32_t qs = qb * TQ, rs = tb * TN;
        const uint32_t qc = min(uint32_t(TQ), a.Q - qs), rc = min(uint32_t(TN), a.N - rs);
        // the tile's squared row norms: loaded now (one register), used after the main loop
        const float xn_t = tid < TN && uint32_t(tid) < rc ? a.xn[uint64_t(rs + uint32_t(tid)) * xs] : 0.0f;
        auto issue = [&](uint32_t s) { issue_with(qres, xres, s); };
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int n = 0; n < NQB; ++n)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[m][n][v] = 0.0f;
        // every wave is past the previous tile's epilogue (its dump in slot 1 is read)
        barrier();
        // per wave and stage: LMIN or LPW direct loads
        issue(1);
        wait_vmcnt<Sh::LMIN>();  // stage 0 (older than stage 1's loads)
        barrier();
        read_frags(0, 0, 0);
        for (uint32_t s = 0; s < nst; ++s) {
            const uint32_t slot = s & 1u;
#pragma unroll
            for (int t = 0; t < KC / 16; ++t) {
                const int cur = t & 1;  // four k-steps per stage: the parity of the global k-step
                if (t < KC / 16 - 1) {
                    read_frags(cur ^ 1, slot, t + 1);
                    mma(cur);
                    interleave();
                } else {
                    // this k-step's fragments are in registers: publish stage s+1, free slot s
                    wait_vmcnt<0>();
                    barrier();
                    // slot s is free from here: its next stage goes first (the slots past the last
                    // stage stay free)
                    if (s + 2 < nst) issue(s + 2);
                    read_frags(cur ^ 1, slot ^ 1u, 0);
                    mma(cur);
                    interleave();
                }
            }
        }
        wait_vmcnt<0>();

        // the tile's row norms from the shadow; flags as in screen_kernel
        if (tid < TN) {
            const uint32_t r = uint32_t(tid);
            const float t = xn_t;
            const float nx = __builtin_amdgcn_sqrtf(t);
            xxs[r] = t;
            const bool flag = !(t < 4.29e9f) || nx < tiny;
            xxp[r] = flag ? __builtin_nanf("") : t;
            nxp[r] = flag ? __builtin_nanf("") : nx;
        }
        // the pre-test constants of the tile's queries, in LDS before the next tile's loads are
        // issued (a wait for a global load after those would wait for them too)
        // (SCREEN_GMIN: the queries' {|q|^2, |q|, 2^-scale, c0q})
        if (tid < TQ)
            ptl[tid] = MODE == SCREEN_GMIN ? a.qinfo[qs + min(uint32_t(tid), qc - 1)] : a.ptc[qs + min(uint32_t(tid), qc - 1)];
        __syncthreads();  // every wave is past the main loop: stage slot 0 is free
        // the next tile's first stage, during this epilogue
        const uint32_t Tn = next_tile(T + gridDim.x);
        if (Tn < total) {
            tile_rsrc(Tn, qres, xres);
            issue_with(qres, xres, 0);
        }
        if constexpr (MODE == SCREEN_GMIN) {
            // per query and 32-row group the smallest of v = alpha acc + beta, screen_kernel's
            // approximate upper bound (cosine: 1 - dot / (|q||x|) + E; L2^2: |q|^2 + |x|^2 - 2 dot
            // + E; -dot: -dot + c1 |q||x|); L2 takes the square root of the group's smallest L2^2.
            // Only a checked threshold comes from these values.  Lane (l32, hh) holds query
            // wq*WQ + 32n + l32 against rows wn*WN + 32m + 8j + 4hh + e: its 16 values of group m,
            // the other 16 in lane l32 + 32.
            const float cE = (a.c1 + a.cn) * (1.0f + 0x1p-20f);
            uint32_t* outk = reinterpret_cast<uint32_t*>(a.out_dot);
            const bool cosine = a.op == OP_COS_DIST, ndot = a.op == OP_NEG_DOT;
#pragma unroll
            for (int n = 0; n < NQB; ++n) {
                const uint32_t ql = uint32_t(wq * WQ + 32 * n + l32);
                const float4 inf = ptl[ql];
                const float an = cosine ? -inf.z / inf.y : ndot ? -inf.z : -2.0f * inf.z;
                const float b = cosine ? 1.0f + cE : ndot ? 0.0f : (1.0f + cE) * inf.x;
                const float bb = cosine ? 0.0f : ndot ? a.c1 * inf.y : 1.0f + cE;
                uint32_t g[MB];
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    float mn = INFINITY;
#pragma unroll
                    for (int t = 0; t < 16; ++t) {
                        const int r = row_of(16 * m + t);
                        const float xx = xxs[r];
                        const float ra = cosine ? __builtin_amdgcn_rsqf(xx) : 1.0f;
                        const float rb = ndot ? __builtin_amdgcn_sqrtf(xx) : xx;
                        const float v = fmaf(an * ra, acc[m][n][t], fmaf(bb, rb, b));
                        mn = uint32_t(r) < rc ? fminf(mn, v) : mn;
                    }
                    mn = fminf(mn, __shfl_xor(mn, 32));
                    if (a.op == OP_L2) mn = __builtin_amdgcn_sqrtf(fmaxf(mn, 0.0f));
                    g[m] = key_of_float(mn);
                }
                if (hh == 0 && ql < qc) {
#pragma unroll
                    for (int m = 0; m < MB; ++m)
                        outk[int64_t(qs + ql) * a.ldo + int64_t(tb) * (TN / 32) + (wn * WN) / 32 + m] = g[m];
                }
            }
            T = Tn;
            continue;
        }
        // the (|x|^2, |x|) box of each 4-row group, NaN when a row of it is flagged: a lane's 32
        // rows are 8 whole groups, so its quick-rejection box is 8 lookups instead of 32 rows'
        // worth of min/max (that loop was a large share of the epilogue's vector work)
        if (tid < TN / 4) {
            float4 b = {INFINITY, -INFINITY, INFINITY, -INFINITY};
            bool f = false;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float xx = xxp[4 * tid + e], nx = nxp[4 * tid + e];
                f |= !(xx == xx) || !(nx == nx);
                b.x = fminf(b.x, xx);
                b.y = fmaxf(b.y, xx);
                b.z = fminf(b.z, nx);
                b.w = fmaxf(b.w, nx);
            }
            if (f) b.x = __builtin_nanf("");
            gbox[tid] = b;
        }
        barrier();  // not __syncthreads: that would wait for the next tile's loads

        // ---- filter epilogue: lane (l32, hh) holds query wq*WQ + 32n + l32 against rows
        // wn*WN + 32m + 8j + 4hh + e in acc[m][n][4j + e]; t = 16m + 4j + e indexes its 16 MB values.
        // One query block at a time; the quick rejection (the right-hand side A|x|^2 + B|x| + C
        // over the lane's rows is bounded below at the corner of their (|x|^2, |x|) box that A's
        // and B's signs select, so a lane whose largest value is below it passes nothing; flagged
        // (NaN) rows disable it) settles most blocks from registers.  Another block goes through
        // the wave's 4 KiB of slot 1 one row block m at a time: the pre-test over
        // its 16 values builds a bit mask without branches; lanes l and l + 32 hold the same query,
        // so one atomic reserves both lanes' places; the appends read the values back from LDS.
        Mask valid = ~Mask(0);
        if (rc < TN) {
            valid = 0;
#pragma unroll 1
            for (int t = 0; t < 16 * MB; ++t) valid |= Mask(uint32_t(row_of(t)) < rc) << t;
        }
        float bxlo = INFINITY, bxhi = -INFINITY, bnlo = INFINITY, bnhi = -INFINITY;
        bool bflag = false;
#pragma unroll
        for (int c = 0; c < 4 * MB; ++c) {
            const float4 b = gbox[row_of(4 * c) >> 2];  // rows 4c .. 4c + 3 of the lane: one group
            bflag |= !(b.x == b.x);
            bxlo = fminf(bxlo, b.x);
            bxhi = fmaxf(bxhi, b.y);
            bnlo = fminf(bnlo, b.z);
            bnhi = fmaxf(bnhi, b.w);
        }
        auto block = [&](auto NC) {
            constexpr int n = decltype(NC)::value;
            const uint32_t qt = uint32_t(wq * WQ + 32 * n + l32);
            const uint32_t qi = qs + min(qt, qc - 1);
            const float4 ptq = ptl[qt];
            const PreTest pt = {ptq.x, ptq.y, ptq.z};
            bool skip = qt >= qc;
            if (!bflag && !skip) {
                const float lo = fmaf(pt.A, pt.A >= 0.0f ? bxlo : bxhi, fmaf(pt.B, pt.B >= 0.0f ? bnlo : bnhi, pt.C));
                float mx = -INFINITY;
#pragma unroll
                for (int t = 0; t < 16 * MB; ++t) mx = fmaxf(mx, acc[t >> 4][n][t & 15]);
                skip = mx < lo;
            }
            // row block m into the dump: values 16m .. 16m + 15
            auto dump_half = [&](auto MC) {
                constexpr int m = decltype(MC)::value;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    f32x4v v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[m][n][4 * c + e];
                    dump[c * 64] = v;
                }
                // re-read the row norms and the dump from LDS below
                asm volatile("" ::: "memory");
            };
            Mask mk = 0;
            if (!skip) {
                auto test_half = [&](auto MC) {
                    constexpr int m = decltype(MC)::value;
                    dump_half(MC);
#pragma unroll 2
                    for (int c = 0; c < 4; ++c) {
                        const int r = row_of(16 * m + 4 * c);
                        const f32x4v xx = *reinterpret_cast<const f32x4v*>(xxp + r);
                        const f32x4v nx = *reinterpret_cast<const f32x4v*>(nxp + r);
                        const f32x4v v = dump[c * 64];
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            mk |= Mask(!(v[e] < fmaf(pt.A, xx[e], fmaf(pt.B, nx[e], pt.C)))) << (16 * m + 4 * c + e);
                    }
                };
                test_half(std::integral_constant<int, 0>());
                test_half(std::integral_constant<int, 1>());
                if constexpr (MB > 2) test_half(std::integral_constant<int, 2>());
                mk &= valid;
            }
            // a block with nothing to append skips the atomic and its wait, which would also wait
            // for the next tile's loads in flight
            if (!__ballot(mk != 0u)) return;
            const uint32_t cnt = uint32_t(__builtin_popcountll(uint64_t(mk)));
            const uint32_t other = uint32_t(__shfl_xor(int(cnt), 32));
            uint32_t base = 0;
            if (hh == 0 && cnt + other) base = atomicAdd(a.cnt + qi, cnt + other);
            uint32_t pos = uint32_t(__shfl(int(base), l32)) + (hh ? other : 0u);
            const float* src = reinterpret_cast<const float*>(dump);
            auto append_half = [&](auto MC) {
                constexpr int m = decltype(MC)::value;
                uint32_t mh = uint32_t(mk >> (16 * m)) & 0xFFFFu;
                if (!__ballot(mh != 0u)) return;
                dump_half(MC);
                while (mh && pos < a.cap) {
                    const int c16 = __builtin_ctz(mh);
                    mh &= mh - 1;
                    const int t = 16 * m + c16;
                    const int r = row_of(t);
                    const int64_t o = int64_t(qi) * a.cap + pos;
                    a.cand_dot[o] = src[(c16 >> 2) * 256 + (c16 & 3)] * ptq.w;
                    a.cand_xx[o] = xxs[r];
                    a.cand_id[o] = a.id_base + rs + uint32_t(r);
                    ++pos;
                }
            };
            append_half(std::integral_constant<int, 0>());
            append_half(std::integral_constant<int, 1>());
            if constexpr (MB > 2) append_half(std::integral_constant<int, 2>());
        };
        block(std::integral_constant<int, 0>());
        block(std::integral_constant<int, 1>());
        if constexpr (NQB > 2) {
            block(std::integral_constant<int, 2>());
            block(std::integral_constant<int, 3>());
        }
        T = Tn;
    }
    wait_vmcnt<0>();
}

// ---- the small-batch screen over the fp16 shadow ------------------------------------------------
// Few queries: streaming the shadow from HBM is the cost, not the MFMA (Q = 1 reads 2 bytes per
// value where the fp32 scan reads 4).  Every wave is an independent worker with no LDS and no
// barrier: it takes tiles of 16 MB rows in turn and computes all 16 NQB (padded) queries against
// them on v_mfma_f32_16x16x32_f16, both operands loaded straight into registers by buffer loads
// (rows from HBM through a descriptor that ends at the tile's last row, so rows past N read
// zeros; queries from L2, zeros past Q) in chunks of 64 L bytes per row, a ring of R chunks (R - 1
// in flight while one computes).  Load i of a chunk: lane (r, g) = (lane % 16, lane / 16) reads
// bytes 64 i + 16 g .. + 15 of its row r of each block (and of its query r): the four lanes of a
// row read 64 contiguous bytes per instruction, and k-step i takes the lane's 8 halves from both
// operands, so row and query pair the same d (the dot is the same sum in any order; the screen's
// bound does not depend on it).  Loads past the last chunk use an offset beyond the descriptors
// (zeros; branch-free, so the compiler's wait counts stay exact).  Epilogue: the pre-test of
// screen16_kernel on each value (flagged rows always pass) and appends from registers.
template <int MODE, int NQB, int MB, int L, int R>
__global__ __launch_bounds__(256, 2) void screen16_small_kernel(ScreenArgs a) {
    constexpr int TNW = 16 * MB;       // rows per wave tile
    constexpr uint32_t CH = 64u * L;   // bytes per chunk of a row
    const int lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const uint32_t pitch = a.Dp * 2u;  // bytes per shadow row (a multiple of 128)
    const uint32_t xpitch = pitch * a.xstride;  // bytes between the rows of the scan
    const uint32_t nch = pitch / CH;
    const uint32_t ntiles = (a.N + TNW - 1) / TNW;
    const __amdgpu_buffer_rsrc_t qres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.qh), 0, int(a.Q * pitch), 0x00020000);
    uint32_t qoff[NQB], roff[MB];
#pragma unroll
    for (int n = 0; n < NQB; ++n) qoff[n] = uint32_t(16 * n + r16) * pitch + 16u * uint32_t(g);
#pragma unroll
    for (int m = 0; m < MB; ++m) roff[m] = uint32_t(16 * m + r16) * xpitch + 16u * uint32_t(g);
    const float tiny = a.op == OP_COS_DIST ? 8.0f * a.c0x : 0.0f;
    h8v rbuf[R][MB][L], qbuf[R][NQB][L];
    f32x4v acc[MB][NQB];
    for (uint32_t tile = blockIdx.x * 4u + uint32_t(wave); tile < ntiles; tile += gridDim.x * 4u) {
        const uint32_t rs = tile * TNW, rc = min(uint32_t(TNW), a.N - rs);
        // (the descriptor ends after the tile's last row: (rc - 1) row strides plus one row)
        const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>(a.xh + int64_t(rs) * a.xstride * a.Dp), 0, int((rc - 1) * xpitch + pitch),
            0x00020000);
        auto load = [&](uint32_t c, h8v(&rb)[MB][L], h8v(&qb)[NQB][L]) {
            const bool ok = c < nch;
            const uint32_t ko = c * CH;
#pragma unroll
            for (int i = 0; i < L; ++i) {
#pragma unroll
                for (int m = 0; m < MB; ++m)
                    rb[m][i] = __builtin_bit_cast(
                        h8v, __builtin_amdgcn_raw_buffer_load_b128(xres, ok ? roff[m] + ko + 64u * i : kDmaSkip, 0, 0));
#pragma unroll
                for (int n = 0; n < NQB; ++n)
                    qb[n][i] = __builtin_bit_cast(
                        h8v, __builtin_amdgcn_raw_buffer_load_b128(qres, ok ? qoff[n] + ko + 64u * i : kDmaSkip, 0, 0));
            }
        };
        auto mma = [&](const h8v(&rb)[MB][L], const h8v(&qb)[NQB][L]) {
#pragma unroll
            for (int i = 0; i < L; ++i)
#pragma unroll
                for (int m = 0; m < MB; ++m)
#pragma unroll
                    for (int n = 0; n < NQB; ++n)
                        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(rb[m][i], qb[n][i], acc[m][n], 0, 0, 0);
        };
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int n = 0; n < NQB; ++n) acc[m][n] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < R - 1; ++r) load(uint32_t(r), rbuf[r], qbuf[r]);
        for (uint32_t c = 0; c < nch; c += R) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                // past the end the loads read zeros (unused) and the MFMAs add nothing
                load(c + uint32_t(r + R - 1), rbuf[(r + R - 1) % R], qbuf[(r + R - 1) % R]);
                mma(rbuf[r], qbuf[r]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // lane (r16, g) holds query 16n + r16 against rows 16m + 4g + v in acc[m][n][v]
        if constexpr (MODE == SCREEN_KEYS) {
            // the threshold sample: every unscaled dot and every row norm
#pragma unroll
            for (int n = 0; n < NQB; ++n) {
                const uint32_t qt = uint32_t(16 * n + r16);
                if (qt >= a.Q) continue;
                const float inv = a.qinfo[qt].z;
#pragma unroll
                for (int m = 0; m < MB; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const uint32_t row = uint32_t(16 * m + 4 * g + v);
                        if (row < rc) a.out_dot[int64_t(qt) * a.ldo + rs + row] = acc[m][n][v] * inv;
                    }
            }
            if (r16 == 0) {
#pragma unroll
                for (int m = 0; m < MB; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const uint32_t row = uint32_t(16 * m + 4 * g + v);
                        if (row < rc) a.out_xx[rs + row] = a.xn[uint64_t(rs + row) * a.xstride];
                    }
            }
            continue;
        }
        // ---- filter epilogue: the row norms one block at a time, a pass mask per query block;
        // the appends re-read the norms of passing rows
        uint32_t mk[NQB];
        float4 pt[NQB];
#pragma unroll
        for (int n = 0; n < NQB; ++n) {
            mk[n] = 0;
            pt[n] = a.ptc[min(uint32_t(16 * n + r16), a.Q - 1)];
        }
#pragma unroll
        for (int m = 0; m < MB; ++m) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t row = uint32_t(16 * m + 4 * g + v);
                const bool in = row < rc;
                const float xx = in ? a.xn[rs + row] : 0.0f;
                const float nx = __builtin_amdgcn_sqrtf(xx);
                const bool flag = !(xx < 4.29e9f) || nx < tiny;
                const float xxp = flag ? __builtin_nanf("") : xx, nxp = flag ? __builtin_nanf("") : nx;
#pragma unroll
                for (int n = 0; n < NQB; ++n)
                    mk[n] |= uint32_t(in & !(acc[m][n][v] < fmaf(pt[n].x, xxp, fmaf(pt[n].y, nxp, pt[n].z))))
                             << (4 * m + v);
            }
        }
#pragma unroll
        for (int n = 0; n < NQB; ++n) {
            const uint32_t qt = uint32_t(16 * n + r16);
            const uint32_t mq = qt < a.Q ? mk[n] : 0u;
            if (!__ballot(mq != 0u)) continue;
            if (!mq) continue;
            uint32_t pos = atomicAdd(a.cnt + qt, uint32_t(__popc(mq)));
#pragma unroll
            for (int m = 0; m < MB; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if ((mq >> (4 * m + v)) & 1u) {
                        if (pos < a.cap) {
                            const uint32_t row = uint32_t(16 * m + 4 * g + v);
                            const int64_t o = int64_t(qt) * a.cap + pos;
                            a.cand_dot[o] = acc[m][n][v] * pt[n].w;
                            a.cand_xx[o] = a.xn[rs + row];
                            a.cand_id[o] = a.id_base + rs + row;
                        }
                        ++pos;
                    }
                }
        }
    }
}

// ---- the fp16 shadow: rows rounded to fp16 (RNE, as the scans round), padded with zeros to Dp,
// and their squared norms in fp32 (one wave per row) ----------------------------------------------
__global__ __launch_bounds__(256) void shadow_kernel(const float* __restrict__ x, int64_t ldx, uint32_t N, uint32_t D,
                                                     uint32_t Dp, _Float16* __restrict__ xh, int64_t ldh,
                                                     float* __restrict__ xn, int vec, float2* __restrict__ xne,
                                                     float* __restrict__ xe) {
    const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= N) return;
    const float* row = x + int64_t(r) * ldx;
    _Float16* out = xh + int64_t(r) * ldh;
    float ss = 0.0f, es = 0.0f;
    for (uint32_t d0 = 0; d0 < Dp; d0 += 256) {
        const uint32_t d = d0 + 4u * uint32_t(lane);
        if (d >= Dp) break;
        f32x4v v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vec && d + 3 < D) {
            v = *reinterpret_cast<const f32x4v*>(row + d);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (d + e < D) v[e] = row[d + e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = fmaf(v[e], v[e], ss);
        const h4v h = __builtin_convertvector(v, h4v);
        *reinterpret_cast<h4v*>(out + d) = h;
        const f32x4v dv = __builtin_convertvector(h, f32x4v) - v;  // exact (inf past the fp16 range)
#pragma unroll
        for (int e = 0; e < 4; ++e) es = fmaf(dv[e], dv[e], es);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if (xne || xe) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) es += __shfl_xor(es, o);
    }
    if (lane == 0) {
        if (xn) xn[r] = ss;
        if (xne) xne[r] = make_float2(ss, err_norm_up(es, D));
        if (xe) xe[r] = err_norm_up(es, D);
    }
}

// ---- exact intervals of the screened pairs -----------------------------------------------------
// Dense (the sample): keys[q * ld + j] = key(hi) from dot[q * ld + j] and xx[j], in place.
// Lists (the scan's candidates): (dot, xx) -> (key(hi), key(lo)), in place, for i < min(cnt, cap).
__global__ __launch_bounds__(256) void screen_bound_kernel(ScreenArgs a, float* dot, const float* xx_dense, float* xx_list,
                                                           const uint32_t* cnt, uint32_t n, int64_t ld) {
    const uint32_t q = blockIdx.y;
    const float4 info = a.qinfo[q];
    const uint32_t m = cnt ? min(cnt[q], n) : n;
    // lists with the measured rounding errors: narrower intervals than the worst case the scan's
    // pre-test used (the list holds a superset of what they would admit)
    const bool measured = cnt && a.xe && a.qerr;
    const BoundV bv{a.vcn, a.vgd, a.vg2d};
    const float eq = measured ? a.qerr[q] : 0.0f;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < m; i += gridDim.x * 256) {
        const int64_t o = int64_t(q) * ld + i;
        const float xx = cnt ? xx_list[o] : xx_dense[i];
        uint32_t klo, khi;
        if (measured) {
            float lo, hi;
            if (screen_bounds_m(bv, a.op, dot[o], info.x, info.y, eq, xx, sqrtf(xx), a.xe[a.cand_id[o]], lo, hi)) {
                klo = key_of_float(lo);
                khi = key_of_float(hi);
            } else {
                klo = 0u;
                khi = 0xFFFFFFFEu;  // the NaN key
            }
        } else {
            screen_keys(a, dot[o], info.x, info.y, xx, sqrtf(xx), info.w, klo, khi);
        }
        reinterpret_cast<uint32_t*>(dot)[o] = khi;
        if (cnt) reinterpret_cast<uint32_t*>(xx_list)[o] = klo;
    }
}

// ---- rerank list: the candidates whose lower bound is within the k-th upper bound -------------
// One workgroup per query.  Lists that overflowed (count > cap), fell short of min_count (both
// listed by the candidate select), whose k-th upper bound exceeds the threshold they were
// filtered with (thr non-null: a threshold below the sample's k-th bound, which holds only when k
// candidates lie within it) or whose rerank list outgrows rcap take the fallback and are left
// empty here; the last two are listed here.
__global__ __launch_bounds__(256) void screen_compact_kernel(const uint32_t* __restrict__ cnt,
                                                             const uint32_t* __restrict__ cand_lo,
                                                             const uint32_t* __restrict__ cand_id,
                                                             const uint32_t* __restrict__ bound, uint32_t cap,
                                                             uint32_t min_count, const uint32_t* __restrict__ thr,
                                                             uint32_t* __restrict__ rr, uint32_t* __restrict__ rcount,
                                                             uint32_t rcap, uint32_t* __restrict__ ovf_cnt,
                                                             uint32_t* __restrict__ ovf_rows,
                                                             uint32_t* __restrict__ max_count) {
    __shared__ uint32_t s_n;
    const uint32_t q = blockIdx.x;
    const int tid = threadIdx.x;
    const uint32_t n = cnt[q];
    if (n > cap || n < min_count) {
        // the candidate select has already listed this query for the fallback
        if (tid == 0) rcount[q] = 0;
        return;
    }
    if (thr && bound[q] > thr[q]) {
        // fewer than k candidates have an upper bound within the threshold: the list may miss
        // a row of the top-k
        if (tid == 0) {
            rcount[q] = 0;
            ovf_rows[atomicAdd(ovf_cnt, 1u)] = q;
        }
        return;
    }
    if (tid == 0) s_n = 0;
    __syncthreads();
    const uint32_t u = bound[q];
    const uint32_t* lo = cand_lo + int64_t(q) * cap;
    const uint32_t* id = cand_id + int64_t(q) * cap;
    uint32_t* out = rr + int64_t(q) * rcap;
    for (uint32_t i0 = 0; i0 < n; i0 += 256) {
        const uint32_t i = i0 + uint32_t(tid);
        const bool p = i < n && lo[i] <= u;
        const uint64_t b = __ballot(p);
        const int lane = tid & 63;
        uint32_t base = 0;
        if (lane == 0 && b) base = atomicAdd(&s_n, uint32_t(__popcll(b)));
        base = __shfl(base, 0);
        if (p) {
            const uint32_t pos = base + uint32_t(__popcll(b & ((1ull << lane) - 1)));
            if (pos < rcap) out[pos] = id[i];
        }
    }
    __syncthreads();
    if (tid == 0) {
        const uint32_t m = s_n;
        if (m > rcap) {
            rcount[q] = 0;
            const uint32_t p = atomicAdd(ovf_cnt, 1u);
            ovf_rows[p] = q;
        } else {
            rcount[q] = m;
            atomicMax(max_count, m);
        }
    }
}

// ---- exact fp32 keys of the rerank lists ------------------------------------------------------
// One wave per (64-row chunk of a query's rerank list, query), persistent and chunk-major (the
// busy chunks spread over every wave); lane l scores row 64c + l with the fp32 scan's per-element
// sequence on the VALU (GemmChain: the fmaf chain every element of the scan's MFMA block follows),
// so every key equals the fp32 scan's.  The rows pass through the wave's LDS slot in coalesced
// 128-byte lines (rows_through_lds).  Needs D % 4 == 0 and 16-byte aligned rows and queries.
template <int R, bool QLDS, int NRG = 8>
__global__ __launch_bounds__(256) void rerank_kernel(const float* __restrict__ q, const float* __restrict__ x,
                                                     uint32_t D, int op, const uint32_t* __restrict__ rr,
                                                     const uint32_t* __restrict__ rcount, uint32_t rcap, uint32_t Q,
                                                     uint32_t* __restrict__ rkey) {
    constexpr uint32_t CH = 8 * NRG;  // rows per chunk (one wave's)
    __shared__ fb_f32x4 slots[4][64 * 8];
    // QLDS: each wave's query staged in LDS (dynamic, 4 x D4 floats), so that a wave alone on its
    // rows does not wait on a load of the query's values for every group
    extern __shared__ __attribute__((aligned(16))) float qstage[];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t D4 = (D + 3) & ~3u;
    const uint32_t nch = (rcap + CH - 1) / CH;
    const uint64_t items = uint64_t(Q) * nch;
    const uint32_t nw = gridDim.x * 4;
    for (uint64_t it = uint64_t(blockIdx.x) * 4 + wave; it < items; it += nw) {
        const uint32_t c = uint32_t(it / Q), qi = uint32_t(it % Q);
        const uint32_t n = min(rcount[qi], rcap);
        if (c * CH >= n) continue;  // (uniform)
        const uint32_t* rl = rr + int64_t(qi) * rcap + c * CH;
        const uint32_t m = min(CH, n - c * CH);
        uint32_t rid[NRG];
        bool rv[NRG];
#pragma unroll
        for (int i = 0; i < NRG; ++i) {
            const uint32_t r = uint32_t(8 * i + (lane >> 3));
            rv[i] = r < m;
            rid[i] = rv[i] ? rl[r] : 0u;
        }
        const float* qp = q + int64_t(qi) * D;
        if constexpr (QLDS) {
            // (the wave writes and then reads only its own region: in order, no barrier)
            float* qw = qstage + wave * D4;
            for (uint32_t d = uint32_t(lane) * 4; d < D; d += 256)
                *reinterpret_cast<fb_f32x4*>(qw + d) = *reinterpret_cast<const fb_f32x4*>(qp + d);
            qp = qw;
        }
        GemmChain ch;
        rows_through_lds<R, NRG>(qp, x, rid, rv, D, slots[wave],
                                 [&](uint32_t j, const fb_f32x4(&xv)[8], const fb_f32x4(&qv)[8]) { ch.group(xv, qv, j, D); });
        if (uint32_t(lane) < m) rkey[int64_t(qi) * rcap + c * CH + lane] = ch.key(op);
    }
}

template <int MODE>
va_status launch_screen(va_context* ctx, const ScreenArgs& a) {
    using namespace scr;
    const uint64_t nqb = (a.Q + TQ - 1) / TQ;
    const uint64_t ntb = (a.N + TN - 1) / TN;
    const uint64_t grid = nqb * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (grid == 0) return VA_OK;
    if (grid > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "screen grid too large (%llu)", (unsigned long long)grid);
    screen_kernel<MODE><<<dim3(uint32_t(grid)), dim3(256), 0, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// Batches of at most kHalfTileQueries queries take a 128-query x 384-row tile of twelve waves
// (the same wave tiles, three waves per SIMD): a 256-query tile would be more than half padding,
// and the kernel is MFMA-bound (1M x 768, Q = 100: screen 0.40 -> 0.33 ms; eight waves of a
// 128 x 256 tile, two per SIMD: 0.36 ms).
constexpr uint32_t kHalfTileQueries = 128;
template <int WAVES, int NQB, int MB, int TQ>
va_status launch_screen16_shape(va_context* ctx, const ScreenArgs& a) {
    using Sh = s16::Shape<WAVES, NQB, MB, TQ>;
    const uint64_t nqb = (a.Q + TQ - 1) / TQ;
    const uint64_t ntb = (a.N + Sh::TN - 1) / Sh::TN;
    const uint64_t tiles = nqb * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (tiles == 0) return VA_OK;
    if (tiles > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "screen grid too large (%llu)", (unsigned long long)tiles);
    // persistent: one workgroup per CU (its LDS fills one), a multiple of the XCD count
    const uint64_t cus = std::max<uint64_t>(uint64_t(ctx->num_cus), kXcds) / kXcds * kXcds;
    const uint64_t grid = std::min(tiles, cus);
    auto kern = &screen16_kernel<WAVES, NQB, MB, TQ>;
    VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, Sh::LDS));
    kern<<<dim3(uint32_t(grid)), dim3(64 * WAVES), Sh::LDS, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}
// The threshold sample's group minima over shadow rows j * a.xstride (false: the row offsets of
// a tile would not fit 32 bits; the caller takes screen_kernel).
bool screen16_gmin_fits(const ScreenArgs& a) {
    return uint64_t(s16::Shape<s16::kWaves, s16::kQueryBlocks, s16::kRowBlocks>::TN) * a.xstride * a.Dp * 2 <
           0x7FFFFFF0ull;
}
va_status launch_screen16_gmin(va_context* ctx, const ScreenArgs& a) {
    using namespace s16;
    using Sh = Shape<kWaves, kQueryBlocks, kRowBlocks, TQ>;
    if (a.Q == 0 || a.N == 0) return VA_OK;
    const uint64_t nqb = (a.Q + TQ - 1) / TQ;
    const uint64_t ntb = (a.N + Sh::TN - 1) / Sh::TN;
    const uint64_t tiles = nqb * ((ntb + kXcds - 1) / kXcds) * kXcds;
    if (tiles > 0x7FFFFFFFull) return fail(ctx, VA_ERR_INVALID_ARG, "screen grid too large (%llu)", (unsigned long long)tiles);
    const uint64_t cus = std::max<uint64_t>(uint64_t(ctx->num_cus), kXcds) / kXcds * kXcds;
    auto kern = &screen16_kernel<kWaves, kQueryBlocks, kRowBlocks, TQ, SCREEN_GMIN>;
    VA_CHECK_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, Sh::LDS));
    kern<<<dim3(uint32_t(std::min(tiles, cus))), dim3(64 * kWaves), Sh::LDS, ctx->stream>>>(a);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}
va_status launch_screen16(va_context* ctx, const ScreenArgs& a) {
    using namespace s16;
    if (a.Q <= kHalfTileQueries)
        return launch_screen16_shape<3 * kWaves / 4, kQueryBlocks, kRowBlocks, int(kHalfTileQueries)>(ctx, a);
    return launch_screen16_shape<kWaves, kQueryBlocks, kRowBlocks, TQ>(ctx, a);
}

// The small-batch screen: NQB 16-query blocks x MB 16-row blocks per wave, chunks of 64 L bytes
// per row, a ring of R chunks, within the registers of two waves per SIMD.  Measured on 1M rows
// of 768 and 1536 values: one query block of 2 row blocks with a 6-deep ring streams the shadow
// at 5.6-5.8 TB/s (4 row blocks, 4 deep: 5.1; 8 row blocks, 2 deep: 4.8); for 17-32 queries 4 row
// blocks 3 deep (3.9 TB/s) beat 2 blocks 6 deep (3.5).
template <int NQB, int MB, int L, int R>
struct Launch {
    static constexpr uint32_t queries = 16u * NQB;  // queries a wave tile covers
    static constexpr uint32_t TNW = 16u * MB;       // rows of a wave tile
};
template <int MODE>
va_status launch_screen16_small(va_context* ctx, const ScreenArgs& a) {
    if (a.Q == 0 || a.N == 0) return VA_OK;
    const uint32_t waves_per_cu = 8;
    auto go = [&](auto kern, uint32_t tnw) -> va_status {
        const uint64_t tiles = (uint64_t(a.N) + tnw - 1) / tnw;
        const uint64_t grid = std::max<uint64_t>(1, std::min<uint64_t>((tiles + 3) / 4,
                                                                        uint64_t(ctx->num_cus) * waves_per_cu / 4));
        kern<<<dim3(uint32_t(grid)), dim3(256), 0, ctx->stream>>>(a);
        VA_CHECK_LAUNCH(ctx);
        return VA_OK;
    };
#ifndef VA_S16S_A
#define VA_S16S_A 1, 2, 2, 6
#endif
#ifndef VA_S16S_B
#define VA_S16S_B 2, 4, 2, 3
#endif
    using KA = Launch<VA_S16S_A>;
    using KB = Launch<VA_S16S_B>;
    static_assert(KB::queries >= kSmallBatchMax, "the small-batch screen covers every batch it is given");
    if (uint64_t(a.Dp) * 2 * a.xstride * (KA::TNW > KB::TNW ? KA::TNW : KB::TNW) > 0x7FFFFFF0ull)
        return fail(ctx, VA_ERR_INVALID_ARG, "launch_screen16_small: tile offsets beyond 32 bits");
    if (a.Q <= KA::queries) return go(&screen16_small_kernel<MODE, VA_S16S_A>, KA::TNW);
    if (a.Q <= KB::queries) return go(&screen16_small_kernel<MODE, VA_S16S_B>, KB::TNW);
    return fail(ctx, VA_ERR_INVALID_ARG, "launch_screen16_small: %u queries (at most %u)", a.Q, kSmallBatchMax);
}

va_status launch_bounds(va_context* ctx, const ScreenArgs& a, float* dot, const float* xx_dense, float* xx_list,
                        const uint32_t* cnt, uint32_t n, int64_t ld, uint32_t rows) {
    if (rows == 0 || n == 0) return VA_OK;
    // lists are short (a few thousand): one block per query row; the dense sample: up to 16
    const uint32_t bx = cnt ? std::min<uint32_t>(4, (n + 255) / 256) : std::min<uint32_t>(16, (n + 255) / 256);
    screen_bound_kernel<<<dim3(bx, rows), dim3(256), 0, ctx->stream>>>(a, dot, xx_dense, xx_list, cnt, n, ld);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

uint32_t padded_dim(uint32_t D) { return (D + scr::DP_ALIGN - 1) / scr::DP_ALIGN * scr::DP_ALIGN; }

// Tile offsets of the scan are 32-bit: 256 rows at stride ldx, and a query block.
bool offsets_fit(uint64_t ldx, uint32_t D) {
    return uint64_t(scr::TN) * ldx * 4 + uint64_t(D) * 4 < 0x7FFFFFF0ull &&
           uint64_t(scr::TQ) * padded_dim(D) * 2 < 0x7FFFFFF0ull;
}

}  // namespace

uint32_t shadow_pitch(uint32_t D) { return padded_dim(D); }

va_status build_shadow(va_context* ctx, const float* x, uint32_t N, uint32_t D, _Float16* shadow, float* norms,
                       float2* norm_err, float* errs) {
    if (N == 0) return VA_OK;
    const uint32_t Dp = padded_dim(D);
    const int vec = (D % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
    shadow_kernel<<<dim3((N + 3) / 4), dim3(256), 0, ctx->stream>>>(x, int64_t(D), N, D, Dp, shadow, int64_t(Dp),
                                                                   norms, vec, norm_err, errs);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status screen_prepare_queries(va_context* ctx, const float* q, uint32_t Q, uint32_t D, _Float16* qh,
                                 float4* qinfo, float c0, float* qerr, uint32_t* zero0, uint32_t n0, uint32_t* zero1,
                                 uint32_t n1) {
    if (Q == 0) return VA_OK;
    const int vec = (D % 4 == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0);
    screen_prep_kernel<<<dim3((Q + 3) / 4), dim3(256), 0, ctx->stream>>>(q, int64_t(D), Q, D, padded_dim(D), qh, qinfo,
                                                                       c0, qerr, vec, zero0, n0, zero1, n1);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

va_status screen_list_bounds(va_context* ctx, const ScreenBound& b, const float4* qinfo, float* dot, float* xx,
                             const uint32_t* cnt, uint32_t cap, uint32_t Q) {
    ScreenArgs a;
    a.op = b.op;
    a.c1 = b.c1;
    a.cn = b.cn;
    a.c0x = b.c0x;
    a.kabs = b.kabs;
    a.qinfo = qinfo;
    return launch_bounds(ctx, a, dot, nullptr, xx, cnt, cap, int64_t(cap), Q);
}

va_status screen_compact(va_context* ctx, const uint32_t* cnt, const uint32_t* cand_lo, const uint32_t* cand_id,
                         const uint32_t* bound, uint32_t cap, uint32_t Q, uint32_t* rr, uint32_t* rcount, uint32_t rcap,
                         uint32_t* ovf_cnt, uint32_t* ovf_rows) {
    screen_compact_kernel<<<dim3(Q), dim3(256), 0, ctx->stream>>>(cnt, cand_lo, cand_id, bound, cap, 0u, nullptr, rr,
                                                                 rcount, rcap, ovf_cnt, ovf_rows, ovf_cnt + 1);
    VA_CHECK_LAUNCH(ctx);
    return VA_OK;
}

// The plan of a screened search: plan_scan's, except that small batches over the fp16 shadow
// sample N/256 rows (at least 4096): for them the sample and its per-row selection are a visible
// share of a search that streams the shadow once, while the screen's band, not the sample's
// threshold, sets the rerank.
ScanPlan screen_plan(const va_context* ctx, const ScreenInput& in, uint32_t k) {
    if (in.xh && in.Q <= kSmallBatchMax && !ctx->opt_sample_rows)
        return plan_scan_for(dense_budget(ctx), std::max<uint64_t>(4096, in.N / 256), ctx->opt_candidate_cap, in.Q,
                             in.N, k);
    return plan_scan(ctx, in.Q, in.N, k);
}

bool screen_applies(const va_context* ctx, const ScreenInput& in, uint32_t k) {
    if (ctx->opt_screen == 1) return false;
    if (in.op != OP_L2SQ && in.op != OP_L2 && in.op != OP_COS_DIST && in.op != OP_NEG_DOT) return false;
    if (in.D % 4 != 0 || (reinterpret_cast<uintptr_t>(in.x) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(in.q) & 15) != 0)
        return false;
    const ScanPlan plan = screen_plan(ctx, in, k);
    if (plan.direct) return false;
    if (!offsets_fit(uint64_t(plan.stride) * in.D, in.D)) return false;
    if (ctx->opt_screen == 2) return true;
    // automatic: over an fp16 shadow every batch (below kSmallBatch queries the small-batch screen
    // streams it at half the fp32 scan's bytes); over fp32 rows enough queries to fill the
    // 256-query tiles of the converting scan
    return in.xh ? true : in.Q >= kSmallBatch;
}

va_status screened_topk_scan(va_context* ctx, const ScreenInput& in, KeyProducer& exact, uint32_t k,
                             const ScanOutputs& out) {
    const uint32_t Q = in.Q, N = in.N, D = in.D;
    const uint32_t Dp = padded_dim(D);
    const ScanPlan plan = screen_plan(ctx, in, k);
    const uint64_t S = plan.S;
    const uint64_t cap = plan.cap;
    // the threshold: the sample's rank-th smallest upper bound (checked in the compaction when
    // rank < k)
    const uint32_t rank = sample_rank(ctx, k, S, N, out.skip != nullptr);
    // rerank capacity: k plus the band of rows whose interval straddles the k-th bound (the
    // launch covers only the longest list actually built)
    const uint64_t rcap = screen_rerank_cap(N, k, cap);
    const Bound bnd = make_bound(D);

    SelectArgs base;
    base.k = k;
    base.out_idx = out.idx;
    base.out_f = out.f;
    base.key_kind = 0;

    ScanPhaseMarks pm(ctx);
    ctx->last_scan = va_scan_timings{};
    VA_CHECK_STATUS(pm.mark(0));

    Scratch s(ctx);
    size_t need = screened_scan_need(Q, Dp, plan, rcap);
    // overflowed queries are finished on the device (no read-back) when the fallback's buffers fit
    const bool device_fb = fb_fits(ctx, need, Q, N, k);
    if (device_fb) need += fb_bytes(Q, N, k);
    VA_CHECK_STATUS(s.reserve(need));
    uint32_t* thr = s.carve<uint32_t>(Q);
    uint32_t* cnt = s.carve<uint32_t>(Q);
    uint32_t* ubound = s.carve<uint32_t>(Q);
    uint32_t* rcount = s.carve<uint32_t>(Q);
    uint32_t* ovf_rows = s.carve<uint32_t>(Q);
    uint32_t* ovf_cnt = s.carve<uint32_t>(64);
    float4* qinfo = s.carve<float4>(Q);
    float4* ptc = s.carve<float4>(Q);
    float* qerr = s.carve<float>(Q);
    _Float16* qh = s.carve<_Float16>(uint64_t(Q) * Dp);
    uint32_t* skeys = s.carve<uint32_t>(uint64_t(plan.qs) * S);
    float* sxx = s.carve<float>(S);
    uint32_t* chi = s.carve<uint32_t>(uint64_t(Q) * cap);
    uint32_t* clo = s.carve<uint32_t>(uint64_t(Q) * cap);
    uint32_t* cid = s.carve<uint32_t>(uint64_t(Q) * cap);
    uint32_t* rr = s.carve<uint32_t>(uint64_t(Q) * rcap);
    uint32_t* rkey = s.carve<uint32_t>(uint64_t(Q) * rcap);
    FbArgs fb;
    if (device_fb) {
        fb = fb_carve(s, Q, N, k);
        fb.n_rows = ovf_cnt;
        fb.rows = ovf_rows;
        fb.skip = out.skip;
    }
    VA_CHECK_STATUS(s.verify(need));

    // ---- 1. queries -> scaled fp16 ---------------------------------------------------------
    // (also clears the scan's list counters and the overflow words: [0] overflowed queries, [1]
    // longest rerank list)
    const bool measured = in.xh && in.xe;  // the candidates' intervals from measured rounding errors
    screen_prep_kernel<<<dim3((Q + 3) / 4), dim3(256), 0, ctx->stream>>>(in.q, int64_t(D), Q, D, Dp, qh, qinfo,
                                                                       bnd.c0, measured ? qerr : nullptr, 1, cnt, Q,
                                                                       ovf_cnt, 2u);
    VA_CHECK_LAUNCH(ctx);

    ScreenArgs sa;
    sa.D = D;
    sa.Dp = Dp;
    sa.op = in.op;
    sa.c1 = bnd.c1;
    sa.cn = bnd.cn;
    sa.c0x = bnd.c0 * 0x1p-25f;
    sa.kabs = bnd.kabs;

    // ---- 2. sample: k-th smallest upper bound over S strided rows ------------------------------
    // A checked rank (rank < k) accepts any threshold, so the sample of a large batch keeps one
    // approximate bound per 32-row group (the scan's epilogue takes the group minimum: no dense
    // keys, no bound pass) and selects among those: the rank-th smallest group minimum is close
    // to the rank-th smallest bound when the rank is far below the group count.
    const bool group_min = rank < k && !(in.xh && Q <= kSmallBatchMax) && S >= 128ull * rank;
    const uint32_t groups = uint32_t((S + scr::TN - 1) / scr::TN * (scr::TN / 32));
    for (uint32_t q0 = 0; q0 < Q; q0 += plan.qs) {
        const uint32_t nq = std::min(plan.qs, Q - q0);
        ScreenArgs a = sa;
        a.x = in.x;
        a.ldx = int64_t(plan.stride) * D;
        a.N = uint32_t(S);
        a.Q = nq;
        a.qh = qh + int64_t(q0) * Dp;
        a.qinfo = qinfo + q0;
        a.out_dot = reinterpret_cast<float*>(skeys);
        a.out_xx = sxx;
        a.ldo = int64_t(S);
        if (group_min) {
            a.ldo = int64_t(groups);
            if (in.xh) {
                // over the fp16 shadow (half the bytes, screen16_kernel's tiles)
                a.xh = in.xh;
                a.xn = in.xn;
                a.xstride = plan.stride;
            }
            if (in.xh && screen16_gmin_fits(a)) VA_CHECK_STATUS(launch_screen16_gmin(ctx, a));
            else VA_CHECK_STATUS(launch_screen<SCREEN_GMIN>(ctx, a));
            SelectArgs sel;
            sel.keys = skeys;
            sel.ld = int64_t(groups);
            sel.n = groups;
            sel.rows = nq;
            sel.k = rank;
            sel.out_kth = thr + q0;
            VA_CHECK_STATUS(launch_select(ctx, sel));
            continue;
        }
        if (in.xh && Q <= kSmallBatchMax) {
            // small batches sample the fp16 shadow (half the bytes, every CU busy)
            a.xh = in.xh;
            a.xn = in.xn;
            a.xstride = plan.stride;
            VA_CHECK_STATUS(launch_screen16_small<SCREEN_KEYS>(ctx, a));
        } else {
            VA_CHECK_STATUS(launch_screen<SCREEN_KEYS>(ctx, a));
        }
        VA_CHECK_STATUS(launch_bounds(ctx, a, reinterpret_cast<float*>(skeys), sxx, nullptr, nullptr, uint32_t(S),
                                      int64_t(S), nq));
        VA_CHECK_STATUS(mask_dense_keys(ctx, skeys, nq, uint32_t(S), int64_t(S), 0, plan.stride, out.skip));
        SelectArgs sel;
        sel.keys = skeys;
        sel.ld = int64_t(S);
        sel.n = uint32_t(S);
        sel.rows = nq;
        sel.k = rank;
        sel.out_kth = thr + q0;
        VA_CHECK_STATUS(launch_select(ctx, sel));
    }
    // ---- 3. screening scan -------------------------------------------------------------------
    VA_CHECK_STATUS(pm.mark(1));
    {
        ScreenArgs a = sa;
        a.x = in.x;
        a.ldx = D;
        a.N = N;
        a.Q = Q;
        a.qh = qh;
        a.qinfo = qinfo;
        a.thr = thr;
        a.cnt = cnt;
        a.cand_dot = reinterpret_cast<float*>(chi);
        a.cand_xx = reinterpret_cast<float*>(clo);
        a.cand_id = cid;
        a.cap = uint32_t(cap);
        if (measured) {
            const BoundV bv = make_bound_v(D);
            a.qerr = qerr;
            a.xe = in.xe;
            a.vcn = bv.cn;
            a.vgd = bv.gd;
            a.vg2d = bv.g2d;
        }
        if (in.xh) {
            a.xh = in.xh;
            a.xn = in.xn;
            a.ptc = ptc;
            pretest_kernel<<<dim3((Q + 255) / 256), dim3(256), 0, ctx->stream>>>(a, Q, ptc);
            VA_CHECK_LAUNCH(ctx);
            if (Q <= kSmallBatchMax)
                VA_CHECK_STATUS(launch_screen16_small<SCREEN_FILTER>(ctx, a));
            else
                VA_CHECK_STATUS(launch_screen16(ctx, a));
        } else {
            VA_CHECK_STATUS(launch_screen<SCREEN_FILTER>(ctx, a));
        }
        VA_CHECK_STATUS(pm.mark(2));
        // (dot, |x|^2) -> (key of hi, key of lo), in place
        VA_CHECK_STATUS(launch_bounds(ctx, a, reinterpret_cast<float*>(chi), nullptr, reinterpret_cast<float*>(clo), cnt,
                                      uint32_t(cap), int64_t(cap), Q));
        VA_CHECK_STATUS(mask_list_keys(ctx, chi, clo, cid, cnt, Q, uint32_t(cap), int64_t(cap), out.skip));
    }
    ctx->last_scan.scan_launches = 1;
    ctx->last_scan.sample_rows = uint32_t(S);
    ctx->last_scan.candidate_cap = uint32_t(cap);
    ctx->last_scan.screened = in.xh ? 2u : 1u;  // 2: screen16_kernel over the fp16 shadow
    // ---- 4. k-th smallest upper bound among the candidates (overflowed lists are listed) ------
    {
        SelectArgs a;
        a.keys = chi;
        a.ids = cid;
        a.counts = cnt;
        a.ld = int64_t(cap);
        a.n = uint32_t(cap);
        a.rows = Q;
        a.k = k;
        a.out_kth = ubound;
        a.overflow_count = ovf_cnt;
        a.overflow_rows = ovf_rows;
        a.min_count = rank < k ? k : 0;
        VA_CHECK_STATUS(launch_select(ctx, a));
    }
    // ---- 5. rerank lists ------------------------------------------------------------------------
    screen_compact_kernel<<<dim3(Q), dim3(256), 0, ctx->stream>>>(cnt, clo, cid, ubound, uint32_t(cap),
                                                                 rank < k ? k : 0u, rank < k ? thr : nullptr, rr,
                                                                 rcount, uint32_t(rcap), ovf_cnt, ovf_rows,
                                                                 ovf_cnt + 1);
    VA_CHECK_LAUNCH(ctx);
    AuxJoinGuard fb_join(ctx, device_fb ? 1 : 0);
    if (device_fb) {
        // ---- 8a. the overflowed queries (listed by steps 4 and 5) take the device fallback's
        // passes on an aux stream, beside the rerank and the selection (a search with none still
        // pays their launches, off the critical path here)
        VA_CHECK_STATUS(aux_fork(ctx, 1));
        StreamScope on_aux(ctx, ctx->aux[0]);
        VA_CHECK_STATUS(fb_passes(ctx, exact, fb));
    }
    // Without the device fallback the overflow count is read back (one synchronisation).
    uint32_t n_ovf = 0;
    if (!device_fb) {
        VA_CHECK_HIP(ctx, hipMemcpyAsync(ctx->host_word, ovf_cnt, 4, hipMemcpyDeviceToHost, ctx->stream));
        VA_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        n_ovf = ctx->host_word[0];
    }
    // ---- 6. exact fp32 keys of the rerank rows ---------------------------------------------------
    {
        const uint64_t items = uint64_t(Q) * ((rcap + 63) / 64);
        const uint32_t blocks = uint32_t(std::min<uint64_t>(2048, (items + 3) / 4));
        // small batches keep few waves busy, each on its own: 8-row chunks (eight times the waves,
        // each streaming an eighth of the rows), the query staged in LDS and eight row groups in
        // flight per wave
        const size_t qlds = size_t(4) * ((D + 3) & ~3u) * 4;
        if (Q <= kSmallBatchMax && qlds <= 64 * 1024) {
            const uint64_t items8 = uint64_t(Q) * ((rcap + 7) / 8);
            rerank_kernel<8, true, 1><<<dim3(uint32_t(std::min<uint64_t>(4096, (items8 + 3) / 4))), dim3(256), qlds,
                                        ctx->stream>>>(in.q, in.x, D, int(in.op), rr, rcount, uint32_t(rcap), Q, rkey);
        } else
            rerank_kernel<2, false><<<dim3(blocks), dim3(256), 0, ctx->stream>>>(in.q, in.x, D, int(in.op), rr,
                                                                                rcount, uint32_t(rcap), Q, rkey);
        VA_CHECK_LAUNCH(ctx);
        VA_CHECK_STATUS(mask_list_keys(ctx, rkey, nullptr, rr, rcount, Q, uint32_t(rcap), int64_t(rcap), out.skip));
    }
    // ---- 7. exact (key, id) top-k ----------------------------------------------------------------
    {
        SelectArgs a = base;
        a.keys = rkey;
        a.ids = rr;
        a.counts = rcount;
        a.ld = int64_t(rcap);
        a.n = uint32_t(rcap);
        a.rows = Q;
        VA_CHECK_STATUS(launch_select(ctx, a));
    }
    // profiling only: rows the exact rerank scored, queries that overflowed
    VA_CHECK_STATUS(pm.count_sum(rcount, Q));
    if (device_fb) VA_CHECK_STATUS(pm.count_overflow(ovf_cnt));
    VA_CHECK_STATUS(pm.mark(3));
    if (device_fb) {
        // ---- 8b. their exact top-k, over the rows step 7 wrote ----------------------------------
        VA_CHECK_STATUS(fb_join.join());
        VA_CHECK_STATUS(fb_select(ctx, fb, base, exact.key_bits()));
        return pm.finish(true, true);
    }
    ctx->last_scan.overflow_rows = n_ovf;
    if (n_ovf == 0) return pm.finish(true, false);
    VA_CHECK_STATUS(rescan_rows(ctx, exact, N, k, base, ovf_rows, n_ovf, out.skip));
    return pm.finish(true, true);
}

}  // namespace va
