// va_screen_bound.hpp — the error bound of the fp16 screening scan and its linear pre-test
// (host and device: the kernels use it, and a host test checks it against fp32 keys computed in
// several summation orders on adversarial inputs).
#pragma once

#include <cfloat>
#include <cmath>
#include <cstdint>

#include "va_keys.hpp"

namespace va {

// The distance families the screen serves (values equal to DistOp's).
enum ScreenOp : int { SOP_L2SQ = 0, SOP_L2 = 1, SOP_COS_DIST = 3, SOP_NEG_DOT = 6 };

// Bound coefficients of a screened search (see make_bound) and its distance family.
struct ScreenBound {
    int op;
    float c1, cn, c0x, kabs;
};

// ---- bound of the screened key ----------------------------------------------------------
// dot: the fp16 dot (already unscaled); qq, nq: fp32 |q|^2, |q|; xx, nx: |x|^2, |x| (fp32, in
// another order than the fp32 scan's); c0q: the query's absolute-rounding coefficient.
// Returns false when the pair cannot be bounded (it is then always a candidate).
VA_HD inline bool screen_bounds(const ScreenBound& a, float dot, float qq, float nq, float xx, float nx,
                                              float c0q, float& lo, float& hi) {
    if (!(fabsf(dot) <= FLT_MAX)) return false;   // non-finite products: entry beyond fp16 range, NaN, inf
    const float cabs = fmaf(c0q, a.kabs, 1e-36f);  // products of two rounding floors, fp32 subnormals
    const float eabs = fmaf(a.c0x, nq, fmaf(c0q, nx, cabs));  // absolute part of the dot bound
    float s, e;
    switch (a.op) {
        case SOP_COS_DIST: {
            const float den = nq * nx;
            if (!(den >= 0x1p-100f)) return false;  // near the FLT_MIN floor (or NaN)
            const float raw = dot / den;
            s = 1.0f - fminf(fmaxf(raw, -1.0f), 1.0f);
            e = a.c1 + a.cn + eabs / den;
            break;
        }
        case SOP_NEG_DOT:
            s = -dot;
            e = fmaf(a.c1, nq * nx, eabs);
            break;
        default: {  // SOP_L2SQ, SOP_L2 (bounded in the squared domain first)
            float v = qq + xx - 2.0f * dot;
            s = v < 0.0f ? 0.0f : v;
            e = fmaf(a.c1 + a.cn, qq + xx, 2.0f * eabs);
            break;
        }
    }
    // room for the rounding of s +- e itself
    e = fmaf(fmaf(0x1p-21f, fabsf(s), e), 1.0f + 0x1p-20f, 0x1p-126f);
    if (!(e <= FLT_MAX) || !(fabsf(s) <= FLT_MAX)) return false;
    lo = s - e;
    hi = s + e;
    if (a.op == SOP_L2) {
        lo = sqrtf(fmaxf(lo, 0.0f)) * (1.0f - 0x1p-22f);
        hi = sqrtf(hi) * (1.0f + 0x1p-22f);
    } else if (a.op == SOP_L2SQ) {
        lo = fmaxf(lo, 0.0f);
    }
    return true;
}

VA_HD inline void screen_keys(const ScreenBound& a, float dot, float qq, float nq, float xx, float nx,
                                            float c0q, uint32_t& klo, uint32_t& khi) {
    float lo, hi;
    if (screen_bounds(a, dot, qq, nq, xx, nx, c0q, lo, hi)) {
        klo = key_of_float(lo);
        khi = key_of_float(hi);
    } else {
        klo = 0u;
        khi = 0xFFFFFFFEu;  // the NaN key
    }
}

// ---- the scan's pre-test ----------------------------------------------------------------------
// A pair whose fp32 key can be <= tau must satisfy  acc >= A |x|^2 + B |x| + C  (acc = the scaled
// fp16 dot).  The constants follow from the same bound as screen_bounds, solved for the dot and
// loosened by 2^-18 of every term (more than the fp32 rounding of the constants and of the two
// fmas); the test is written !(acc < rhs), so a NaN rhs (a flagged row) always passes.  Queries
// the form cannot serve get C = -inf (every row passes).
struct PreTest {
    float A, B, C;
};
VA_HD inline PreTest pretest_consts(const ScreenBound& a, float qq, float nq, float inv, float c0q, uint32_t thr_key) {
    const PreTest all = {0.0f, 0.0f, -INFINITY};
    if (thr_key >= 0xFFFFFFFEu) return all;  // the NaN key (or no threshold): every key passes
    const float tau = float_of_key(thr_key);
    if (!(fabsf(tau) <= FLT_MAX) || !(qq <= FLT_MAX)) return all;
    const float sig = 1.0f / inv;  // 2^scale, exact
    const float cabs = fmaf(c0q, a.kabs, 1e-36f);
    const float w = 1.0f + 0x1p-20f;
    const float r = 0x1p-18f;
    float A = 0.0f, B, C;
    switch (a.op) {
        case SOP_COS_DIST: {
            // clamp(dot/den) >= 1 - tau - E with 1 - tau - E > -1 (tau < 1.5 and the query and row
            // terms of E below 1/8 each; rows with |x| < 8 c0x are flagged)
            if (tau >= 1.5f || c0q > 0.125f * nq) return all;
            const float e0 = (a.c1 + a.cn + 0x1p-20f) * w;
            B = sig * ((1.0f - tau - e0) * nq - w * c0q - 0x1p-126f * nq);
            C = -sig * w * fmaf(a.c0x, nq, cabs);
            B = B - fabsf(B) * r - sig * nq * 0x1p-20f;
            C = C - fabsf(C) * r;
            break;
        }
        case SOP_NEG_DOT: {
            // -dot <= tau + E_dot
            B = -sig * w * fmaf(a.c1, nq, c0q);
            C = -sig * (tau + w * fmaf(a.c0x, nq, cabs));
            B = B - fabsf(B) * r;
            C = C - fabsf(C) * r - sig * fabsf(tau) * 0x1p-21f;
            break;
        }
        default: {
            // |q|^2 + |x|^2 - 2 dot <= tau + E (L2: tau squared, with room for the sqrt's rounding)
            const float t = a.op == SOP_L2 ? tau * tau * (1.0f + 0x1p-20f) : tau;
            const float alpha = (a.c1 + a.cn + 0x1p-20f) * w;
            A = sig * (1.0f - alpha) * 0.5f;
            B = -sig * w * c0q;
            C = sig * 0.5f * ((1.0f - alpha) * qq - t - 2.0f * w * fmaf(a.c0x, nq, cabs) - 0x1p-126f);
            A = A * (1.0f - r);
            B = B - fabsf(B) * r;
            C = C - fabsf(C) * r - sig * (qq + fabsf(t)) * 0x1p-21f;
            break;
        }
    }
    if (!(fabsf(A) <= FLT_MAX) || !(fabsf(B) <= FLT_MAX) || !(fabsf(C) <= FLT_MAX)) return all;
    return PreTest{A, B, C};
}

// Coefficients of the bound for dimension D (host, double precision; every term rounded up by
// 1/16): c1 relative to |q||x| for the fp16 roundings and the two fp32 accumulations, cn
// relative to |q|^2 + |x|^2 (or 1 for cosine) for the norms' two orders and the key formula, c0
// the absolute floor of fp16 subnormals scaled by sqrt(D) (c0x = c0 * 2^-25 on the row side),
// kabs the product of the two floors.
struct Bound {
    float c1, cn, c0, kabs;
};
inline Bound make_bound(uint32_t D) {
    const double u = std::ldexp(1.0, -11);   // fp16 unit roundoff
    const double up = std::ldexp(1.0, -23);  // any fp32 rounding (nearest or toward zero)
    auto gam = [&](double n) { return n * up / (1.0 - n * up); };
    const double gD = gam(D), g2D = gam(2.0 * D);
    const double slack = 1.0625;
    Bound b;
    // |dot16 - dot| + |dot32 - dot| <= c1 |q||x| + c0 (2^-25 |q| + eta_q |x|) + ...
    b.c1 = float(slack * (2 * u + u * u + gD * (1 + 3 * u) + g2D));
    // the two orders of the norms and the key formula's roundings (relative to |q|^2 + |x|^2, or
    // to 1 for cosine)
    b.cn = float(slack * (2 * gD + std::ldexp(1.0, -20)));
    b.c0 = float(slack * (1 + u) * (1 + gD) * std::sqrt(double(D)));
    // the product of the two absolute floors: D * 2^-25 * eta_q = c0q * D * 2^-25 / c0
    b.kabs = float(slack * double(D) * std::ldexp(1.0, -25) / double(b.c0));
    return b;
}

// ---- the L2^2 bound with measured rounding errors ---------------------------------------------
// When each vector's fp16 rounding error is known (eq >= |q~ - q| for the query, unscaled, and
// ex >= |x~ - x| for the row), the fp16 part of the bound is the exact expansion
//     |q~.x~ - q.x| = |dq.x + q.dx + dq.dx| <= eq |x| + |q| ex + eq ex
// instead of its worst case 2u |q||x| (typical rounding errors are about 0.4u of the norm).  The
// fp32 accumulation of the exact fp16 products adds gd |q~||x~| <= gd (|q| + eq)(|x| + ex), the
// fp32 scan's own dot g2d |q||x| (any order, products rounded), and cn (|q|^2 + |x|^2) covers the
// norms computed in two orders and the key formula, as in screen_bounds.  The result is linear in
// the row's |x|^2, |x| and ex, so the pre-test keeps its form with one more term.
struct BoundV {
    float cn, gd, g2d;
};
inline BoundV make_bound_v(uint32_t D) {
    const double up = std::ldexp(1.0, -23);
    auto gam = [&](double n) { return n * up / (1.0 - n * up); };
    const double slack = 1.0625;
    BoundV b;
    b.cn = float(slack * (2 * gam(D) + std::ldexp(1.0, -20)));
    b.gd = float(slack * gam(D));
    b.g2d = float(slack * gam(2.0 * D));
    return b;
}

// An upper bound of the norm of a rounding-error vector from ss, the fp32 sum (any order) of the
// squares of its D entries (each entry, the difference of a float and its fp16 image, is exact in
// fp32): the sum's and the squares' roundings, squares lost to underflow, the sqrt's rounding.
VA_HD inline float err_norm_up(float ss, uint32_t D) {
    return sqrtf(fmaf(ss, 1.0f + float(D) * 0x1p-22f, 0x1p-110f)) * (1.0f + 0x1p-20f);
}

// coefficients of |x| and of ex in the bound of |2 (dot16 - dot32)|; the factor 1 + 2^-9 covers
// their own rounding and the relative error of the fp32 norms |q|, |x| they multiply
VA_HD inline float boundv_nx(const BoundV& b, float nq, float eq) {
    return 2.0f * fmaf(b.gd, nq + eq, fmaf(b.g2d, nq, eq)) * (1.0f + 0x1p-9f);
}
VA_HD inline float boundv_ex(const BoundV& b, float nq, float eq) {
    return 2.0f * (1.0f + b.gd) * (nq + eq) * (1.0f + 0x1p-9f);
}

// The interval [lo, hi] of the fp32 L2^2 key from the fp16 dot (already unscaled); false when the
// pair cannot be bounded (non-finite dot, query or row outside the fp16 range).
VA_HD inline bool screen_bounds_v(const BoundV& b, float dot, float qq, float nq, float eq, float xx, float nx,
                                  float ex, float& lo, float& hi) {
    if (!(fabsf(dot) <= FLT_MAX) || !(eq <= FLT_MAX) || !(ex <= FLT_MAX) || !(qq <= FLT_MAX) || !(xx <= FLT_MAX))
        return false;
    const float v = qq + xx - 2.0f * dot;
    const float s = v < 0.0f ? 0.0f : v;
    float e = fmaf(b.cn, qq + xx, fmaf(boundv_nx(b, nq, eq), nx, boundv_ex(b, nq, eq) * ex));
    e = fmaf(fmaf(0x1p-21f, fabsf(s), e), 1.0f + 0x1p-20f, 0x1p-126f);  // rounding of s and e
    if (!(e <= FLT_MAX) || !(fabsf(s) <= FLT_MAX)) return false;
    lo = fmaxf(s - e, 0.0f);
    hi = s + e;
    return true;
}

// Every distance family with measured rounding errors.  K = |dot16 - dot32| bounded as in
// screen_bounds_v (half its eq/ex part): the exact expansion of the fp16 roundings, the MFMA's
// accumulation and the fp32 scan's own dot.  The key's interval then follows screen_bounds with
// its worst-case dot terms (c1 |q||x| and the absolute floors, which the measured norms include)
// replaced by K: cosine e = K / (|q||x|) + cn, -dot e = K, L2^2 e = cn (|q|^2 + |x|^2) + 2K (the
// value screen_bounds_v uses).  The clamp of the cosine is 1-Lipschitz, the norms' two orders
// and the key formula stay in cn, the final roundings as in screen_bounds.
VA_HD inline bool screen_bounds_m(const BoundV& b, int op, float dot, float qq, float nq, float eq, float xx, float nx,
                                  float ex, float& lo, float& hi) {
    if (!(fabsf(dot) <= FLT_MAX) || !(eq <= FLT_MAX) || !(ex <= FLT_MAX) || !(qq <= FLT_MAX) || !(xx <= FLT_MAX))
        return false;
    const float k2 = fmaf(boundv_nx(b, nq, eq), nx, boundv_ex(b, nq, eq) * ex);  // 2K
    float s, e;
    switch (op) {
        case SOP_COS_DIST: {
            const float den = nq * nx;
            if (!(den >= 0x1p-100f)) return false;  // near the FLT_MIN floor (or NaN)
            const float raw = dot / den;
            s = 1.0f - fminf(fmaxf(raw, -1.0f), 1.0f);
            e = 0.5f * k2 / den + b.cn;
            break;
        }
        case SOP_NEG_DOT:
            s = -dot;
            e = 0.5f * k2;
            break;
        default: {  // SOP_L2SQ, SOP_L2 (bounded in the squared domain first)
            const float v = qq + xx - 2.0f * dot;
            s = v < 0.0f ? 0.0f : v;
            e = fmaf(b.cn, qq + xx, k2);
            break;
        }
    }
    e = fmaf(fmaf(0x1p-21f, fabsf(s), e), 1.0f + 0x1p-20f, 0x1p-126f);  // rounding of s and e
    if (!(e <= FLT_MAX) || !(fabsf(s) <= FLT_MAX)) return false;
    lo = s - e;
    hi = s + e;
    if (op == SOP_L2) {
        lo = sqrtf(fmaxf(lo, 0.0f)) * (1.0f - 0x1p-22f);
        hi = sqrtf(hi) * (1.0f + 0x1p-22f);
    } else if (op == SOP_L2SQ) {
        lo = fmaxf(lo, 0.0f);
    }
    return true;
}

// The pre-test of screen_bounds_v: a pair whose lower bound can be <= tau satisfies
//     acc >= A |x|^2 + B |x| + E ex + C      (acc = the scaled fp16 dot, sig = 2^scale = 1/inv)
// (from 2 dot >= |q|^2 + |x|^2 - e - tau, with the rounding room 2^-21 |s| <= 2^-21 (|tau| + e)
// of a pair at the boundary folded into e), each term loosened by 2^-18 for the fp32 rounding of
// the constants and of the kernel's fma chain; written !(acc < rhs), so a NaN rhs (a flagged row)
// passes.  Thresholds the form cannot serve give C = -inf (every pair passes).
struct PreTestV {
    float A, B, E, C;
};
VA_HD inline PreTestV pretest_v(const BoundV& b, float qq, float nq, float eq, float inv, uint32_t thr_key) {
    const PreTestV all = {0.0f, 0.0f, 0.0f, -INFINITY};
    if (thr_key >= 0xFFFFFFFEu) return all;  // the NaN key (or no threshold): every key passes
    const float tau = float_of_key(thr_key);
    if (!(fabsf(tau) <= FLT_MAX) || !(qq <= FLT_MAX) || !(eq <= FLT_MAX)) return all;
    const float sig = 1.0f / inv;  // 2^scale, exact
    const float w = 1.0f + 0x1p-19f;
    const float r = 0x1p-18f;
    const float a1 = 1.0f - b.cn * w;
    float A = sig * 0.5f * a1;
    float B = -sig * 0.5f * w * boundv_nx(b, nq, eq);
    float E = -sig * 0.5f * w * boundv_ex(b, nq, eq);
    float C = sig * 0.5f * (a1 * qq - tau - w * 0x1p-21f * fabsf(tau) - 0x1p-125f);
    A = A * (1.0f - r);
    B = B - fabsf(B) * r;
    E = E - fabsf(E) * r;
    C = C - fabsf(C) * r - sig * (qq + fabsf(tau)) * 0x1p-21f;
    if (!(fabsf(A) <= FLT_MAX) || !(fabsf(B) <= FLT_MAX) || !(fabsf(E) <= FLT_MAX) || !(fabsf(C) <= FLT_MAX))
        return all;
    return PreTestV{A, B, E, C};
}

// The power-of-two scale of a query (largest |entry| m, any entry non-finite: bad): 2^sc puts
// the largest entry in [2^14, 2^15), at most 2^40 so the pre-test constants stay finite.
VA_HD inline int query_scale_exponent(float m, bool bad) {
    int sc = 0;
    if (!bad && m > 0.0f) {
        int e = 0;
        (void)frexpf(m, &e);  // m in [2^(e-1), 2^e)
        sc = 15 - e < 40 ? 15 - e : 40;
    }
    return sc;
}

}  // namespace va
