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
