// Host build of the screening scan's error bound (vectoraccelerate_amd/csrc/va_screen_bound.hpp),
// the same source the kernels compile, exported for tests/test_screen_bound.py (ctypes).
#include "../../vectoraccelerate_amd/csrc/va_screen_bound.hpp"

extern "C" {

void sb_make_bound(uint32_t D, float* out4) {
    const va::Bound b = va::make_bound(D);
    out4[0] = b.c1;
    out4[1] = b.cn;
    out4[2] = b.c0;
    out4[3] = b.kabs;
}

int sb_query_scale(float maxabs, int bad) { return va::query_scale_exponent(maxabs, bad != 0); }

// lo_hi[0..1] = the interval of the fp32 key; returns 0 when the pair cannot be bounded
int sb_bounds(int op, const float* bound4, float dot, float qq, float nq, float xx, float nx, float c0q, float* lo_hi) {
    const va::ScreenBound b{op, bound4[0], bound4[1], bound4[2] * 0x1p-25f, bound4[3]};
    return va::screen_bounds(b, dot, qq, nq, xx, nx, c0q, lo_hi[0], lo_hi[1]) ? 1 : 0;
}

// abc[0..2] = the pre-test's constants for threshold key thr_key
void sb_pretest(int op, const float* bound4, float qq, float nq, float inv, float c0q, uint32_t thr_key, float* abc) {
    const va::ScreenBound b{op, bound4[0], bound4[1], bound4[2] * 0x1p-25f, bound4[3]};
    const va::PreTest p = va::pretest_consts(b, qq, nq, inv, c0q, thr_key);
    abc[0] = p.A;
    abc[1] = p.B;
    abc[2] = p.C;
}

uint32_t sb_key(float f) { return va::key_of_float(f); }

// the L2^2 bound with measured rounding errors: b3 = {cn, gd, g2d}
void sb_make_bound_v(uint32_t D, float* b3) {
    const va::BoundV b = va::make_bound_v(D);
    b3[0] = b.cn;
    b3[1] = b.gd;
    b3[2] = b.g2d;
}

float sb_err_norm_up(float ss, uint32_t D) { return va::err_norm_up(ss, D); }

int sb_bounds_v(const float* b3, float dot, float qq, float nq, float eq, float xx, float nx, float ex, float* lo_hi) {
    const va::BoundV b{b3[0], b3[1], b3[2]};
    return va::screen_bounds_v(b, dot, qq, nq, eq, xx, nx, ex, lo_hi[0], lo_hi[1]) ? 1 : 0;
}

// every distance family with measured rounding errors (the flat screen's candidate intervals)
int sb_bounds_m(const float* b3, int op, float dot, float qq, float nq, float eq, float xx, float nx, float ex,
                float* lo_hi) {
    const va::BoundV b{b3[0], b3[1], b3[2]};
    return va::screen_bounds_m(b, op, dot, qq, nq, eq, xx, nx, ex, lo_hi[0], lo_hi[1]) ? 1 : 0;
}

// abce[0..3] = the pre-test's constants A, B, E, C for threshold key thr_key
void sb_pretest_v(const float* b3, float qq, float nq, float eq, float inv, uint32_t thr_key, float* abce) {
    const va::BoundV b{b3[0], b3[1], b3[2]};
    const va::PreTestV p = va::pretest_v(b, qq, nq, eq, inv, thr_key);
    abce[0] = p.A;
    abce[1] = p.B;
    abce[2] = p.E;
    abce[3] = p.C;
}

}  // extern "C"
