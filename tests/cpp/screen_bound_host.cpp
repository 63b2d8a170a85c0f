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

}  // extern "C"
