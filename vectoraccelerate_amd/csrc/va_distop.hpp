// va_distop.hpp — the fp32 distance of the search path from its three parts (q.x, |q|^2, |x|^2).
// Shared by the distance GEMM and the overflow fallback, which must produce identical keys.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>

#include "va_internal.hpp"

namespace va {

__device__ __forceinline__ float apply_op(int op, float dot, float qq, float xx) {
    switch (op) {
        case OP_L2SQ:
        case OP_L2: {
            // cancellation can leave a tiny negative: clamp at 0, but let NaN through
            float v = qq + xx - 2.0f * dot;
            v = (v < 0.0f) ? 0.0f : v;
            return op == OP_L2 ? sqrtf(v) : v;
        }
        case OP_COS_SIM:
        case OP_COS_DIST: {
            // cosine_similarity finalisation (DistanceShaders.metal:300-319)
            float denom = sqrtf(qq) * sqrtf(xx);
            float raw = (denom < FLT_MIN) ? 0.0f : dot / denom;
            float s = (raw != raw) ? raw : fminf(fmaxf(raw, -1.0f), 1.0f);
            return op == OP_COS_SIM ? s : 1.0f - s;
        }
        case OP_DOT: return dot;
        case OP_ABS_DOT: return fabsf(dot);
        default: return -dot;
    }
}

}  // namespace va
