// Per-pixel term of the residual pass (odie/residual_cuda.cu:20-33, odie/selection.py:58-73):
// t = byte / 255 (correctly rounded fp32 division) or the fp32 target, d = p - t in fp32,
// rgb = (double(d0*d0) + double(d1*d1)) + double(d2*d2), term = rgb / 3.0 in fp64.  Shared by
// the streamed residual (residual.hip) and the fused reconstruction (reconstruct.hip).
#pragma once
#include "common.h"

namespace odie {

__device__ inline float byte_target(uint8_t value) { return static_cast<float>(value) / 255.0f; }

__device__ inline double residual_term(float p0, float p1, float p2, float t0, float t1, float t2) {
    const float d0 = p0 - t0, d1 = p1 - t1, d2 = p2 - t2;
    double rgb = static_cast<double>(d0 * d0) + static_cast<double>(d1 * d1);
    rgb = rgb + static_cast<double>(d2 * d2);
    return rgb / 3.0;
}

}  // namespace odie
