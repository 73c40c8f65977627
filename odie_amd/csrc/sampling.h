// Stratified pixel sampling (odie/data.py:63-80), shared by odie_stratified_ids and the
// route's stratified variant so both evaluate the same fp32 expression.
#pragma once
#include "common.h"

namespace odie {

// Slot j of a side x side stratified batch, with the slot's two uniforms u: stratum
// (j % side, j / side); uv = u / side + stratum / side in fp32 (side a power of two: both
// quotients exact); pixel = trunc(uv * (W, H)) clamped to the image; id = y * W + x.
__device__ inline int64_t stratified_id(float2 u, int64_t j, int side, float inv_side, int width, int height) {
    const float sx = static_cast<float>(j % side) * inv_side, sy = static_cast<float>(j / side) * inv_side;
    const float ux = u.x * inv_side + sx, uy = u.y * inv_side + sy;
    const float fx = ux * static_cast<float>(width), fy = uy * static_cast<float>(height);
    // .long() truncates toward zero; the clamps follow (odie/data.py:79-80)
    int64_t x = static_cast<int64_t>(fx), y = static_cast<int64_t>(fy);
    x = x < 0 ? 0 : (x > width - 1 ? width - 1 : x);
    y = y < 0 ? 0 : (y > height - 1 ? height - 1 : y);
    return y * width + x;
}

}  // namespace odie
