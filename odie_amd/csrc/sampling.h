// Stratified pixel sampling (odie/data.py:63-80), shared by odie_stratified_ids and the
// route's stratified variant so both evaluate the same fp32 expression.
#pragma once
#include "common.h"

namespace odie {

// fp32 -> int32 truncated toward zero, saturating at the int32 range, NaN -> 0 (v_cvt_i32_f32).
__device__ inline int32_t truncate_to_int(float v) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Slot j of a side x side stratified batch, with the slot's two uniforms u: stratum
// (j % side, j / side); uv = u / side + stratum / side in fp32 (side a power of two: both
// quotients exact); pixel = trunc(uv * (W, H)) clamped to the image; id = y * W + x.  With
// j < side^2 <= 2^31 the stratum comes from a mask and a shift of 32-bit j; the truncation
// saturates at the int32 range, which the clamp into the image then maps as the reference's
// 64-bit truncation does (and a NaN to 0, as its clamp of the minimum int64 does).
__device__ inline int64_t stratified_id(float2 u, int64_t j, int side, float inv_side, int width, int height) {
    const uint32_t slot = static_cast<uint32_t>(j);
    const float sx = static_cast<float>(static_cast<int32_t>(slot & static_cast<uint32_t>(side - 1))) * inv_side;
    const float sy = static_cast<float>(static_cast<int32_t>(slot >> __builtin_ctz(static_cast<uint32_t>(side)))) * inv_side;
    const float ux = u.x * inv_side + sx, uy = u.y * inv_side + sy;
    const float fx = ux * static_cast<float>(width), fy = uy * static_cast<float>(height);
    // .long() truncates toward zero; the clamps follow (odie/data.py:79-80)
    int32_t x = truncate_to_int(fx), y = truncate_to_int(fy);
    x = x < 0 ? 0 : (x > width - 1 ? width - 1 : x);
    y = y < 0 ? 0 : (y > height - 1 ? height - 1 : y);
    return static_cast<int64_t>(y) * width + x;
}

}  // namespace odie
