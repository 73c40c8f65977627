// Stratified pixel sampling (odie/data.py:63-80): one pixel per square stratum of a side x side
// grid, side = sqrt(batch).  Slot j's stratum is (j % side, j / side); with the slot's two
// uniforms u, uv = u / side + stratum / side in fp32 (side is a power of two: both quotients
// are exact), pixel = trunc(uv * (W, H)) clamped to the image, id = y * W + x -- the reference's
// torch expression, evaluated per slot.
#include "common.h"
#include "sampling.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

__global__ __launch_bounds__(256) void stratified_kernel(const float* uniforms, int batch, int side, float inv_side,
                                                         int width, int height, int64_t* ids) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= batch) return;
    ids[j] = stratified_id(reinterpret_cast<const float2*>(uniforms)[j], j, side, inv_side, width, height);
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_stratified_ids(const float* uniforms, int batch, int width, int height, int64_t* ids,
                                 uint64_t stream) {
    if (batch < 1 || (batch & (batch - 1))) return fail("odie_stratified_ids: batch must be a power of two");
    int side = 1;
    while (side * side < batch) side *= 2;
    if (side * side != batch) return fail("Stratified sampling requires a square power-of-two batch size");
    if (width < 1 || height < 1) return fail("odie_stratified_ids: empty image");
    if (!uniforms || !ids) return fail("odie_stratified_ids: null pointer");
    if (reinterpret_cast<uintptr_t>(uniforms) % 8) return fail("odie_stratified_ids: uniforms must be 8-byte aligned");
    stratified_kernel<<<(batch + 255) / 256, 256, 0, as_stream(stream)>>>(uniforms, batch, side, 1.0f / side, width,
                                                                          height, ids);
    return check_launch("odie_stratified_ids");
}
