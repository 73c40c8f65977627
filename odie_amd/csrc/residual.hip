// Residual pass: per-cell FP64 squared-error totals in raster order, bit-exact with the
// reference's rule (odie/residual_cuda.cu:11-43, odie/selection.py:58-73).
//
// Per pixel: t = byte / 255 (correctly rounded fp32 division) or the fp32 target itself,
// d = p - t in fp32, rgb = (double(d0*d0) + double(d1*d1)) + double(d2*d2) in fp64, and the
// cell total grows by rgb / 3.0 in fp64 -- sequentially, in raster order within each cell,
// continued across streamed chunks.  An FP64 sum is order dependent, so each cell is one
// sequential chain; the parallelism is across cells.  To keep the chain's latency the only
// serial part, every thread first computes the per-pixel terms of the next run of pixels of
// its row (independent work the scheduler can overlap) and then folds them in order.
#include "residual.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kResidualBlock = 128;
constexpr int kRun = 8;   // pixel terms computed ahead of the sequential fold

template <bool RGB8>
__device__ inline double pixel_term(const float* prediction, const void* target, int64_t p) {
    float t0, t1, t2;
    if constexpr (RGB8) {
        const uint8_t* bytes = static_cast<const uint8_t*>(target);
        t0 = byte_target(bytes[p]);
        t1 = byte_target(bytes[p + 1]);
        t2 = byte_target(bytes[p + 2]);
    } else {
        const float* values = static_cast<const float*>(target);
        t0 = values[p];
        t1 = values[p + 1];
        t2 = values[p + 2];
    }
    return residual_term(prediction[p], prediction[p + 1], prediction[p + 2], t0, t1, t2);
}

template <bool RGB8>
__global__ __launch_bounds__(kResidualBlock) void accumulate_kernel(const float* prediction, const void* target,
                                                                    int64_t begin, int64_t end, int width,
                                                                    int resolution, int first_y, int active_cells,
                                                                    const int* xb, const int* yb, double* totals) {
    const int t = blockIdx.x * kResidualBlock + threadIdx.x;
    if (t >= active_cells) return;
    const int cx = t % resolution, cy = first_y + t / resolution;
    const int64_t cell = static_cast<int64_t>(cy) * resolution + cx;
    const int64_t first_row = begin / width, last_row = (end - 1) / width + 1;
    const int64_t y0 = yb[cy] > first_row ? yb[cy] : first_row;
    const int64_t y1 = yb[cy + 1] < last_row ? yb[cy + 1] : last_row;
    double sum = totals[cell];
    for (int64_t y = y0; y < y1; ++y) {
        const int64_t row = y * width;
        const int64_t x0 = xb[cx] > begin - row ? xb[cx] : begin - row;
        const int64_t x1 = xb[cx + 1] < end - row ? xb[cx + 1] : end - row;
        int64_t x = x0;
        for (; x + kRun <= x1; x += kRun) {
            double terms[kRun];
#pragma unroll
            for (int j = 0; j < kRun; ++j) terms[j] = pixel_term<RGB8>(prediction, target, (row + x + j - begin) * 3);
#pragma unroll
            for (int j = 0; j < kRun; ++j) sum = sum + terms[j];
        }
        for (; x < x1; ++x) sum = sum + pixel_term<RGB8>(prediction, target, (row + x - begin) * 3);
    }
    totals[cell] = sum;
}

// Cell bounds of the native geometry cells along one axis of `size` pixels (the pixel -> cell map of
// odie/selection.py:44-55 and odie/gpu_residual.py:49-62): pixel p has the coordinate
// x = fp32(p) / fp32(size - 1) (correctly rounded division) and the cell floor(fmaf(R - 1, x, 0.5))
// -- the encode's own geometry -- so bounds[c] is the first pixel whose cell is >= c and
// bounds[R] = size.  Cells grow with p, so each thread writes the bounds of the cells its pixel
// opens.
__device__ inline int native_cell(int p, int size, int resolution) {
    const float x = __fdiv_rn(static_cast<float>(p), static_cast<float>(size - 1));
    const int cell = static_cast<int>(floorf(__builtin_fmaf(static_cast<float>(resolution - 1), x, 0.5f)));
    return cell < resolution - 1 ? cell : resolution - 1;
}

__global__ __launch_bounds__(256) void cell_bounds_kernel(int size, int resolution, int32_t* bounds) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= size) return;
    const int cell = native_cell(p, size, resolution);
    const int before = p ? native_cell(p - 1, size, resolution) : -1;
    for (int c = before + 1; c <= cell; ++c) bounds[c] = p;
    if (p == size - 1) bounds[resolution] = size;
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_cell_bounds(int width, int height, int resolution, int32_t* xb, int32_t* yb, uint64_t stream) {
    if (width < 2 || height < 2) return fail("odie_cell_bounds: width and height must be at least 2");
    if (resolution < 2 || resolution > (1 << 23)) return fail("odie_cell_bounds: resolution must be within [2, 2^23]");
    if (!xb || !yb) return fail("odie_cell_bounds: null pointer");
    const hipStream_t s = as_stream(stream);
    cell_bounds_kernel<<<static_cast<uint32_t>((width + 255) / 256), 256, 0, s>>>(width, resolution, xb);
    cell_bounds_kernel<<<static_cast<uint32_t>((height + 255) / 256), 256, 0, s>>>(height, resolution, yb);
    return check_launch("odie_cell_bounds");
}

// Same signature and meaning as score_chunk (odie/residual_cuda.cu:45-52): pixels [begin, end)
// of a width-wide image, prediction fp32 [end-begin, 3], target uint8 or fp32 [end-begin, 3],
// cells of rows first_y.. (active_cells of them) with column/row bounds xb[R+1], yb[R+1];
// totals (fp64 [R*R]) are read and updated.  Returns 0, or the runtime's error code as the
// reference does (hipErrorInvalidValue for a refused argument; the message in odie_error()).
ODIE_API int score_chunk(const float* prediction, const void* target, int64_t begin, int64_t end, int width,
                         int resolution, int first_y, int active_cells, const int* xb, const int* yb, double* totals,
                         bool rgb8, uint64_t stream) {
    if (width < 1 || resolution < 1) return fail_code("score_chunk: width and resolution must be positive");
    if (begin < 0 || end < begin) return fail_code("score_chunk: need 0 <= begin <= end");
    if (first_y < 0 || active_cells < 0 || first_y + (active_cells + resolution - 1) / resolution > resolution)
        return fail_code("score_chunk: cell rows out of range");
    if (end == begin || active_cells == 0) return 0;
    if (!prediction || !target || !xb || !yb || !totals) return fail_code("score_chunk: null pointer");
    const uint32_t blocks = static_cast<uint32_t>((active_cells + kResidualBlock - 1) / kResidualBlock);
    const hipStream_t s = as_stream(stream);
    if (rgb8)
        accumulate_kernel<true><<<blocks, kResidualBlock, 0, s>>>(prediction, target, begin, end, width, resolution,
                                                                  first_y, active_cells, xb, yb, totals);
    else
        accumulate_kernel<false><<<blocks, kResidualBlock, 0, s>>>(prediction, target, begin, end, width, resolution,
                                                                   first_y, active_cells, xb, yb, totals);
    return launch_code("score_chunk");
}
