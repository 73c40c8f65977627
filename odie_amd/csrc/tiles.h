// The expert tiles of an image: a regions_x x regions_y grid with integer bounds
// x0[r] = ceil(r * W / regions_x) (y likewise), and each tile's pixel -> coordinate scale
// fp32(1 / (tile_width - 1)), the reference's convention (odie/native/runtime.cu:35-36) applied
// to the tile.  Shared by the router and the fused reconstruction.
#pragma once
#include <cstdint>

namespace odie {

constexpr int kMaxTiles = 64;   // tiles per axis

struct TileBounds {
    int32_t x0[kMaxTiles + 1];
    int32_t y0[kMaxTiles + 1];
    float rx[kMaxTiles];
    float ry[kMaxTiles];
};

inline void make_tile_bounds(int width, int height, int regions_x, int regions_y, TileBounds& b) {
    for (int r = 0; r <= kMaxTiles; ++r) {
        const int rxx = r < regions_x ? r : regions_x, ryy = r < regions_y ? r : regions_y;
        b.x0[r] = static_cast<int32_t>((static_cast<int64_t>(rxx) * width + regions_x - 1) / regions_x);
        b.y0[r] = static_cast<int32_t>((static_cast<int64_t>(ryy) * height + regions_y - 1) / regions_y);
    }
    for (int r = 0; r < kMaxTiles; ++r) {
        const int tw = r < regions_x ? b.x0[r + 1] - b.x0[r] : 2;
        const int th = r < regions_y ? b.y0[r + 1] - b.y0[r] : 2;
        b.rx[r] = static_cast<float>(1.0 / static_cast<double>(tw - 1));
        b.ry[r] = static_cast<float>(1.0 / static_cast<double>(th - 1));
    }
}

// Largest r < regions with bounds[r] <= v.
__device__ inline int tile_of(const int32_t* bounds, int regions, uint32_t v) {
    int lo = 0, hi = regions - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (static_cast<uint32_t>(bounds[mid]) <= v) lo = mid; else hi = mid - 1;
    }
    return lo;
}

}  // namespace odie
