// The expert tiles of an image: a regions_x x regions_y grid with integer bounds
// x0[r] = ceil(r * W / regions_x) (y likewise), and each tile's pixel -> coordinate scale
// fp32(1 / (tile_width - 1)), the reference's convention (odie/native/runtime.cu:35-36) applied
// to the tile.  Shared by the router and the fused reconstruction.
#pragma once
#include <cstdint>

namespace odie {

constexpr int kMaxTiles = 64;   // tiles per axis

// Unsigned 32-bit division by an invariant divisor d >= 1 with one multiply-high: Granlund and
// Montgomery, "Division by invariant integers using multiplication" (PLDI 1994), Figure 4.1:
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, then n / d = (t + ((n - t) >> sh1)) >> sh2
// with t = mulhi(m, n), sh1 = min(l, 1), sh2 = max(l - 1, 0), exact for every 32-bit n.
struct Divisor {
    uint32_t magic;
    uint32_t sh1, sh2;
};

inline Divisor make_divisor(uint32_t d) {
    uint32_t l = 0;
    while (l < 32 && (uint64_t{1} << l) < d) ++l;
    const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1;
    return Divisor{static_cast<uint32_t>(m), l < 1 ? l : 1u, l > 1 ? l - 1 : 0u};
}

__device__ inline uint32_t divide(uint32_t n, const Divisor& d) {
    const uint32_t t = __umulhi(d.magic, n);
    return (t + ((n - t) >> d.sh1)) >> d.sh2;
}

struct TileBounds {
    int32_t x0[kMaxTiles + 1];
    int32_t y0[kMaxTiles + 1];
    float rx[kMaxTiles];
    float ry[kMaxTiles];
    float sx, sy;   // fp32(regions_x / width), fp32(regions_y / height): tile_of's estimate
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
    b.sx = static_cast<float>(static_cast<double>(regions_x) / width);
    b.sy = static_cast<float>(static_cast<double>(regions_y) / height);
}

// Largest r < regions with bounds[r] <= v.  With bounds[r] = ceil(r * extent / regions) that is
// floor(v * regions / extent) (bounds[r] <= v iff r * extent <= v * regions for integer v),
// capped at regions - 1.  The fp32 estimate v * scale (scale = fp32(regions / extent)) is within
// 2^-16 of v * regions / extent for r < 64, so its floor is off by at most one, either way: one
// comparison of exact 64-bit products each way fixes it, with no table and no branch.
__device__ inline int tile_of(int regions, uint32_t extent, float scale, uint32_t v) {
    int r = static_cast<int>(static_cast<float>(v) * scale);
    r = r < 0 ? 0 : (r > regions - 1 ? regions - 1 : r);
    const uint32_t ur = static_cast<uint32_t>(r);
    const uint64_t scaled = static_cast<uint64_t>(v) * static_cast<uint32_t>(regions);
    const bool up = (ur + 1 < static_cast<uint32_t>(regions)) & (static_cast<uint64_t>(ur + 1) * extent <= scaled);
    const bool down = static_cast<uint64_t>(ur) * extent > scaled;
    return r + static_cast<int>(up) - static_cast<int>(down);
}

}  // namespace odie
