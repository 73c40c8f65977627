// Fused reconstruction of an image through the multi-expert hash-grid model: for every pixel
// of a raster range, its expert tile and tile coordinate (the router's convention), the 16-level
// fp16 encode from that expert's table and the decoder MLP, in one kernel, so the features never
// reach memory.  The streamed full-image inference the residual pass scores
// (odie/evaluation.py:12-36, odie/gpu_residual.py:130-179: prediction = model(coordinates(ids))
// for ids in raster order).
//
// One wave per tile of 32 consecutive pixels.  Lane (g, s) encodes pixel s's levels
// 8*kt + 4*g + j (kt = 0, 1; j = 0..3): exactly the features 16*kt + 8*g + e that the decoder's
// first MFMA takes from that lane as its B operand, so the encode feeds the MLP in registers.
// Every value is computed with the arithmetic of odie_grid_forward (fp16 table, fp16 FMA chain,
// half2_level) and odie_mlp_forward (forward_tile): the same bits as those two entry points on
// the routed coordinates.
#include "grid.h"
#include "mlp.h"
#include "residual.h"
#include "tiles.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kLevels = 16;
constexpr int kReconBlock = kMlpBlock;
constexpr int kReconWaves = kReconBlock / 64;

struct ReconArgs {
    int64_t begin;
    int64_t n;
    uint32_t width;
    Divisor by_width;      // id / width with one multiply-high
    uint32_t height;
    int regions_x;
    int regions_y;
    int experts;
    const int32_t* slots;      // table slot of each tile, < 0: no expert (null: slot = tile)
    const uint32_t* table;     // fp16 pairs
    int64_t expert_pairs;      // pairs per expert
    const uint16_t* weights;
    float* prediction;         // [n][3] or null
    uint16_t* features;        // [n][32] or null
    uint16_t* output;          // [n][16] or null
    DevLevel level[kLevels];
};

// Per-block copies of the decoder's forward weights, the tile bounds and the level descriptors
// (read from LDS, the descriptors stay out of the scalar registers the unrolled levels would
// otherwise spill).
__device__ inline void stage_model(const ReconArgs& a, const TileBounds& bounds, _Float16* w, TileBounds& tb,
                                   DevLevel* levels) {
    stage_forward_weights<2>(a.weights, w);
    constexpr int kLevelWords = kLevels * static_cast<int>(sizeof(DevLevel) / 4);
    static_assert(kLevelWords <= kReconBlock, "one thread per descriptor word");
    if (static_cast<int>(threadIdx.x) < kLevelWords)
        reinterpret_cast<uint32_t*>(levels)[threadIdx.x] = reinterpret_cast<const uint32_t*>(a.level)[threadIdx.x];
    for (int j = threadIdx.x; j <= kMaxTiles; j += kReconBlock) {
        tb.x0[j] = bounds.x0[j];
        tb.y0[j] = bounds.y0[j];
        if (j < kMaxTiles) {
            tb.rx[j] = bounds.rx[j];
            tb.ry[j] = bounds.ry[j];
        }
    }
    if (threadIdx.x == 0) {
        tb.sx = bounds.sx;
        tb.sy = bounds.sy;
    }
    __syncthreads();
}

// The wave's 32 pixels (pixel s of lane (g, s) is `id`, `valid` when it is real): the encode of
// lane (g, s)'s eight levels (pairs) and the decoder output rows of lane group g (out).
__device__ inline void predict(const ReconArgs& a, const TileBounds& tb, const DevLevel* levels, const _Float16* w,
                               uint32_t id, bool valid,
                               int g, int s, uint32_t pairs[2][4], half8& out) {
    uint32_t y = divide(id, a.by_width);
    const uint32_t x = id - y * a.width;
    if (y >= a.height) y = a.height - 1;
    const int tx = tile_of(a.regions_x, a.width, tb.sx, x), ty = tile_of(a.regions_y, a.height, tb.sy, y);
    const int t = ty * a.regions_x + tx;
    int slot = a.slots ? a.slots[t] : t;
    if (slot >= a.experts || !valid) slot = -1;
    const float u = static_cast<float>(x - static_cast<uint32_t>(tb.x0[tx])) * tb.rx[tx];
    const float v = static_cast<float>(y - static_cast<uint32_t>(tb.y0[ty])) * tb.ry[ty];
    const uint32_t* table = a.table + (slot >= 0 ? static_cast<int64_t>(slot) * a.expert_pairs : 0);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // lane group g encodes level 8kt + 4g + j
            const DevLevel lv = levels[8 * kt + 4 * g + j];
            uint32_t idx[4];
            float wk[4];
            grid_corners(lv, u, v, idx, wk);
            uint32_t e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) e[k] = slot >= 0 ? table[lv.offset + idx[k]] : 0u;
            pairs[kt][j] = slot >= 0 ? half2_level(e, wk) : 0u;
        }
    }
    half8 xb[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
        xb[kt] = __builtin_bit_cast(half8, u32x4{pairs[kt][0], pairs[kt][1], pairs[kt][2], pairs[kt][3]});
    half8 h1[4], h2[4];
    f32x16 acc3;
    forward_tile<2>(w, g, s, xb, h1, h2, acc3);
    out = round8(acc3, 0);
}

// Output rows 0..2 (the RGB prediction) are elements 0..2 of lane group 0.
__device__ inline void rgb_of(const half8& out, float& r, float& gr, float& b) {
    const u32x4 bits = __builtin_bit_cast(u32x4, out);   // element 2i in the low half of dword i
    r = __half2float(bits_to_half(static_cast<uint16_t>(bits.x & 0xffffu)));
    gr = __half2float(bits_to_half(static_cast<uint16_t>(bits.x >> 16)));
    b = __half2float(bits_to_half(static_cast<uint16_t>(bits.y & 0xffffu)));
}

__global__ __launch_bounds__(kReconBlock) void reconstruct_kernel(ReconArgs a, TileBounds bounds) {
    __shared__ _Float16 w[kForwardHalfs];
    __shared__ TileBounds tb;
    __shared__ DevLevel levels[kLevels];
    stage_model(a, bounds, w, tb, levels);
    const int lane = threadIdx.x % 64, g = lane / 32, s = lane % 32;
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kReconWaves;
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kReconWaves + threadIdx.x / 64; tile < tiles;
         tile += waves) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        uint32_t pairs[2][4];
        half8 out;
        predict(a, tb, levels, w, static_cast<uint32_t>(a.begin + (valid ? row : 0)), valid, g, s, pairs, out);
        if (!valid) continue;
        if (a.features) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                *reinterpret_cast<uint4*>(a.features + row * 32 + 16 * kt + 8 * g) =
                    make_uint4(pairs[kt][0], pairs[kt][1], pairs[kt][2], pairs[kt][3]);
        }
        if (a.output) {
            const u32x4 bits = __builtin_bit_cast(u32x4, out);
            uint16_t* p = a.output + row * 16;
            *reinterpret_cast<uint2*>(p + 4 * g) = make_uint2(bits.x, bits.y);
            *reinterpret_cast<uint2*>(p + 8 + 4 * g) = make_uint2(bits.z, bits.w);
        }
        if (a.prediction && g == 0) {
            float* p = a.prediction + row * 3;
            rgb_of(out, p[0], p[1], p[2]);
        }
    }
}

struct ScoreArgs {
    const uint8_t* target;   // RGB8 [H*W][3]
    int resolution;
    const int32_t* xb;       // cell column / row bounds [R+1]
    const int32_t* yb;
    double* totals;          // fp64 [R*R], continued
    double* squares;         // fp64 [R*R] or null: sum of (p - byte*(1/255))^2 over the cell's channels
};

__device__ inline double lane_double(double value, int lane) {
    const uint64_t bits = __double_as_longlong(value);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(bits), lane);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(bits >> 32), lane);
    return __longlong_as_double((static_cast<uint64_t>(hi) << 32) | lo);
}

// One wave per residual cell: the cell's pixels in raster order, 32 at a time, predicted as in
// reconstruct_kernel; each pixel's residual term (residual_term, the streamed pass's
// arithmetic) is folded into the cell total in order -- row by row, left to right -- so the
// total is the reference's sequential fp64 sum bit for bit, with no prediction in memory.
__global__ __launch_bounds__(kReconBlock) void score_kernel(ReconArgs a, TileBounds bounds, ScoreArgs sc) {
    __shared__ _Float16 w[kForwardHalfs];
    __shared__ TileBounds tb;
    __shared__ DevLevel levels[kLevels];
    stage_model(a, bounds, w, tb, levels);
    const int lane = threadIdx.x % 64, g = lane / 32, s = lane % 32;
    const int cells = sc.resolution * sc.resolution;
    const float inv255 = 1.0f / 255.0f;
    for (int cell = blockIdx.x * kReconWaves + threadIdx.x / 64; cell < cells; cell += gridDim.x * kReconWaves) {
        const int cx = cell % sc.resolution, cy = cell / sc.resolution;
        const int x0 = max(sc.xb[cx], 0), x1 = min(sc.xb[cx + 1], static_cast<int>(a.width));
        const int y0 = max(sc.yb[cy], 0), y1 = min(sc.yb[cy + 1], static_cast<int>(a.height));
        double sum = sc.totals[cell], squares = 0.0;
        for (int y = y0; y < y1; ++y) {
            for (int xs = x0; xs < x1; xs += 32) {
                const int count = min(32, x1 - xs);
                const bool valid = s < count;
                const uint32_t id = static_cast<uint32_t>(y) * a.width + static_cast<uint32_t>(xs + (valid ? s : 0));
                uint32_t pairs[2][4];
                half8 out;
                predict(a, tb, levels, w, id, valid, g, s, pairs, out);
                double term = 0.0;
                if (g == 0 && valid) {
                    float p0, p1, p2;
                    rgb_of(out, p0, p1, p2);
                    const uint8_t* px = sc.target + 3ull * id;
                    const uint8_t b0 = px[0], b1 = px[1], b2 = px[2];
                    term = residual_term(p0, p1, p2, byte_target(b0), byte_target(b1), byte_target(b2));
                    const float e0 = p0 - static_cast<float>(b0) * inv255, e1 = p1 - static_cast<float>(b1) * inv255,
                                e2 = p2 - static_cast<float>(b2) * inv255;
                    squares += static_cast<double>(e0 * e0);
                    squares += static_cast<double>(e1 * e1);
                    squares += static_cast<double>(e2 * e2);
                    if (a.prediction) {
                        float* p = a.prediction + 3ull * id;
                        p[0] = p0;
                        p[1] = p1;
                        p[2] = p2;
                    }
                }
                for (int j = 0; j < count; ++j) sum = sum + lane_double(term, j);
            }
        }
        for (int step = 32; step; step >>= 1) squares += __shfl_xor(squares, step);
        if (lane == 0) {
            sc.totals[cell] = sum;
            if (sc.squares) sc.squares[cell] = squares;
        }
    }
}

}  // namespace
}  // namespace odie

using namespace odie;

// Validates the model arguments shared by both entry points and fills a (everything but the
// pixel range and the outputs).  Returns 0 or -1 with the error set.
static int model_args(const char* what, int width, int height, int regions_x, int regions_y, const int32_t* slots,
                      int experts, const uint16_t* table, int64_t expert_params, const odie_grid_level* levels,
                      int n_levels, const uint16_t* weights, ReconArgs& a, TileBounds& bounds) {
    const std::string w(what);
    if (regions_x < 1 || regions_y < 1 || regions_x > kMaxTiles || regions_y > kMaxTiles)
        return fail(w + ": regions per axis must be within 1..64");
    if (width < 2 * regions_x || height < 2 * regions_y)
        return fail(w + ": every tile needs at least two pixels per axis");
    if (static_cast<uint64_t>(width) * static_cast<uint64_t>(height) > (uint64_t{1} << 32))
        return fail(w + ": images are limited to 2^32 pixels");
    if (n_levels != kLevels) return fail(w + ": the fused decoder takes 16 levels x 2 features");
    if (experts < 1) return fail(w + ": experts must be >= 1");
    if (!levels) return fail(w + ": levels is null");
    uint64_t entries = 0;
    if (make_dev_levels(what, levels, n_levels, a.level, entries)) return -1;
    if (expert_params < static_cast<int64_t>(entries) * 2 || expert_params % 2)
        return fail(w + ": expert_params must be even and hold the levels' table");
    if (!table || !weights) return fail(w + ": null pointer");
    if (reinterpret_cast<uintptr_t>(table) % 4) return fail(w + ": table must be 4-byte aligned");
    a.width = static_cast<uint32_t>(width);
    a.by_width = make_divisor(a.width);
    a.height = static_cast<uint32_t>(height);
    a.regions_x = regions_x;
    a.regions_y = regions_y;
    a.experts = experts;
    a.slots = slots;
    a.table = reinterpret_cast<const uint32_t*>(table);
    a.expert_pairs = expert_params / 2;
    a.weights = weights;
    make_tile_bounds(width, height, regions_x, regions_y, bounds);
    return 0;
}

ODIE_API int odie_reconstruct(int64_t begin, int64_t n, int width, int height, int regions_x, int regions_y,
                              const int32_t* slots, int experts, const uint16_t* table, int64_t expert_params,
                              const odie_grid_level* levels, int n_levels, const uint16_t* weights, float* prediction,
                              uint16_t* features, uint16_t* output, uint64_t stream) {
    if (n < 0 || begin < 0) return fail("odie_reconstruct: begin and n must be nonnegative");
    ReconArgs a{};
    TileBounds bounds;
    if (model_args("odie_reconstruct", width, height, regions_x, regions_y, slots, experts, table, expert_params,
                   levels, n_levels, weights, a, bounds))
        return -1;
    if (static_cast<uint64_t>(begin) + static_cast<uint64_t>(n) > static_cast<uint64_t>(width) * height)
        return fail("odie_reconstruct: the pixel range runs past the image");
    if (n == 0) return 0;
    if (!prediction && !features && !output) return fail("odie_reconstruct: no output");
    if ((features && reinterpret_cast<uintptr_t>(features) % 16) || (output && reinterpret_cast<uintptr_t>(output) % 8))
        return fail("odie_reconstruct: features must be 16-byte and output 8-byte aligned");
    a.begin = begin;
    a.n = n;
    a.prediction = prediction;
    a.features = features;
    a.output = output;
    const int64_t tiles = (n + 31) / 32;
    int64_t blocks = (tiles + kReconWaves - 1) / kReconWaves;
    if (blocks > 4096) blocks = 4096;
    reconstruct_kernel<<<static_cast<uint32_t>(blocks), kReconBlock, 0, as_stream(stream)>>>(a, bounds);
    return check_launch("odie_reconstruct");
}

ODIE_API int odie_reconstruct_scores(int width, int height, int regions_x, int regions_y, const int32_t* slots,
                                     int experts, const uint16_t* table, int64_t expert_params,
                                     const odie_grid_level* levels, int n_levels, const uint16_t* weights,
                                     const uint8_t* target, int resolution, const int32_t* xb, const int32_t* yb,
                                     double* totals, double* squares, float* prediction, uint64_t stream) {
    ReconArgs a{};
    TileBounds bounds;
    if (model_args("odie_reconstruct_scores", width, height, regions_x, regions_y, slots, experts, table,
                   expert_params, levels, n_levels, weights, a, bounds))
        return -1;
    if (resolution < 1 || resolution > 65536) return fail("odie_reconstruct_scores: resolution must be within 1..65536");
    if (!target || !xb || !yb || !totals) return fail("odie_reconstruct_scores: null pointer");
    a.prediction = prediction;
    ScoreArgs sc{target, resolution, xb, yb, totals, squares};
    const int64_t cells = static_cast<int64_t>(resolution) * resolution;
    int64_t blocks = (cells + kReconWaves - 1) / kReconWaves;
    if (blocks > 65536) blocks = 65536;
    score_kernel<<<static_cast<uint32_t>(blocks), kReconBlock, 0, as_stream(stream)>>>(a, bounds, sc);
    return check_launch("odie_reconstruct_scores");
}
