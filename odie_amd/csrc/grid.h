// Device helpers shared by the grid encode kernels: level descriptors and the
// tiny-cuda-nn grid geometry (corner indices and bilinear weights).
#pragma once
#include <type_traits>

#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {

struct DevLevel {
    float scale;
    uint32_t res;
    uint32_t size;
    uint32_t mask;    // size - 1 when size is a power of two, else 0
    uint32_t offset;  // first entry of the level
    uint32_t hashed;
    uint32_t prime;   // hash multiplier: 2654435761 & mask when 0 < mask < 2^24, else 2654435761
};

// Row term of the spatial hash, y * 2654435761 reduced mod the (power-of-two) table size.
// When the table has at most 2^24 entries only the low 24 bits of the product survive the
// mask, and those depend only on the low 24 bits of both factors, so the full-rate 24-bit
// multiply gives exactly the bits the 32-bit product would.
__device__ inline uint32_t hash_row(uint32_t y, const DevLevel& lv) {
    if (lv.mask && lv.mask < (1u << 24)) return __umul24(y, lv.prime);
    return y * 2654435761u;
}

__device__ inline uint32_t wrap_index(uint32_t v, const DevLevel& lv) {
    if (lv.mask) return v & lv.mask;
    if (v < lv.size) return v;
    v -= lv.size;
    return v < lv.size ? v : v % lv.size;
}

// The four corner indices of one level reduced mod the table size (wrap_index on each): a mask
// for power-of-two tables; otherwise one conditional subtraction, and the remainder only when a
// lane's index is still out of range after it (coordinates far off the unit square).
__device__ inline void wrap_corners(uint32_t idx[4], const DevLevel& lv) {
    if (lv.mask) {
#pragma unroll
        for (int k = 0; k < 4; ++k) idx[k] &= lv.mask;
        return;
    }
    bool far = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        idx[k] = idx[k] >= lv.size ? idx[k] - lv.size : idx[k];
        far |= idx[k] >= lv.size;
    }
    if (far) {
#pragma unroll
        for (int k = 0; k < 4; ++k) idx[k] = idx[k] < lv.size ? idx[k] : idx[k] % lv.size;
    }
}

// tiny-cuda-nn grid geometry: p = fma(scale, x, 0.5), corner = floor(p), fraction p - floor(p);
// corners (0,0),(1,0),(0,1),(1,1); dense index x + y*res, hashed x ^ y*2654435761, mod size.
// The row terms are formed once per row of corners.
__device__ inline void grid_corners(const DevLevel& lv, float x, float y, uint32_t idx[4], float w[4]) {
    const float px = __builtin_fmaf(lv.scale, x, 0.5f);
    const float py = __builtin_fmaf(lv.scale, y, 0.5f);
    const float flx = floorf(px), fly = floorf(py);
    const uint32_t gx = static_cast<uint32_t>(static_cast<int32_t>(flx));
    const uint32_t gy = static_cast<uint32_t>(static_cast<int32_t>(fly));
    const float fx = px - flx, fy = py - fly;
    w[0] = (1.0f - fx) * (1.0f - fy);
    w[1] = fx * (1.0f - fy);
    w[2] = (1.0f - fx) * fy;
    w[3] = fx * fy;
    if (lv.hashed) {
        const uint32_t h0 = hash_row(gy, lv), h1 = hash_row(gy + 1u, lv);
        idx[0] = gx ^ h0;
        idx[1] = (gx + 1u) ^ h0;
        idx[2] = gx ^ h1;
        idx[3] = (gx + 1u) ^ h1;
    } else {
        const uint32_t base = gx + gy * lv.res;
        idx[0] = base;
        idx[1] = base + 1u;
        idx[2] = base + lv.res;
        idx[3] = base + lv.res + 1u;
    }
    wrap_corners(idx, lv);
}

// One fp16 level of 2 features: acc = fma(fp16(w_k), entry_k, acc) over the corners in order,
// from +0, on both features at once (v_pk_fma_f16); entries and the result are fp16 pairs
// (feature 0 in the low half).  The forward's arithmetic (odie/packed_kernels.cu:52-62).
__device__ inline uint32_t half2_level(const uint32_t g[4], const float w[4]) {
    __half2 acc = __half2(__float2half(0.0f), __float2half(0.0f));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const __half2 value = __halves2half2(bits_to_half(static_cast<uint16_t>(g[k] & 0xffffu)),
                                             bits_to_half(static_cast<uint16_t>(g[k] >> 16)));
        acc = __hfma2(__float2half2_rn(keep_fp32(w[k])), value, acc);
    }
    return static_cast<uint32_t>(half_to_bits(__low2half(acc))) |
           (static_cast<uint32_t>(half_to_bits(__high2half(acc))) << 16);
}

template <bool HALF>
using Elem = typename std::conditional<HALF, __half, float>::type;

// Packed xy planes (odie/packed_kernels.cu:12-88 semantics).  Descriptor row d of a level:
// d[0] resolution R, d[1] points, d[2] plane offset, d[3] node word offset, d[4] cell bitmap
// byte offset, d[5] features, d[6] feature offset, d[7] direct (1: row = node).
//
// Geometry at integer resolution R: p = fma(R-1, x, 0.5), cell = floor(px) + floor(py)*R.
// The cell's integer corner is clamped into the plane so that any input addresses memory
// inside the layout; for x, y in [0,1] the clamp never changes the corner.
__device__ inline void plane_geometry(float x, float y, int r, int& cell, float w[4]) {
    const float px = __builtin_fmaf(static_cast<float>(r - 1), x, 0.5f);
    const float py = __builtin_fmaf(static_cast<float>(r - 1), y, 0.5f);
    int ix = static_cast<int>(floorf(px)), iy = static_cast<int>(floorf(py));
    const float fx = px - static_cast<float>(ix), fy = py - static_cast<float>(iy);
    ix = ix < 0 ? 0 : (ix > r - 1 ? r - 1 : ix);
    iy = iy < 0 ? 0 : (iy > r - 1 ? r - 1 : iy);
    cell = ix + iy * r;
    w[0] = (1.0f - fx) * (1.0f - fy);
    w[1] = fx * (1.0f - fy);
    w[2] = (1.0f - fx) * fy;
    w[3] = fx * fy;
}

// Parameter of feature c of corner k of `cell`: node (cell + k%2 + (k/2) R) mod points, its row
// (the node itself, or its rank among the stored nodes: word prefix + popcount below it),
// plane offset + row * features + c, clamped into the parameters.
// Row of corner k of `cell` (the first half of packed_param; the same for every feature).
__device__ inline int packed_row(const int32_t* d, const uint64_t* node_bitmap, const int32_t* prefix, int cell,
                                 int k) {
    const int node = (cell + (k & 1) + (k >> 1) * d[0]) % d[1];
    if (d[7]) return node;
    const int word = d[3] + (node >> 6), bit = node & 63;
    const uint64_t mask = (uint64_t{1} << bit) - uint64_t{1};
    return prefix[word] + __popcll(node_bitmap[word] & mask);
}

// Parameter of feature c of a corner in row `row`, clamped into the parameters.
__device__ inline int64_t packed_at(const int32_t* d, int64_t params, int row, int c) {
    const int64_t p = static_cast<int64_t>(d[2]) + static_cast<int64_t>(row) * d[5] + c;
    return p < 0 ? 0 : (p >= params ? params - 1 : p);
}

__device__ inline int64_t packed_param(const int32_t* d, const uint64_t* node_bitmap, const int32_t* prefix,
                                       int64_t params, int cell, int k, int c) {
    return packed_at(d, params, packed_row(d, node_bitmap, prefix, cell, k), c);
}

__device__ inline bool cell_visible(const int32_t* d, const uint8_t* bitmap, int cell) {
    return (bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1;
}

// Host: device rows of an odie_grid_level table (levels contiguous from entry 0); entries
// receives the table's entry count.  Returns 0, or -1 with the error set.
inline int make_dev_levels(const char* what, const odie_grid_level* levels, int n_levels, DevLevel* out,
                           uint64_t& entries) {
    const std::string w(what);
    entries = 0;
    for (int l = 0; l < n_levels; ++l) {
        const odie_grid_level& lv = levels[l];
        if (lv.size == 0 || lv.resolution == 0) return fail(w + ": level size and resolution must be positive");
        if (!(lv.scale == lv.scale)) return fail(w + ": level scale is NaN");
        if (lv.offset != entries) return fail(w + ": level offsets must be contiguous from 0");
        entries += lv.size;
        DevLevel& d = out[l];
        d.scale = lv.scale;
        d.res = lv.resolution;
        d.size = lv.size;
        d.mask = (lv.size & (lv.size - 1)) == 0 ? lv.size - 1 : 0;
        d.offset = lv.offset;
        d.hashed = lv.hashed ? 1u : 0u;
        d.prime = (d.mask && d.mask < (1u << 24)) ? (2654435761u & d.mask) : 2654435761u;
    }
    return 0;
}

// Host-side description of one owner-computes backward launch (backward.hip).
struct AdamStep;

// What the encode forward can hand the owner backward of the same batch (the handoff buffer),
// from the owner's own plan: its slice masks when its passes are unbanded, or its band lists
// when they are banded (else nothing, bytes 0).
//   masks: plane p (`stride` bytes, stride >= n) belongs to level level[p]; its byte i has bit s
//     set when a corner of coordinate i lands in the aligned block s of 2^bits[p] entries;
//   lists: at byte 0 each expert's slot starts [experts][kBandSlots + 1] and the `ordered` word,
//     at list_at the coordinate index of every list position [n] (int32), at sorted_at that
//     coordinate's (x, y) [n] (float2); the band kernels' counts go to the library's workspace.
constexpr int kMaxMaskPlanes = 16;
struct HandoffPlan {
    int planes;
    int level[kMaxMaskPlanes];
    int bits[kMaxMaskPlanes];
    int64_t stride;
    int lists;        // 1: band lists (and no masks)
    int parts;        // band counting parts per expert
    int64_t ordered_at, list_at, sorted_at;
    int64_t bytes;    // the handoff buffer's length
};

struct OwnerLaunch {
    const float* coords;
    const int32_t* offsets;   // null for a single grid
    const void* upstream;     // [n, up_width] row-major
    int up_half;
    int up_width;
    float* grad;
    int accumulate;
    int64_t n;
    int64_t expert_params;
    int experts;
    int n_levels;
    int features;
    const DevLevel* levels;   // host array [n_levels]
    int64_t lds_bytes;
    int remap;
    int banded;               // fine passes walk y-band lists: 0 never, 1 always, 2 when they pay
    int masks;                // unbanded hashed slices walk only coordinates whose slice mask reaches them
    int64_t split_target;     // banded: coordinate-level visits per work item (0: chosen per launch)
    hipStream_t stream;
    const AdamStep* adam;   // non-null: apply this optimizer step instead of writing grad
    const void* planes;       // non-null: upstream already level-major [n_levels][n][features]
    const float* blockmax;    // with planes: max |upstream| per 128-row record and level
    HandoffPlan* plan_out;    // non-null: only fill in the handoff plan (no launch, no workspace)
    const uint8_t* handoff;   // non-null: the handoff buffer, already filled (by the forward) per the
                              // plan, handoff_bytes long; else the backward forms masks or lists itself
    int64_t handoff_bytes;
};
int launch_owner_backward(const OwnerLaunch& launch);
// The band lists of a banded plan into `handoff` (plan.lists), for the forward to walk and the
// backward to reuse: the owner's own band kernels on in.coords / in.offsets.
int launch_band_lists(const OwnerLaunch& in, const HandoffPlan& plan, uint8_t* handoff);

// Owner-computes backward of packed xy planes (backward.hip): gradient [params] fp32, every
// value written once.  upstream fp16 [n][width]; descriptors device [levels][8].
int launch_packed_owner(const float* coords, int64_t n, const uint16_t* upstream, int width, const int32_t* desc,
                        int levels, const uint64_t* node_bitmap, const int32_t* node_prefix, const uint8_t* bitmap,
                        float* gradient, int64_t params, int64_t lds_bytes, int64_t splits, hipStream_t stream);

// odie_grid_backward_adam with the optimizer step already formed (adam.h), so that callers
// can set fields the C ABI does not expose (the fp16 gradient store).
int grid_backward_adam_internal(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                                const odie_grid_level* levels, int n_levels, int features, const AdamStep& adam,
                                hipStream_t stream);

// grid_backward_adam_internal on an upstream already in the owner's layout (fp16 level-major
// planes and their 128-row maxima, as the decoder's training kernel can write them).
int grid_backward_adam_planes_internal(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                       const uint32_t* planes, const float* blockmax, int64_t expert_params,
                                       const odie_grid_level* levels, int n_levels, int features,
                                       const AdamStep& adam, hipStream_t stream);

// The packed-plane forward with the native step's active prefix (levels >= active are off)
// and the fp16 bits written past the last level (the runtime pads with 1.0).  levels16x2: the
// caller guarantees 16 levels of 2 features at output offsets 2l (the faster kernel applies).
// pairs: the caller guarantees 2 features at output offset 2l for every level but the last,
// which has 1 or 2 (the pairs kernel applies when the row is a multiple of 16 columns).
// odie_packed_backward on `s`; zeroed: the caller has already cleared `gradient` (the atomics
// path then adds into it without clearing it first).
int packed_backward_internal(const float* coords, int64_t n, const uint16_t* upstream, int up_width,
                             const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                             const int32_t* node_prefix, const uint8_t* bitmap, float* gradient,
                             int64_t parameter_count, hipStream_t s, bool zeroed);

int packed_forward_internal(const float* coords, int64_t n, const float* grid, int64_t parameter_count,
                            const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                            const int32_t* node_prefix, const uint8_t* bitmap, int width, int active, uint16_t pad,
                            uint16_t* features, uint8_t* visibility, hipStream_t stream, bool levels16x2 = false,
                            bool pairs = false);


}  // namespace odie
