// Expert routing and compaction for gfx950.
//
// A pixel id is split into (x, y) = (id % W, id / W) with 32-bit arithmetic, as the
// reference's batch kernel does (odie/native/runtime.cu:33-36).  The image is cut into a
// regions_x x regions_y grid of tiles with integer bounds x0[r] = ceil(r*W/regions_x) (and
// the same for y); expert = ry*regions_x + rx.  Each expert fits its tile as a sub-image,
// so the coordinate it sees is the reference's pixel -> coordinate convention applied to
// the tile: u = fp32(x - x0[rx]) * fp32(1/(tile_width-1)) (fp32 product of the fp32
// reciprocal of the exact double quotient, runtime.cu:35-36), same for v.
//
// Compaction is a stable counting sort by expert: coordinates end up grouped by expert,
// in their original order inside each expert (numpy argsort(kind='stable') order, the tie
// rule the reference uses for rankings, odie/selection.py:116).
//   pass 1  each wave counts the experts of its own sub-chunk (LDS histogram per wave)
//   pass 2  a parallel scan of the counts, expert-major then sub-chunk order
//   pass 3  the scatter: lanes sharing an expert get their order from one ballot per bit of
//           the expert id, a running count in LDS carries it across groups of 64, and the
//           staged form writes each expert's run of a group of sub-chunks out in one piece.
//           No global atomics, so the result is deterministic.
#include <map>
#include <mutex>
#include <set>
#include <string>

#include "common.h"
#include "sampling.h"
#include "tiles.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kRouteBlock = 256;
constexpr int kWaves = kRouteBlock / 64;
constexpr int kCountThreads = 512;   // the grouped count pass's workgroup (2048 id pairs per round either way)
constexpr int kMaxRegions = kMaxTiles;
constexpr int kMaxExperts = kMaxRegions * kMaxRegions;

struct RouteArgs {
    const int64_t* ids;
    const float* uniforms;  // in place of ids: slot i is the pixel of stratified slot i (side x side strata)
    int side;
    float inv_side;
    int32_t* expert_out;
    int32_t* perm;
    float* coords;
    int32_t* offsets;
    const uint8_t* rgb;     // image bytes [height*width][3], or null
    uint32_t* colors;       // packed r | g << 8 | b << 16 of each slot's pixel, or null
    int32_t* counts;   // [experts * parts]
    int32_t* block_sums;  // [ceil(experts * parts / kScanSegment)]
    uint32_t* scan_ticket; // with the one-launch scan: block_sums + its segments (block_sums hold sum + 1)
    int scan_segments;     // with the one-launch scan: its blocks
    const int32_t* slots; // tile -> expert, or null (expert = tile); with slots, bucket `owned` holds
                          // the ids of tiles without an expert (slot outside [0, owned))
    int owned;            // experts owning tiles (with slots; experts = owned + 1 buckets)
    int64_t n;
    uint32_t width;
    uint32_t height;
    Divisor by_width;      // id / width with one multiply-high
    int regions_x;
    int regions_y;
    int experts;       // buckets of the counting sort
    int expert_bits;   // bits of the largest bucket id
    int part;          // ids per wave sub-chunk (multiple of 64)
    int parts;         // number of sub-chunks
    int per_column;    // sub-chunks per column of the counts (1, or the staged scatter's group)
    int columns;       // columns of the expert-major counts: ceil(parts / per_column)
    int32_t x0[kMaxRegions + 1];
    int32_t y0[kMaxRegions + 1];
    float rx[kMaxRegions];   // fp32(1/(tile_width-1))
    float ry[kMaxRegions];
    float sx, sy;            // fp32(regions_x / width), fp32(regions_y / height)
};

struct Bounds {
    int32_t x0[kMaxRegions + 1];
    int32_t y0[kMaxRegions + 1];
};

// The walks below load kAhead groups of 64 ids per wave before placing any of them (the direct
// scatter kDirectAhead: on stratified batches, whose draw it forms itself, more loads in flight
// paid; the count and staged walks measured faster with fewer).
constexpr int kAhead = 4;
constexpr int kDirectAhead = 8;

// Pixel ids (their low 32 bits: ids are below 2^32 once clamped into the image) of inputs
// first + k * stride (k < K), each index past `last` clamped to it; slot i of a stratified batch
// is the pixel its uniforms draw.  The choice between stored ids and the draw is made once for
// all K, so that every load is issued before any of them is used.
template <int K>
__device__ inline void pixel_ids(const RouteArgs& a, int64_t first, int64_t stride, int64_t last, uint32_t id[K]) {
    if (a.uniforms) {
        float2 u[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int64_t i = first + k * stride < last ? first + k * stride : last;
            u[k] = reinterpret_cast<const float2*>(a.uniforms)[i];
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int64_t i = first + k * stride < last ? first + k * stride : last;
            id[k] = static_cast<uint32_t>(stratified_id(u[k], i, a.side, a.inv_side, static_cast<int>(a.width),
                                                        static_cast<int>(a.height)));
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k) id[k] = static_cast<uint32_t>(a.ids[first + k * stride < last ? first + k * stride : last]);
    }
}

__device__ inline void locate_id(const RouteArgs& a, uint32_t id, int& expert, uint32_t& x,
                                 uint32_t& y, int& rx, int& ry) {
    y = divide(id, a.by_width);
    x = id - y * a.width;
    if (y >= a.height) y = a.height - 1;  // ids past the image clamp to its last row
    rx = tile_of(a.regions_x, a.width, a.sx, x);
    ry = tile_of(a.regions_y, a.height, a.sy, y);
    expert = ry * a.regions_x + rx;
    if (a.slots) {
        const int32_t slot = a.slots[expert];
        expert = slot >= 0 && slot < a.owned ? slot : a.owned;
    }
}

// The expert reported for an id in bucket `expert`: -1 for the bucket of tiles without one.
__device__ inline int32_t reported(const RouteArgs& a, int expert) {
    return a.slots && expert == a.owned ? -1 : expert;
}

__device__ inline void load_bounds(const RouteArgs& a, Bounds& b) {
    for (int j = threadIdx.x; j <= kMaxRegions; j += blockDim.x) {
        b.x0[j] = a.x0[j];
        b.y0[j] = a.y0[j];
    }
    __syncthreads();
}

// Counts per expert of every sub-chunk (per_column 1: each wave counts one sub-chunk, and the
// block's kWaves counts of each expert are consecutive in the expert-major array, so they are
// written as one run), or of every group of per_column consecutive sub-chunks (GROUPED: a block
// per group, its waves taking the group's sub-chunks in turn; the staged scatter needs no finer
// offsets, and the scans then run over per_column times fewer counts).
template <bool GROUPED, int T = kRouteBlock>
__global__ __launch_bounds__(T) void route_count_kernel(RouteArgs a) {
    extern __shared__ int32_t hist[];  // [experts][kWaves] counts of the block's sub-chunks, or [experts]
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    constexpr int kSlots = GROUPED ? 1 : kWaves;
    const int first = static_cast<int>(blockIdx.x) * (GROUPED ? a.per_column : kWaves);
    const int members = GROUPED ? a.per_column : kWaves;
    if (a.scan_ticket)   // the one-launch scan's published sums (0: not yet) and its ticket
        for (int j = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); j <= a.scan_segments;
             j += static_cast<int>(gridDim.x * blockDim.x))
            a.block_sums[j] = 0;
    if constexpr (GROUPED) {
        // the group's ids as 16-byte pairs (ids 16-byte aligned: checked by the host), every
        // pair of a round of kPairs per thread loaded before any is used; the first round is
        // issued before the histogram is cleared, so its loads fly over the clear and the barrier
        constexpr int kPairs = 2048 / T;
        const int64_t begin = static_cast<int64_t>(first) * a.part;
        const int64_t group_end = begin + static_cast<int64_t>(members) * a.part;
        const int64_t end = group_end < a.n ? group_end : a.n;
        const int4* pairs = reinterpret_cast<const int4*>(a.ids + begin);
        const int64_t count = end - begin, npairs = count / 2;   // whole pairs; an odd last id alone
        int4 two[kPairs];
        auto fetch = [&](int64_t round) {
#pragma unroll
            for (int k = 0; k < kPairs; ++k) {
                const int64_t q = round + k * T + threadIdx.x;
                two[k] = pairs[q < npairs ? q : npairs - 1];
            }
        };
        if (npairs > 0) fetch(0);
        for (int j = threadIdx.x; j < a.experts; j += T) hist[j] = 0;
        __syncthreads();
        for (int64_t round = 0; round < npairs; round += T * kPairs) {
            if (round > 0) fetch(round);
#pragma unroll
            for (int k = 0; k < kPairs; ++k) {
                const int64_t q = round + k * T + threadIdx.x;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    int expert, rx, ry;
                    uint32_t x, y;
                    locate_id(a, static_cast<uint32_t>(h ? two[k].z : two[k].x), expert, x, y, rx, ry);
                    if (q < npairs) atomicAdd(hist + expert, 1);
                }
            }
        }
        if ((count & 1) && threadIdx.x == 0) {
            int expert, rx, ry;
            uint32_t x, y;
            locate_id(a, static_cast<uint32_t>(a.ids[end - 1]), expert, x, y, rx, ry);
            atomicAdd(hist + expert, 1);
        }
    }
    if constexpr (!GROUPED) {
        for (int j = threadIdx.x; j < a.experts * kSlots; j += kRouteBlock) hist[j] = 0;
        __syncthreads();
    }
    for (int k = wave; !GROUPED && k < members && first + k < a.parts; k += kWaves) {
        const int64_t begin = static_cast<int64_t>(first + k) * a.part;
        const int64_t end = begin + a.part < a.n ? begin + a.part : a.n;
        int32_t* counter = hist + (GROUPED ? 0 : wave);
        for (int64_t g = begin; g < end; g += 64 * kAhead) {
            uint32_t id[kAhead];
            pixel_ids<kAhead>(a, g + lane, 64, end - 1, id);
#pragma unroll
            for (int j = 0; j < kAhead; ++j) {
                int expert, rx, ry;
                uint32_t x, y;
                locate_id(a, id[j], expert, x, y, rx, ry);
                if (g + j * 64 + lane < end) atomicAdd(counter + expert * kSlots, 1);
            }
        }
    }
    __syncthreads();
    if constexpr (GROUPED) {
        for (int e = threadIdx.x; e < a.experts; e += T)
            a.counts[static_cast<int64_t>(e) * a.columns + blockIdx.x] = hist[e];
    } else {
        for (int j = threadIdx.x; j < a.experts * kWaves; j += kRouteBlock) {
            const int e = j / kWaves, k = j % kWaves;
            if (first + k < a.parts) a.counts[static_cast<int64_t>(e) * a.columns + first + k] = hist[j];
        }
    }
}

// Exclusive scan of counts (expert-major) in place: every block sums a segment of kScanSegment
// counts; then every block rescans its segment from its offset, the sum of the segments before
// it (added up by the block itself when there are at most 1024 segments, else scanned by one
// block in a launch between the two).  offsets[e] = first slot of expert e; offsets[E] = n.
constexpr int kScanBlock = 256;
constexpr int kScanSegment = 1024;  // counts per scan block (4 per thread)

__device__ inline int32_t block_exclusive_scan(int32_t value, int32_t* shared, int32_t& total) {
    // Inclusive scan of one value per thread over the block (kScanBlock threads) in LDS.
    shared[threadIdx.x] = value;
    __syncthreads();
    for (int stride = 1; stride < kScanBlock; stride <<= 1) {
        const int32_t add = threadIdx.x >= stride ? shared[threadIdx.x - stride] : 0;
        __syncthreads();
        shared[threadIdx.x] += add;
        __syncthreads();
    }
    total = shared[kScanBlock - 1];
    const int32_t inclusive = shared[threadIdx.x];
    __syncthreads();
    return inclusive - value;
}

__global__ __launch_bounds__(kScanBlock) void route_scan_reduce_kernel(RouteArgs a) {
    __shared__ int32_t shared[kScanBlock];
    const int64_t total = static_cast<int64_t>(a.experts) * a.columns;
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * kScanSegment + threadIdx.x * (kScanSegment / kScanBlock);
    int32_t sum = 0;
    for (int j = 0; j < kScanSegment / kScanBlock; ++j)
        if (begin + j < total) sum += a.counts[begin + j];
    int32_t block_total;
    block_exclusive_scan(sum, shared, block_total);
    if (threadIdx.x == 0) a.block_sums[blockIdx.x] = block_total;
}

__global__ __launch_bounds__(kScanBlock) void route_scan_top_kernel(RouteArgs a, int blocks) {
    __shared__ int32_t shared[kScanBlock];
    const int per = (blocks + kScanBlock - 1) / kScanBlock;
    int32_t sum = 0;
    for (int j = 0; j < per; ++j) {
        const int b = threadIdx.x * per + j;
        if (b < blocks) sum += a.block_sums[b];
    }
    int32_t total;
    int32_t running = block_exclusive_scan(sum, shared, total);
    for (int j = 0; j < per; ++j) {
        const int b = threadIdx.x * per + j;
        if (b < blocks) {
            const int32_t value = a.block_sums[b];
            a.block_sums[b] = running;
            running += value;
        }
    }
    if (threadIdx.x == 0 && !a.slots) a.offsets[a.experts] = static_cast<int32_t>(a.n);
}

// SUMS_SCANNED: block_sums already holds each segment's offset (route_scan_top_kernel ran);
// otherwise every block adds up the sums of the segments before its own (few segments).
template <bool SUMS_SCANNED>
__global__ __launch_bounds__(kScanBlock) void route_scan_apply_kernel(RouteArgs a) {
    __shared__ int32_t shared[kScanBlock];
    int32_t offset;
    if constexpr (SUMS_SCANNED) {
        offset = a.block_sums[blockIdx.x];
    } else {
        int32_t before = 0;
        for (uint32_t b = threadIdx.x; b < blockIdx.x; b += kScanBlock) before += a.block_sums[b];
        block_exclusive_scan(before, shared, offset);
        if (blockIdx.x == 0 && threadIdx.x == 0 && !a.slots) a.offsets[a.experts] = static_cast<int32_t>(a.n);
    }
    const int64_t total = static_cast<int64_t>(a.experts) * a.columns;
    constexpr int kPer = kScanSegment / kScanBlock;
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * kScanSegment + threadIdx.x * kPer;
    int32_t values[kPer];
    int32_t sum = 0;
    for (int j = 0; j < kPer; ++j) {
        values[j] = begin + j < total ? a.counts[begin + j] : 0;
        sum += values[j];
    }
    int32_t block_total;
    int32_t running = offset + block_exclusive_scan(sum, shared, block_total);
    for (int j = 0; j < kPer; ++j) {
        const int64_t k = begin + j;
        if (k < total) {
            a.counts[k] = running;
            if (k % a.columns == 0) a.offsets[k / a.columns] = running;
        }
        running += values[j];
    }
}

// The two scan launches in one, when there are few segments: each block draws a ticket (its
// segment), sums the segment, publishes the sum + 1 with a device-coherent store, then adds the
// sums its predecessors published.  A block waits only for segments of lower tickets, whose
// blocks started before it and publish before they wait, so every wait ends.
// (The wait is bounded so that the kernel always ends; the scatters store only slots inside
// [0, n), so even counts scanned after an expired wait cannot send a store outside the outputs.)
constexpr int kScanSpinLimit = 1 << 22;
constexpr int kScanWaves = kScanBlock / 64;

// Exclusive scan of one value per thread over the block with wave shuffles and one barrier;
// `totals` ([2][kScanWaves], alternated by `round` so that consecutive scans need no barrier
// between them) receives the waves' sums, `total` the block's.
__device__ inline int32_t block_scan_shuffled(int32_t value, int32_t* totals, int round, int32_t& total) {
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    int32_t inclusive = value;
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t other = __shfl_up(inclusive, d);
        if (lane >= d) inclusive += other;
    }
    int32_t* mine = totals + (round & 1) * kScanWaves;
    if (lane == 63) mine[wave] = inclusive;
    __syncthreads();
    int32_t before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w) {
        const int32_t t = mine[w];
        if (w < wave) before += t;
        total += t;
    }
    return before + inclusive - value;
}

__global__ __launch_bounds__(kScanBlock) void route_scan_kernel(RouteArgs a) {
    __shared__ int32_t totals[2 * kScanWaves];
    __shared__ uint32_t drawn;
    if (threadIdx.x == 0) drawn = atomicAdd(a.scan_ticket, 1u);
    __syncthreads();
    const uint32_t segment = drawn;
    const int64_t total = static_cast<int64_t>(a.experts) * a.columns;
    constexpr int kPer = kScanSegment / kScanBlock;
    const int64_t begin = static_cast<int64_t>(segment) * kScanSegment + threadIdx.x * kPer;
    int32_t values[kPer];
    int32_t sum = 0;
    for (int j = 0; j < kPer; ++j) {
        values[j] = begin + j < total ? a.counts[begin + j] : 0;
        sum += values[j];
    }
    int32_t block_total;
    const int32_t inside = block_scan_shuffled(sum, totals, 0, block_total);
    uint32_t* sums = reinterpret_cast<uint32_t*>(a.block_sums);
    if (threadIdx.x == 0)
        __hip_atomic_store(sums + segment, static_cast<uint32_t>(block_total) + 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    int32_t before = 0;
    for (uint32_t q = threadIdx.x; q < segment; q += kScanBlock) {
        uint32_t v = __hip_atomic_load(sums + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int spins = 0; v == 0u && spins < kScanSpinLimit; ++spins) {
            __builtin_amdgcn_s_sleep(2);
            v = __hip_atomic_load(sums + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        before += static_cast<int32_t>(v - 1u);
    }
    int32_t offset;
    block_scan_shuffled(before, totals, 1, offset);
    int32_t running = offset + inside;
    for (int j = 0; j < kPer; ++j) {
        const int64_t k = begin + j;
        if (k < total) {
            a.counts[k] = running;
            if (k % a.columns == 0) a.offsets[k / a.columns] = running;
        }
        running += values[j];
    }
    if (segment == 0 && threadIdx.x == 0 && !a.slots) a.offsets[a.experts] = static_cast<int32_t>(a.n);
}

__global__ __launch_bounds__(kRouteBlock) void route_scatter_kernel(RouteArgs a) {
    extern __shared__ int32_t running[];  // [kWaves][experts]
    __shared__ Bounds bounds;
    load_bounds(a, bounds);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int part = blockIdx.x * kWaves + wave;
    int32_t* mine = running + wave * a.experts;
    for (int e = lane; e < a.experts; e += 64) mine[e] = 0;
    __syncthreads();
    if (part >= a.parts) return;
    const int64_t begin = static_cast<int64_t>(part) * a.part;
    const int64_t end = begin + a.part < a.n ? begin + a.part : a.n;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    for (int64_t ahead = begin; ahead < end; ahead += 64 * kDirectAhead) {
        uint32_t ids[kDirectAhead];
        pixel_ids<kDirectAhead>(a, ahead + lane, 64, end - 1, ids);
#pragma unroll
        for (int k = 0; k < kDirectAhead; ++k) {
            const int64_t group = ahead + k * 64;
            const int64_t i = group + lane;
            const bool valid = i < end;
            int expert = -1, rx = 0, ry = 0;
            uint32_t x = 0, y = 0;
            if (valid) locate_id(a, ids[k], expert, x, y, rx, ry);
            // Lanes holding the same expert: the AND over the id's bits of ballot(bit) or its
            // complement (one ballot per bit, whatever the number of distinct experts).  Every
            // lane reads the running count of its expert, then the lowest lane of each expert
            // advances it; the LDS reads of one instruction precede its writes in the wave.
            uint64_t same = __ballot(valid);
            for (int bit = 0; bit < a.expert_bits; ++bit) {
                const uint64_t ones = __ballot(valid && ((expert >> bit) & 1));
                same &= ((expert >> bit) & 1) ? ones : ~ones;
            }
            int32_t base = 0, rank = 0;
            if (valid) {
                rank = __popcll(same & below);
                base = mine[expert];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            if (valid && rank == 0) mine[expert] = base + __popcll(same);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int64_t slot =
                valid ? static_cast<int64_t>(a.counts[static_cast<int64_t>(expert) * a.columns + part]) + base + rank : 0;
            if (valid && slot >= 0 && slot < a.n) {
                a.perm[slot] = static_cast<int32_t>(i);
                const float u = static_cast<float>(x - static_cast<uint32_t>(bounds.x0[rx])) * a.rx[rx];
                const float v = static_cast<float>(y - static_cast<uint32_t>(bounds.y0[ry])) * a.ry[ry];
                reinterpret_cast<float2*>(a.coords)[slot] = make_float2(u, v);
                if (a.expert_out) a.expert_out[i] = reported(a, expert);
                // the pixel's index for route_colors_kernel (below 2^32: the image size is bounded)
                if (a.colors) a.colors[slot] = y * a.width + x;
            }
        }
    }
}

// Target colors in slot order.  route_scatter leaves each slot's pixel index in colors; the
// slots of one expert are contiguous and lie in one tile of the image, and consecutive chunks
// of slots run on one XCD (xcd_major), so each XCD gathers the bytes of its own run of tiles
// through its L2 instead of fetching a line of the image for every id.  One slot per thread: the
// most blocks in flight (measured against 2, 4, 8 and 16 slots per thread: 19.7 against
// 20.2-22.8 us at 2^22 slots, 359 against 364-388 us for 2^24 slots of a 3.2 GB image).
constexpr int kColorsPer = 1;
constexpr int kColorsChunk = kRouteBlock * kColorsPer;

__global__ __launch_bounds__(kRouteBlock) void route_colors_kernel(const uint8_t* rgb, uint32_t* colors, int64_t n,
                                                                  uint64_t image_bytes, bool words) {
    const int64_t begin = static_cast<int64_t>(xcd_major(blockIdx.x, gridDim.x)) * kColorsChunk + threadIdx.x;
    uint32_t pixel[kColorsPer];
#pragma unroll
    for (int k = 0; k < kColorsPer; ++k) {
        const int64_t i = begin + k * kRouteBlock;
        pixel[k] = i < n ? colors[i] : 0u;
    }
    // A pixel's three bytes from the 8-byte window at the dword below them (one load; the base
    // is 4-byte aligned when `words`), or byte by byte where that window would pass the image's end.
    uint32_t c[kColorsPer];
#pragma unroll
    for (int k = 0; k < kColorsPer; ++k) {
        const uint64_t at = 3 * static_cast<uint64_t>(pixel[k]);
        const uint64_t word = at & ~uint64_t{3};
        if (words && word + 8 <= image_bytes) {
            const uint2 w = *reinterpret_cast<const uint2*>(rgb + word);
            const uint64_t both = (static_cast<uint64_t>(w.y) << 32) | w.x;
            c[k] = static_cast<uint32_t>(both >> (8 * (at - word))) & 0xffffffu;
        } else {
            c[k] = rgb[at] | (static_cast<uint32_t>(rgb[at + 1]) << 8) | (static_cast<uint32_t>(rgb[at + 2]) << 16);
        }
    }
#pragma unroll
    for (int k = 0; k < kColorsPer; ++k) {
        const int64_t i = begin + k * kRouteBlock;
        if (i < n) colors[i] = c[k];
    }
}

// The scatter with a block of W waves staging a group of consecutive sub-chunks in LDS.  The
// sub-chunks' runs of one expert are consecutive in the output (the scanned counts are
// expert-major, then sub-chunk order), so the group's ids form one run per expert.  The block
//   1. copies the group's pixel ids (32 bits each) into LDS with coalesced loads;
//   2. cuts the group into W slices, one per wave, and each wave locates the ids of its slice,
//      keeps each id's expert and counts its slice's ids per expert;
//   3. scans those counts (expert-major, then slice order) into each slice's first position
//      for each expert inside the group's expert-ordered output;
//   4. each wave places the ids of its slice in order (lanes sharing an expert take their order
//      from ballots), recording only the id's offset inside the group;
//   5. the block's lanes take consecutive positions, fetch those ids from LDS, locate them
//      again and store them at consecutive slots of the output.
// Same slots as route_scatter_kernel; the stores are whole runs, the ids are read from memory
// once, and the serial placement is split W ways.
constexpr int kStagedMaxWaves = 8;

inline size_t staging_bytes(int experts, int part, int waves, int group) {
    return static_cast<size_t>(4) * experts * (1 + waves) + static_cast<size_t>(8) * part * group;
}

template <int W>
__global__ __launch_bounds__(64 * W) void route_scatter_staged_kernel(RouteArgs a, int group) {
    extern __shared__ int32_t lds[];
    __shared__ Bounds bounds;
    __shared__ int32_t wave_sums[W];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int tid = static_cast<int>(threadIdx.x);
    const int first = static_cast<int>(xcd_major(blockIdx.x, gridDim.x)) * group;   // the group's first sub-chunk
    if (first >= a.parts) return;
    // the tile bounds (used at the write-out) loaded beside the counts and ids, not ahead of them
    // behind a barrier of their own
    static_assert(64 * W > kMaxRegions, "one bound per thread");
    const bool bounder = tid <= kMaxRegions;
    int32_t bound_x = 0, bound_y = 0;
    if (bounder) {
        bound_x = a.x0[tid];
        bound_y = a.y0[tid];
    }
    const int members = a.parts - first < group ? a.parts - first : group;
    const int64_t group_begin = static_cast<int64_t>(first) * a.part;
    const int64_t group_end = group_begin + static_cast<int64_t>(members) * a.part;
    const int32_t count = static_cast<int32_t>((group_end < a.n ? group_end : a.n) - group_begin);
    const int experts = a.experts;
    const int32_t ids_cap = group * a.part;
    int32_t* base = lds;                                                   // [experts]
    uint32_t* hist = reinterpret_cast<uint32_t*>(lds + experts);           // [W][experts]
    uint32_t* held = hist + W * experts;                                   // [ids_cap] the group's ids
    uint16_t* tag = reinterpret_cast<uint16_t*>(held + ids_cap);           // [ids_cap] expert of id j
    uint16_t* local = tag + ids_cap;                                       // [ids_cap] offset of position j's id
    // base[e] = slot of the group's first id of expert e: the scanned count of (e, first)
    for (int e = tid; e < experts; e += 64 * W) {
        base[e] = a.counts[static_cast<int64_t>(e) * a.columns + first / a.per_column];
#pragma unroll
        for (int w = 0; w < W; ++w) hist[w * experts + e] = 0u;
    }
    for (int32_t j0 = 0; j0 < count; j0 += 64 * W * 2 * kAhead) {
        // stored ids only: stratified batches take the direct scatter
        uint32_t ids[2 * kAhead];
#pragma unroll
        for (int k = 0; k < 2 * kAhead; ++k) {
            const int32_t j = j0 + k * 64 * W + tid;
            ids[k] = j < count ? static_cast<uint32_t>(a.ids[group_begin + j]) : 0u;
        }
#pragma unroll
        for (int k = 0; k < 2 * kAhead; ++k) {
            const int32_t j = j0 + k * 64 * W + tid;
            if (j < count) held[j] = ids[k];
        }
    }
    if (bounder) {
        bounds.x0[tid] = bound_x;
        bounds.y0[tid] = bound_y;
    }
    __syncthreads();
    // slices of whole groups of 64 ids
    const int32_t slice = ((count + W - 1) / W + 63) / 64 * 64;
    const int32_t begin = wave * slice < count ? wave * slice : count;
    const int32_t end = begin + slice < count ? begin + slice : count;
    uint32_t* mine = hist + wave * experts;
    for (int32_t ahead = begin; ahead < end; ahead += 64 * kAhead) {
        uint32_t ids[kAhead];
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
            const int32_t j = ahead + k * 64 + lane;
            ids[k] = held[j < end ? j : end - 1];
        }
        int tags[kAhead];
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
            int rx, ry;
            uint32_t x, y;
            locate_id(a, ids[k], tags[k], x, y, rx, ry);
        }
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
            const int32_t j = ahead + k * 64 + lane;
            if (j < end) {
                tag[j] = static_cast<uint16_t>(tags[k]);
                atomicAdd(&mine[tags[k]], 1u);
            }
        }
    }
    __syncthreads();
    // exclusive scan over (expert, slice): thread t takes experts [t*per, (t+1)*per)
    {
        const int per = (experts + 64 * W - 1) / (64 * W);
        int32_t sum = 0;
        for (int q = 0; q < per; ++q) {
            const int e = tid * per + q;
            if (e < experts) {
#pragma unroll
                for (int w = 0; w < W; ++w) sum += static_cast<int32_t>(hist[w * experts + e]);
            }
        }
        int32_t inclusive = sum;
        for (int d = 1; d < 64; d <<= 1) {
            const int32_t other = __shfl_up(inclusive, d);
            if (lane >= d) inclusive += other;
        }
        if (lane == 63) wave_sums[wave] = inclusive;
        __syncthreads();
        int32_t at = inclusive - sum;
        for (int w = 0; w < wave; ++w) at += wave_sums[w];
        for (int q = 0; q < per; ++q) {
            const int e = tid * per + q;
            if (e < experts) {
                base[e] -= at;
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    const int32_t c = static_cast<int32_t>(hist[w * experts + e]);
                    hist[w * experts + e] = static_cast<uint32_t>(at);
                    at += c;
                }
            }
        }
    }
    __syncthreads();
    {
        const uint64_t below = (uint64_t{1} << lane) - 1;
        for (int32_t ahead = begin; ahead < end; ahead += 64 * kAhead) {
            int tags[kAhead];
#pragma unroll
            for (int k = 0; k < kAhead; ++k) {
                const int32_t j = ahead + k * 64 + lane;
                const int t = static_cast<int>(tag[j < end ? j : end - 1]);
                tags[k] = j < end ? t : -1;
            }
            // lanes sharing an expert, for the kAhead groups at once (independent ballots)
            uint64_t same[kAhead];
#pragma unroll
            for (int k = 0; k < kAhead; ++k) same[k] = __ballot(tags[k] >= 0);
            for (int bit = 0; bit < a.expert_bits; ++bit) {
#pragma unroll
                for (int k = 0; k < kAhead; ++k) {
                    const bool one = (tags[k] >> bit) & 1;
                    const uint64_t ones = __ballot(tags[k] >= 0 && one);
                    same[k] &= one ? ones : ~ones;
                }
            }
#pragma unroll
            for (int k = 0; k < kAhead; ++k) {
                const int32_t j = ahead + k * 64 + lane;
                const bool valid = j < end;
                const int expert = tags[k];
                int32_t position = 0, rank = 0;
                if (valid) {
                    rank = __popcll(same[k] & below);
                    position = static_cast<int32_t>(mine[expert]);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                if (valid && rank == 0) mine[expert] = static_cast<uint32_t>(position + __popcll(same[k]));
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (valid) {
                    local[position + rank] = static_cast<uint16_t>(j);
                    if (a.expert_out) a.expert_out[group_begin + j] = reported(a, expert);
                }
            }
        }
    }
    __syncthreads();
    for (int32_t j0 = 0; j0 < count; j0 += 64 * W * kAhead) {
        int32_t at[kAhead];
        uint32_t ids[kAhead];
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
            const int32_t j = j0 + k * 64 * W + tid;
            at[k] = static_cast<int32_t>(local[j < count ? j : count - 1]);
        }
#pragma unroll
        for (int k = 0; k < kAhead; ++k) ids[k] = held[at[k]];
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
            const int32_t j = j0 + k * 64 * W + tid;
            int expert, rx, ry;
            uint32_t x, y;
            locate_id(a, ids[k], expert, x, y, rx, ry);
            const int64_t slot = static_cast<int64_t>(base[expert]) + j;
            if (j < count && slot >= 0 && slot < a.n) {
                a.perm[slot] = static_cast<int32_t>(group_begin + at[k]);
                const float u = static_cast<float>(x - static_cast<uint32_t>(bounds.x0[rx])) * a.rx[rx];
                const float v = static_cast<float>(y - static_cast<uint32_t>(bounds.y0[ry])) * a.ry[ry];
                reinterpret_cast<float2*>(a.coords)[slot] = make_float2(u, v);
                // the pixel's index for route_colors_kernel
                if (a.colors) a.colors[slot] = y * a.width + x;
            }
        }
    }
}

// Waves per staged-scatter block and sub-chunks per group: 8 waves if the staging of one
// sub-chunk then fits the LDS budget (two blocks per CU), else 4; and the most sub-chunks, up to
// 8, that still fit.  waves = 0 when not even one sub-chunk with 4 waves fits.
constexpr size_t kStagingBudget = 72 * 1024;

void staged_shape(int experts, int part, int& waves, int& group) {
    const size_t budget = kStagingBudget - sizeof(Bounds) - kStagedMaxWaves * 4;
    for (waves = kStagedMaxWaves; waves >= 4; waves /= 2)
        for (group = 8; group >= 1; group /= 2)
            if (staging_bytes(experts, part, waves, group) <= budget) return;
    waves = 0;
    group = 0;
}

// The staged scatter's dynamic LDS limit, raised to the whole staging budget once per device
// and kernel shape (not per call: a call under graph capture then makes no attribute change).
template <int W>
int allow_staging() {
    static std::mutex lock;
    static std::set<int> devices;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return fail("odie_route: no current device");
    std::lock_guard<std::mutex> guard(lock);
    if (devices.count(device)) return 0;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(route_scatter_staged_kernel<W>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kStagingBudget)) != hipSuccess)
        return fail("odie_route: LDS attribute of the staged scatter");
    devices.insert(device);
    return 0;
}

template <int W>
int launch_staged(const RouteArgs& a, int group, hipStream_t s) {
    const uint32_t groups = round_up(static_cast<uint32_t>((a.parts + group - 1) / group), kXcds);
    const size_t staging = staging_bytes(a.experts, a.part, W, group);
    if (allow_staging<W>()) return -1;
    route_scatter_staged_kernel<W><<<groups, 64 * W, staging, s>>>(a, group);
    return 0;
}

int& route_one_scan() {
    static int enabled = 1;
    return enabled;
}

int& route_min_part() {
    static int part = 512;
    return part;
}

int route_plan(int64_t n, int experts, int& part, int& parts) {
    // Sub-chunks of at least route_min_part() ids, few enough that experts*parts stays <= 2^22
    // (16 MiB of counts): a wave walks its sub-chunk serially, so short ones keep more waves on
    // every CU.
    int64_t p = route_min_part();
    while ((n + p - 1) / p * experts > (int64_t{1} << 22)) p *= 2;
    part = static_cast<int>(p);
    parts = static_cast<int>((n + p - 1) / p);
    if (parts < 1) parts = 1;
    return 0;
}

}  // namespace

int set_route_tuning(const std::string& key, int value) {
    // the workspace size follows the part, so a caller sizes it after the setting
    if (key == "route_part" && value >= 64 && value <= (1 << 16) && (value & (value - 1)) == 0) route_min_part() = value;
    else if (key == "route_one_scan" && (value == 0 || value == 1)) route_one_scan() = value;
    else return fail("odie_set_tuning: unknown key or value out of range: " + key);
    return 0;
}

}  // namespace odie

using namespace odie;

int64_t scan_blocks(int64_t n, int experts) {
    int part, parts;
    route_plan(n, experts, part, parts);
    return (static_cast<int64_t>(experts) * parts + kScanSegment - 1) / kScanSegment;
}

ODIE_API int64_t odie_route_workspace(int64_t n, int experts) {
    if (n < 0 || n > (int64_t{1} << 31) - 1 || experts < 1 || experts > kMaxExperts) return -1;
    int part, parts;
    route_plan(n, experts, part, parts);
    const int64_t counts = (static_cast<int64_t>(experts) * parts * 4 + 255) / 256 * 256;
    return counts + scan_blocks(n, experts) * 4;
}

namespace odie {
namespace {

// Checks the arguments common to odie_route and odie_route_noalloc (nothing is queued).
int route_check(const void* ids, int64_t n, int width, int height, int regions_x, int regions_y, int32_t* perm,
                float* coords, int32_t* offsets, const uint8_t* rgb, uint32_t* colors) {
    if (n < 0 || n > (int64_t{1} << 31) - 1) return fail("odie_route: n must be within [0, 2^31-1]");
    if (regions_x < 1 || regions_y < 1 || regions_x > kMaxRegions || regions_y > kMaxRegions)
        return fail("odie_route: regions per axis must be within 1..64");
    if (width < 2 * regions_x || height < 2 * regions_y)
        return fail("odie_route: every tile needs at least two pixels per axis");
    if (static_cast<uint64_t>(width) * static_cast<uint64_t>(height) > (uint64_t{1} << 32))
        return fail("odie_route: images are limited to 2^32 pixels (32-bit pixel ids)");
    if (!offsets) return fail("odie_route: offsets is null");
    if (n > 0 && (!ids || !perm || !coords)) return fail("odie_route: ids, perm and coords must be non-null");
    if (rgb && !colors) return fail("odie_route: rgb needs colors");
    if (reinterpret_cast<uintptr_t>(coords) % 8) return fail("odie_route: coords must be 8-byte aligned");
    return 0;
}

// Queues the route on `stream` with `workspace` (odie_route_workspace(n, E) bytes, checked by
// the caller) as its scratch.
int route_launch(const int64_t* ids, int64_t n, int width, int height, int regions_x, int regions_y,
                 int32_t* expert, int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb,
                 uint32_t* colors, void* workspace, uint64_t stream, const float* uniforms = nullptr, int side = 0,
                 const int32_t* slots = nullptr, int owned = 0) {
    // buckets of the counting sort: one per tile, or one per expert and the one of tiles without
    const int experts = slots ? owned + 1 : regions_x * regions_y;
    RouteArgs a{};
    a.slots = slots;
    a.owned = owned;
    a.ids = ids;
    a.uniforms = uniforms;
    a.side = side;
    a.inv_side = side > 0 ? 1.0f / static_cast<float>(side) : 0.0f;
    a.expert_out = expert;
    a.perm = perm;
    a.coords = coords;
    a.offsets = offsets;
    a.rgb = rgb;
    a.colors = colors;
    a.counts = static_cast<int32_t*>(workspace);
    {
        int part, parts;
        route_plan(n, experts, part, parts);
        const int64_t counts = (static_cast<int64_t>(experts) * parts * 4 + 255) / 256 * 256;
        a.block_sums = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + counts);
    }
    a.n = n;
    a.width = static_cast<uint32_t>(width);
    a.by_width = make_divisor(a.width);
    a.height = static_cast<uint32_t>(height);
    a.regions_x = regions_x;
    a.regions_y = regions_y;
    a.experts = experts;
    a.expert_bits = 0;
    while ((1 << a.expert_bits) < experts) ++a.expert_bits;
    route_plan(n, experts, a.part, a.parts);
    // staged scatter when a group's staging fits the LDS budget.  A stratified batch lists its
    // strata row by row, so consecutive ids mostly share an expert and the direct scatter's stores
    // already come in runs.
    int waves = 0, group = 0;
    staged_shape(experts, a.part, waves, group);
    // (the grouped count reads the ids as 16-byte pairs)
    const bool staged = !uniforms && waves > 0 && reinterpret_cast<uintptr_t>(ids) % 16 == 0;
    a.per_column = staged ? group : 1;
    a.columns = (a.parts + a.per_column - 1) / a.per_column;
    {
        TileBounds tb;
        make_tile_bounds(width, height, regions_x, regions_y, tb);
        for (int r = 0; r <= kMaxRegions; ++r) {
            a.x0[r] = tb.x0[r];
            a.y0[r] = tb.y0[r];
        }
        for (int r = 0; r < kMaxRegions; ++r) {
            a.rx[r] = tb.rx[r];
            a.ry[r] = tb.ry[r];
        }
        a.sx = tb.sx;
        a.sy = tb.sy;
    }
    const hipStream_t s = as_stream(stream);
    const size_t shmem = static_cast<size_t>(kWaves) * experts * 4;
    if (shmem + sizeof(Bounds) > 64 * 1024) return fail("odie_route: too many experts for the LDS histogram");
    const uint32_t blocks = static_cast<uint32_t>((a.parts + kWaves - 1) / kWaves);
    if (n == 0) return launch_fill_zero(reinterpret_cast<float*>(offsets), slots ? owned + 1 : experts + 1, s);
    const int sblocks = static_cast<int>((static_cast<int64_t>(experts) * a.columns + kScanSegment - 1) / kScanSegment);
    if (sblocks > kScanBlock * 64) return fail("odie_route: too many counts to scan");
    // one scan launch when its segments' sums and ticket fit the workspace's block sums
    if (route_one_scan() && sblocks <= kScanBlock * 4 && sblocks + 1 <= scan_blocks(n, experts)) {
        a.scan_segments = sblocks;
        a.scan_ticket = reinterpret_cast<uint32_t*>(a.block_sums + sblocks);
    }
    if (staged) route_count_kernel<true, kCountThreads><<<a.columns, kCountThreads, static_cast<size_t>(experts) * 4, s>>>(a);
    else route_count_kernel<false><<<blocks, kRouteBlock, shmem, s>>>(a);
    if (a.scan_ticket) {
        route_scan_kernel<<<sblocks, kScanBlock, 0, s>>>(a);
    } else if (sblocks <= kScanBlock * 4) {
        route_scan_reduce_kernel<<<sblocks, kScanBlock, 0, s>>>(a);
        route_scan_apply_kernel<false><<<sblocks, kScanBlock, 0, s>>>(a);
    } else {
        route_scan_reduce_kernel<<<sblocks, kScanBlock, 0, s>>>(a);
        route_scan_top_kernel<<<1, kScanBlock, 0, s>>>(a, sblocks);
        route_scan_apply_kernel<true><<<sblocks, kScanBlock, 0, s>>>(a);
    }
    if (staged) {
        if ((waves == 8 ? launch_staged<8>(a, group, s) : launch_staged<4>(a, group, s)) != 0) return -1;
    } else {
        route_scatter_kernel<<<blocks, kRouteBlock, shmem, s>>>(a);
    }
    if (rgb) {
        const uint32_t chunks = round_up(static_cast<uint32_t>((n + kColorsChunk - 1) / kColorsChunk), kXcds);
        const uint64_t image_bytes = 3 * static_cast<uint64_t>(width) * static_cast<uint64_t>(height);
        const bool words = reinterpret_cast<uintptr_t>(rgb) % 4 == 0;
        route_colors_kernel<<<chunks, kRouteBlock, 0, s>>>(rgb, colors, n, image_bytes, words);
    }
    return check_launch("odie_route");
}

// Scratch of odie_route_noalloc: one copy per device, held until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a stand-in for the device
// variable); it uses the per-device address from hipGetSymbolAddress.
constexpr int64_t kRouteScratchBytes = ODIE_ROUTE_NOALLOC_BYTES;
static __device__ __align__(256) uint8_t scratch[kRouteScratchBytes];

void* scratch_address() {
    static std::mutex lock;
    static std::map<int, void*> addresses;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        fail("odie_route_noalloc: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(lock);
    auto found = addresses.find(device);
    if (found != addresses.end()) return found->second;
    void* address = nullptr;
    const hipError_t status = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (status != hipSuccess || !address) {
        fail(std::string("odie_route_noalloc: hipGetSymbolAddress failed: ") + hipGetErrorString(status));
        return nullptr;
    }
    addresses[device] = address;
    return address;
}

}  // namespace
}  // namespace odie

ODIE_API int odie_route(const int64_t* ids, int64_t n, int width, int height, int regions_x, int regions_y,
                        int32_t* expert, int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb,
                        uint32_t* colors, void* workspace, int64_t workspace_bytes, uint64_t stream) {
    if (route_check(ids, n, width, height, regions_x, regions_y, perm, coords, offsets, rgb, colors)) return -1;
    if (n > 0 && (!workspace || workspace_bytes < odie_route_workspace(n, regions_x * regions_y)))
        return fail("odie_route: workspace must hold odie_route_workspace(n, experts) bytes");
    return route_launch(ids, n, width, height, regions_x, regions_y, expert, perm, coords, offsets, rgb, colors,
                        workspace, stream);
}

ODIE_API int odie_route_stratified(const float* uniforms, int64_t n, int width, int height, int regions_x,
                                   int regions_y, int32_t* expert, int32_t* perm, float* coords, int32_t* offsets,
                                   const uint8_t* rgb, uint32_t* colors, void* workspace, int64_t workspace_bytes,
                                   uint64_t stream) {
    if (route_check(uniforms, n, width, height, regions_x, regions_y, perm, coords, offsets, rgb, colors)) return -1;
    int side = 1;
    while (static_cast<int64_t>(side) * side < n) side *= 2;
    if (n < 1 || static_cast<int64_t>(side) * side != n)
        return fail("Stratified sampling requires a square power-of-two batch size");
    if (reinterpret_cast<uintptr_t>(uniforms) % 8) return fail("odie_route_stratified: uniforms must be 8-byte aligned");
    if (!workspace || workspace_bytes < odie_route_workspace(n, regions_x * regions_y))
        return fail("odie_route: workspace must hold odie_route_workspace(n, experts) bytes");
    return route_launch(nullptr, n, width, height, regions_x, regions_y, expert, perm, coords, offsets, rgb, colors,
                        workspace, stream, uniforms, side);
}

ODIE_API int odie_route_allocated(const int64_t* ids, const float* uniforms, int64_t n, int width, int height,
                                  int regions_x, int regions_y, const int32_t* slots, int experts, int32_t* expert,
                                  int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb, uint32_t* colors,
                                  void* workspace, int64_t workspace_bytes, uint64_t stream) {
    if ((ids == nullptr) == (uniforms == nullptr) && n > 0)
        return fail("odie_route_allocated: give exactly one of ids and uniforms");
    if (route_check(ids ? static_cast<const void*>(ids) : uniforms, n, width, height, regions_x, regions_y, perm,
                    coords, offsets, rgb, colors))
        return -1;
    if (experts < 1 || experts >= kMaxExperts) return fail("odie_route_allocated: experts must be within 1..4095");
    if (!slots) return fail("odie_route_allocated: slots is null");
    int side = 0;
    if (uniforms) {
        side = 1;
        while (static_cast<int64_t>(side) * side < n) side *= 2;
        if (static_cast<int64_t>(side) * side != n)
            return fail("Stratified sampling requires a square power-of-two batch size");
        if (reinterpret_cast<uintptr_t>(uniforms) % 8) return fail("odie_route_allocated: uniforms must be 8-byte aligned");
    }
    if (n > 0 && (!workspace || workspace_bytes < odie_route_workspace(n, experts + 1)))
        return fail("odie_route_allocated: workspace must hold odie_route_workspace(n, experts + 1) bytes");
    return route_launch(ids, n, width, height, regions_x, regions_y, expert, perm, coords, offsets, rgb, colors,
                        workspace, stream, uniforms, side, slots, experts);
}

ODIE_API int odie_route_noalloc(const int64_t* ids, int64_t n, int width, int height, int regions_x, int regions_y,
                                int32_t* expert, int32_t* perm, float* coords, int32_t* offsets, const uint8_t* rgb,
                                uint32_t* colors, uint64_t stream) {
    if (route_check(ids, n, width, height, regions_x, regions_y, perm, coords, offsets, rgb, colors)) return -1;
    const int64_t need = odie_route_workspace(n, regions_x * regions_y);
    if (need > kRouteScratchBytes)
        return fail("odie_route_noalloc: " + std::to_string(n) + " ids over " + std::to_string(regions_x * regions_y) +
                    " experts need " + std::to_string(need) + " bytes of scratch, more than its " +
                    std::to_string(kRouteScratchBytes) + "; use odie_route with a workspace");
    void* space = scratch_address();
    if (!space) return -1;
    return route_launch(ids, n, width, height, regions_x, regions_y, expert, perm, coords, offsets, rgb, colors, space,
                        stream);
}
