// B1 on the device: the reference's select_mean_rank (odie/selection.py:108-126).  The cells are
// ranked by descending score, ties by ascending cell id (the stable argsort of -score), and
// walked in rank order: a cell is admitted when the closure nodes it adds -- those of its four
// corners (cell + {0, 1, R, R + 1}) mod align8(R^2) not yet taken, a corner listed twice counted
// twice -- keep the running count within the cap.
//
//   ranking  a stable LSD radix sort of (key, cell) pairs, eight passes of 8-bit digits: key =
//            (2^63 - 1) - (score bits with the sign cleared), so ascending keys are descending
//            scores (-0 ties +0, the GPU selector's key, odie/native/selection_cuda.cu:14-17) and
//            equal keys keep ascending cell ids.
//   phase 1  as long as every cell so far was admitted, a cell's new nodes are the corners it
//            is the first (lowest rank) to touch.  So the lowest rank of every node, a prefix
//            count of those first touches over the ranking, and the first rank K where it passes
//            the cap give the walk exactly up to K: every rank below K admitted, K refused.
//   phase 2  after K fewer than 4 node slots remain (K's at most 4 new nodes did not fit), so at
//            most 3 more cells that add nodes can be admitted.  One workgroup walks the ranks from
//            K in tiles of 1024: every cell that adds no node is admitted (nodes unchanged), the
//            first that adds between 1 and the remaining count is admitted and its nodes kept in
//            LDS, and the tile is evaluated again from the next rank.
#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kSortBlock = 1024;            // threads per block = elements per tile
constexpr int kSortWaves = kSortBlock / 64;
constexpr int kDigits = 256;
constexpr int kPasses = 8;
constexpr int64_t kMaxCells = int64_t{1} << 24;
constexpr int kMaxEventNodes = 16;          // nodes added in phase 2: at most 3 cells x 4 corners

struct SortArgs {
    const uint64_t* keys_in;
    const int32_t* values_in;
    uint64_t* keys_out;
    int32_t* values_out;
    int32_t* counts;    // [kDigits][tiles]: the tile's count of each digit, then its first slot
    int64_t n;
    int tiles;
    int shift;
};

__global__ __launch_bounds__(256) void rank_keys_kernel(const double* scores, int64_t n, uint64_t* keys,
                                                        int32_t* values) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const uint64_t bits = static_cast<uint64_t>(__double_as_longlong(scores[i])) & 0x7fffffffffffffffull;
    keys[i] = 0x7fffffffffffffffull - bits;
    values[i] = static_cast<int32_t>(i);
}

__global__ __launch_bounds__(kSortBlock) void digit_count_kernel(SortArgs a) {
    __shared__ int32_t hist[kDigits];
    if (threadIdx.x < kDigits) hist[threadIdx.x] = 0;
    __syncthreads();
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kSortBlock + threadIdx.x;
    if (i < a.n) atomicAdd(&hist[(a.keys_in[i] >> a.shift) & 0xff], 1);
    __syncthreads();
    if (threadIdx.x < kDigits) a.counts[static_cast<int64_t>(threadIdx.x) * a.tiles + blockIdx.x] = hist[threadIdx.x];
}

// Exclusive prefix of one value per thread over the block; total receives the block's sum.
__device__ inline int64_t block_exclusive(int64_t value, int64_t* shared, int64_t& total) {
    shared[threadIdx.x] = value;
    __syncthreads();
    for (int stride = 1; stride < kSortBlock; stride <<= 1) {
        const int64_t add = static_cast<int>(threadIdx.x) >= stride ? shared[threadIdx.x - stride] : 0;
        __syncthreads();
        shared[threadIdx.x] += add;
        __syncthreads();
    }
    total = shared[kSortBlock - 1];
    const int64_t inclusive = shared[threadIdx.x];
    __syncthreads();
    return inclusive - value;
}

// One block: the digit-major counts become every (digit, tile)'s first slot of the pass output.
__global__ __launch_bounds__(kSortBlock) void digit_scan_kernel(SortArgs a) {
    __shared__ int64_t shared[kSortBlock];
    const int64_t total = static_cast<int64_t>(kDigits) * a.tiles;
    const int64_t per = (total + kSortBlock - 1) / kSortBlock;
    const int64_t j0 = threadIdx.x * per < total ? threadIdx.x * per : total;
    const int64_t j1 = j0 + per < total ? j0 + per : total;
    int64_t sum = 0;
    for (int64_t j = j0; j < j1; ++j) sum += a.counts[j];
    int64_t all;
    int64_t run = block_exclusive(sum, shared, all);
    for (int64_t j = j0; j < j1; ++j) {
        const int32_t c = a.counts[j];
        a.counts[j] = static_cast<int32_t>(run);
        run += c;
    }
}

// Stable scatter of one tile: an element's slot is its (digit, tile)'s first slot, plus the
// elements of that digit in the tile's earlier waves, plus those in its own wave before it
// (lanes sharing a digit found with one ballot per digit bit).
__global__ __launch_bounds__(kSortBlock) void digit_scatter_kernel(SortArgs a) {
    __shared__ int32_t waves[kSortWaves][kDigits];
    for (int j = threadIdx.x; j < kSortWaves * kDigits; j += kSortBlock) (&waves[0][0])[j] = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kSortBlock + threadIdx.x;
    const bool valid = i < a.n;
    const uint64_t key = valid ? a.keys_in[i] : 0ull;
    const int32_t value = valid ? a.values_in[i] : 0;
    const int digit = static_cast<int>((key >> a.shift) & 0xff);
    uint64_t same = __ballot(valid);
    for (int bit = 0; bit < 8; ++bit) {
        const bool one = (digit >> bit) & 1;
        const uint64_t ones = __ballot(valid && one);
        same &= one ? ones : ~ones;
    }
    const int rank = __popcll(same & ((uint64_t{1} << lane) - 1));
    if (valid && rank == 0) waves[wave][digit] = __popcll(same);
    __syncthreads();
    if (threadIdx.x < kDigits) {
        int32_t run = 0;
        for (int w = 0; w < kSortWaves; ++w) {
            const int32_t c = waves[w][threadIdx.x];
            waves[w][threadIdx.x] = run;
            run += c;
        }
    }
    __syncthreads();
    if (valid) {
        const int64_t slot = static_cast<int64_t>(a.counts[static_cast<int64_t>(digit) * a.tiles + blockIdx.x]) +
                             waves[wave][digit] + rank;
        a.keys_out[slot] = key;
        a.values_out[slot] = value;
    }
}

struct AdmitArgs {
    const int32_t* order;    // [n]: the cell at every rank
    int32_t* first;          // [points]: the lowest rank touching every node
    int64_t* prefix;         // [n]: new nodes up to every rank (inclusive) while every cell is admitted
    int64_t* tile_sums;      // [tiles]
    int32_t* cut;            // [1]: K, the first rank whose prefix passes the cap (n if none)
    uint8_t* chosen;         // [n]
    uint8_t* nodes;          // [points]
    int64_t* stats;          // [2]: nodes counted against the cap, cells walked
    int64_t n;
    int64_t points;
    int64_t resolution;
    int64_t cap;
    int tiles;
};

__device__ inline void corners(const AdmitArgs& a, int64_t cell, int64_t c[4]) {
    c[0] = cell % a.points;
    c[1] = (cell + 1) % a.points;
    c[2] = (cell + a.resolution) % a.points;
    c[3] = (cell + a.resolution + 1) % a.points;
}

__global__ __launch_bounds__(256) void admit_reset_kernel(AdmitArgs a) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; j < a.points; j += stride) {
        a.first[j] = 0x7fffffff;
        a.nodes[j] = 0;
        if (j < a.n) a.chosen[j] = 0;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) a.cut[0] = static_cast<int32_t>(a.n);
}

__global__ __launch_bounds__(256) void first_touch_kernel(AdmitArgs a) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= a.n) return;
    int64_t c[4];
    corners(a, a.order[r], c);
#pragma unroll
    for (int j = 0; j < 4; ++j) atomicMin(a.first + c[j], static_cast<int32_t>(r));
}

// The new nodes of every rank (the corners it touches first, duplicates counted) and their
// inclusive prefix within each tile of kSortBlock ranks.
__global__ __launch_bounds__(kSortBlock) void first_count_kernel(AdmitArgs a) {
    __shared__ int64_t shared[kSortBlock];
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kSortBlock + threadIdx.x;
    int64_t added = 0;
    if (r < a.n) {
        int64_t c[4];
        corners(a, a.order[r], c);
#pragma unroll
        for (int j = 0; j < 4; ++j) added += a.first[c[j]] == static_cast<int32_t>(r);
    }
    int64_t total;
    const int64_t before = block_exclusive(added, shared, total);
    if (r < a.n) a.prefix[r] = before + added;
    if (threadIdx.x == 0) a.tile_sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(kSortBlock) void tile_scan_kernel(AdmitArgs a) {
    __shared__ int64_t shared[kSortBlock];
    const int per = (a.tiles + kSortBlock - 1) / kSortBlock;
    const int t0 = static_cast<int>(threadIdx.x) * per < a.tiles ? static_cast<int>(threadIdx.x) * per : a.tiles;
    const int t1 = t0 + per < a.tiles ? t0 + per : a.tiles;
    int64_t sum = 0;
    for (int t = t0; t < t1; ++t) sum += a.tile_sums[t];
    int64_t all;
    int64_t run = block_exclusive(sum, shared, all);
    for (int t = t0; t < t1; ++t) {
        const int64_t s = a.tile_sums[t];
        a.tile_sums[t] = run;
        run += s;
    }
}

__global__ __launch_bounds__(kSortBlock) void cut_kernel(AdmitArgs a) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kSortBlock + threadIdx.x;
    if (r >= a.n) return;
    const int64_t p = a.prefix[r] + a.tile_sums[blockIdx.x];
    a.prefix[r] = p;
    if (p > a.cap) atomicMin(a.cut, static_cast<int32_t>(r));
}

// Every rank below K: admitted, its corners taken (several writers of one node all write 1).
__global__ __launch_bounds__(256) void admit_prefix_kernel(AdmitArgs a) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= a.n || r >= a.cut[0]) return;
    const int64_t cell = a.order[r];
    a.chosen[cell] = 1;
    int64_t c[4];
    corners(a, cell, c);
#pragma unroll
    for (int j = 0; j < 4; ++j) a.nodes[c[j]] = 1;
}

// Phase 2, one workgroup.  The nodes array holds phase 1's nodes and is only read here; the nodes
// of the (at most three) cells admitted here that add nodes live in LDS and are written at the end.
__global__ __launch_bounds__(kSortBlock) void admit_rest_kernel(AdmitArgs a) {
    __shared__ int64_t taken[kMaxEventNodes];
    __shared__ int taken_count;
    __shared__ int32_t event;
    __shared__ int64_t remaining;
    const int64_t k = a.cut[0];
    if (threadIdx.x == 0) {
        taken_count = 0;
        remaining = a.cap - (k > 0 ? a.prefix[k - 1] : 0);
    }
    __syncthreads();
    for (int64_t base = k; base < a.n; base += kSortBlock) {
        int64_t start = base;   // ranks below start in this tile are decided
        for (;;) {
            if (threadIdx.x == 0) event = 0x7fffffff;
            __syncthreads();
            const int64_t r = base + threadIdx.x;
            const bool open = r < a.n && r >= start;
            int64_t added = 0, cell = 0;
            if (open) {
                cell = a.order[r];
                int64_t c[4];
                corners(a, cell, c);
                const int count = taken_count;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bool have = a.nodes[c[j]] != 0;
                    for (int q = 0; q < count; ++q) have = have || taken[q] == c[j];
                    added += !have;
                }
                if (added >= 1 && added <= remaining) atomicMin(&event, static_cast<int32_t>(r));
            }
            __syncthreads();
            const int64_t stop = event;   // the first rank that adds nodes and fits, or none
            if (open && r < stop && added == 0) a.chosen[cell] = 1;
            __syncthreads();
            if (stop == 0x7fffffff) break;
            if (r == stop) {
                a.chosen[cell] = 1;
                int64_t c[4];
                corners(a, cell, c);
                int count = taken_count;
                for (int j = 0; j < 4; ++j) {
                    bool have = a.nodes[c[j]] != 0;
                    for (int q = 0; q < count; ++q) have = have || taken[q] == c[j];
                    if (!have) taken[count++] = c[j];   // a corner listed twice is stored once
                }
                taken_count = count;
                remaining -= added;
            }
            __syncthreads();
            start = stop + 1;
        }
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < taken_count) a.nodes[taken[threadIdx.x]] = 1;
    if (threadIdx.x == 0) {
        a.stats[0] = a.cap - remaining;
        a.stats[1] = a.n;
    }
}

struct Layout {
    size_t keys[2], values[2], counts, first, prefix, tile_sums, cut, total;
};

Layout layout_of(int64_t n, int64_t points) {
    const auto align = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const int64_t tiles = (n + kSortBlock - 1) / kSortBlock;
    Layout l{};
    size_t at = 0;
    for (int b = 0; b < 2; ++b) {
        l.keys[b] = at;
        at += align(static_cast<size_t>(n) * 8);
    }
    for (int b = 0; b < 2; ++b) {
        l.values[b] = at;
        at += align(static_cast<size_t>(n) * 4);
    }
    l.counts = at;
    at += align(static_cast<size_t>(kDigits) * tiles * 4);
    l.first = at;
    at += align(static_cast<size_t>(points) * 4);
    l.prefix = at;
    at += align(static_cast<size_t>(n) * 8);
    l.tile_sums = at;
    at += align(static_cast<size_t>(tiles) * 8);
    l.cut = at;
    at += 256;
    l.total = at;
    return l;
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int64_t odie_select_mean_rank_workspace(int resolution) {
    if (resolution < 1 || static_cast<int64_t>(resolution) * resolution > kMaxCells) return -1;
    const int64_t n = static_cast<int64_t>(resolution) * resolution;
    return static_cast<int64_t>(layout_of(n, (n + 7) / 8 * 8).total);
}

ODIE_API int odie_select_mean_rank(const double* scores, int resolution, int cap, uint8_t* chosen, uint8_t* nodes,
                                   int64_t* stats, void* workspace, int64_t workspace_bytes, uint64_t stream) {
    if (resolution < 1 || static_cast<int64_t>(resolution) * resolution > kMaxCells)
        return fail("odie_select_mean_rank: resolution^2 must be within 1..2^24");
    const int64_t n = static_cast<int64_t>(resolution) * resolution;
    const int64_t points = (n + 7) / 8 * 8;
    if (cap < 0 || cap % 8 || cap > points)
        return fail("odie_select_mean_rank: Node cap must be 8-aligned and within the native plane");
    if (!scores || !chosen || !nodes || !stats) return fail("odie_select_mean_rank: null pointer");
    const Layout l = layout_of(n, points);
    if (!workspace || workspace_bytes < static_cast<int64_t>(l.total))
        return fail("odie_select_mean_rank: workspace must hold odie_select_mean_rank_workspace(resolution) bytes");
    char* space = static_cast<char*>(workspace);
    const hipStream_t s = as_stream(stream);
    const int tiles = static_cast<int>((n + kSortBlock - 1) / kSortBlock);
    const uint32_t blocks256 = static_cast<uint32_t>((n + 255) / 256);
    uint64_t* keys[2] = {reinterpret_cast<uint64_t*>(space + l.keys[0]), reinterpret_cast<uint64_t*>(space + l.keys[1])};
    int32_t* values[2] = {reinterpret_cast<int32_t*>(space + l.values[0]), reinterpret_cast<int32_t*>(space + l.values[1])};
    rank_keys_kernel<<<blocks256, 256, 0, s>>>(scores, n, keys[0], values[0]);
    SortArgs sa{};
    sa.counts = reinterpret_cast<int32_t*>(space + l.counts);
    sa.n = n;
    sa.tiles = tiles;
    for (int pass = 0; pass < kPasses; ++pass) {
        sa.keys_in = keys[pass % 2];
        sa.values_in = values[pass % 2];
        sa.keys_out = keys[(pass + 1) % 2];
        sa.values_out = values[(pass + 1) % 2];
        sa.shift = 8 * pass;
        digit_count_kernel<<<tiles, kSortBlock, 0, s>>>(sa);
        digit_scan_kernel<<<1, kSortBlock, 0, s>>>(sa);
        digit_scatter_kernel<<<tiles, kSortBlock, 0, s>>>(sa);
    }
    AdmitArgs aa{};
    aa.order = values[kPasses % 2];
    aa.first = reinterpret_cast<int32_t*>(space + l.first);
    aa.prefix = reinterpret_cast<int64_t*>(space + l.prefix);
    aa.tile_sums = reinterpret_cast<int64_t*>(space + l.tile_sums);
    aa.cut = reinterpret_cast<int32_t*>(space + l.cut);
    aa.chosen = chosen;
    aa.nodes = nodes;
    aa.stats = stats;
    aa.n = n;
    aa.points = points;
    aa.resolution = resolution;
    aa.cap = cap;
    aa.tiles = tiles;
    const uint32_t point_blocks = static_cast<uint32_t>((points + 255) / 256 < 4096 ? (points + 255) / 256 : 4096);
    admit_reset_kernel<<<point_blocks, 256, 0, s>>>(aa);
    first_touch_kernel<<<blocks256, 256, 0, s>>>(aa);
    first_count_kernel<<<tiles, kSortBlock, 0, s>>>(aa);
    tile_scan_kernel<<<1, kSortBlock, 0, s>>>(aa);
    cut_kernel<<<tiles, kSortBlock, 0, s>>>(aa);
    admit_prefix_kernel<<<blocks256, 256, 0, s>>>(aa);
    admit_rest_kernel<<<1, kSortBlock, 0, s>>>(aa);
    return check_launch("odie_select_mean_rank");
}
