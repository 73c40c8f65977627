// B2 exact greedy support selection (odie/selection.py:129-207) for gfx950.
//
// The rule: repeatedly take the free cell (all four closure nodes already present) with the
// smallest id; otherwise the cell with the best score/cost over costs 1..min(4, cap-used),
// compared by cross-multiplication in fp64 and ties to the lower id; each taken cell adds
// its missing nodes and lowers the cost of the cells that share them.
//
// Layout and work split:
//  * a tournament tree per cost category 1..4 with fan 64 (one wave per node): level 0 nodes
//    hold, for 64 consecutive cells, the best cell of that category (largest sign-cleared
//    fp64 score key, then lowest id; -1 if none), higher levels the best of 64 nodes below;
//  * the levels whose nodes fit in 64 KiB live in LDS for the whole launch (loaded at entry,
//    written back at exit); lower levels stay in the caller's tree buffer;
//  * one workgroup runs the sequential choices; per choice it re-scans only the tree nodes
//    on the paths of the cells whose category changed (one wave per node, in parallel).
// Free cells never need the tree: a free cell adds no node and so changes no other cell's
// cost, hence every cell freed by a choice is taken right after it, in ascending id, exactly
// where the reference's "free first" rule takes them.  Category 0 is therefore not stored,
// and iteration counts, choices and trace order are those of the reference rule.
#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kFan = 64;
constexpr int kCats = 4;                // cost categories 1..4
constexpr int kGreedyBlock = 512;
constexpr int kGreedyWaves = kGreedyBlock / 64;
constexpr int kMaxLevels = 8;
constexpr int kLdsTreeInts = 12288;     // 48 KiB of tree ids in LDS
constexpr int kMaxTasks = 64;

struct TreeShape {
    int levels;
    int first_lds;                      // levels >= first_lds are kept in LDS during a launch
    int64_t size[kMaxLevels];           // nodes per level
    int64_t offset[kMaxLevels];         // first int of a level in the tree buffer (4 per node)
    int lds_ints;                       // ints of the LDS-resident levels
};

TreeShape tree_shape(int64_t n) {
    TreeShape t{};
    int64_t children = n, offset = 0;
    int levels = 0;
    do {
        const int64_t parents = (children + kFan - 1) / kFan;
        t.size[levels] = parents;
        t.offset[levels] = offset;
        offset += parents * kCats;
        children = parents;
        ++levels;
    } while (children > 1 && levels < kMaxLevels);
    t.levels = levels;
    t.first_lds = levels - 1;
    int64_t ints = t.size[levels - 1] * kCats;
    while (t.first_lds > 0 && ints + t.size[t.first_lds - 1] * kCats <= kLdsTreeInts) {
        --t.first_lds;
        ints += t.size[t.first_lds] * kCats;
    }
    t.lds_ints = static_cast<int>(ints);
    return t;
}

int64_t tree_ints(const TreeShape& t) { return t.offset[t.levels - 1] + t.size[t.levels - 1] * kCats; }

__device__ inline uint64_t score_key(const double* scores, int id) {
    return static_cast<uint64_t>(__double_as_longlong(scores[id])) & 0x7fffffffffffffffull;
}

__device__ inline bool better(int a, uint64_t ka, int b, uint64_t kb) {
    if (a < 0) return false;
    if (b < 0) return true;
    return ka > kb || (ka == kb && a < b);
}

// Best (id, key) over the wave: lane values in, result in every lane.
__device__ inline int wave_best(int id, uint64_t key) {
    for (int step = 32; step; step >>= 1) {
        const int other = __shfl_xor(id, step);
        const uint64_t other_key = __shfl_xor(key, step);
        if (better(other, other_key, id, key)) {
            id = other;
            key = other_key;
        }
    }
    return id;
}

// Offset of closure corner k (0..3) from its cell: 0, 1, R, R+1 (odie/selection.py:158).
__device__ inline int corner_delta(int k, int resolution) { return (k & 1) + (k >> 1) * resolution; }

struct GreedyArgs {
    const double* scores;
    int* missing;
    uint8_t* chosen;
    uint8_t* nodes;
    int* tree;
    int64_t* stats;
    int* trace;
    int n;
    int points;
    int resolution;
    int cap;
    int normalized;
    int chunk;
    TreeShape shape;
};

__device__ inline int& tree_at(const GreedyArgs& a, int* lds_tree, int level, int64_t node, int cat) {
    if (level >= a.shape.first_lds)
        return lds_tree[a.shape.offset[level] - a.shape.offset[a.shape.first_lds] + node * kCats + (cat - 1)];
    return a.tree[a.shape.offset[level] + node * kCats + (cat - 1)];
}

// Best cell of category `cat` under level-`level` node `node`, computed by one wave from the
// level below (cells for level 0).
__device__ inline int rescan(const GreedyArgs& a, int* lds_tree, int level, int64_t node, int cat) {
    const int lane = threadIdx.x % 64;
    const int64_t child = node * kFan + lane;
    int id = -1;
    if (level == 0) {
        if (child < a.n && !a.chosen[child] && a.missing[child] == cat) id = static_cast<int>(child);
    } else if (child < a.shape.size[level - 1]) {
        id = tree_at(a, lds_tree, level - 1, child, cat);
    }
    const uint64_t key = id >= 0 ? score_key(a.scores, id) : 0;
    return wave_best(id, key);
}

__global__ __launch_bounds__(kGreedyBlock) void init_kernel(GreedyArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kGreedyBlock + threadIdx.x;
    if (i < a.n) {
        a.missing[i] = 4;
        a.chosen[i] = 0;
    }
    if (i < a.points) a.nodes[i] = 0;
    if (i < 4) a.stats[i] = 0;
}

// One wave per (node, category) of one level; level 0 reads the cells.
__global__ __launch_bounds__(256) void build_kernel(GreedyArgs a, int level) {
    const int64_t task = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / 64;
    const int64_t node = task / kCats;
    const int cat = static_cast<int>(task % kCats) + 1;
    if (node >= a.shape.size[level]) return;  // the whole wave takes the same branch
    const int lane = threadIdx.x % 64;
    const int64_t child = node * kFan + lane;
    int id = -1;
    if (level == 0) {
        if (child < a.n && !a.chosen[child] && a.missing[child] == cat) id = static_cast<int>(child);
    } else if (child < a.shape.size[level - 1]) {
        id = a.tree[a.shape.offset[level - 1] + child * kCats + (cat - 1)];
    }
    const uint64_t key = id >= 0 ? score_key(a.scores, id) : 0;
    id = wave_best(id, key);
    if (lane == 0) a.tree[a.shape.offset[level] + node * kCats + (cat - 1)] = id;
}

__global__ __launch_bounds__(kGreedyBlock) void greedy_kernel(GreedyArgs a) {
    extern __shared__ int lds_tree[];
    __shared__ int cell, cost, stop, nadded, added[4], naffected, affected[16], old_cat[16], new_cat[16];
    __shared__ int nfree, freed[16], ntasks, tasks_node[kMaxTasks], tasks_cat[kMaxTasks];
    __shared__ int changed[kMaxTasks];
    __shared__ int halted, invalid;
    __shared__ long long used, iterations;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int64_t lds_base = a.shape.offset[a.shape.first_lds];
    for (int j = tid; j < a.shape.lds_ints; j += kGreedyBlock) lds_tree[j] = a.tree[lds_base + j];
    if (tid == 0) {
        used = a.stats[0];
        iterations = a.stats[1];
        halted = a.stats[2] != 0 || a.stats[3] != 0;
        stop = 0;
        invalid = 0;
    }
    __syncthreads();
    const int top = a.shape.levels - 1;
    // `stop` is read only right after a barrier, before thread 0 can write it again
    for (int step = 0; step < a.chunk && !halted; ++step) {
        // A. choose the best costly cell: the root winners of costs 1..min(4, cap-used),
        // score/cost compared by cross-multiplication, ties to the lower id
        if (tid == 0) {
            const int64_t remaining = static_cast<int64_t>(a.cap) - used;
            int best = -1, best_cost = 0;
            double best_score = 0.0;
            for (int c = 1; c <= 4 && c <= remaining; ++c) {
                const int candidate = tree_at(a, lds_tree, top, 0, c);
                if (candidate < 0) continue;
                const double score = a.scores[candidate];
                if (best >= 0) {
                    const double left = a.normalized ? score * static_cast<double>(best_cost) : score;
                    const double right = a.normalized ? best_score * static_cast<double>(c) : best_score;
                    if (!(left > right || (left == right && candidate < best))) continue;
                }
                best = candidate;
                best_cost = c;
                best_score = score;
            }
            cell = best;
            cost = best_cost;
            stop = best < 0;
        }
        __syncthreads();
        if (stop) break;
        // B. take it: mark its closure nodes, count the new ones
        if (wave == 0) {
            int node = 0;
            bool fresh = false;
            if (lane < 4) {
                node = static_cast<int>((static_cast<int64_t>(cell) + corner_delta(lane, a.resolution)) % a.points);
                fresh = a.nodes[node] == 0;
            }
            const uint64_t fresh_mask = __ballot(lane < 4 && fresh);
            if (lane < 4 && fresh) {
                a.nodes[node] = 1;
                added[__popcll(fresh_mask & ((uint64_t{1} << lane) - 1))] = node;
            }
            if (lane == 0) {
                nadded = __popcll(fresh_mask);
                a.chosen[cell] = 1;
                if (a.trace) a.trace[iterations] = cell;
                iterations += 1;
                used += nadded;
                invalid = nadded != cost;
                if (invalid) a.stats[3] = 1;
            }
        }
        __syncthreads();
        if (invalid) break;
        // C. cells sharing the new nodes lose one missing node per shared corner
        if (wave == 0) {
            int inc = -1;
            if (lane < 4 * nadded) {
                const int node = added[lane / 4];
                inc = static_cast<int>((static_cast<int64_t>(node) - corner_delta(lane % 4, a.resolution) + a.points) % a.points);
                if (inc >= a.n || a.chosen[inc]) inc = -1;
            }
            // distinct cells among the 16 lanes; the first lane of each counts the duplicates
            int dup = 0;
            bool first = inc >= 0;
            for (int j = 0; j < 16; ++j) {
                const int other = __shfl(inc, j);
                if (inc >= 0 && other == inc) {
                    ++dup;
                    if (j < lane) first = false;
                }
            }
            const uint64_t firsts = __ballot(first);
            int old = 0, now = 0;
            if (first) {
                old = a.missing[inc];
                now = old - dup;
                a.missing[inc] = now;
                const int slot = __popcll(firsts & ((uint64_t{1} << lane) - 1));
                affected[slot] = inc;
                old_cat[slot] = old;
                new_cat[slot] = now;
            }
            // cells freed by this choice are taken now, in ascending id
            const bool frees = first && now == 0;
            const uint64_t free_mask = __ballot(frees);
            int rank = 0;
            for (int j = 0; j < 16; ++j) {
                const int other = __shfl(inc, j);
                if (((free_mask >> j) & 1) && other < inc) ++rank;
            }
            if (frees) {
                freed[rank] = inc;
                a.chosen[inc] = 1;
            }
            if (lane == 0) {
                naffected = __popcll(firsts);
                nfree = __popcll(free_mask);
            }
        }
        __syncthreads();
        if (tid == 0) {
            for (int j = 0; j < nfree; ++j) {
                if (a.trace) a.trace[iterations] = freed[j];
                iterations += 1;
            }
            // D. tree tasks at level 0: the taken cell leaves category `cost`; every affected
            // cell leaves its old category and joins its new one (none if freed).
            int count = 0;
            auto add_task = [&](int node, int cat) {
                if (cat < 1 || cat > 4) return;
                for (int j = 0; j < count; ++j)
                    if (tasks_node[j] == node && tasks_cat[j] == cat) return;
                tasks_node[count] = node;
                tasks_cat[count] = cat;
                ++count;
            };
            add_task(cell / kFan, cost);
            for (int j = 0; j < naffected; ++j) {
                add_task(affected[j] / kFan, old_cat[j]);
                add_task(affected[j] / kFan, new_cat[j]);
            }
            ntasks = count;
        }
        __syncthreads();
        for (int level = 0; level <= top; ++level) {
            for (int t = wave; t < ntasks; t += kGreedyWaves) {
                const int node = tasks_node[t], cat = tasks_cat[t];
                const int best = rescan(a, lds_tree, level, node, cat);
                if (lane == 0) {
                    int& slot = tree_at(a, lds_tree, level, node, cat);
                    changed[t] = slot != best;
                    slot = best;
                }
            }
            __syncthreads();
            if (tid == 0) {
                int count = 0;
                for (int t = 0; t < ntasks; ++t) {
                    if (!changed[t]) continue;
                    const int node = tasks_node[t] / kFan, cat = tasks_cat[t];
                    bool seen = false;
                    for (int j = 0; j < count; ++j) seen |= tasks_node[j] == node && tasks_cat[j] == cat;
                    if (!seen) {
                        tasks_node[count] = node;
                        tasks_cat[count] = cat;
                        ++count;
                    }
                }
                ntasks = level < top ? count : 0;
            }
            __syncthreads();
            if (ntasks == 0) break;
        }
    }
    __syncthreads();
    for (int j = tid; j < a.shape.lds_ints; j += kGreedyBlock) a.tree[lds_base + j] = lds_tree[j];
    if (tid == 0) {
        a.stats[0] = used;
        a.stats[1] = iterations;
        if (stop && !invalid) a.stats[2] = 1;
    }
}

int check_common(const char* what, const double* scores, int n, int points, int* missing, uint8_t* chosen,
                 uint8_t* nodes, int* tree, int64_t* stats) {
    const std::string w(what);
    if (n < 1) return fail(w + ": n must be positive");
    if (points < n || points % 8) return fail(w + ": points must be an 8-aligned count >= n");
    if (!scores || !missing || !chosen || !nodes || !tree || !stats) return fail(w + ": null pointer");
    return 0;
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int64_t odie_selection_tree_ints(int n) {
    if (n < 1) return -1;
    return tree_ints(tree_shape(n));
}

// Same signature as selection_init (odie/native/selection_cuda.cu:208-220), and the same failure
// value: the runtime's error code (hipErrorInvalidValue for a refused argument), the message in
// odie_error().  host_offsets /
// host_sizes / levels describe the caller's fan-32 tree allocation; this selector lays out its
// own fan-64 tree, which needs no more ints than that allocation (checked when given).
ODIE_API int selection_init(const double* scores, int n, int points, int* missing, uint8_t* chosen, uint8_t* nodes,
                            int* tree, int64_t* stats, const int* host_offsets, const int* host_sizes, int levels,
                            uint64_t stream) {
    if (check_common("selection_init", scores, n, points, missing, chosen, nodes, tree, stats)) return hipErrorInvalidValue;
    const TreeShape shape = tree_shape(n);
    if (host_offsets && host_sizes && levels > 0) {
        const int64_t available = static_cast<int64_t>(host_offsets[levels - 1]) + 5LL * host_sizes[levels - 1];
        if (available < tree_ints(shape)) return fail_code("selection_init: tree buffer too small");
    }
    GreedyArgs a{};
    a.scores = scores;
    a.missing = missing;
    a.chosen = chosen;
    a.nodes = nodes;
    a.tree = tree;
    a.stats = stats;
    a.n = n;
    a.points = points;
    a.shape = shape;
    const hipStream_t s = as_stream(stream);
    const int64_t count = points > n ? points : n;
    init_kernel<<<static_cast<uint32_t>((count + kGreedyBlock - 1) / kGreedyBlock), kGreedyBlock, 0, s>>>(a);
    for (int level = 0; level < shape.levels; ++level) {
        const int64_t waves = shape.size[level] * kCats;
        build_kernel<<<static_cast<uint32_t>((waves + 3) / 4), 256, 0, s>>>(a, level);
    }
    return launch_code("selection_init");
}

// Same signature as selection_chunk (odie/native/selection_cuda.cu:222-230); offsets, sizes and
// levels (the caller's fan-32 layout) are not needed.  Runs up to `chunk` choices (a choice's
// freed cells are taken with it); stats = {used nodes, iterations, done, invariant error}.
ODIE_API int selection_chunk(const double* scores, int n, int points, int resolution, int cap, bool normalized,
                             int* missing, uint8_t* chosen, uint8_t* nodes, int* tree, const int* offsets,
                             const int* sizes, int levels, int chunk, int64_t* stats, int* trace, uint64_t stream) {
    (void)offsets;
    (void)sizes;
    (void)levels;
    if (check_common("selection_chunk", scores, n, points, missing, chosen, nodes, tree, stats)) return hipErrorInvalidValue;
    if (resolution < 2 || static_cast<int64_t>(resolution) * resolution != n)
        return fail_code("selection_chunk: n must be resolution^2");
    if (cap < 0 || cap % 8 || cap > points) return fail_code("selection_chunk: cap must be 8-aligned within points");
    if (chunk < 1) return fail_code("selection_chunk: chunk must be positive");
    GreedyArgs a{};
    a.scores = scores;
    a.missing = missing;
    a.chosen = chosen;
    a.nodes = nodes;
    a.tree = tree;
    a.stats = stats;
    a.trace = trace;
    a.n = n;
    a.points = points;
    a.resolution = resolution;
    a.cap = cap;
    a.normalized = normalized ? 1 : 0;
    a.chunk = chunk;
    a.shape = tree_shape(n);
    greedy_kernel<<<1, kGreedyBlock, static_cast<size_t>(a.shape.lds_ints) * 4, as_stream(stream)>>>(a);
    return launch_code("selection_chunk");
}
