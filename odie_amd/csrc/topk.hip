// Top-k tile selection: the k cells with the largest scores, ties to the lower id, returned in
// ascending id order -- the ranking rule of the reference ("descending score, ascending
// native cell ID", odie/selection.py:103,116), with scores compared as sign-cleared FP64 bit
// patterns so -0 and +0 tie (odie/native/selection_cuda.cu:14-17).
//
// One workgroup.  A radix select over the 64-bit keys (eight 8-bit digits, most significant
// first) finds the key of the k-th element; every element strictly above it is taken, and
// among those equal to it the lowest ids fill the remaining places.  Selected ids are then
// written in ascending order by a block-wide prefix count over the id range -- no sort.
#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kTopkBlock = 1024;

__device__ inline uint64_t topk_key(const double* scores, int64_t i) {
    // larger score -> larger key; sign cleared so that -0 == +0
    return static_cast<uint64_t>(__double_as_longlong(scores[i])) & 0x7fffffffffffffffull;
}

// Inclusive prefix of one int per thread over the block; returns the exclusive prefix and the
// block total.
__device__ inline int64_t block_prefix(int64_t value, int64_t* shared, int64_t& total) {
    shared[threadIdx.x] = value;
    __syncthreads();
    for (int stride = 1; stride < kTopkBlock; stride <<= 1) {
        const int64_t add = threadIdx.x >= stride ? shared[threadIdx.x - stride] : 0;
        __syncthreads();
        shared[threadIdx.x] += add;
        __syncthreads();
    }
    total = shared[kTopkBlock - 1];
    const int64_t inclusive = shared[threadIdx.x];
    __syncthreads();
    return inclusive - value;
}

__global__ __launch_bounds__(kTopkBlock) void topk_kernel(const double* scores, int64_t n, int64_t k, int32_t* ids) {
    __shared__ uint32_t histogram[256];
    __shared__ int64_t shared[kTopkBlock];
    __shared__ uint64_t prefix_key;
    __shared__ int64_t remaining;   // how many of the top-k are still to be found below the prefix
    if (threadIdx.x == 0) {
        prefix_key = 0;
        remaining = k;
    }
    __syncthreads();
    // Radix select of the k-th largest key, most significant digit first.
    for (int digit = 7; digit >= 0; --digit) {
        for (int b = threadIdx.x; b < 256; b += kTopkBlock) histogram[b] = 0;
        __syncthreads();
        const int shift = digit * 8;
        const uint64_t high_mask = digit == 7 ? 0ull : ~((uint64_t{1} << (shift + 8)) - 1);
        const uint64_t prefix = prefix_key;
        for (int64_t i = threadIdx.x; i < n; i += kTopkBlock) {
            const uint64_t key = topk_key(scores, i);
            if ((key & high_mask) == prefix) atomicAdd(&histogram[(key >> shift) & 0xff], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int64_t need = remaining;
            int bin = 255;
            for (; bin > 0; --bin) {
                if (histogram[bin] >= need) break;
                need -= histogram[bin];
            }
            prefix_key = prefix | (static_cast<uint64_t>(bin) << shift);
            remaining = need;
        }
        __syncthreads();
    }
    // threshold = key of the k-th largest; take every key above it and the `remaining`
    // lowest ids among keys equal to it.
    const uint64_t threshold = prefix_key;
    const int64_t ties = remaining;
    int64_t seen_ties = 0;  // equal keys before this thread's current chunk
    int64_t written = 0;    // selected ids before this thread's current chunk
    const int64_t per = (n + kTopkBlock - 1) / kTopkBlock;
    // Each thread owns a contiguous id range so that prefix counts give ascending order.
    const int64_t i0 = threadIdx.x * per < n ? threadIdx.x * per : n;
    const int64_t i1 = i0 + per < n ? i0 + per : n;
    int64_t my_equal = 0, my_above = 0;
    for (int64_t i = i0; i < i1; ++i) {
        const uint64_t key = topk_key(scores, i);
        my_equal += key == threshold;
        my_above += key > threshold;
    }
    int64_t total;
    seen_ties = block_prefix(my_equal, shared, total);
    // selected in my range: all above, plus equal ones whose rank among equals is < ties
    int64_t my_taken_equal = ties - seen_ties;
    my_taken_equal = my_taken_equal < 0 ? 0 : (my_taken_equal > my_equal ? my_equal : my_taken_equal);
    written = block_prefix(my_above + my_taken_equal, shared, total);
    int64_t equal_rank = seen_ties;
    for (int64_t i = i0; i < i1; ++i) {
        const uint64_t key = topk_key(scores, i);
        bool take = key > threshold;
        if (key == threshold) {
            take = equal_rank < ties;
            ++equal_rank;
        }
        if (take) ids[written++] = static_cast<int32_t>(i);
    }
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_topk(const double* scores, int64_t n, int64_t k, int32_t* ids, uint64_t stream) {
    if (n < 0 || n > (int64_t{1} << 31) - 1) return fail("odie_topk: n must be within [0, 2^31-1]");
    if (k < 0 || k > n) return fail("odie_topk: k must be within [0, n]");
    if (k == 0) return 0;
    if (!scores || !ids) return fail("odie_topk: null pointer");
    topk_kernel<<<1, kTopkBlock, 0, as_stream(stream)>>>(scores, n, k, ids);
    return check_launch("odie_topk");
}
