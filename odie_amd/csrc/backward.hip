// Grid-encode backward without global atomics ("owner computes").
//
// Measured on MI355X: global fp32 atomics saturate near 21 G op/s and LDS fp32 atomics
// near 0.2 T op/s, while LDS 64-bit integer atomics (ds_add_u64) reach ~2.4 T op/s.  So the
// gradient is not scattered into HBM at all:
//   1. transpose  the upstream rows [N, L*F] into level-major planes [L][N][F] and record
//                 the largest |upstream| of every 1024-row block and level;
//   2. owner      one workgroup owns one slice of one expert's gradient (a group of coarse
//                 levels, or a part of one finer level) that fits in LDS.  It walks every
//                 coordinate of its expert, evaluates the geometry of its level(s) and adds
//                 the contributions that land in its slice as 64-bit fixed-point integers
//                 (ds_add_u64).  The fixed-point scale 2^S is chosen per workgroup from
//                 max|upstream| over its coordinates and levels: every contribution stays
//                 below 2^31 and 4*count of them below 2^62, so nothing can overflow; each
//                 contribution is the fp32 product w_k * upstream (as in the reference,
//                 odie/packed_kernels.cu:84) rounded to the nearest multiple of 2^-S.  The
//                 slice is then converted to fp32 and written with plain coalesced stores.
//                 Integer sums are associative, so the gradient does not depend on the
//                 order in which lanes add.
//   3. reduce     only when one expert's coordinates are split over several workgroups per
//                 slice (few experts, many coordinates): partial slices are summed.
// Every gradient entry is written by exactly one workgroup, so no clearing pass is needed.
#include "grid.h"

namespace odie {
namespace {

constexpr int kTransposeBlock = 256;
constexpr int kTransposeRows = 1024;  // rows per transpose block (and per max-record)
constexpr int kOwnerBlock = 1024;
constexpr int kBatch = 4;             // coordinates per thread per owner-loop iteration

struct TransposeArgs {
    const void* upstream;
    void* planes;
    float* blockmax;
    int64_t n;
    int width;
    int n_levels;
    int vec_rows;
};

template <int F, bool HALF, int LMAX>
__global__ __launch_bounds__(kTransposeBlock) void transpose_kernel(TransposeArgs a) {
    using U = Elem<HALF>;
    __shared__ float waves[kTransposeBlock / 64][LMAX];
    float peak[LMAX];
#pragma unroll
    for (int l = 0; l < LMAX; ++l) peak[l] = 0.0f;
    const int used = a.n_levels * F;
    for (int r = 0; r < kTransposeRows / kTransposeBlock; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        if (i >= a.n) break;
        const U* row = reinterpret_cast<const U*>(a.upstream) + static_cast<size_t>(i) * a.width;
        U vals[LMAX * F];
        if (a.vec_rows) {
            constexpr int kPer = 16 / sizeof(U);
            constexpr int kChunks = (LMAX * F + kPer - 1) / kPer;
#pragma unroll
            for (int j = 0; j < kChunks; ++j) {
                if (j * kPer < used) {
                    const uint4 v = reinterpret_cast<const uint4*>(row)[j];
                    const U* parts = reinterpret_cast<const U*>(&v);
#pragma unroll
                    for (int q = 0; q < kPer; ++q)
                        if (j * kPer + q < LMAX * F) vals[j * kPer + q] = parts[q];
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < LMAX * F; ++c)
                if (c < used) vals[c] = row[c];
        }
        U* planes = reinterpret_cast<U*>(a.planes);
#pragma unroll
        for (int l = 0; l < LMAX; ++l) {
            if (l < a.n_levels) {
                U* dst = planes + (static_cast<size_t>(l) * a.n + i) * F;
                if constexpr (HALF && F == 2) {
                    const uint32_t word = static_cast<uint32_t>(half_to_bits(vals[l * F])) |
                                          (static_cast<uint32_t>(half_to_bits(vals[l * F + 1])) << 16);
                    *reinterpret_cast<uint32_t*>(dst) = word;
                } else {
#pragma unroll
                    for (int c = 0; c < F; ++c) dst[c] = vals[l * F + c];
                }
#pragma unroll
                for (int c = 0; c < F; ++c) {
                    const float v = fabsf(static_cast<float>(vals[l * F + c]));
                    peak[l] = (v > peak[l] || v != v) ? v : peak[l];
                }
            }
        }
    }
    // NaN is kept by the comparisons below (not fmaxf) so the owner pass sees a non-finite bound.
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
        if (l < a.n_levels) {
            float m = peak[l];
            for (int step = 32; step; step >>= 1) {
                const float other = __shfl_xor(m, step);
                m = (other > m || other != other) ? other : m;
            }
            if (lane == 0) waves[wave][l] = m;
        }
    }
    __syncthreads();
    if (threadIdx.x < a.n_levels) {
        float m = 0.0f;
        for (int w = 0; w < kTransposeBlock / 64; ++w) {
            const float other = waves[w][threadIdx.x];
            m = (other > m || other != other) ? other : m;
        }
        a.blockmax[static_cast<size_t>(blockIdx.x) * a.n_levels + threadIdx.x] = m;
    }
}

struct OwnerArgs {
    const float* coords;
    const int32_t* offsets;
    const void* planes;
    const float* blockmax;
    float* grad;
    float* partial;
    int64_t n;
    int64_t expert_params;
    int experts;
    int n_levels;
    int group;        // pass 0 covers levels [0, group) when group > 0
    int passes;       // passes per expert
    int splits;       // coordinate splits per pass
    int accumulate;   // 1: grad += slice
    int remap;
    DevLevel level[ODIE_MAX_LEVELS];
    int first_pass[ODIE_MAX_LEVELS];
    int slices[ODIE_MAX_LEVELS];
    int slice_entries[ODIE_MAX_LEVELS];
};

template <int F, bool HALF>
__global__ __launch_bounds__(kOwnerBlock) void owner_kernel(OwnerArgs a) {
    extern __shared__ unsigned long long acc[];
    __shared__ float reduce[kOwnerBlock / 64];
    using U = Elem<HALF>;
    const uint32_t total = static_cast<uint32_t>(a.experts) * a.passes * a.splits;
    const uint32_t work = a.remap ? xcd_major(blockIdx.x, gridDim.x) : blockIdx.x;
    if (work >= total) return;
    const int e = work / (a.passes * a.splits);
    const int p = (work / a.splits) % a.passes;
    const int s = work % a.splits;

    // Pass -> levels [l0, l1) and the slice [lo, hi) of the expert's gradient (in floats).
    int l0, l1;
    uint32_t lo, hi;
    if (a.group > 0 && p == 0) {
        l0 = 0;
        l1 = a.group;
        lo = 0;
        hi = (a.level[a.group - 1].offset + a.level[a.group - 1].size) * F;
    } else {
        int l = a.group;
        while (l + 1 < a.n_levels && a.first_pass[l + 1] <= p) ++l;
        const int slice = p - a.first_pass[l];
        const uint32_t first = static_cast<uint32_t>(slice) * a.slice_entries[l];
        uint32_t last = first + a.slice_entries[l];
        if (last > a.level[l].size) last = a.level[l].size;
        l0 = l;
        l1 = l + 1;
        lo = (a.level[l].offset + first) * F;
        hi = (a.level[l].offset + last) * F;
    }
    const uint32_t span = hi - lo;

    // Coordinates of this expert (and split).
    int64_t base = 0, stop = a.n;
    if (a.offsets) {
        base = a.offsets[e];
        stop = a.offsets[e + 1];
        if (stop < base) stop = base;
        if (stop > a.n) stop = a.n;
        if (base > stop) base = stop;
    }
    const int64_t share = (stop - base + a.splits - 1) / a.splits;
    const int64_t b0 = base + share * s < stop ? base + share * s : stop;
    const int64_t b1 = b0 + share < stop ? b0 + share : stop;

    // Fixed-point scale from the bound 4 * count * max|upstream| over this range and levels.
    float bound = 0.0f;
    if (b1 > b0) {
        const int64_t r0 = b0 / kTransposeRows, r1 = (b1 - 1) / kTransposeRows;
        const int levels = l1 - l0;
        for (int64_t t = threadIdx.x; t < (r1 - r0 + 1) * levels; t += kOwnerBlock) {
            const float v = a.blockmax[(r0 + t / levels) * a.n_levels + l0 + t % levels];
            bound = (v > bound || v != v) ? v : bound;
        }
    }
    for (int step = 32; step; step >>= 1) {
        const float other = __shfl_xor(bound, step);
        bound = (other > bound || other != other) ? other : bound;
    }
    if (threadIdx.x % 64 == 0) reduce[threadIdx.x / 64] = bound;
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) acc[j] = 0ull;
    __syncthreads();
    float peak = 0.0f;
    for (int w = 0; w < kOwnerBlock / 64; ++w) peak = (reduce[w] > peak || reduce[w] != reduce[w]) ? reduce[w] : peak;
    // Scale 2^shift: every contribution |w*u| <= peak maps below 2^31 (so it converts with one
    // rint + cvt_i32), and 4*count contributions of that size stay below 2^62 in the int64 sum.
    const double limit = 4.0 * static_cast<double>(b1 - b0) * static_cast<double>(peak);
    int shift = 60;
    if (peak > 0.0f && limit <= 1.0e300) {
        const int by_value = 30 - ilogb(peak);
        const int by_sum = 61 - ilogb(limit);
        shift = by_value < by_sum ? by_value : by_sum;
    }
    if (shift > 120) shift = 120;
    const float scale = ldexpf(1.0f, shift);
    const bool finite = !(peak != peak) && peak <= 3.0e38f;

    // Each thread takes kBatch coordinates per iteration (strided by the block so every load
    // stays coalesced) and issues all their loads before any arithmetic, keeping several
    // L2/HBM requests in flight per lane.
    const U* planes = reinterpret_cast<const U*>(a.planes);
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kBatch * kOwnerBlock) {
        float2 xy[kBatch];
        bool valid[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int64_t ii = i + b * kOwnerBlock;
            valid[b] = ii < b1;
            xy[b] = valid[b] ? reinterpret_cast<const float2*>(a.coords)[ii] : make_float2(0.f, 0.f);
        }
        for (int l = l0; l < l1; ++l) {
            float u[kBatch][F];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int64_t ii = i + b * kOwnerBlock;
                const U* src = planes + (static_cast<size_t>(l) * a.n + (valid[b] ? ii : b0)) * F;
                if constexpr (HALF && F == 2) {
                    const uint32_t word = valid[b] ? *reinterpret_cast<const uint32_t*>(src) : 0u;
                    u[b][0] = __half2float(bits_to_half(static_cast<uint16_t>(word & 0xffffu)));
                    u[b][1] = __half2float(bits_to_half(static_cast<uint16_t>(word >> 16)));
                } else {
#pragma unroll
                    for (int c = 0; c < F; ++c) u[b][c] = valid[b] ? static_cast<float>(src[c]) : 0.0f;
                }
            }
            const DevLevel& lv = a.level[l];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                bool any = false;
#pragma unroll
                for (int c = 0; c < F; ++c) any |= u[b][c] != 0.0f;
                if (!any) continue;
                uint32_t idx[4];
                float w[4];
                grid_corners(lv, xy[b].x, xy[b].y, idx, w);
                // Convert all contributions before the (divergent) slice test so that the
                // masked part of the wave is only the LDS add itself.
                int32_t q[4][F];
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int c = 0; c < F; ++c) q[k][c] = static_cast<int32_t>(rintf((w[k] * u[b][c]) * scale));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t slot = (lv.offset + idx[k]) * F - lo;
                    if (slot >= span) continue;
#pragma unroll
                    for (int c = 0; c < F; ++c)
                        if (q[k][c] != 0)
                            atomicAdd(acc + slot + c, static_cast<unsigned long long>(static_cast<long long>(q[k][c])));
                }
            }
        }
    }
    __syncthreads();
    const double unscale = ldexp(1.0, -shift);
    float* out = a.splits == 1 ? a.grad + static_cast<size_t>(e) * a.expert_params + lo
                               : a.partial + static_cast<size_t>(s) * a.experts * a.expert_params +
                                     static_cast<size_t>(e) * a.expert_params + lo;
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) {
        float v = static_cast<float>(static_cast<double>(static_cast<long long>(acc[j])) * unscale);
        if (!finite) v = __builtin_nanf("");
        if (a.splits == 1 && a.accumulate) v += out[j];
        out[j] = v;
    }
}

__global__ __launch_bounds__(256) void split_reduce_kernel(const float* partial, float* grad, int64_t total, int splits,
                                                           int accumulate) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t x = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; x < total; x += stride) {
        float v = accumulate ? grad[x] : 0.0f;
        for (int s = 0; s < splits; ++s) v += partial[static_cast<size_t>(s) * total + x];
        grad[x] = v;
    }
}

template <typename Kernel>
int allow_lds(Kernel kernel, size_t bytes) {
    const hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (status != hipSuccess) return fail(std::string("LDS attribute: ") + hipGetErrorString(status));
    return 0;
}

}  // namespace

int launch_owner_backward(const OwnerLaunch& in) {
    const int F = in.features;
    const int L = in.n_levels;
    const bool half = in.up_half != 0;
    const size_t elem = half ? 2 : 4;
    const int64_t lds_bytes = in.lds_bytes;
    const int64_t cap = lds_bytes / 8 - F;  // floats per slice (int64 accumulators), minus entry rounding
    if (cap < 64) return fail("odie_grid_backward: LDS budget too small for the owner backward");

    OwnerArgs o{};
    o.coords = in.coords;
    o.offsets = in.offsets;
    o.n = in.n;
    o.expert_params = in.expert_params;
    o.experts = in.experts;
    o.n_levels = L;
    o.accumulate = in.accumulate;
    o.remap = in.remap;
    int group = 0;
    int64_t grouped = 0;
    while (group < L && grouped + static_cast<int64_t>(in.levels[group].size) * F <= cap) {
        grouped += static_cast<int64_t>(in.levels[group].size) * F;
        ++group;
    }
    int passes = group > 0 ? 1 : 0;
    for (int l = 0; l < L; ++l) {
        o.level[l] = in.levels[l];
        if (l < group) continue;
        const int64_t floats = static_cast<int64_t>(in.levels[l].size) * F;
        const int64_t slices = (floats + cap - 1) / cap;
        o.slices[l] = static_cast<int>(slices);
        o.slice_entries[l] = static_cast<int>((in.levels[l].size + slices - 1) / slices);
        o.first_pass[l] = passes;
        passes += static_cast<int>(slices);
    }
    o.group = group;
    o.passes = passes;
    const int64_t per_pass = static_cast<int64_t>(in.experts) * passes;
    int splits = 1;
    if (per_pass < 512) {
        const int64_t want = (512 + per_pass - 1) / per_pass;
        const int64_t most = in.n / (static_cast<int64_t>(in.experts) * 16384);
        splits = static_cast<int>(want < most ? want : (most > 1 ? most : 1));
    }
    o.splits = splits;

    // Workspace: level-major planes, block maxima, split partials.
    const int64_t row_blocks = (in.n + kTransposeRows - 1) / kTransposeRows;
    const size_t planes_bytes = (static_cast<size_t>(in.n) * L * F * elem + 255) / 256 * 256;
    const size_t max_bytes = (static_cast<size_t>(row_blocks) * L * 4 + 255) / 256 * 256;
    const size_t total_params = static_cast<size_t>(in.experts) * in.expert_params;
    const size_t partial_bytes = splits > 1 ? static_cast<size_t>(splits) * total_params * 4 : 0;
    char* space = static_cast<char*>(workspace(planes_bytes + max_bytes + partial_bytes, in.stream));
    if (!space) return -1;
    o.planes = space;
    o.blockmax = reinterpret_cast<float*>(space + planes_bytes);
    o.partial = reinterpret_cast<float*>(space + planes_bytes + max_bytes);
    o.grad = in.grad;

    TransposeArgs t{};
    t.upstream = in.upstream;
    t.planes = space;
    t.blockmax = reinterpret_cast<float*>(space + planes_bytes);
    t.n = in.n;
    t.width = in.up_width;
    t.n_levels = L;
    t.vec_rows = (reinterpret_cast<uintptr_t>(in.upstream) % 16 == 0) && (in.up_width * elem) % 16 == 0 &&
                 (L * F * elem) % 16 == 0;
    const uint32_t tblocks = static_cast<uint32_t>(row_blocks);
    const size_t shmem = static_cast<size_t>(cap + F) * 8;
    const uint32_t total = static_cast<uint32_t>(per_pass * splits);
    const uint32_t oblocks = round_up(total, kXcds);
    hipStream_t s = in.stream;

#define ODIE_TRANSPOSE(FF, HH)                                                                          \
    do {                                                                                                \
        if (L <= 16) transpose_kernel<FF, HH, 16><<<tblocks, kTransposeBlock, 0, s>>>(t);               \
        else transpose_kernel<FF, HH, 32><<<tblocks, kTransposeBlock, 0, s>>>(t);                       \
    } while (0)
#define ODIE_OWNER(FF, HH)                                                                              \
    do {                                                                                                \
        if (allow_lds(owner_kernel<FF, HH>, shmem)) return -1;                                          \
        owner_kernel<FF, HH><<<oblocks, kOwnerBlock, shmem, s>>>(o);                                    \
    } while (0)
#define ODIE_BOTH(FF)                                                                                   \
    do {                                                                                                \
        if (half) { ODIE_TRANSPOSE(FF, true); ODIE_OWNER(FF, true); }                                   \
        else { ODIE_TRANSPOSE(FF, false); ODIE_OWNER(FF, false); }                                      \
    } while (0)
    switch (F) {
        case 1: ODIE_BOTH(1); break;
        case 2: ODIE_BOTH(2); break;
        case 4: ODIE_BOTH(4); break;
        default: ODIE_BOTH(8); break;
    }
#undef ODIE_BOTH
#undef ODIE_OWNER
#undef ODIE_TRANSPOSE
    if (splits > 1) {
        int64_t blocks = (static_cast<int64_t>(total_params) + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        split_reduce_kernel<<<static_cast<uint32_t>(blocks), 256, 0, s>>>(o.partial, in.grad,
                                                                          static_cast<int64_t>(total_params), splits,
                                                                          in.accumulate);
    }
    return check_launch("odie_grid_backward");
}

}  // namespace odie
