// Multiresolution grid encode for gfx950: hash grid (single grid or packed experts) and
// packed xy planes, forward and gradient scatter.
//
// Work decomposition: one lane per coordinate, all levels in registers, so a row of
// features is produced and stored with 16-byte stores and the upstream row is loaded the
// same way.  Blocks own contiguous chunks of the (expert-compacted) coordinate array and
// their block ids are remapped so consecutive chunks -- and therefore one expert's table
// -- stay on one XCD and its L2.  The backward accumulates the coarse levels of the
// chunk's expert in LDS (ds_add_f32) and flushes them once per chunk with global fp32
// atomics; finer levels go straight to global_atomic_add_f32.
#include "grid.h"
#include "adam.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kBlock = 256;
// Word 3 of a raw buffer resource on CDNA (gfx9 layout): DATA_FORMAT 32 in bits 15..18 (a zero
// data format would make untyped buffer loads return zero), the rest (swizzle, index stride) 0.
constexpr int kRawBufferWord3 = 0x00020000;

struct GridArgs {
    const float* coords;
    const int32_t* offsets;
    const void* params;
    void* out;
    const void* upstream;
    float* grad;
    int64_t n;
    int64_t expert_params;
    int experts;
    int n_levels;
    int width;       // output (forward) or upstream (backward) row width in elements
    int chunk;       // coordinates per block
    int vec_rows;    // rows are 16-byte aligned and a multiple of 16 bytes
    int lds_levels;  // backward: levels accumulated in LDS
    int lds_floats;  // backward: LDS accumulator size in floats
    int remap;       // 1: XCD-major block order
    int paired;      // forward, fp16 F=2: 16-byte group loads (table 16-byte aligned, entries % 4 == 0)
    int stage_levels;   // forward, fp16 F=2: coarse levels read from an LDS copy of the expert's table
    int stage_entries;  // entries staged (multiple of 4)
    uint8_t* masks;     // forward: the owner backward's slice masks written on the way (HandoffPlan), or null
    int64_t mask_stride;
    const int32_t* list;     // forward: walk the owner's band lists (list position j: coordinate list[j]
    const float2* sorted;    // at sorted[j]; its row is written at list[j]) when *ordered, or null
    const int32_t* ordered;
    int32_t mask_info[ODIE_MAX_LEVELS];   // level l: its mask plane | bits << 8, or -1
    DevLevel level[ODIE_MAX_LEVELS];
};

// Tuning knobs (set through odie_set_tuning; defaults chosen by measurement).
struct Tuning {
    int forward_chunk = 0;           // forward: coordinates per block (0: 1024 when at least half of
                                     // the table is staged in LDS, so that the staging is amortized, else 256)
    int backward_chunk = 8192;
    int lds_bytes = 65536;
    int xcd_remap = 1;
    int backward_mode = 1;          // 0: LDS + global fp32 atomics, 1: owner computes
    int banded = 2;                 // owner: fine passes walk y-band lists (0 never, 1 always, 2 when they pay)
    int split_target = 0;           // owner, banded: coordinate-level visits per work item (0: automatic)
    int owner_masks = 1;            // owner, unbanded: hashed slices walk only the coordinates whose
                                    // slice mask reaches them (0: every coordinate)
    int packed_owner = 0;           // packed backward: 1 owner computes (deterministic), 0 global atomics
                                    // (measured faster on the 65536-id native steps: 0.30 vs 0.56 ms)
    int packed_splits = 0;          // packed owner: coordinate splits per slice (0: automatic)
    int packed_lds = 1;             // packed backward with atomics: coarse levels accumulated in LDS
    int packed_blocks = 256;        // packed backward with LDS: most blocks (each flushes its partials once)
    int paired_loads = 2;           // forward: 16-byte corner-pair loads (0 off, 1 on, 2: expert tables past 1 MB)
    int forward_lds_bytes = 28672;  // forward: LDS budget for staged coarse levels (0: off)
    int owner_lds_bytes = 162816;   // 160 KiB minus the owner kernel's static 1 KiB (its Adam rate table)
};
Tuning& tuning() {
    static Tuning t;
    return t;
}

// Largest expert e with offsets[e] <= i, clamped to a valid expert.
__device__ inline int expert_at(const GridArgs& a, int64_t i) {
    if (!a.offsets) return 0;
    int lo = 0, hi = a.experts - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.offsets[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// End of the expert segment containing i, clipped to [i+1, end].
__device__ inline int64_t segment_end(const GridArgs& a, int e, int64_t i, int64_t end) {
    if (!a.offsets) return end;
    int64_t stop = a.offsets[e + 1];
    if (stop > end) stop = end;
    if (stop <= i) stop = end;  // malformed offsets: finish the chunk as this expert
    return stop;
}

// First row past every expert: rows from offsets[experts] on (the ids of tiles without an
// expert, as odie_route_allocated leaves them) belong to none -- zero features, no gradient.
__device__ inline int64_t owned_end(const GridArgs& a) {
    if (!a.offsets) return a.n;
    const int64_t last = a.offsets[a.experts];
    return last < 0 ? 0 : (last > a.n ? a.n : last);
}

__device__ inline uint32_t pick4(const uint4& v, uint32_t j) {
    const uint32_t low = (j & 1u) ? v.y : v.x;
    const uint32_t high = (j & 1u) ? v.w : v.z;
    return (j & 2u) ? high : low;
}

// Row `row` of the output from coordinate p (slot i of the walk: row i, or list[i] in band order;
// the masks, written only in slot order, at i).
template <int F, bool HALF, int LMAX>
__device__ inline void encode_row(const GridArgs& a, const DevLevel* levels, const int32_t* mask_info,
                                  const Elem<HALF>* table, __amdgpu_buffer_rsrc_t entries_rsrc,
                                  const uint32_t* staged, int64_t i, float2 p, int64_t row_at) {
    using T = Elem<HALF>;
    T vals[LMAX * F];
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
        if (l < a.n_levels) {
            const DevLevel lv = levels[l];
            uint32_t idx[4];
            float w[4];
            grid_corners(lv, p.x, p.y, idx, w);
            if (a.masks) {
                // the owner backward's slice mask of this level: the aligned blocks of 2^bits
                // entries that the corners land in (the level-local indices it forms itself)
                const int32_t info = __builtin_amdgcn_readfirstlane(mask_info[l]);
                if (info >= 0) {
                    const uint32_t bits = static_cast<uint32_t>(info) >> 8;
                    uint32_t byte = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) byte |= 1u << (idx[k] >> bits);
                    a.masks[static_cast<int64_t>(info & 0xff) * a.mask_stride + i] = static_cast<uint8_t>(byte);
                }
            }
            const T* t = table + static_cast<size_t>(lv.offset) * F;
            if constexpr (HALF && F == 2) {
                // Corners (0,1) and (2,3) usually sit in one aligned 16-byte group of four
                // entries (x and x+1 differ only in their low bits, dense or hashed): fetch
                // the group of the even corner and load the odd corner alone only when it
                // falls outside.  Values and FMA order are unchanged.
                uint32_t g[4];
                if (l < a.stage_levels) {
                    // coarse level staged in LDS by the block
#pragma unroll
                    for (int k = 0; k < 4; ++k) g[k] = staged[lv.offset + idx[k]];
                } else if (!lv.hashed) {
                    // dense: corners (x, y) and (x+1, y) are adjacent entries (but where the index
                    // wraps at the level's end), so one 8-byte load fetches both: two vector
                    // memory instructions per level instead of four.  A raw buffer load over the
                    // expert's table takes the 4-byte aligned offset as one dwordx2 (a global
                    // load at that alignment is split in two).
                    const uint32_t* entries = reinterpret_cast<const uint32_t*>(t);
#pragma unroll
                    for (int k = 0; k < 4; k += 2) {
                        if (idx[k + 1] == idx[k] + 1u) {
                            const auto two =
                                __builtin_amdgcn_raw_buffer_load_b64(entries_rsrc, (lv.offset + idx[k]) * 4u, 0, 0);
                            g[k] = two[0];
                            g[k + 1] = two[1];
                        } else {
                            g[k] = entries[idx[k]];
                            g[k + 1] = entries[idx[k + 1]];
                        }
                    }
                } else if (a.paired) {
                    const uint32_t* entries = reinterpret_cast<const uint32_t*>(table);
#pragma unroll
                    for (int k = 0; k < 4; k += 2) {
                        const uint32_t first = lv.offset + idx[k], second = lv.offset + idx[k + 1];
                        const uint32_t base = first & ~3u;
                        const uint4 group = *reinterpret_cast<const uint4*>(entries + base);
                        g[k] = pick4(group, first & 3u);
                        g[k + 1] = (second & ~3u) == base ? pick4(group, second & 3u) : entries[second];
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) g[k] = reinterpret_cast<const uint32_t*>(t)[idx[k]];
                }
                const uint32_t pair = half2_level(g, w);
                vals[l * F] = bits_to_half(static_cast<uint16_t>(pair & 0xffffu));
                vals[l * F + 1] = bits_to_half(static_cast<uint16_t>(pair >> 16));
            } else if constexpr (HALF && F % 2 == 0) {
                __half2 acc[F / 2];
#pragma unroll
                for (int c = 0; c < F / 2; ++c) acc[c] = __half2(__float2half(0.0f), __float2half(0.0f));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const __half2* src = reinterpret_cast<const __half2*>(t + static_cast<size_t>(idx[k]) * F);
                    const __half2 wk = __float2half2_rn(keep_fp32(w[k]));
#pragma unroll
                    for (int c = 0; c < F / 2; ++c) acc[c] = __hfma2(wk, src[c], acc[c]);
                }
#pragma unroll
                for (int c = 0; c < F / 2; ++c) {
                    vals[l * F + 2 * c] = __low2half(acc[c]);
                    vals[l * F + 2 * c + 1] = __high2half(acc[c]);
                }
            } else if constexpr (HALF) {
                __half acc = __float2half(0.0f);
#pragma unroll
                for (int k = 0; k < 4; ++k) acc = __hfma(__float2half_rn(keep_fp32(w[k])), t[idx[k]], acc);
                vals[l] = acc;
            } else {
                float acc[F];
#pragma unroll
                for (int c = 0; c < F; ++c) acc[c] = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float* src = t + static_cast<size_t>(idx[k]) * F;
#pragma unroll
                    for (int c = 0; c < F; ++c) acc[c] = __builtin_fmaf(w[k], src[c], acc[c]);
                }
#pragma unroll
                for (int c = 0; c < F; ++c) vals[l * F + c] = acc[c];
            }
        } else {
#pragma unroll
            for (int c = 0; c < F; ++c) vals[l * F + c] = T(0.0f);
        }
    }
    T* row = reinterpret_cast<T*>(a.out) + static_cast<size_t>(row_at) * a.width;
    const int used = a.n_levels * F;
    if (a.vec_rows && (used * static_cast<int>(sizeof(T))) % 16 == 0) {
        constexpr int kPer = 16 / sizeof(T);
        constexpr int kChunks = (LMAX * F + kPer - 1) / kPer;
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            if (j * kPer < used) {
                uint32_t words[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if constexpr (HALF) {
                        const int e0 = j * kPer + 2 * q;
                        const uint32_t lo = e0 < LMAX * F ? half_to_bits(vals[e0]) : 0u;
                        const uint32_t hi = e0 + 1 < LMAX * F ? half_to_bits(vals[e0 + 1]) : 0u;
                        words[q] = lo | (hi << 16);
                    } else {
                        const int e0 = j * kPer + q;
                        words[q] = e0 < LMAX * F ? __float_as_uint(vals[e0]) : 0u;
                    }
                }
                reinterpret_cast<uint4*>(row)[j] = make_uint4(words[0], words[1], words[2], words[3]);
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < LMAX * F; ++c)
            if (c < used) row[c] = vals[c];
    }
    for (int c = used; c < a.width; ++c) row[c] = T(0.0f);
}

template <int F, bool HALF, int LMAX>
__global__ __launch_bounds__(kBlock) void grid_forward_kernel(GridArgs a) {
    // The level descriptors are read from an LDS copy: taken from the kernel arguments, sixteen
    // levels' descriptors would be held in scalar registers across the whole unrolled row and
    // spilled, and every basic block of the row would reload them lane by lane.
    __shared__ DevLevel levels[LMAX];
    __shared__ int32_t mask_info[LMAX];
    constexpr int kLevelWords = LMAX * static_cast<int>(sizeof(DevLevel) / 4);
    static_assert(kLevelWords <= kBlock, "one thread per descriptor word");
    if (static_cast<int>(threadIdx.x) < kLevelWords)
        reinterpret_cast<uint32_t*>(levels)[threadIdx.x] = reinterpret_cast<const uint32_t*>(a.level)[threadIdx.x];
    if (static_cast<int>(threadIdx.x) < LMAX) mask_info[threadIdx.x] = a.mask_info[threadIdx.x];
    __syncthreads();
    const uint32_t block = a.remap ? xcd_major(blockIdx.x, gridDim.x) : blockIdx.x;
    int64_t begin = static_cast<int64_t>(block) * a.chunk;
    if (begin >= a.n) return;
    int64_t end = begin + a.chunk < a.n ? begin + a.chunk : a.n;
    extern __shared__ uint32_t staged[];
    // band order when the lists are exact and cover every owned position: expert ranges in order
    // from position 0 (each expert's list positions are then its own range, so a position's
    // expert is the same either way)
    const bool by_list = a.list && *a.ordered && (!a.offsets || a.offsets[0] <= 0);
    const int64_t owned = owned_end(a);
    for (int64_t i = (begin > owned ? begin : owned) + threadIdx.x; i < end; i += kBlock) {
        Elem<HALF>* row = reinterpret_cast<Elem<HALF>*>(a.out) + static_cast<size_t>(i) * a.width;
        for (int c = 0; c < a.width; ++c) row[c] = Elem<HALF>(0.0f);
    }
    if (owned < end) {
        if (owned <= begin) return;
        end = owned;
    }
    while (begin < end) {
        const int e = expert_at(a, begin);
        const int64_t stop = segment_end(a, e, begin, end);
        const Elem<HALF>* table = reinterpret_cast<const Elem<HALF>*>(a.params) + static_cast<size_t>(e) * a.expert_params;
        // the expert's table as a raw buffer (scalar registers; out-of-range offsets read 0).
        // readfirstlane returns an int: each half goes back through uint32_t, so that the low
        // half is not sign-extended over the high one when bit 31 of the address is set.
        const uint64_t at = reinterpret_cast<uint64_t>(table);
        const uint32_t at_hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(at >> 32)));
        const uint32_t at_lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(at)));
        const uint64_t base = (static_cast<uint64_t>(at_hi) << 32) | at_lo;
        const uint64_t bytes = static_cast<uint64_t>(a.expert_params) * sizeof(Elem<HALF>);
        const __amdgpu_buffer_rsrc_t entries_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void*>(base), 0, static_cast<int>(bytes < 0xffffffffull ? bytes : 0xffffffffull),
            kRawBufferWord3);
        if (a.stage_levels > 0) {
            // Stage the expert's coarse levels (fp16 x2 entries as dwords) in LDS.
            __syncthreads();
            const uint4* src = reinterpret_cast<const uint4*>(table);
            for (int j = threadIdx.x; j < a.stage_entries / 4; j += kBlock) reinterpret_cast<uint4*>(staged)[j] = src[j];
            __syncthreads();
        }
        for (int64_t i = begin + threadIdx.x; i < stop; i += kBlock) {
            const float2 p = by_list ? a.sorted[i] : reinterpret_cast<const float2*>(a.coords)[i];
            const int64_t row_at = by_list ? static_cast<int64_t>(a.list[i]) : i;
            if (row_at < 0 || row_at >= a.n) continue;   // (a list entry is always a coordinate index)
            encode_row<F, HALF, LMAX>(a, levels, mask_info, table, entries_rsrc, staged, i, p, row_at);
        }
        begin = stop;
    }
}

template <int F, bool HALF_UP, int LMAX>
__global__ __launch_bounds__(kBlock) void grid_backward_kernel(GridArgs a) {
    extern __shared__ float lds[];
    using U = Elem<HALF_UP>;
    const uint32_t block = a.remap ? xcd_major(blockIdx.x, gridDim.x) : blockIdx.x;
    int64_t begin = static_cast<int64_t>(block) * a.chunk;
    if (begin >= a.n) return;
    int64_t end = begin + a.chunk < a.n ? begin + a.chunk : a.n;
    const int used = a.n_levels * F;
    const int64_t owned = owned_end(a);
    if (owned <= begin) return;
    if (owned < end) end = owned;
    while (begin < end) {
        const int e = expert_at(a, begin);
        const int64_t stop = segment_end(a, e, begin, end);
        float* grad = a.grad + static_cast<size_t>(e) * a.expert_params;
        if (a.lds_levels > 0) {
            for (int j = threadIdx.x; j < a.lds_floats; j += kBlock) lds[j] = 0.0f;
            __syncthreads();
        }
        for (int64_t i = begin + threadIdx.x; i < stop; i += kBlock) {
            const U* urow = reinterpret_cast<const U*>(a.upstream) + static_cast<size_t>(i) * a.width;
            float up[LMAX * F];
            if (a.vec_rows && (used * static_cast<int>(sizeof(U))) % 16 == 0) {
                constexpr int kPer = 16 / sizeof(U);
                constexpr int kChunks = (LMAX * F + kPer - 1) / kPer;
#pragma unroll
                for (int j = 0; j < kChunks; ++j) {
                    if (j * kPer < used) {
                        const uint4 v = reinterpret_cast<const uint4*>(urow)[j];
                        const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            if constexpr (HALF_UP) {
                                const int e0 = j * kPer + 2 * q;
                                if (e0 < LMAX * F) up[e0] = __half2float(bits_to_half(static_cast<uint16_t>(words[q] & 0xffffu)));
                                if (e0 + 1 < LMAX * F) up[e0 + 1] = __half2float(bits_to_half(static_cast<uint16_t>(words[q] >> 16)));
                            } else {
                                const int e0 = j * kPer + q;
                                if (e0 < LMAX * F) up[e0] = __uint_as_float(words[q]);
                            }
                        }
                    }
                }
            } else {
#pragma unroll
                for (int c = 0; c < LMAX * F; ++c) up[c] = c < used ? static_cast<float>(urow[c]) : 0.0f;
            }
            const float2 p = reinterpret_cast<const float2*>(a.coords)[i];
#pragma unroll
            for (int l = 0; l < LMAX; ++l) {
                if (l < a.n_levels) {
                    const DevLevel& lv = a.level[l];
                    uint32_t idx[4];
                    float w[4];
                    grid_corners(lv, p.x, p.y, idx, w);
                    const bool local = l < a.lds_levels;
                    float* base = local ? lds : grad;
#pragma unroll
                    for (int c = 0; c < F; ++c) {
                        const float value = up[l * F + c];
                        if (value == 0.0f) continue;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            float* target = base + (static_cast<size_t>(lv.offset) + idx[k]) * F + c;
                            atomicAdd(target, w[k] * value);
                        }
                    }
                }
            }
        }
        if (a.lds_levels > 0) {
            __syncthreads();
            for (int j = threadIdx.x; j < a.lds_floats; j += kBlock) {
                const float v = lds[j];
                if (v != 0.0f) atomicAdd(grad + j, v);
            }
            __syncthreads();
        }
        begin = stop;
    }
}

// Clears `count` floats (a fill kernel rather than hipMemsetAsync so that the backward can
// be captured in a graph).
__global__ __launch_bounds__(kBlock) void fill_zero_kernel(float* data, int64_t count) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * 4;
    for (int64_t i = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 4; i < count; i += stride) {
        if (i + 4 <= count && (reinterpret_cast<uintptr_t>(data + i) & 15) == 0) {
            *reinterpret_cast<float4*>(data + i) = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            for (int64_t j = i; j < i + 4 && j < count; ++j) data[j] = 0.0f;
        }
    }
}

int validate_grid(const char* what, const float* coords, int64_t n, const int32_t* offsets, int experts,
                  int64_t expert_params, const odie_grid_level* levels, int n_levels, int features,
                  GridArgs& a) {
    const std::string w(what);
    if (n < 0 || n > (int64_t{1} << 31) - 1) return fail(w + ": n must be within [0, 2^31-1]");
    if (n > 0 && !coords) return fail(w + ": coords is null");
    if (experts < 1) return fail(w + ": experts must be >= 1");
    if (experts > 1 && !offsets) return fail(w + ": offsets are required when experts > 1");
    if (!levels) return fail(w + ": levels is null");
    if (n_levels < 1 || n_levels > ODIE_MAX_LEVELS) return fail(w + ": n_levels must be within 1..32");
    if (features != 1 && features != 2 && features != 4 && features != 8)
        return fail(w + ": features per level must be 1, 2, 4 or 8");
    uint64_t entries = 0;
    if (make_dev_levels(what, levels, n_levels, a.level, entries)) return -1;
    if (expert_params < static_cast<int64_t>(entries) * features)
        return fail(w + ": expert_params is smaller than the levels' table");
    a.coords = coords;
    a.offsets = experts > 1 ? offsets : nullptr;
    a.n = n;
    a.expert_params = expert_params;
    a.experts = experts;
    a.n_levels = n_levels;
    return 0;
}

#define ODIE_GRID_DISPATCH(KERNEL, F, HALF, LMAX, GRID, SHMEM, STREAM, ARGS)                              \
    do {                                                                                                  \
        if (LMAX <= 16) {                                                                                 \
            switch (F) {                                                                                  \
                case 1: if (HALF) KERNEL<1, true, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);             \
                        else KERNEL<1, false, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
                case 2: if (HALF) KERNEL<2, true, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);             \
                        else KERNEL<2, false, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
                case 4: if (HALF) KERNEL<4, true, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);             \
                        else KERNEL<4, false, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
                default: if (HALF) KERNEL<8, true, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);            \
                        else KERNEL<8, false, 16><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
            }                                                                                             \
        } else {                                                                                          \
            switch (F) {                                                                                  \
                case 1: if (HALF) KERNEL<1, true, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);             \
                        else KERNEL<1, false, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
                case 2: if (HALF) KERNEL<2, true, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);             \
                        else KERNEL<2, false, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
                case 4: if (HALF) KERNEL<4, true, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);             \
                        else KERNEL<4, false, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
                default: if (HALF) KERNEL<8, true, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS);            \
                        else KERNEL<8, false, 32><<<GRID, kBlock, SHMEM, STREAM>>>(ARGS); break;          \
            }                                                                                             \
        }                                                                                                 \
    } while (0)

uint32_t grid_blocks(int64_t n, int chunk) {
    const uint64_t blocks = (static_cast<uint64_t>(n) + chunk - 1) / chunk;
    return round_up(static_cast<uint32_t>(blocks), kXcds);
}

// ---------------------------------------------------------------------------------------
// Packed xy planes (odie/packed_kernels.cu:12-88 semantics).
// ---------------------------------------------------------------------------------------

struct PackedArgs {
    const float* coords;
    const float* grid;
    const int32_t* desc;
    const uint64_t* node_bitmap;
    const int32_t* prefix;
    const uint8_t* bitmap;
    const uint16_t* upstream;
    uint16_t* features;
    uint8_t* visibility;
    float* gradient;
    int64_t n;
    int64_t params;
    int levels;
    int width;
    int active;          // levels >= active are off (the native step's active prefix)
    uint16_t pad;        // fp16 bits written to columns past the last level
};

__device__ inline int64_t plane_param(const PackedArgs& a, const int32_t* d, int cell, int k, int c) {
    return packed_param(d, a.node_bitmap, a.prefix, a.params, cell, k, c);
}

__global__ __launch_bounds__(kBlock) void packed_forward_kernel(PackedArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= a.n) return;
    const float2 p = reinterpret_cast<const float2*>(a.coords)[i];
    uint16_t* row = a.features + static_cast<size_t>(i) * a.width;
    int written = 0;
    uint32_t vis[ODIE_MAX_LEVELS / 4];
#pragma unroll
    for (int q = 0; q < ODIE_MAX_LEVELS / 4; ++q) vis[q] = 0;
#pragma unroll
    for (int l = 0; l < ODIE_MAX_LEVELS; ++l) {
        if (l < a.levels) {
            const int32_t* d = a.desc + 8 * l;
            int cell;
            float w[4];
            plane_geometry(p.x, p.y, d[0], cell, w);
            const bool on = l < a.active && ((a.bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1);
            vis[l / 4] |= static_cast<uint32_t>(on) << (8 * (l % 4));
            int rows[4] = {0, 0, 0, 0};
            if (on) {
#pragma unroll
                for (int k = 0; k < 4; ++k) rows[k] = packed_row(d, a.node_bitmap, a.prefix, cell, k);
            }
            for (int c = 0; c < d[5]; ++c) {
                __half v = __float2half(0.0f);
                if (on) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        v = __hfma(__float2half_rn(keep_fp32(w[k])),
                                   __float2half_rn(a.grid[packed_at(d, a.params, rows[k], c)]), v);
                }
                row[d[6] + c] = half_to_bits(v);
            }
            const int top = d[6] + d[5];
            written = top > written ? top : written;
        }
    }
    for (int c = written; c < a.width; ++c) row[c] = a.pad;
    uint8_t* vrow = a.visibility + static_cast<size_t>(i) * a.levels;
#pragma unroll
    for (int l = 0; l < ODIE_MAX_LEVELS; ++l)
        if (l < a.levels) vrow[l] = static_cast<uint8_t>(vis[l / 4] >> (8 * (l % 4)));
}

// packed_forward_kernel for 16 levels of 2 features in level order (width 32): both features of
// a corner in one 8-byte load, the row kept in registers and written with 16-byte stores, the
// visibility bytes with one.  Same arithmetic, same bits.
__global__ __launch_bounds__(kBlock) void packed_forward16x2_kernel(PackedArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= a.n) return;
    const float2 p = reinterpret_cast<const float2*>(a.coords)[i];
    uint32_t pairs[16];
    uint32_t vis[4] = {0, 0, 0, 0};
#pragma unroll
    for (int l = 0; l < 16; ++l) {
        const int32_t* d = a.desc + 8 * l;
        int cell;
        float w[4];
        plane_geometry(p.x, p.y, d[0], cell, w);
        const bool on = l < a.active && ((a.bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1);
        vis[l / 4] |= static_cast<uint32_t>(on) << (8 * (l % 4));
        __half v0 = __float2half(0.0f), v1 = __float2half(0.0f);
        if (on) {
            float2 g[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t at = plane_param(a, d, cell, k, 0);   // even: both features are inside
                g[k] = *reinterpret_cast<const float2*>(a.grid + (at < a.params - 1 ? at : a.params - 2));
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const __half wk = __float2half_rn(keep_fp32(w[k]));
                v0 = __hfma(wk, __float2half_rn(g[k].x), v0);
                v1 = __hfma(wk, __float2half_rn(g[k].y), v1);
            }
        }
        pairs[l] = static_cast<uint32_t>(half_to_bits(v0)) | (static_cast<uint32_t>(half_to_bits(v1)) << 16);
    }
    uint4* row = reinterpret_cast<uint4*>(a.features + static_cast<size_t>(i) * 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) row[j] = make_uint4(pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2], pairs[4 * j + 3]);
    reinterpret_cast<uint4*>(a.visibility)[i] = make_uint4(vis[0], vis[1], vis[2], vis[3]);
}

// packed_forward_kernel for rows of fp16 pairs: every level 2 features at output offset 2l but the
// last, which may hold one (the reference's F2 layouts with an F1 finest level, rows of align16
// of the features, PAIRS = width / 2).  The row is kept in registers and written with 16-byte
// stores, the visibility bytes in 4-byte words where they fall on word boundaries.  Same
// arithmetic, same bits.
template <int PAIRS>
__global__ __launch_bounds__(kBlock) void packed_forward_pairs_kernel(PackedArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= a.n) return;
    const float2 p = reinterpret_cast<const float2*>(a.coords)[i];
    const uint32_t pad = a.pad;
    uint32_t pairs[PAIRS];
    uint32_t vis[PAIRS / 4];
#pragma unroll
    for (int q = 0; q < PAIRS / 4; ++q) vis[q] = 0;
#pragma unroll
    for (int l = 0; l < PAIRS; ++l) {
        pairs[l] = pad | (pad << 16);
        if (l < a.levels) {
            const int32_t* d = a.desc + 8 * l;
            int cell;
            float w[4];
            plane_geometry(p.x, p.y, d[0], cell, w);
            const bool on = l < a.active && ((a.bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1);
            vis[l / 4] |= static_cast<uint32_t>(on) << (8 * (l % 4));
            const bool two = d[5] == 2;
            __half v0 = __float2half(0.0f), v1 = __float2half(0.0f);
            if (on) {
                float2 g[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int64_t at = plane_param(a, d, cell, k, 0);
                    if (two) {
                        // even, both features inside; a clamped index (descriptors out of step with
                        // the bitmaps) stays an aligned pair inside the grid (params is a multiple of 8)
                        g[k] = *reinterpret_cast<const float2*>(a.grid + (at < a.params - 1 ? at : a.params - 2));
                    } else {
                        g[k].x = a.grid[at];
                        g[k].y = 0.0f;
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const __half wk = __float2half_rn(keep_fp32(w[k]));
                    v0 = __hfma(wk, __float2half_rn(g[k].x), v0);
                    v1 = __hfma(wk, __float2half_rn(g[k].y), v1);
                }
            }
            pairs[l] = static_cast<uint32_t>(half_to_bits(v0)) |
                       ((two ? static_cast<uint32_t>(half_to_bits(v1)) : pad) << 16);
        }
    }
    uint4* row = reinterpret_cast<uint4*>(a.features + static_cast<size_t>(i) * (2 * PAIRS));
#pragma unroll
    for (int j = 0; j < PAIRS / 4; ++j) row[j] = make_uint4(pairs[4 * j], pairs[4 * j + 1], pairs[4 * j + 2], pairs[4 * j + 3]);
    uint8_t* vrow = a.visibility + static_cast<size_t>(i) * a.levels;
    if (a.levels % 4 == 0) {
#pragma unroll
        for (int q = 0; q < PAIRS / 4; ++q)
            if (4 * q < a.levels) reinterpret_cast<uint32_t*>(vrow)[q] = vis[q];
    } else {
#pragma unroll
        for (int l = 0; l < PAIRS; ++l)
            if (l < a.levels) vrow[l] = static_cast<uint8_t>(vis[l / 4] >> (8 * (l % 4)));
    }
}

__global__ __launch_bounds__(kBlock) void packed_backward_kernel(PackedArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= a.n) return;
    const float2 p = reinterpret_cast<const float2*>(a.coords)[i];
    const uint16_t* urow = a.upstream + static_cast<size_t>(i) * a.width;
    for (int l = 0; l < a.levels; ++l) {
        const int32_t* d = a.desc + 8 * l;
        int cell;
        float w[4];
        plane_geometry(p.x, p.y, d[0], cell, w);
        if (!((a.bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1)) continue;
        int rows[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) rows[k] = packed_row(d, a.node_bitmap, a.prefix, cell, k);
        for (int c = 0; c < d[5]; ++c) {
            const int col = d[6] + c;
            if (col >= a.width) continue;
            const float value = __half2float(bits_to_half(urow[col]));
            if (value == 0.0f) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) atomicAdd(a.gradient + packed_at(d, a.params, rows[k], c), w[k] * value);
        }
    }
}

// Packed backward with the coarse levels accumulated in LDS: the levels whose parameters lie in
// the first lds_floats values (found from the descriptors' plane offsets) take LDS atomics, and
// the block adds its partial sums to the gradient once at the end; the finer, sparsely updated
// levels take global atomics directly.  A block walks a contiguous chunk of coordinates.
constexpr int kPackedLdsFloats = 16384;

__global__ __launch_bounds__(kBlock) void packed_backward_lds_kernel(PackedArgs a, int64_t chunk) {
    __shared__ float lds[kPackedLdsFloats];
    // coarse levels: the longest prefix of levels that ends within the LDS budget
    int lds_levels = 0;
    while (lds_levels + 1 < a.levels && a.desc[8 * (lds_levels + 1) + 2] <= kPackedLdsFloats &&
           a.desc[8 * (lds_levels + 1) + 2] >= 0)
        ++lds_levels;
    const int lds_floats = lds_levels > 0 ? a.desc[8 * lds_levels + 2] : 0;
    for (int j = threadIdx.x; j < lds_floats; j += kBlock) lds[j] = 0.0f;
    __syncthreads();
    const int64_t b0 = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t b1 = b0 + chunk < a.n ? b0 + chunk : a.n;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kBlock) {
        const float2 p = reinterpret_cast<const float2*>(a.coords)[i];
        const uint16_t* urow = a.upstream + static_cast<size_t>(i) * a.width;
        for (int l = 0; l < a.levels; ++l) {
            const int32_t* d = a.desc + 8 * l;
            int cell;
            float w[4];
            plane_geometry(p.x, p.y, d[0], cell, w);
            if (!((a.bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1)) continue;
            // the corners' rows once for all features of the level
            int rows[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) rows[k] = packed_row(d, a.node_bitmap, a.prefix, cell, k);
            for (int c = 0; c < d[5]; ++c) {
                const int col = d[6] + c;
                if (col >= a.width) continue;
                const float value = __half2float(bits_to_half(urow[col]));
                if (value == 0.0f) continue;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int64_t param = packed_at(d, a.params, rows[k], c);
                    if (l < lds_levels && param < lds_floats) atomicAdd(lds + param, w[k] * value);
                    else atomicAdd(a.gradient + param, w[k] * value);
                }
            }
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < lds_floats; j += kBlock)
        if (lds[j] != 0.0f) atomicAdd(a.gradient + j, lds[j]);
}

}  // namespace

int launch_fill_zero(float* data, int64_t count, hipStream_t stream) {
    if (count <= 0) return 0;
    int64_t blocks = (count + 4 * kBlock - 1) / (4 * kBlock);
    if (blocks > 8192) blocks = 8192;
    fill_zero_kernel<<<static_cast<uint32_t>(blocks), kBlock, 0, stream>>>(data, count);
    return check_launch("fill_zero");
}

int set_grid_tuning(const std::string& key, int value) {
    Tuning& t = tuning();
    if (key == "forward_chunk" && value >= 0 && value % kBlock == 0) t.forward_chunk = value;
    else if (key == "backward_chunk" && value >= kBlock && value % kBlock == 0) t.backward_chunk = value;
    else if (key == "lds_bytes" && value >= 0 && value <= 160 * 1024) t.lds_bytes = value;
    else if (key == "xcd_remap" && (value == 0 || value == 1)) t.xcd_remap = value;
    else if (key == "backward_mode" && (value == 0 || value == 1)) t.backward_mode = value;
    else if (key == "banded" && value >= 0 && value <= 2) t.banded = value;
    else if (key == "owner_masks" && (value == 0 || value == 1)) t.owner_masks = value;
    else if (key == "split_target" && value >= 0) t.split_target = value;
    else if (key == "packed_owner" && (value == 0 || value == 1)) t.packed_owner = value;
    else if (key == "packed_splits" && value >= 0 && value <= 64) t.packed_splits = value;
    else if (key == "packed_lds" && (value == 0 || value == 1)) t.packed_lds = value;
    else if (key == "packed_blocks" && value >= 1 && value <= 65536) t.packed_blocks = value;
    else if (key == "paired_loads" && value >= 0 && value <= 2) t.paired_loads = value;
    else if (key == "forward_lds_bytes" && value >= 0 && value <= 65536) t.forward_lds_bytes = value;
    else if (key == "owner_lds_bytes" && value >= 4096 && value <= 162816) t.owner_lds_bytes = value;
    else return fail("odie_set_tuning: unknown key or value out of range: " + key);
    return 0;
}

}  // namespace odie

using namespace odie;

namespace {

// The owner backward's launch for this grid and batch under the current tuning, as far as its
// planning reads it.
OwnerLaunch planning_launch(const float* coords, int64_t n, const int32_t* offsets, int experts, int64_t expert_params,
                            const GridArgs& a, int n_levels, int features, hipStream_t stream) {
    const Tuning& t = tuning();
    OwnerLaunch o{};
    o.coords = coords;
    o.offsets = offsets;
    o.stream = stream;
    o.n = n;
    o.experts = experts;
    o.expert_params = expert_params;
    o.n_levels = n_levels;
    o.features = features;
    o.levels = a.level;
    o.lds_bytes = t.owner_lds_bytes;
    o.remap = t.xcd_remap;
    o.banded = t.banded;
    o.masks = t.owner_masks;
    o.split_target = t.split_target;
    o.up_half = 1;
    o.up_width = n_levels * features;
    return o;
}

// The handoff plan of the owner backward for this grid and batch (its own planning, asked for
// the plan alone).
int handoff_plan(int64_t n, int experts, int64_t expert_params, const GridArgs& a, int n_levels, int features,
                 HandoffPlan& plan) {
    OwnerLaunch o = planning_launch(nullptr, n, nullptr, experts, expert_params, a, n_levels, features, nullptr);
    o.plan_out = &plan;
    return launch_owner_backward(o);
}

// odie_grid_forward, filling the owner backward's handoff on the way when `handoff` is non-null
// (handoff_bytes long, at least odie_grid_handoff_bytes): the slice masks, written by the
// forward kernel, or the band lists, built first and then walked by the forward kernel.
int grid_forward(const char* who, const float* coords, int64_t n, const int32_t* offsets, int experts,
                 const void* params, int64_t expert_params, int param_dtype, const odie_grid_level* levels,
                 int n_levels, int features, void* out, int out_width, uint8_t* handoff, int64_t handoff_bytes,
                 uint64_t stream) {
    GridArgs a{};
    if (validate_grid(who, coords, n, offsets, experts, expert_params, levels, n_levels, features, a))
        return -1;
    for (int l = 0; l < ODIE_MAX_LEVELS; ++l) a.mask_info[l] = -1;
    HandoffPlan plan{};
    if (handoff && n > 0) {
        if (handoff_plan(n, experts, expert_params, a, n_levels, features, plan)) return -1;
        if (plan.bytes > 0 && handoff_bytes < plan.bytes)
            return fail(std::string(who) + ": handoff is shorter than odie_grid_handoff_bytes");
        if (plan.planes > 0) {
            a.masks = handoff;
            a.mask_stride = plan.stride;
            for (int p = 0; p < plan.planes; ++p) a.mask_info[plan.level[p]] = p | (plan.bits[p] << 8);
        }
    }
    const std::string w(who);
    if (param_dtype != ODIE_F32 && param_dtype != ODIE_F16) return fail(w + ": param_dtype must be 0 (fp32) or 1 (fp16)");
    if (out_width < n_levels * features) return fail(w + ": out_width is smaller than n_levels*features");
    if (n == 0) return 0;
    if (!params || !out) return fail(w + ": params and out must be non-null");
    const bool half = param_dtype == ODIE_F16;
    const size_t elem = half ? 2 : 4;
    a.params = params;
    a.out = out;
    a.width = out_width;
    a.chunk = tuning().forward_chunk;
    a.remap = tuning().xcd_remap;
    {
        const uint64_t entries = static_cast<uint64_t>(levels[n_levels - 1].offset) + levels[n_levels - 1].size;
        // Corner pairs from one 16-byte group load: one request for corners (x, y) and (x+1, y)
        // instead of two.  Measured: one expert of 2^19-entry levels (11 MB) 0.611 -> 0.581 ms;
        // 64 experts of 2^16-entry levels (2.2 MB each) 0.462 -> 0.453 ms; 1024 experts of
        // 32 KB tables 3.49 -> 3.52 ms per stratified gigapixel step (small tables: mostly dense
        // levels, which fetch their pairs with 8-byte loads either way).  So pairs from 1 MB up.
        const int mode = tuning().paired_loads;
        const bool past_l2 = expert_params * 2 > (int64_t{1} << 20);
        a.paired = (mode == 1 || (mode == 2 && past_l2)) && half && features == 2 &&
                   reinterpret_cast<uintptr_t>(params) % 16 == 0 && entries % 4 == 0 && (expert_params * 2) % 16 == 0;
        // Stage the longest prefix of levels that fits the budget (entries of 4 bytes).
        if (half && features == 2 && reinterpret_cast<uintptr_t>(params) % 16 == 0 && (expert_params * 2) % 16 == 0) {
            int64_t staged = 0;
            for (int l = 0; l < n_levels; ++l) {
                const int64_t next = static_cast<int64_t>(levels[l].offset) + levels[l].size;
                if (next * 4 > tuning().forward_lds_bytes || next % 4) break;
                a.stage_levels = l + 1;
                staged = next;
            }
            a.stage_entries = static_cast<int>(staged);
        }
    }
    if (a.chunk == 0) {
        // Each block copies the staged levels into LDS once: with most of a small table staged
        // (the 1024-expert gigapixel grid: 28 of its 32 KB) that copy dominates 256 rows; with a
        // large table (2.2 MB at the 64-expert headline) the other levels' gathers go through L2,
        // where 256-row blocks measured faster.
        const int64_t entries = static_cast<int64_t>(levels[n_levels - 1].offset) + levels[n_levels - 1].size;
        a.chunk = 2 * static_cast<int64_t>(a.stage_entries) >= entries ? 1024 : 256;
    }
    a.vec_rows = (reinterpret_cast<uintptr_t>(out) % 16 == 0) && (out_width * elem) % 16 == 0;
    if (reinterpret_cast<uintptr_t>(coords) % 8) return fail(w + ": coords must be 8-byte aligned");
    const uint32_t blocks = grid_blocks(n, a.chunk);
    const hipStream_t s = as_stream(stream);
    if (plan.lists) {
        const OwnerLaunch o = planning_launch(coords, n, a.offsets, experts, expert_params, a, n_levels, features, s);
        if (launch_band_lists(o, plan, handoff)) return -1;
        a.list = reinterpret_cast<const int32_t*>(handoff + plan.list_at);
        a.sorted = reinterpret_cast<const float2*>(handoff + plan.sorted_at);
        a.ordered = reinterpret_cast<const int32_t*>(handoff + plan.ordered_at);
    }
    ODIE_GRID_DISPATCH(grid_forward_kernel, features, half, n_levels, blocks,
                       static_cast<size_t>(a.stage_entries) * 4, s, a);
    return check_launch(who);
}

}  // namespace

ODIE_API int odie_grid_forward(const float* coords, int64_t n, const int32_t* offsets, int experts,
                               const void* params, int64_t expert_params, int param_dtype,
                               const odie_grid_level* levels, int n_levels, int features,
                               void* out, int out_width, uint64_t stream) {
    return grid_forward("odie_grid_forward", coords, n, offsets, experts, params, expert_params, param_dtype, levels,
                        n_levels, features, out, out_width, nullptr, 0, stream);
}

ODIE_API int64_t odie_grid_handoff_bytes(int64_t n, int experts, int64_t expert_params,
                                         const odie_grid_level* levels, int n_levels, int features) {
    const std::string w("odie_grid_handoff_bytes");
    if (n < 0 || n > (int64_t{1} << 31) - 1) return fail(w + ": n must be within [0, 2^31-1]");
    if (experts < 1) return fail(w + ": experts must be >= 1");
    if (!levels) return fail(w + ": levels is null");
    if (n_levels < 1 || n_levels > ODIE_MAX_LEVELS) return fail(w + ": n_levels must be within 1..32");
    if (features != 1 && features != 2 && features != 4 && features != 8)
        return fail(w + ": features per level must be 1, 2, 4 or 8");
    GridArgs a{};
    uint64_t entries = 0;
    if (make_dev_levels("odie_grid_handoff_bytes", levels, n_levels, a.level, entries)) return -1;
    if (expert_params < static_cast<int64_t>(entries) * features)
        return fail(w + ": expert_params is smaller than the levels' table");
    if (n == 0) return 0;
    HandoffPlan plan;
    if (handoff_plan(n, experts, expert_params, a, n_levels, features, plan)) return -1;
    return plan.bytes;
}

ODIE_API int odie_grid_forward_handoff(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                       const void* params, int64_t expert_params, int param_dtype,
                                       const odie_grid_level* levels, int n_levels, int features, void* out,
                                       int out_width, void* handoff, int64_t handoff_bytes, uint64_t stream) {
    if (n > 0 && !handoff && handoff_bytes > 0) return fail("odie_grid_forward_handoff: handoff is null");
    return grid_forward("odie_grid_forward_handoff", coords, n, offsets, experts, params, expert_params, param_dtype,
                        levels, n_levels, features, out, out_width, static_cast<uint8_t*>(handoff), handoff_bytes,
                        stream);
}

namespace {

// odie_grid_backward, reading the forward's handoff (odie_grid_forward_handoff) when non-null.
int grid_backward(const float* coords, int64_t n, const int32_t* offsets, int experts, const void* upstream,
                  int up_dtype, int up_width, int64_t expert_params, const odie_grid_level* levels, int n_levels,
                  int features, float* gradient, int zero_first, const uint8_t* handoff, int64_t handoff_bytes,
                  uint64_t stream) {
    GridArgs a{};
    if (validate_grid("odie_grid_backward", coords, n, offsets, experts, expert_params, levels, n_levels, features, a))
        return -1;
    if (up_dtype != ODIE_F32 && up_dtype != ODIE_F16) return fail("odie_grid_backward: up_dtype must be 0 (fp32) or 1 (fp16)");
    if (up_width < n_levels * features) return fail("odie_grid_backward: up_width is smaller than n_levels*features");
    if (!gradient) return fail("odie_grid_backward: gradient is null");
    if (n > 0 && !upstream) return fail("odie_grid_backward: upstream is null");
    if (reinterpret_cast<uintptr_t>(coords) % 8) return fail("odie_grid_backward: coords must be 8-byte aligned");
    const hipStream_t s = as_stream(stream);
    const int64_t total = expert_params * experts;
    const Tuning& t = tuning();
    if (static_cast<int64_t>(a.level[n_levels - 1].offset + a.level[n_levels - 1].size) * features >= (int64_t{1} << 31))
        return fail("odie_grid_backward: one table must hold fewer than 2^31 values");
    if (n == 0) return zero_first ? launch_fill_zero(gradient, total, s) : 0;
    if (t.backward_mode == 1) {
        if (expert_params != static_cast<int64_t>(a.level[n_levels - 1].offset + a.level[n_levels - 1].size) * features) {
            // values past the levels' tables are not owned by any slice: clear them up front
            if (zero_first && launch_fill_zero(gradient, total, s)) return -1;
            zero_first = 0;
        }
        OwnerLaunch o{};
        o.coords = coords;
        o.offsets = a.offsets;
        o.upstream = upstream;
        o.up_half = up_dtype == ODIE_F16;
        o.up_width = up_width;
        o.grad = gradient;
        o.accumulate = zero_first ? 0 : 1;
        o.n = n;
        o.expert_params = expert_params;
        o.experts = experts;
        o.n_levels = n_levels;
        o.features = features;
        o.levels = a.level;
        o.lds_bytes = t.owner_lds_bytes;
        o.remap = t.xcd_remap;
        o.banded = t.banded;
        o.masks = t.owner_masks;
        o.split_target = t.split_target;
        o.stream = s;
        o.handoff = handoff;
        o.handoff_bytes = handoff_bytes;
        return launch_owner_backward(o);
    }
    if (zero_first && launch_fill_zero(gradient, total, s)) return -1;
    const bool half = up_dtype == ODIE_F16;
    const size_t elem = half ? 2 : 4;
    a.upstream = upstream;
    a.grad = gradient;
    a.width = up_width;
    a.chunk = t.backward_chunk;
    a.remap = t.xcd_remap;
    a.vec_rows = (reinterpret_cast<uintptr_t>(upstream) % 16 == 0) && (up_width * elem) % 16 == 0;
    // Coarse levels whose table is small next to the chunk's corner count are accumulated
    // in LDS: the flush costs one atomic per entry instead of one per corner.
    int lds_levels = 0;
    int64_t lds_floats = 0;
    for (int l = 0; l < n_levels; ++l) {
        const int64_t floats = static_cast<int64_t>(levels[l].size) * features;
        if ((lds_floats + floats) * 4 > t.lds_bytes) break;
        if (static_cast<int64_t>(levels[l].size) > 2 * static_cast<int64_t>(a.chunk)) break;
        lds_floats += floats;
        lds_levels = l + 1;
    }
    a.lds_levels = lds_levels;
    a.lds_floats = static_cast<int>(lds_floats);
    const size_t shmem = static_cast<size_t>(lds_floats) * 4;
    const uint32_t blocks = grid_blocks(n, a.chunk);
    ODIE_GRID_DISPATCH(grid_backward_kernel, features, half, n_levels, blocks, shmem, s, a);
    return check_launch("odie_grid_backward");
}

}  // namespace

ODIE_API int odie_grid_backward(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                                const odie_grid_level* levels, int n_levels, int features,
                                float* gradient, int zero_first, uint64_t stream) {
    return grid_backward(coords, n, offsets, experts, upstream, up_dtype, up_width, expert_params, levels, n_levels,
                         features, gradient, zero_first, nullptr, 0, stream);
}

// Encode backward fused with the optimizer step: every parameter's gradient is formed in
// LDS by the owner-computes backward and the Adam update (adam.h) is applied where it is
// flushed, so the gradient never reaches HBM.  Same result as odie_grid_backward followed
// by odie_adam_step on the gradient, bit for bit.
namespace odie {

namespace {

// Shared body of the fused entry points and of odie_grid_backward_planes: upstream rows
// (transposed by the owner launch) or, with planes set, the level-major fp16 planes and their
// 128-row column maxima; with adam the optimizer step is applied in the owner's flush, without
// it the gradient is written (zero_first = 0: added) to `gradient`.
int backward_adam(const char* name, const float* coords, int64_t n, const int32_t* offsets, int experts,
                  const void* upstream, int up_dtype, int up_width, const uint32_t* planes, const float* blockmax,
                  int64_t expert_params, const odie_grid_level* levels, int n_levels, int features,
                  const AdamStep* adam, float* gradient, int zero_first, hipStream_t s,
                  const uint8_t* handoff = nullptr, int64_t handoff_bytes = 0) {
    GridArgs a{};
    if (validate_grid(name, coords, n, offsets, experts, expert_params, levels, n_levels, features, a)) return -1;
    if (planes || blockmax) {
        if (features != 2) return fail(std::string(name) + ": planes carry 2 fp16 features per level");
        if (n > 0 && (!planes || !blockmax)) return fail(std::string(name) + ": planes and blockmax must be non-null");
        if (reinterpret_cast<uintptr_t>(planes) % 4) return fail(std::string(name) + ": planes must be 4-byte aligned");
    } else {
        if (up_dtype != ODIE_F32 && up_dtype != ODIE_F16)
            return fail(std::string(name) + ": up_dtype must be 0 (fp32) or 1 (fp16)");
        if (up_width < n_levels * features) return fail(std::string(name) + ": up_width is smaller than n_levels*features");
        if (n > 0 && !upstream) return fail(std::string(name) + ": upstream is null");
    }
    if (reinterpret_cast<uintptr_t>(coords) % 8) return fail(std::string(name) + ": coords must be 8-byte aligned");
    if (!adam && !gradient) return fail(std::string(name) + ": gradient is null");
    const int64_t table = static_cast<int64_t>(a.level[n_levels - 1].offset + a.level[n_levels - 1].size) * features;
    if (table >= (int64_t{1} << 31)) return fail(std::string(name) + ": one table must hold fewer than 2^31 values");
    if (expert_params != table) return fail(std::string(name) + ": expert_params must equal the levels' table size");
    const int64_t total = expert_params * experts;
    if (n == 0) {   // every gradient is zero
        if (!adam) return zero_first ? launch_fill_zero(gradient, total, s) : 0;
        float* zero = static_cast<float*>(workspace(static_cast<size_t>(total) * 4, s));
        if (!zero || launch_fill_zero(zero, total, s)) return -1;
        return launch_adam(*adam, zero, 0, total, s);
    }
    const Tuning& t = tuning();
    OwnerLaunch o{};
    o.coords = coords;
    o.offsets = a.offsets;
    o.upstream = planes ? nullptr : upstream;
    o.up_half = planes ? 1 : up_dtype == ODIE_F16;
    o.up_width = planes ? n_levels * features : up_width;
    o.planes = planes;
    o.blockmax = blockmax;
    o.grad = adam ? nullptr : gradient;
    o.accumulate = adam || zero_first ? 0 : 1;
    o.n = n;
    o.expert_params = expert_params;
    o.experts = experts;
    o.n_levels = n_levels;
    o.features = features;
    o.levels = a.level;
    o.lds_bytes = t.owner_lds_bytes;
    o.remap = t.xcd_remap;
    o.banded = t.banded;
    o.masks = t.owner_masks;
    o.split_target = t.split_target;
    o.stream = s;
    o.adam = adam;
    o.handoff = handoff;
    o.handoff_bytes = handoff_bytes;
    return launch_owner_backward(o);
}

}  // namespace

int grid_backward_adam_internal(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                                const odie_grid_level* levels, int n_levels, int features, const AdamStep& adam,
                                hipStream_t s) {
    return backward_adam("odie_grid_backward_adam", coords, n, offsets, experts, upstream, up_dtype, up_width, nullptr,
                         nullptr, expert_params, levels, n_levels, features, &adam, nullptr, 0, s);
}

int grid_backward_adam_planes_internal(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                       const uint32_t* planes, const float* blockmax, int64_t expert_params,
                                       const odie_grid_level* levels, int n_levels, int features,
                                       const AdamStep& adam, hipStream_t s) {
    return backward_adam("odie_grid_backward_adam_planes", coords, n, offsets, experts, nullptr, ODIE_F16, 0, planes,
                         blockmax, expert_params, levels, n_levels, features, &adam, nullptr, 0, s);
}

}  // namespace odie

ODIE_API int odie_grid_backward_adam(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                     const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                                     const odie_grid_level* levels, int n_levels, int features, float* master,
                                     uint16_t* half_copy, float* m, float* v, uint32_t* steps, int variant, int64_t step,
                                     float lr, float beta1, float beta2, float eps, float loss_scale, uint64_t stream) {
    AdamStep adam;
    if (make_adam_step("odie_grid_backward_adam", master, half_copy, m, v, steps, variant, step, lr, beta1, beta2, eps,
                       loss_scale, true, adam))
        return -1;
    return grid_backward_adam_internal(coords, n, offsets, experts, upstream, up_dtype, up_width, expert_params, levels,
                                       n_levels, features, adam, as_stream(stream));
}

ODIE_API int odie_grid_backward_adam_planes(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                            const uint32_t* planes, const float* blockmax, int64_t expert_params,
                                            const odie_grid_level* levels, int n_levels, int features, float* master,
                                            uint16_t* half_copy, float* m, float* v, uint32_t* steps, int variant,
                                            int64_t step, float lr, float beta1, float beta2, float eps,
                                            float loss_scale, uint64_t stream) {
    AdamStep adam;
    if (make_adam_step("odie_grid_backward_adam_planes", master, half_copy, m, v, steps, variant, step, lr, beta1,
                       beta2, eps, loss_scale, true, adam))
        return -1;
    return grid_backward_adam_planes_internal(coords, n, offsets, experts, planes, blockmax, expert_params, levels,
                                              n_levels, features, adam, as_stream(stream));
}

ODIE_API int odie_grid_backward_adam_planes_handoff(const float* coords, int64_t n, const int32_t* offsets,
                                                    int experts, const uint32_t* planes, const float* blockmax,
                                                    int64_t expert_params, const odie_grid_level* levels,
                                                    int n_levels, int features, float* master, uint16_t* half_copy,
                                                    float* m, float* v, uint32_t* steps, int variant, int64_t step,
                                                    float lr, float beta1, float beta2, float eps, float loss_scale,
                                                    const void* handoff, int64_t handoff_bytes, uint64_t stream) {
    AdamStep adam;
    if (make_adam_step("odie_grid_backward_adam_planes_handoff", master, half_copy, m, v, steps, variant, step, lr,
                       beta1, beta2, eps, loss_scale, true, adam))
        return -1;
    if (n > 0 && !handoff && handoff_bytes > 0) return fail("odie_grid_backward_adam_planes_handoff: handoff is null");
    return backward_adam("odie_grid_backward_adam_planes_handoff", coords, n, offsets, experts, nullptr, ODIE_F16, 0,
                         planes, blockmax, expert_params, levels, n_levels, features, &adam, nullptr, 0,
                         as_stream(stream), static_cast<const uint8_t*>(handoff), handoff_bytes);
}

ODIE_API int odie_grid_backward_handoff(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                        const void* upstream, int up_dtype, int up_width, int64_t expert_params,
                                        const odie_grid_level* levels, int n_levels, int features, float* gradient,
                                        int zero_first, const void* handoff, int64_t handoff_bytes,
                                        uint64_t stream) {
    if (n > 0 && !handoff && handoff_bytes > 0) return fail("odie_grid_backward_handoff: handoff is null");
    // (with the atomics backward, tuning key backward_mode 0, the handoff goes unread)
    return grid_backward(coords, n, offsets, experts, upstream, up_dtype, up_width, expert_params, levels, n_levels,
                         features, gradient, zero_first, static_cast<const uint8_t*>(handoff), handoff_bytes, stream);
}

ODIE_API int odie_grid_backward_planes(const float* coords, int64_t n, const int32_t* offsets, int experts,
                                       const uint32_t* planes, const float* blockmax, int64_t expert_params,
                                       const odie_grid_level* levels, int n_levels, int features, float* gradient,
                                       int zero_first, uint64_t stream) {
    return backward_adam("odie_grid_backward_planes", coords, n, offsets, experts, nullptr, ODIE_F16, 0, planes,
                         blockmax, expert_params, levels, n_levels, features, nullptr, gradient, zero_first,
                         as_stream(stream));
}

ODIE_API int odie_set_tuning(const char* key, int value) {
    if (!key) return fail("odie_set_tuning: key is null");
    if (std::string(key).rfind("route_", 0) == 0) return set_route_tuning(key, value);
    return set_grid_tuning(key, value);
}

namespace odie {

int packed_forward_internal(const float* coords, int64_t n, const float* grid, int64_t parameter_count,
                            const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                            const int32_t* node_prefix, const uint8_t* bitmap, int width, int active, uint16_t pad,
                            uint16_t* features, uint8_t* visibility, hipStream_t stream, bool levels16x2,
                            bool pairs) {
    if (n < 0 || n > (int64_t{1} << 31) - 1) return fail("odie_packed_forward: n must be within [0, 2^31-1]");
    if (levels < 2 || levels > ODIE_MAX_LEVELS) return fail("odie_packed_forward: descriptor must have 2..32 levels");
    if (width < 2 || width > 128) return fail("odie_packed_forward: feature width must be within 2..128");
    if (parameter_count <= 0) return fail("odie_packed_forward: parameter_count must be positive");
    if (n == 0) return 0;
    if (!coords || !grid || !descriptors || !bitmap || !features || !visibility)
        return fail("odie_packed_forward: null pointer");
    if (reinterpret_cast<uintptr_t>(coords) % 8) return fail("odie_packed_forward: coords must be 8-byte aligned");
    PackedArgs a{};
    a.coords = coords;
    a.grid = grid;
    a.desc = descriptors;
    a.node_bitmap = node_bitmap;
    a.prefix = node_prefix;
    a.bitmap = bitmap;
    a.features = features;
    a.visibility = visibility;
    a.n = n;
    a.params = parameter_count;
    a.levels = levels;
    a.width = width;
    a.active = active;
    a.pad = pad;
    const uint32_t blocks = static_cast<uint32_t>((n + kBlock - 1) / kBlock);
    const bool aligned = reinterpret_cast<uintptr_t>(features) % 16 == 0 && reinterpret_cast<uintptr_t>(grid) % 8 == 0;
    if (levels16x2 && levels == 16 && width == 32 && aligned && reinterpret_cast<uintptr_t>(visibility) % 16 == 0) {
        packed_forward16x2_kernel<<<blocks, kBlock, 0, stream>>>(a);
    } else if (pairs && aligned && reinterpret_cast<uintptr_t>(visibility) % 4 == 0 && width % 16 == 0 &&
               width >= 2 * levels && width <= 80) {
        switch (width / 2) {
            case 8: packed_forward_pairs_kernel<8><<<blocks, kBlock, 0, stream>>>(a); break;
            case 16: packed_forward_pairs_kernel<16><<<blocks, kBlock, 0, stream>>>(a); break;
            case 24: packed_forward_pairs_kernel<24><<<blocks, kBlock, 0, stream>>>(a); break;
            case 32: packed_forward_pairs_kernel<32><<<blocks, kBlock, 0, stream>>>(a); break;
            default: packed_forward_pairs_kernel<40><<<blocks, kBlock, 0, stream>>>(a); break;
        }
    } else {
        packed_forward_kernel<<<blocks, kBlock, 0, stream>>>(a);
    }
    return check_launch("odie_packed_forward");
}

}  // namespace odie

using namespace odie;

ODIE_API int odie_packed_forward(const float* coords, int64_t n, const float* grid, int64_t parameter_count,
                                 const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                                 const int32_t* node_prefix, const uint8_t* bitmap, int width,
                                 uint16_t* features, uint8_t* visibility, uint64_t stream) {
    return packed_forward_internal(coords, n, grid, parameter_count, descriptors, levels, node_bitmap, node_prefix,
                                   bitmap, width, levels, 0, features, visibility, as_stream(stream));
}

namespace odie {

int packed_backward_internal(const float* coords, int64_t n, const uint16_t* upstream, int up_width,
                             const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                             const int32_t* node_prefix, const uint8_t* bitmap, float* gradient,
                             int64_t parameter_count, hipStream_t s, bool zeroed) {
    if (n < 0 || n > (int64_t{1} << 31) - 1) return fail("odie_packed_backward: n must be within [0, 2^31-1]");
    if (levels < 2 || levels > ODIE_MAX_LEVELS) return fail("odie_packed_backward: descriptor must have 2..32 levels");
    if (up_width < 2 || up_width > 128) return fail("odie_packed_backward: upstream width must be within 2..128");
    if (parameter_count < 0) return fail("odie_packed_backward: parameter count must be nonnegative");
    if (parameter_count > 0 && !gradient) return fail("odie_packed_backward: gradient is null");
    if (n == 0 || parameter_count == 0) return zeroed ? 0 : launch_fill_zero(gradient, parameter_count, s);
    if (!coords || !upstream || !descriptors || !bitmap) return fail("odie_packed_backward: null pointer");
    if (reinterpret_cast<uintptr_t>(coords) % 8) return fail("odie_packed_backward: coords must be 8-byte aligned");
    const Tuning& t = tuning();
    if (t.packed_owner)   // owner computes: every value written once, deterministic order
        return launch_packed_owner(coords, n, upstream, up_width, descriptors, levels, node_bitmap, node_prefix, bitmap,
                                   gradient, parameter_count, t.owner_lds_bytes, t.packed_splits, s);
    if (!zeroed && launch_fill_zero(gradient, parameter_count, s)) return -1;
    PackedArgs a{};
    a.coords = coords;
    a.desc = descriptors;
    a.node_bitmap = node_bitmap;
    a.prefix = node_prefix;
    a.bitmap = bitmap;
    a.upstream = upstream;
    a.gradient = gradient;
    a.n = n;
    a.params = parameter_count;
    a.levels = levels;
    a.width = up_width;
    if (t.packed_lds) {
        // few large chunks: each block flushes its coarse partials once
        int64_t blocks = (n + 255) / 256;
        if (blocks > t.packed_blocks) blocks = t.packed_blocks;
        const int64_t chunk = (n + blocks - 1) / blocks;
        packed_backward_lds_kernel<<<static_cast<uint32_t>(blocks), kBlock, 0, s>>>(a, chunk);
    } else {
        const uint32_t blocks = static_cast<uint32_t>((n + kBlock - 1) / kBlock);
        packed_backward_kernel<<<blocks, kBlock, 0, s>>>(a);
    }
    return check_launch("odie_packed_backward");
}

}  // namespace odie

ODIE_API int odie_packed_backward(const float* coords, int64_t n, const uint16_t* upstream, int up_width,
                                  const int32_t* descriptors, int levels, const uint64_t* node_bitmap,
                                  const int32_t* node_prefix, const uint8_t* bitmap, float* gradient,
                                  int64_t parameter_count, uint64_t stream) {
    return packed_backward_internal(coords, n, upstream, up_width, descriptors, levels, node_bitmap, node_prefix,
                                    bitmap, gradient, parameter_count, as_stream(stream), false);
}
