// Grid-encode backward without global atomics ("owner computes").
//
// Measured on MI355X: global fp32 atomics saturate near 21 G op/s and LDS fp32 atomics
// near 0.2 T op/s, while LDS 64-bit integer atomics (ds_add_u64) reach ~2.4 T op/s.  So the
// gradient is not scattered into HBM at all:
//   1. transpose  the upstream rows [N, L*F] into level-major planes [L][N][F] and record
//                 the largest |upstream| of every 128-row record and column (level, feature);
//   2. owner      one workgroup owns one slice of one expert's gradient (a group of coarse
//                 levels, or a part of one finer level) that fits in LDS.  It walks every
//                 coordinate of its expert, evaluates the geometry of its level(s) and adds
//                 the contributions that land in its slice as 64-bit fixed-point integers
//                 (ds_add_u64).  Every (level, feature) of the slice has its own fixed-point
//                 scale 2^S, chosen from max|upstream| of that column over the workgroup's
//                 coordinates: every contribution stays below 2^31 and 4*count of them below
//                 2^62, so nothing can overflow; each contribution is the fp32 product
//                 w_k * upstream (as in the reference, odie/packed_kernels.cu:84) rounded to the
//                 nearest multiple of 2^-S, so its error is at most 2^-31 of the largest |u| of
//                 its own level and feature, whatever the other columns hold.  The slice is
//                 then converted to fp32 and written with plain coalesced stores.
//                 Integer sums are associative, so the gradient does not depend on the
//                 order in which lanes add.
//   3. reduce     only when one expert's coordinates are split over several workgroups per
//                 slice (few experts, many coordinates): partial slices are summed.
// Every gradient entry is written by exactly one workgroup, so no clearing pass is needed.
#include <cmath>

#include "grid.h"
#include "adam.h"

namespace odie {
namespace {

constexpr int kTransposeBlock = 256;
constexpr int kTransposeRows = 1024;  // rows per transpose block
constexpr int kMaxRows = 128;         // rows per |upstream| maximum record (two waves of a pass)
constexpr int kOwnerBlock = 1024;
constexpr int kBatch = 4;             // coordinates per thread per owner-loop iteration
constexpr int kGroupBatch = 2;        // the same in the coarse-group pass, whose adds all land
constexpr int kWaves = kOwnerBlock / 64;

// Band lists.  A coordinate with x and y in [0, 1] falls in y-band floor(y * kBands) (clamped);
// any other coordinate (outside the unit square, or NaN) in the last slot, kBands.  A table row
// of a dense level, or of a hashed one whose slices are aligned blocks wider than a row of
// corners, is reached only from the cells just above and below it, so a slice of such a level
// is reached only from a few bands plus that last slot.
constexpr int kBands = 2047;
constexpr int kBandSlots = kBands + 1;       // 2048 slots: 64 bitmap words, one per lane
constexpr int kBandWords = kBandSlots / 32;
constexpr int kBandBlock = 1024;
constexpr int kBandPart = 16384;             // coordinates per counting workgroup
constexpr int kMaxBandParts = 256;
constexpr int kMaxRuns = kBandSlots / 2;     // runs of marked slots in 2048 bits
// LDS after a banded pass's accumulators: slot bitmap, run list ranges, piece prefix, scan scratch
constexpr int kReserveInts = kBandWords + 2 * kMaxRuns + (kMaxRuns + 1) + kWaves + 4;
constexpr int kReserveBytes = (kReserveInts * 4 + 255) / 256 * 256;
static_assert(kBandBlock == kOwnerBlock, "the block scan serves both kernels");

struct TransposeArgs {
    const void* upstream;
    void* planes;
    float* blockmax;
    int64_t n;
    int width;
    int n_levels;
    int vec_rows;
    // with the band lists: position i of the planes takes upstream row list[i] when *ordered (the
    // lists then hold every coordinate of its expert once), so that the owner's banded walk reads
    // its upstream values in list order, as it reads the sorted coordinates; row i otherwise
    const int32_t* list;
    const int32_t* ordered;
    const int32_t* offsets;   // the experts' ranges (null: one expert over [0, n))
    int experts;
};

// Positions [lo, hi) the band lists cover when *ordered: from the first expert's first
// coordinate to the last one's end, clamped as the owner clamps the ranges.  Positions outside
// (ids routed to no expert) have no list entry and keep their own row.
__device__ inline void listed_range(const TransposeArgs& a, int64_t& lo, int64_t& hi) {
    lo = 0;
    hi = a.n;
    if (!a.offsets) return;
    const int64_t first = a.offsets[0], last = a.offsets[a.experts];
    lo = first < 0 ? 0 : (first > a.n ? a.n : first);
    hi = last > a.n ? a.n : (last < lo ? lo : last);
}

// Upstream row of plane position i.
__device__ inline int64_t source_row(const TransposeArgs& a, bool by_list, int64_t lo, int64_t hi, int64_t i) {
    return by_list && i >= lo && i < hi ? static_cast<int64_t>(a.list[i]) : i;
}

// Maximum of two |upstream| records; NaN wins, so the owner pass sees a non-finite bound.
__device__ inline float nan_max(float a, float b) { return (b > a || b != b) ? b : a; }

// Record q of the block (rows q*128.. of its 1024) is waves 2*(q%2) and 2*(q%2)+1 of pass q/2;
// `waves` holds `stride` column maxima per wave, of which the first `columns` are used.
__device__ inline void write_records(const TransposeArgs& a, const float* waves, int stride, int columns) {
    constexpr int kRecords = kTransposeRows / kMaxRows;
    for (int t = threadIdx.x; t < kRecords * columns; t += kTransposeBlock) {
        const int q = t / columns, j = t % columns;
        const int64_t record = static_cast<int64_t>(blockIdx.x) * kRecords + q;
        if (record * kMaxRows >= a.n) continue;
        const float* pass = waves + (q / 2) * (kTransposeBlock / 64) * stride;
        const int w = 2 * (q % 2);
        a.blockmax[record * columns + j] = nan_max(pass[w * stride + j], pass[(w + 1) * stride + j]);
    }
}

// Rows [N, width] -> level-major planes [L][N][F], and the largest |upstream| of every 128-row
// record and column (level l, feature c: column l*F + c).
template <int F, bool HALF, int LMAX>
__global__ __launch_bounds__(kTransposeBlock) void transpose_kernel(TransposeArgs a) {
    using U = Elem<HALF>;
    constexpr int kPasses = kTransposeRows / kTransposeBlock;
    constexpr int kColumns = LMAX * F;
    __shared__ float waves[kPasses][kTransposeBlock / 64][kColumns];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int used = a.n_levels * F;
    const bool by_list = a.list && *a.ordered;
    int64_t lo, hi;
    listed_range(a, lo, hi);
    for (int r = 0; r < kPasses; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        const bool valid = i < a.n;
        U vals[kColumns];
        if (valid) {
            const U* row = reinterpret_cast<const U*>(a.upstream) + static_cast<size_t>(source_row(a, by_list, lo, hi, i)) * a.width;
            if (a.vec_rows) {
                constexpr int kPer = 16 / sizeof(U);
                constexpr int kChunks = (kColumns + kPer - 1) / kPer;
#pragma unroll
                for (int j = 0; j < kChunks; ++j) {
                    if (j * kPer < used) {
                        const uint4 v = reinterpret_cast<const uint4*>(row)[j];
                        const U* parts = reinterpret_cast<const U*>(&v);
#pragma unroll
                        for (int q = 0; q < kPer; ++q)
                            if (j * kPer + q < kColumns) vals[j * kPer + q] = parts[q];
                    }
                }
            } else {
#pragma unroll
                for (int c = 0; c < kColumns; ++c)
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
                }
            }
        }
        // the wave's 64 rows lie in one record of kMaxRows = 128 rows
#pragma unroll
        for (int j = 0; j < kColumns; ++j) {
            if (j < used) {
                float m = valid ? fabsf(static_cast<float>(vals[j])) : 0.0f;
                for (int step = 32; step; step >>= 1) m = nan_max(m, __shfl_xor(m, step));
                if (lane == 0) waves[r][wave][j] = m;
            }
        }
    }
    __syncthreads();
    write_records(a, &waves[0][0][0], kColumns, used);
}

// fp16 pairs (F = 2), levels a multiple of 4 and 16-byte rows: every thread loads its four
// rows first (16-byte loads), then writes one dword per level and row; the per-feature |u|
// maxima of each level (two 16-bit magnitudes per dword) are reduced over the 32 lanes of each
// lane group eight levels at a time (group_max8), then over the record's two waves and four lane
// groups.
template <int LMAX>
__global__ __launch_bounds__(kTransposeBlock) void transpose_half2_kernel(TransposeArgs a) {
    constexpr int kPasses = kTransposeRows / kTransposeBlock;
    constexpr int kChunks = LMAX / 4;  // 16-byte chunks per row (4 levels each)
    __shared__ uint32_t waves[kPasses][kTransposeBlock / 64][2][LMAX];   // per lane group and level
    uint4 rows[kPasses][kChunks];
    const int chunks = a.n_levels / 4;
    const bool by_list = a.list && *a.ordered;
    int64_t lo, hi;
    listed_range(a, lo, hi);
    int64_t source[kPasses];   // every pass's row index loaded before any row
#pragma unroll
    for (int r = 0; r < kPasses; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        source[r] = source_row(a, by_list, lo, hi, i < a.n ? i : 0);
    }
#pragma unroll
    for (int r = 0; r < kPasses; ++r) {
        const uint4* row = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.upstream) +
                                                          static_cast<size_t>(source[r]) * a.width);
#pragma unroll
        for (int j = 0; j < kChunks; ++j) rows[r][j] = j < chunks ? row[j] : make_uint4(0, 0, 0, 0);
    }
    uint32_t* planes = reinterpret_cast<uint32_t*>(a.planes);
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, g = lane / 32, s = lane % 32;
#pragma unroll
    for (int r = 0; r < kPasses; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        const bool valid = i < a.n;
        uint32_t peak[LMAX];
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const uint32_t words[4] = {rows[r][j].x, rows[r][j].y, rows[r][j].z, rows[r][j].w};
            if (valid && j < chunks) {
#pragma unroll
                for (int q = 0; q < 4; ++q) planes[static_cast<size_t>(4 * j + q) * a.n + i] = words[q];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) peak[4 * j + q] = valid ? pair_magnitudes(words[q]) : 0u;
        }
#pragma unroll
        for (int k = 0; k < LMAX / 8; ++k) {
            if (8 * k < a.n_levels) {   // uniform: the whole wave takes part in group_max8
                const uint32_t m = group_max8(peak + 8 * k, lane);
                if (s < 8) waves[r][wave][g][8 * k + s] = m;
            }
        }
    }
    __syncthreads();
    constexpr int kRecords = kTransposeRows / kMaxRows;
    const int columns = 2 * a.n_levels;
    for (int t = threadIdx.x; t < kRecords * columns; t += kTransposeBlock) {
        const int q = t / columns, j = t % columns, l = j / 2, f = j % 2;
        const int64_t record = static_cast<int64_t>(blockIdx.x) * kRecords + q;
        if (record * kMaxRows >= a.n) continue;
        const int w = 2 * (q % 2);
        const auto& pass = waves[q / 2];
        const uint32_t both = pair_max(pair_max(pass[w][0][l], pass[w][1][l]), pair_max(pass[w + 1][0][l], pass[w + 1][1][l]));
        a.blockmax[record * columns + j] = __half2float(bits_to_half(static_cast<uint16_t>(both >> (16 * f))));
    }
}

// Work items.  Every expert has `items` of them, in this order: the coarse-group pass (levels
// [0, group), when group > 0) split `group_splits` ways, then for each finer level l its
// `slices[l]` slices, each split `splits[l]` ways (item first_item[l] + slice * splits[l] + s).
// A split takes one share of the pass's coordinates.  Unbanded, split s of a pass walks the
// s-th index range of the expert's coordinates and writes fp32 partial slices, summed by
// split_reduce_kernel.  Banded, the fine passes walk only the coordinates listed in the y-band
// slots their table rows can reach (band lists below), every pass bounds its fixed-point scale
// over all of the expert's coordinates, and splits write the raw 64-bit sums, added exactly by
// banded_reduce_kernel: the gradient does not depend on how a pass is split.  Every column
// (level, feature) of an expert has one fixed-point scale, from its peak over the expert's
// coordinates (column_peaks_kernel), shared by every pass and split that covers it.
struct OwnerArgs {
    const float* coords;
    const int32_t* offsets;
    const void* planes;
    const float* blockmax;      // [records][n_levels * features]: max |upstream| per 128-row record and column
    float* grad;
    float* partial;             // unbanded splits: fp32 [max split][experts][expert_params]
    long long* partial64;       // banded splits: int64 [max split][experts][partial_floats]
    const uint32_t* peaks;      // [experts][n_levels * features]: max |upstream| of each column over the
                                // records that meet the expert's coordinates (float bits; NaN above all)
    int64_t partial_floats;
    int64_t n;
    int64_t expert_params;
    int experts;
    int n_levels;
    int features;
    int group;        // pass 0 covers levels [0, group) when group > 0
    int items;        // work items per expert
    int group_splits;
    int heavy;        // leading items of every expert scheduled first (work_of)
    int accumulate;   // 1: grad += slice
    int remap;
    int banded;
    DevLevel level[ODIE_MAX_LEVELS];
    int first_item[ODIE_MAX_LEVELS];
    int slices[ODIE_MAX_LEVELS];
    int splits[ODIE_MAX_LEVELS];
    int slice_entries[ODIE_MAX_LEVELS];
    int row_bits[ODIE_MAX_LEVELS];   // > 0: slices are aligned 2^row_bits blocks (hashed levels)
    int cap;                         // int64 accumulators in LDS; the band workspace follows them
    int fused;                       // 1: apply the optimizer step instead of writing the gradient
    AdamStep adam;
    // band lists (banded): coordinate indices of expert e ordered by y-band slot, slot b at
    // list[start[e * (kBandSlots + 1) + b] .. start[... + b + 1]); valid when *ordered
    const int32_t* band_start;
    const int32_t* band_list;
    const float2* band_sorted;
    const int32_t* ordered;
    // 1: the planes (and their record maxima) are in band-list order when *ordered (the backward
    // transposed them so); every pass then reads coordinates from band_sorted and upstream values
    // at the same list position
    int band_planes;
    // slice masks (unbanded levels cut into at most 8 aligned blocks of 2^row_bits entries):
    // byte i of plane mask_plane[l] (planes mask_stride bytes apart) has bit s set when a corner
    // of coordinate i lands in block s
    const uint8_t* masks;
    int64_t mask_stride;
    int mask_plane[ODIE_MAX_LEVELS];   // -1: no mask for the level
    int ring_at;                       // byte offset of the waves' rings in the dynamic LDS
};

constexpr int32_t kNonFinite = 1 << 30;   // shift of a column whose upstream bound is not finite

// Fixed-point shift of a column whose contributions are w * u with |u| <= peak (the bits of a
// non-negative float, or a NaN), `count` coordinates of them: 2^shift * peak stays below 2^31, so
// one contribution converts with one rint + cvt_i32, and 4 * count of them below 2^62 in the
// int64 sum.  The quantum is 2^-shift <= 2^-30 peak (count < 2^29).  kNonFinite for a NaN or
// infinite peak.
__device__ inline int32_t column_shift(uint32_t peak_bits, int64_t count) {
    const float peak = __uint_as_float(peak_bits);
    if (!(peak <= 3.0e38f)) return kNonFinite;
    int shift = 60;
    if (peak > 0.0f) {
        const int by_value = 30 - ilogb(peak);
        const int by_sum = 61 - ilogb(4.0 * static_cast<double>(count) * static_cast<double>(peak));
        shift = by_value < by_sum ? by_value : by_sum;
    }
    return shift > 120 ? 120 : shift;
}

// 2^shift as the multiplier of the upstream values (1 for a non-finite column: its values are NaN).
__device__ inline float shift_scale(int32_t shift) { return shift == kNonFinite ? 1.0f : ldexpf(1.0f, shift); }

// The fp32 gradient value of a raw 64-bit fixed-point sum at `shift`.
__device__ inline float unscaled(long long sum, int32_t shift) {
    if (shift == kNonFinite) return __builtin_nanf("");
    return static_cast<float>(static_cast<double>(sum) * ldexp(1.0, -shift));
}

enum LevelKind { kDense = 0, kHashedPow2 = 1, kGeneric = 2, kHashed24 = 3 };

// Nearest integer, halves rounded up (floor(x + 0.5)) in one instruction.  |x| < 2^31 here.
// Any rounding to nearest keeps each fixed-point contribution within half a quantum.
__device__ inline int32_t round_to_int(float x) {
    int32_t r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

// Table entries of the four corners of grid cell (gx, gy) (grid_corners' indices, per level kind).
template <int KIND>
__device__ inline void corner_index(uint32_t gx, uint32_t gy, const DevLevel& lv, uint32_t idx[4]) {
    if constexpr (KIND == kHashed24) {
        // power-of-two table of at most 2^24 entries: 24-bit row multiply (see hash_row)
        const uint32_t h0 = __umul24(gy, lv.prime), h1 = __umul24(gy + 1u, lv.prime);
        idx[0] = (gx ^ h0) & lv.mask;
        idx[1] = ((gx + 1u) ^ h0) & lv.mask;
        idx[2] = (gx ^ h1) & lv.mask;
        idx[3] = ((gx + 1u) ^ h1) & lv.mask;
    } else if constexpr (KIND == kHashedPow2) {
        const uint32_t h0 = gy * 2654435761u, h1 = (gy + 1u) * 2654435761u;
        idx[0] = (gx ^ h0) & lv.mask;
        idx[1] = ((gx + 1u) ^ h0) & lv.mask;
        idx[2] = (gx ^ h1) & lv.mask;
        idx[3] = ((gx + 1u) ^ h1) & lv.mask;
    } else if constexpr (KIND == kDense) {
        const uint32_t base = gx + gy * lv.res;
        idx[0] = wrap_index(base, lv);
        idx[1] = wrap_index(base + 1u, lv);
        idx[2] = wrap_index(base + lv.res, lv);
        idx[3] = wrap_index(base + lv.res + 1u, lv);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t cx = gx + static_cast<uint32_t>(k & 1), cy = gy + static_cast<uint32_t>(k >> 1);
            idx[k] = wrap_index(cx ^ hash_row(cy, lv), lv);
        }
    }
}

__device__ inline int level_kind(const DevLevel& lv) {
    if (lv.hashed && lv.mask && lv.mask < (1u << 24)) return kHashed24;
    if (lv.hashed && lv.mask) return kHashedPow2;
    return lv.hashed ? kGeneric : kDense;
}

// Adds one coordinate's contributions at one level to the LDS slice [lo, lo+span).
// us[c] = upstream feature c times the fixed-point scale 2^S ((w*u)*2^S == w*(u*2^S) exactly:
// scaling by a power of two commutes with rounding).  Contributions are rounded to integers
// before the (divergent) slice test so the masked part of the wave is only the LDS add.
// Bilinear weights and table entries of the four corners of (x, y) at one level (the forward's
// grid_corners, per level kind).
template <int KIND>
__device__ inline void corner_geometry(float x, float y, const DevLevel& lv, uint32_t idx[4], float w[4]) {
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
    corner_index<KIND>(gx, gy, lv, idx);
}

template <int F, int KIND>
__device__ inline void contribute(float x, float y, const float* us, const DevLevel& lv, uint32_t lo, uint32_t span,
                                  unsigned long long* acc) {
    float w[4];
    uint32_t idx[4];
    corner_geometry<KIND>(x, y, lv, idx, w);
    int32_t q[4][F];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int c = 0; c < F; ++c) q[k][c] = round_to_int(w[k] * us[c]);
    // feature-planar slice (feature c of entry e at c * entries + e): the 64-bit adds of one
    // instruction spread over every bank pair, where entry-major order would use every fourth
    const uint32_t entries = span / F;
    const uint32_t shift = lv.offset - lo / F;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t entry = idx[k] + shift;
        if (entry >= entries) continue;
#pragma unroll
        for (int c = 0; c < F; ++c)
            atomicAdd(acc + c * entries + entry, static_cast<unsigned long long>(static_cast<long long>(q[k][c])));
    }
}

// LDS accumulator of value j (entry j / F, feature j % F) of a slice of `span` values.
template <int F>
__device__ inline uint32_t planar(uint32_t j, uint32_t span) { return (j % F) * (span / F) + j / F; }

template <int F, bool HALF>
__device__ inline void load_upstream(const Elem<HALF>* plane, int64_t at, const float* scale, bool valid, float* us) {
    if constexpr (HALF && F == 2) {
        const uint32_t word = *reinterpret_cast<const uint32_t*>(plane + at * F);
        us[0] = __half2float(bits_to_half(static_cast<uint16_t>(word & 0xffffu)));
        us[1] = __half2float(bits_to_half(static_cast<uint16_t>(word >> 16)));
    } else {
#pragma unroll
        for (int c = 0; c < F; ++c) us[c] = static_cast<float>(plane[at * F + c]);
    }
#pragma unroll
    for (int c = 0; c < F; ++c) us[c] = valid ? us[c] * scale[c] : 0.0f;
}

// Offset of this thread's coordinate within each run of kOwnerBlock.  Hashed levels take the
// thread index: one wave reads 64 consecutive coordinates, fully coalesced.  Dense levels have
// few, large cells, and a spatially ordered batch (the stratified draw lists its strata row by
// row) would put a whole wave on two or three of them, where its 64-bit LDS adds to one
// address serialize.  There a wave takes 16 runs of 4 consecutive coordinates, 16 coordinates
// apart, from a quarter of the block:
//   offset = (wave / 4) * 256 + (wave % 4 + 4 * (lane / 4)) * 4 + lane % 4,
// a permutation of [0, 1024) whose loads still come in 32-byte runs.  A 65536-id stratified
// batch has 256 strata per row, so the wave's runs land 16 strata apart along a row.
template <int KIND>
__device__ inline int64_t lane_offset() {
    static_assert(kOwnerBlock == 1024, "the spread order covers 16 waves");
    if constexpr (KIND != kDense) {
        return threadIdx.x;
    } else {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        return (wave >> 2) * 256 + ((wave & 3) + 4 * (lane >> 2)) * 4 + (lane & 3);
    }
}

// Every coordinate of [b0, b1) against one level: each thread takes kBatch coordinates per
// iteration, kOwnerBlock apart, at lane_offset<KIND>() within each run; loads are issued
// unconditionally (clamped index) before any arithmetic.  A thread stops once its first
// coordinate is past b1: its later ones are too.
template <int F, bool HALF, int KIND, int B = kBatch>
__device__ inline void accumulate_level(const float* coords, const Elem<HALF>* plane, const DevLevel lv, int64_t b0,
                                        int64_t b1, uint32_t lo, uint32_t span, const float* scale,
                                        unsigned long long* acc) {
    for (int64_t i = b0 + lane_offset<KIND>(); i < b1; i += B * kOwnerBlock) {
        float2 xy[B];
        float us[B][F];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int64_t ii = i + b * kOwnerBlock;
            const int64_t at = ii < b1 ? ii : b0;
            xy[b] = reinterpret_cast<const float2*>(coords)[at];
            load_upstream<F, HALF>(plane, at, scale, ii < b1, us[b]);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) contribute<F, KIND>(xy[b].x, xy[b].y, us[b], lv, lo, span, acc);
    }
}

// A masked slice: each wave scans its runs of 256 of the coordinates [b0, b1) through their mask
// bytes (the next run's bytes loaded before the current run is used), queues those with a corner
// in block `block` of the level in a ring of kRing indices in LDS (ballot positions, no barrier:
// the ring is the wave's own), and evaluates kTake queued coordinates at a time, six per lane
// with all their loads issued first -- so the geometry runs only for coordinates that land
// (about 1.9 of a hashed level's 8 blocks per coordinate, 1 to 2 of a dense level's) instead of
// for all of them.
constexpr int kRing = 384;                  // >= kTake - 1 + 64: a group of 64's hits always fit
constexpr int kTake = 256;
constexpr int kRingBytes = kWaves * kRing * 4;
static_assert(kRing >= kTake - 1 + 64 && kRing <= 2 * kTake, "ring bound and single-subtraction wrap");

__device__ inline uint32_t ring_slot(uint32_t at) { return at < kRing ? at : at - kRing; }   // at < 2 kRing

template <int F, bool HALF, int KIND>
__device__ inline void accumulate_masked(const float* coords, const Elem<HALF>* plane, const uint8_t* mask,
                                         const DevLevel lv, int64_t b0, int64_t b1, uint32_t block, uint32_t lo,
                                         uint32_t span, const float* scale, unsigned long long* acc,
                                         int32_t* ring) {
    constexpr int kPer = kTake / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    uint32_t head = 0, count = 0;   // wave-uniform; head < kRing
    const auto evaluate = [&](uint32_t take) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        int32_t at[kPer];
        bool ok[kPer];
#pragma unroll
        for (int b = 0; b < kPer; ++b) {
            const uint32_t k = static_cast<uint32_t>(lane) + 64u * b;
            ok[b] = k < take;
            at[b] = ring[ring_slot(head + (ok[b] ? k : 0u))];
        }
        float2 xy[kPer];
        float us[kPer][F];
#pragma unroll
        for (int b = 0; b < kPer; ++b) {
            xy[b] = reinterpret_cast<const float2*>(coords)[at[b]];
            load_upstream<F, HALF>(plane, at[b], scale, ok[b], us[b]);
        }
#pragma unroll
        for (int b = 0; b < kPer; ++b)
            if (64u * b < take) contribute<F, KIND>(xy[b].x, xy[b].y, us[b], lv, lo, span, acc);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        head = ring_slot(head + take);
        count -= take;
    };
    const auto load_run = [&](int64_t run, uint32_t m[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t i = run + 64 * q + lane;
            m[q] = i < b1 ? mask[i] : 0u;
        }
    };
    uint32_t next[4];
    int64_t run = b0 + 256 * wave;
    if (run < b1) load_run(run, next);
    for (; run < b1; run += 256 * kWaves) {
        uint32_t m[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) m[q] = next[q];
        if (run + 256 * kWaves < b1) load_run(run + 256 * kWaves, next);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool hit = (m[q] >> block) & 1u;
            const uint64_t ballot = __ballot(hit);
            if (hit) ring[ring_slot(head + count + static_cast<uint32_t>(__popcll(ballot & below)))] =
                static_cast<int32_t>(run + 64 * q + lane);
            count += static_cast<uint32_t>(__popcll(ballot));
            if (count >= kTake) evaluate(kTake);
        }
    }
    while (count > 0) evaluate(count < kTake ? count : kTake);
}

// Mask bytes of the masked levels: plane p, byte i = the aligned blocks of 2^bits[p] entries of
// level level[p] that the corners of coordinate i land in (bit s: block s).  Planes are `stride`
// bytes apart.  The launch also clears the column peaks (zero words).

struct MaskArgs {
    const float* coords;
    uint8_t* masks;
    uint32_t* peaks;     // cleared here for column_peaks_kernel
    int64_t peak_words;
    int64_t n;
    int64_t stride;
    int planes;
    int bits[kMaxMaskPlanes];
    DevLevel level[kMaxMaskPlanes];
};

// One coordinate per thread, every plane (measured on MI355X: 44 us for 2^22 coordinates and 10
// planes; a shortcut that takes a hashed level's blocks from the row hashes alone, four
// coordinates per thread with word stores, descriptors from LDS, or one plane per block row were
// all slower, 58-90 us).
__global__ __launch_bounds__(256) void slice_mask_kernel(MaskArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    for (int64_t j = i; j < a.peak_words; j += static_cast<int64_t>(gridDim.x) * 256) a.peaks[j] = 0u;
    if (i >= a.n) return;
    const float2 xy = reinterpret_cast<const float2*>(a.coords)[i];
    for (int p = 0; p < a.planes; ++p) {
        const DevLevel lv = a.level[p];
        uint32_t idx[4];
        float w[4];
        switch (level_kind(lv)) {
            case kHashed24: corner_geometry<kHashed24>(xy.x, xy.y, lv, idx, w); break;
            case kHashedPow2: corner_geometry<kHashedPow2>(xy.x, xy.y, lv, idx, w); break;
            case kGeneric: corner_geometry<kGeneric>(xy.x, xy.y, lv, idx, w); break;
            default: corner_geometry<kDense>(xy.x, xy.y, lv, idx, w); break;
        }
        uint32_t byte = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) byte |= 1u << (idx[k] >> a.bits[p]);
        a.masks[static_cast<int64_t>(p) * a.stride + i] = static_cast<uint8_t>(byte);
    }
}

// Coordinates [base, stop) of expert e: offsets clamped into [0, n] and to a non-empty order.
__device__ inline void expert_range(const int32_t* offsets, int64_t n, int e, int64_t& base, int64_t& stop) {
    base = 0;
    stop = n;
    if (!offsets) return;
    base = offsets[e] > 0 ? offsets[e] : 0;
    stop = offsets[e + 1];
    if (base > n) base = n;
    if (stop > n) stop = n;
    if (stop < base) stop = base;
}

__device__ inline int band_slot(float x, float y) {
    if (!(x >= 0.0f && x <= 1.0f && y >= 0.0f && y <= 1.0f)) return kBands;
    const int b = static_cast<int>(y * static_cast<float>(kBands));
    return b < kBands ? b : kBands - 1;
}

// Exclusive prefix of v over the block's threads in thread order; total receives the block's sum.
__device__ inline int32_t block_exclusive(int32_t v, int32_t* waves, int32_t& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int32_t x = v;
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) waves[wave] = x;
    __syncthreads();
    int32_t before = 0;
    total = 0;
    for (int w = 0; w < kWaves; ++w) {
        const int32_t s = waves[w];
        if (w < wave) before += s;
        total += s;
    }
    __syncthreads();
    return before + x - v;
}

struct BandArgs {
    const float* coords;
    const int32_t* offsets;
    int64_t n;
    int experts;
    int parts;        // counting workgroups per expert
    int32_t* counts;  // [experts][parts][kBandSlots]: a part's slot counts, then its share's first offsets
    int32_t* start;   // [experts][kBandSlots + 1]: list position of every slot of the expert, then its end
    int32_t* list;    // [n]: coordinate index at every list position
    float2* sorted;   // [n]: that coordinate's (x, y)
    int32_t* ordered; // 1 when the expert ranges are in order (the lists are then exact)
};

// COUNT: every part of every expert counts its coordinates per slot.  PLACE (after
// band_columns_kernel and band_start_kernel): the part writes its coordinates' indices and
// (x, y) at the slots' cursors.  The order within a slot is free: the owner's integer sums do
// not depend on it.
// The grid is a multiple of kXcds; block -> (expert, part) is XCD-major, so the parts of an
// expert run on one XCD and the lines of its list fill in that XCD's L2.
template <bool PLACE>
__global__ __launch_bounds__(kBandBlock) void band_kernel(BandArgs a) {
    __shared__ int32_t slots[kBandSlots];
    const uint32_t item = xcd_major(blockIdx.x, gridDim.x);
    if (item >= static_cast<uint32_t>(a.experts) * a.parts) return;
    const int e = item / a.parts, part = item % a.parts;
    int64_t base, stop;
    expert_range(a.offsets, a.n, e, base, stop);
    const int64_t share = (stop - base + a.parts - 1) / a.parts;
    const int64_t b0 = base + share * part < stop ? base + share * part : stop;
    const int64_t b1 = b0 + share < stop ? b0 + share : stop;
    int32_t* row = a.counts + (static_cast<int64_t>(e) * a.parts + part) * kBandSlots;
    const int32_t* first = a.start + static_cast<int64_t>(e) * (kBandSlots + 1);
    for (int t = threadIdx.x; t < kBandSlots; t += kBandBlock) slots[t] = PLACE ? first[t] + row[t] : 0;
    __syncthreads();
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kBandBlock) {
        const float2 xy = reinterpret_cast<const float2*>(a.coords)[i];
        const int32_t at = atomicAdd(&slots[band_slot(xy.x, xy.y)], 1);
        if constexpr (PLACE) {
            a.list[at] = static_cast<int32_t>(i);
            a.sorted[at] = xy;
        }
    }
    if constexpr (!PLACE) {
        __syncthreads();
        for (int t = threadIdx.x; t < kBandSlots; t += kBandBlock) row[t] = slots[t];
    }
}

// Per-slot scan over the parts: a group of `group` lanes (a power of two, at most 64) takes one
// slot of one expert, each lane `per` consecutive parts.  Every part's count becomes its offset
// within the slot (counts, in place) and the slot's total goes to start, for band_start_kernel.
__global__ __launch_bounds__(kBandBlock) void band_columns_kernel(BandArgs a, int group, int per) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int slots_per_wave = 64 / group;
    const int64_t column = wave * slots_per_wave + lane / group;   // expert * kBandSlots + slot
    if (column >= static_cast<int64_t>(a.experts) * kBandSlots) return;   // whole groups leave together
    const int e = static_cast<int>(column / kBandSlots), slot = static_cast<int>(column % kBandSlots);
    const int j = lane % group;
    const int p0 = j * per < a.parts ? j * per : a.parts;
    const int p1 = p0 + per < a.parts ? p0 + per : a.parts;
    int32_t* rows = a.counts + static_cast<int64_t>(e) * a.parts * kBandSlots + slot;
    int32_t sum = 0;
    for (int part = p0; part < p1; ++part) sum += rows[static_cast<int64_t>(part) * kBandSlots];
    int32_t x = sum;
    for (int d = 1; d < group; d <<= 1) {
        const int32_t y = __shfl_up(x, d, group);
        if (j >= d) x += y;
    }
    int32_t run = x - sum;
    for (int part = p0; part < p1; ++part) {
        int32_t* c = rows + static_cast<int64_t>(part) * kBandSlots;
        const int32_t count = *c;
        *c = run;
        run += count;
    }
    if (j == group - 1) a.start[static_cast<int64_t>(e) * (kBandSlots + 1) + slot] = x;
}

// One workgroup per expert: the slot totals become the list position of every slot, from the
// expert's first coordinate (and the end after them).  Block 0 records whether the offsets are
// in order.
__global__ __launch_bounds__(kBandBlock) void band_start_kernel(BandArgs a) {
    __shared__ int32_t waves[kWaves];
    const int e = blockIdx.x;
    int64_t base, stop;
    expert_range(a.offsets, a.n, e, base, stop);
    if (e == 0) {
        int bad = 0;
        if (a.offsets)
            for (int k = threadIdx.x; k < a.experts; k += kBandBlock) bad |= a.offsets[k] > a.offsets[k + 1];
        bad = __syncthreads_or(bad);
        if (threadIdx.x == 0) *a.ordered = !bad;
    }
    int32_t* first = a.start + static_cast<int64_t>(e) * (kBandSlots + 1);
    constexpr int kPer = kBandSlots / kBandBlock;
    int32_t total[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) total[k] = first[threadIdx.x + k * kBandBlock];
    int32_t sum = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        int32_t all;
        const int32_t before = block_exclusive(total[k], waves, all);
        first[threadIdx.x + k * kBandBlock] = static_cast<int32_t>(base) + sum + before;
        sum += all;
    }
    if (threadIdx.x == 0) first[kBandSlots] = static_cast<int32_t>(base) + sum;
}

// Bitmap word w's bits for the slots [lo, hi].
__device__ inline uint32_t word_bits(int w, int lo, int hi) {
    const int a = lo > 32 * w ? lo - 32 * w : 0;
    const int b = hi < 32 * w + 31 ? hi - 32 * w : 31;
    if (b < a) return 0u;
    const uint32_t upto = b == 31 ? 0xffffffffu : (2u << b) - 1u;
    return upto & ~((1u << a) - 1u);
}

// Slots [lo, hi] holding every coordinate in [0, 1]^2 whose cell row at this level,
// floor(fma(scale, y, 0.5)), lies in [g0, g1].  fma rounds once (|error| <= 2^-24 (scale + 1)
// in cell units) and y * kBands once (<= 2^-13 slots); the bounds are widened by both.
__device__ inline void row_slots(const DevLevel& lv, int64_t g0, int64_t g1, int& lo, int& hi) {
    const double s = lv.scale;
    const double slack = ldexp(s + 1.0, -24);
    double y0 = ((static_cast<double>(g0) - 0.5 - slack) / s) * kBands - 0x1p-12;
    double y1 = ((static_cast<double>(g1) + 0.5 + slack) / s) * kBands + 0x1p-12;
    y0 = y0 < 0.0 ? 0.0 : (y0 > kBands - 1 ? kBands - 1 : y0);
    y1 = y1 < 0.0 ? 0.0 : (y1 > kBands - 1 ? kBands - 1 : y1);
    lo = static_cast<int>(floor(y0));
    hi = static_cast<int>(floor(y1));
}

// Cell rows reached by table entries [a, b) of a dense level through raw corner indices
// cx + cy * res with 0 <= cx, cy <= cmax: cy in [ceil((a - cmax) / res), floor((b - 1) / res)],
// and the cells just below those corners.
__device__ inline void dense_rows(int64_t a, int64_t b, int64_t res, int64_t cmax, int64_t& g0, int64_t& g1) {
    const int64_t over = a - cmax;
    const int64_t cy0 = over <= 0 ? 0 : (over + res - 1) / res;
    g0 = cy0 - 1;
    g1 = (b - 1) / res;
}

// Fills the LDS slot bitmap `bits` of the slice [first, last) of level lv (row_bits > 0: the
// aligned block `slice` of 2^row_bits entries of a hashed level).  Every thread takes part.
__device__ inline void mark_slice(const DevLevel& lv, uint32_t first, uint32_t last, int row_bits, uint32_t slice,
                                  uint32_t* bits) {
    const float top = __builtin_fmaf(lv.scale, 1.0f, 0.5f);   // largest p: x, y in [0, 1], fma is monotone
    const bool usable = lv.scale >= 1.0f && top < 16777216.0f;
    const int64_t gmax = usable ? static_cast<int64_t>(floorf(top)) : 0;   // largest cell row or column
    const int64_t cmax = gmax + 1;                                          // largest corner
    const int64_t res = lv.res, size = lv.size;
    bool all = !usable;
    if (!lv.hashed) {
        all |= cmax + cmax * res >= 2 * size;   // wrap_index's single subtraction covers every corner
    } else {
        all |= row_bits <= 0 || lv.mask == 0;
    }
    if (all || !lv.hashed) {
        // one word per thread of wave 0; dense: the two raw ranges [first, last), [first, last) + size
        int lo0 = 0, hi0 = kBands - 1, lo1 = 1, hi1 = 0;
        if (!all) {
            int64_t g0, g1;
            dense_rows(first, last, res, cmax, g0, g1);
            g0 = g0 < 0 ? 0 : g0;
            g1 = g1 > gmax ? gmax : g1;
            if (g0 <= g1) row_slots(lv, g0, g1, lo0, hi0); else { lo0 = 1; hi0 = 0; }
            const int64_t a = first + size, b = last + size < cmax + cmax * res + 1 ? last + size : cmax + cmax * res + 1;
            if (a < b) {
                dense_rows(a, b, res, cmax, g0, g1);
                g0 = g0 < 0 ? 0 : g0;
                g1 = g1 > gmax ? gmax : g1;
                if (g0 <= g1) row_slots(lv, g0, g1, lo1, hi1);
            }
        }
        if (threadIdx.x < kBandWords) {
            uint32_t w = word_bits(threadIdx.x, lo0, hi0) | word_bits(threadIdx.x, lo1, hi1);
            if (threadIdx.x == kBandWords - 1) w |= 1u << 31;   // the slot of coordinates outside [0, 1]^2
            bits[threadIdx.x] = w;
        }
        __syncthreads();
        return;
    }
    // hashed, aligned blocks of 2^row_bits entries: corner (cx, cy) lies in block
    // (((cy * prime) & mask) >> row_bits) ^ (cx >> row_bits) (within the mask), and cx >> row_bits
    // takes the values 0 .. cmax >> row_bits; so row cy reaches block `slice` only when
    // (((cy * prime) & mask) >> row_bits) ^ slice is one of them.  Cells cy - 1 and cy reach row cy.
    if (threadIdx.x < kBandWords) bits[threadIdx.x] = threadIdx.x == kBandWords - 1 ? 1u << 31 : 0u;
    __syncthreads();
    const uint32_t columns = static_cast<uint32_t>(cmax >> row_bits);
    for (int64_t cy = threadIdx.x; cy <= cmax; cy += kOwnerBlock) {
        if ((((hash_row(static_cast<uint32_t>(cy), lv) & lv.mask) >> row_bits) ^ slice) > columns) continue;
        int lo, hi;
        row_slots(lv, cy - 1 > 0 ? cy - 1 : 0, cy < gmax ? cy : gmax, lo, hi);
        for (int w = lo >> 5; w <= (hi >> 5); ++w) atomicOr(bits + w, word_bits(w, lo, hi));
    }
    __syncthreads();
}

// Turns the slot bitmap into runs of consecutive marked slots: the first list position of every
// run (run_k0) and the runs' sizes concatenated (prefix[r]: list entries before run r, prefix[runs]:
// all of them).  Returns the number of runs.
__device__ inline int slice_runs(const uint32_t* bits, const int32_t* start, int32_t* run_k0, int32_t* run_k1,
                                 int32_t* prefix, int32_t* scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int32_t* count = scratch + kWaves;
    if (wave == 0) {
        const uint32_t w = bits[lane];
        const uint32_t below = __shfl_up(w, 1), above = __shfl_down(w, 1);
        const uint32_t carry_in = lane > 0 ? below >> 31 : 0u;
        const uint32_t carry_out = lane < kBandWords - 1 ? above & 1u : 0u;
        uint32_t starts = w & ~((w << 1) | carry_in);
        uint32_t ends = w & ~((w >> 1) | (carry_out << 31));
        // a run may end in a later word: starts and ends are numbered separately
        const int32_t cs = __popc(starts), ce = __popc(ends);
        int32_t xs = cs, xe = ce;
        for (int d = 1; d < 64; d <<= 1) {
            const int32_t ys = __shfl_up(xs, d), ye = __shfl_up(xe, d);
            if (lane >= d) {
                xs += ys;
                xe += ye;
            }
        }
        for (int32_t r = xs - cs; starts; starts &= starts - 1, ++r) run_k0[r] = 32 * lane + __ffs(starts) - 1;
        for (int32_t r = xe - ce; ends; ends &= ends - 1, ++r) run_k1[r] = 32 * lane + __ffs(ends) - 1;
        if (lane == 63) *count = xs;
    }
    __syncthreads();
    const int runs = *count;
    int32_t size = 0;
    if (threadIdx.x < runs) {
        const int32_t k0 = start[run_k0[threadIdx.x]], k1 = start[run_k1[threadIdx.x] + 1];
        run_k0[threadIdx.x] = k0;
        size = k1 - k0;
    }
    int32_t total;
    const int32_t before = block_exclusive(size, scratch, total);
    if (threadIdx.x < runs) prefix[threadIdx.x] = before;
    if (threadIdx.x == 0) prefix[runs] = total;
    __syncthreads();
    return runs;
}

// Run holding concatenated position v: the largest r < runs with prefix[r] <= v.
__device__ inline int find_run(const int32_t* prefix, int runs, int32_t v) {
    int lo = 0, hi = runs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (prefix[mid] <= v) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Concatenated run positions [v0, v1) of a banded slice against one level.  Position v of run r
// is list entry run_k0[r] + v - prefix[r]: its coordinate's (x, y) in `sorted`, its upstream at
// the same entry of band-ordered planes (by_list), else at its index in `list`.  Each wave walks its own contiguous share of [v0, v1), kBatch
// positions per lane per iteration, 64 apart; a lane's run only moves forward.
template <int F, bool HALF, int KIND>
__device__ inline void accumulate_runs(const float2* sorted, bool by_list, const Elem<HALF>* plane, const DevLevel lv,
                                       const int32_t* list, const int32_t* run_k0, const int32_t* prefix, int runs,
                                       int32_t v0, int32_t v1, uint32_t lo, uint32_t span, const float* scale,
                                       unsigned long long* acc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int32_t w0 = v0 + static_cast<int32_t>(static_cast<int64_t>(v1 - v0) * wave / kWaves);
    const int32_t w1 = v0 + static_cast<int32_t>(static_cast<int64_t>(v1 - v0) * (wave + 1) / kWaves);
    if (w0 >= w1) return;
    int r = find_run(prefix, runs, w0);
    for (int32_t v = w0 + lane; v < w1; v += kBatch * 64) {
        int32_t k[kBatch];
        bool ok[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int32_t p = v + b * 64 < w1 ? v + b * 64 : w1 - 1;
            while (r + 1 < runs && prefix[r + 1] <= p) ++r;
            k[b] = run_k0[r] + (p - prefix[r]);
            ok[b] = v + b * 64 < w1;
        }
        float2 xy[kBatch];
        float us[kBatch][F];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            xy[b] = sorted[k[b]];
            load_upstream<F, HALF>(plane, by_list ? k[b] : list[k[b]], scale, ok[b], us[b]);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) contribute<F, KIND>(xy[b].x, xy[b].y, us[b], lv, lo, span, acc);
    }
}

// Block -> work item.  Remapped (with at least one expert per XCD), each XCD takes a contiguous
// chunk of the items (an expert's slices share its coordinates in that XCD's L2).  Inside a chunk the heavy items -- the
// splits of every expert's coarse-group pass, `heavy` per expert, which walk all coordinates
// through several fully landing levels and take about six times as long as a fine slice --
// come first, so that they start at once instead of finishing after everything else.  A
// permutation of [0, blocks) that keeps every item in its chunk.
__device__ inline uint32_t work_of(uint32_t block, uint32_t blocks, int remap, uint32_t per_expert,
                                   uint32_t heavy) {
    uint32_t chunk = blocks, q = block, o = 0;
    if (remap) {
        chunk = blocks / kXcds;
        o = (block % kXcds) * chunk;
        q = block / kXcds;
    }
    if (heavy == 0 || heavy >= per_expert) return o + q;
    const auto heavy_before = [&](uint32_t w) {
        const uint32_t r = w % per_expert;
        return (w / per_expert) * heavy + (r < heavy ? r : heavy);
    };
    const uint32_t f0 = heavy_before(o), count = heavy_before(o + chunk) - f0;
    if (q < count) {
        const uint32_t k = f0 + q;
        return (k / heavy) * per_expert + k % heavy;
    }
    const uint32_t light = per_expert - heavy, m = (o - f0) + (q - count);
    return (m / light) * per_expert + heavy + m % light;
}

// Largest |upstream| of every column (level l, feature c: l * F + c) of every expert, over the
// 128-row records that meet the expert's coordinates, as float bits (non-negative floats and NaN
// order as unsigned integers).  Block (x, e) takes every gridDim.x-th run of kPeakRecords of
// expert e's records; thread t takes column t % columns of every (kPeakBlock / columns)-th
// record of the run; one LDS, then one global maximum per column.  peaks must be zero on entry.
constexpr int kPeakBlock = 256;
constexpr int kPeakRecords = 32;

__global__ __launch_bounds__(kPeakBlock) void column_peaks_kernel(OwnerArgs a, uint32_t* peaks) {
    __shared__ uint32_t block_peak[kPeakBlock];
    const int e = blockIdx.y;
    const int columns = a.n_levels * a.features;   // <= kPeakBlock (checked at launch)
    block_peak[threadIdx.x] = 0u;
    __syncthreads();
    int64_t base, stop;
    expert_range(a.offsets, a.n, e, base, stop);
    uint32_t mine = 0u;
    const int per = kPeakBlock / columns;
    const int column = threadIdx.x % columns, first = threadIdx.x / columns;
    if (stop > base && first < per) {
        const int64_t r0 = base / kMaxRows, r1 = (stop - 1) / kMaxRows;
        for (int64_t run = r0 + static_cast<int64_t>(blockIdx.x) * kPeakRecords; run <= r1;
             run += static_cast<int64_t>(gridDim.x) * kPeakRecords) {
            const int64_t end = run + kPeakRecords - 1 < r1 ? run + kPeakRecords - 1 : r1;
            for (int64_t q = run + first; q <= end; q += per) {
                const uint32_t v = __float_as_uint(a.blockmax[q * columns + column]) & 0x7fffffffu;
                mine = v > mine ? v : mine;
            }
        }
    }
    if (mine) atomicMax(block_peak + column, mine);
    __syncthreads();
    if (threadIdx.x < columns && block_peak[threadIdx.x])
        atomicMax(peaks + static_cast<int64_t>(e) * columns + threadIdx.x, block_peak[threadIdx.x]);
}

// Fixed-point shifts of level l's F columns of expert e, whose count coordinates the peaks cover.
template <int F>
__device__ inline void level_shifts(const OwnerArgs& a, int e, int l, int64_t count, int32_t* shift) {
    const uint32_t* peak = a.peaks + (static_cast<int64_t>(e) * a.n_levels + l) * F;
#pragma unroll
    for (int c = 0; c < F; ++c) shift[c] = column_shift(peak[c], count);
}

template <int F, bool HALF>
__global__ __launch_bounds__(kOwnerBlock) void owner_kernel(OwnerArgs a) {
    extern __shared__ unsigned long long acc[];
    __shared__ float rates[kRateTable];   // fused flush: the optimizer's step size of the recent ages
    using U = Elem<HALF>;
    const uint32_t per_expert = static_cast<uint32_t>(a.items);
    const uint32_t total = static_cast<uint32_t>(a.experts) * per_expert;
    const uint32_t work = work_of(blockIdx.x, gridDim.x, a.remap, per_expert, static_cast<uint32_t>(a.heavy));
    if (work >= total) return;
    const int e = work / per_expert;
    const int r = work % per_expert;

    // Item -> pass p, split s of `splits`, levels [l0, l1) and the slice [lo, hi) of the
    // expert's gradient (in floats).
    const bool grouped = r < a.group_splits;
    int s, splits, l0, l1, slice = 0;
    uint32_t lo, hi;
    if (grouped) {
        s = r;
        splits = a.group_splits;
        l0 = 0;
        l1 = a.group;
        lo = 0;
        hi = (a.level[a.group - 1].offset + a.level[a.group - 1].size) * F;
    } else {
        int l = a.group;
        while (l + 1 < a.n_levels && a.first_item[l + 1] <= r) ++l;
        splits = a.splits[l];
        slice = (r - a.first_item[l]) / splits;
        s = (r - a.first_item[l]) % splits;
        const uint32_t first = static_cast<uint32_t>(slice) * a.slice_entries[l];
        uint32_t last = first + a.slice_entries[l];
        if (last > a.level[l].size) last = a.level[l].size;
        l0 = l;
        l1 = l + 1;
        lo = (a.level[l].offset + first) * F;
        hi = (a.level[l].offset + last) * F;
    }
    const uint32_t span = hi - lo;

    // Coordinates of this expert, and this split's index range of them.  The scales are the
    // expert's (its column peaks and coordinate count), whichever share a split walks.
    int64_t base, stop;
    expert_range(a.offsets, a.n, e, base, stop);
    const int64_t share = (stop - base + splits - 1) / splits;
    const int64_t b0 = base + share * s < stop ? base + share * s : stop;
    const int64_t b1 = b0 + share < stop ? b0 + share : stop;
    const int64_t count = stop - base;
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) acc[j] = 0ull;
    if (a.fused && a.adam.variant != 0 && threadIdx.x < kRateTable)
        rates[threadIdx.x] = adam_rate(a.adam, a.adam.rate_first + threadIdx.x);
    __syncthreads();

    // A banded fine pass walks the pieces of its share of the band-list runs its rows reach.
    const bool banded = a.banded && !grouped && *a.ordered;
    int32_t* reserve = reinterpret_cast<int32_t*>(acc + a.cap);
    uint32_t* bits = reinterpret_cast<uint32_t*>(reserve);
    int32_t* run_k0 = reserve + kBandWords;
    int32_t* run_k1 = run_k0 + kMaxRuns;
    int32_t* prefix = run_k1 + kMaxRuns;
    int32_t* scratch = prefix + kMaxRuns + 1;
    int runs = 0;
    int64_t q0 = 0, q1 = 0;
    if (banded) {
        const DevLevel& lv = a.level[l0];
        mark_slice(lv, lo / F - lv.offset, hi / F - lv.offset, a.row_bits[l0], static_cast<uint32_t>(slice), bits);
        runs = slice_runs(bits, a.band_start + static_cast<int64_t>(e) * (kBandSlots + 1), run_k0, run_k1, prefix,
                          scratch);
        const int64_t listed = prefix[runs];
        q0 = listed * s / splits;
        q1 = listed * (s + 1) / splits;
    }

    // band-ordered planes: coordinates and upstream values at the same list positions, in every
    // pass (an expert's list positions are its index range, so the passes' ranges are unchanged)
    const bool by_list = a.band_planes && *a.ordered;
    const float* coords = by_list ? reinterpret_cast<const float*>(a.band_sorted) : a.coords;
    for (int l = l0; l < l1; ++l) {
        const DevLevel lv = a.level[l];
        const U* plane = reinterpret_cast<const U*>(a.planes) + static_cast<size_t>(l) * a.n * F;
        const int kind = level_kind(lv);
        int32_t shift[F];
        level_shifts<F>(a, e, l, count, shift);
        float scale[F];
#pragma unroll
        for (int c = 0; c < F; ++c) scale[c] = shift_scale(shift[c]);
        if (banded) {
            if (runs == 0) break;
            switch (kind) {
                case kHashed24: accumulate_runs<F, HALF, kHashed24>(a.band_sorted, by_list, plane, lv, a.band_list, run_k0, prefix, runs, static_cast<int32_t>(q0), static_cast<int32_t>(q1), lo, span, scale, acc); break;
                case kHashedPow2: accumulate_runs<F, HALF, kHashedPow2>(a.band_sorted, by_list, plane, lv, a.band_list, run_k0, prefix, runs, static_cast<int32_t>(q0), static_cast<int32_t>(q1), lo, span, scale, acc); break;
                case kGeneric: accumulate_runs<F, HALF, kGeneric>(a.band_sorted, by_list, plane, lv, a.band_list, run_k0, prefix, runs, static_cast<int32_t>(q0), static_cast<int32_t>(q1), lo, span, scale, acc); break;
                default: accumulate_runs<F, HALF, kDense>(a.band_sorted, by_list, plane, lv, a.band_list, run_k0, prefix, runs, static_cast<int32_t>(q0), static_cast<int32_t>(q1), lo, span, scale, acc); break;
            }
        } else if (!grouped && a.masks && a.mask_plane[l] >= 0) {
            const uint8_t* mask = a.masks + static_cast<int64_t>(a.mask_plane[l]) * a.mask_stride;
            int32_t* ring = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(acc) + a.ring_at) + (threadIdx.x >> 6) * kRing;
            switch (kind) {
                case kHashed24: accumulate_masked<F, HALF, kHashed24>(a.coords, plane, mask, lv, b0, b1, static_cast<uint32_t>(slice), lo, span, scale, acc, ring); break;
                case kHashedPow2: accumulate_masked<F, HALF, kHashedPow2>(a.coords, plane, mask, lv, b0, b1, static_cast<uint32_t>(slice), lo, span, scale, acc, ring); break;
                case kGeneric: accumulate_masked<F, HALF, kGeneric>(a.coords, plane, mask, lv, b0, b1, static_cast<uint32_t>(slice), lo, span, scale, acc, ring); break;
                default: accumulate_masked<F, HALF, kDense>(a.coords, plane, mask, lv, b0, b1, static_cast<uint32_t>(slice), lo, span, scale, acc, ring); break;
            }
        } else {
            switch (kind) {
                case kHashed24:
                    if (grouped) accumulate_level<F, HALF, kHashed24, kGroupBatch>(coords, plane, lv, b0, b1, lo, span, scale, acc);
                    else accumulate_level<F, HALF, kHashed24>(coords, plane, lv, b0, b1, lo, span, scale, acc);
                    break;
                case kHashedPow2: accumulate_level<F, HALF, kHashedPow2>(coords, plane, lv, b0, b1, lo, span, scale, acc); break;
                case kGeneric: accumulate_level<F, HALF, kGeneric>(coords, plane, lv, b0, b1, lo, span, scale, acc); break;
                default:
                    if (grouped) accumulate_level<F, HALF, kDense, kGroupBatch>(coords, plane, lv, b0, b1, lo, span, scale, acc);
                    else accumulate_level<F, HALF, kDense>(coords, plane, lv, b0, b1, lo, span, scale, acc);
                    break;
            }
        }
    }
    __syncthreads();
    if (splits > 1 && a.banded) {
        // raw 64-bit sums: banded_reduce_kernel adds the splits exactly and applies the scales
        long long* out = a.partial64 + (static_cast<int64_t>(s) * a.experts + e) * a.partial_floats + lo;
        for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) out[j] = static_cast<long long>(acc[planar<F>(j, span)]);
        return;
    }
    // Value j of the slice is feature j % F of entry lo / F + j / F.  A thread's j only grows, so
    // its level (and the shifts of that level's columns) only moves forward.
    int level = l0;
    int32_t shift[F];
    level_shifts<F>(a, e, level, count, shift);
    const auto shift_of = [&](uint32_t j) {
        const uint32_t entry = lo / F + j / F;
        if (level + 1 < l1 && a.level[level + 1].offset <= entry) {
            while (level + 1 < l1 && a.level[level + 1].offset <= entry) ++level;
            level_shifts<F>(a, e, level, count, shift);
        }
        return shift[j % F];
    };
    if (a.fused && splits == 1) {
        // The final gradient of these parameters is in LDS: update them right here.  One
        // workgroup holds the CU, so the loads of four elements per thread are issued before
        // any of them is used, to keep memory latency off the critical path.
        const AdamStep& o = a.adam;
        const int64_t first = static_cast<int64_t>(e) * a.expert_params + lo;
        for (uint32_t j0 = threadIdx.x; j0 < span; j0 += kBatch * kOwnerBlock) {
            float g[kBatch], w[kBatch], m[kBatch], v[kBatch];
            uint32_t age[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const uint32_t j = j0 + k * kOwnerBlock;
                const int64_t i = first + (j < span ? j : 0);
                w[k] = o.master[i];
                m[k] = o.m[i];
                v[k] = o.v[i];
                age[k] = o.variant != 0 ? o.steps[i] : 0u;
                const uint32_t jj = j < span ? j : 0;
                g[k] = unscaled(static_cast<long long>(acc[planar<F>(jj, span)]), j < span ? shift_of(j) : 0);
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const uint32_t j = j0 + k * kOwnerBlock;
                if (j >= span) continue;
                const int64_t i = first + j;
                if (adam_math(o, g[k], w[k], m[k], v[k], age[k], rates)) {
                    o.master[i] = w[k];
                    o.m[i] = m[k];
                    o.v[i] = v[k];
                    if (o.variant != 0) o.steps[i] = age[k];
                }
                if (o.half_copy) o.half_copy[i] = half_to_bits(__float2half_rn(w[k]));
            }
        }
        return;
    }
    float* out = splits == 1 ? a.grad + static_cast<size_t>(e) * a.expert_params + lo
                               : a.partial + static_cast<size_t>(s) * a.experts * a.expert_params +
                                     static_cast<size_t>(e) * a.expert_params + lo;
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) {
        float v = unscaled(static_cast<long long>(acc[planar<F>(j, span)]), shift_of(j));
        if (splits == 1 && a.accumulate) v += out[j];
        out[j] = v;
    }
}

// Banded splits: every entry of the first partial_floats values of every expert whose pass is
// split gets the exact sum of its splits' 64-bit partials, scaled by its column's 2^-shift (the
// same in every pass and split of the level: each bounds it over all of the expert's
// coordinates), and is written (added with accumulate) or handed to the optimizer step, as the
// owner does unsplit.
__global__ __launch_bounds__(256) void banded_reduce_kernel(OwnerArgs a) {
    const int64_t count = static_cast<int64_t>(a.experts) * a.partial_floats;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t y = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; y < count; y += stride) {
        const int e = static_cast<int>(y / a.partial_floats);
        const int64_t x = y % a.partial_floats;
        const uint32_t entry = static_cast<uint32_t>(x / a.features);
        int l = 0;
        while (l + 1 < a.n_levels && a.level[l + 1].offset <= entry) ++l;
        const int splits = l >= a.group ? a.splits[l] : a.group_splits;
        if (splits <= 1) continue;
        // eight independent loads in flight per round: the splits' partials are far apart
        const long long* column = a.partial64 + static_cast<int64_t>(e) * a.partial_floats + x;
        const int64_t step = static_cast<int64_t>(a.experts) * a.partial_floats;
        long long sum = 0;
        int s = 0;
        for (; s + 8 <= splits; s += 8) {
            long long v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = column[(s + k) * step];
#pragma unroll
            for (int k = 0; k < 8; ++k) sum += v[k];
        }
        for (; s < splits; ++s) sum += column[s * step];
        int64_t base, stop;
        expert_range(a.offsets, a.n, e, base, stop);
        const uint32_t peak = a.peaks[(static_cast<int64_t>(e) * a.n_levels + l) * a.features + x % a.features];
        float v = unscaled(sum, column_shift(peak, stop - base));
        const int64_t i = static_cast<int64_t>(e) * a.expert_params + x;
        if (a.fused) {
            adam_update(a.adam, i, v);
        } else {
            if (a.accumulate) v += a.grad[i];
            a.grad[i] = v;
        }
    }
}

// Sums the split partials of the first `prefix` values of every expert (prefix = expert_params:
// all of them) and writes the gradient or applies the optimizer step.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* partial, float* grad, int64_t total, int splits,
                                                           int accumulate, int fused, AdamStep adam,
                                                           int64_t expert_params, int64_t prefix) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t count = total / expert_params * prefix;
    for (int64_t y = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; y < count; y += stride) {
        const int64_t x = y / prefix * expert_params + y % prefix;
        float v = accumulate ? grad[x] : 0.0f;
        for (int s = 0; s < splits; ++s) v += partial[static_cast<size_t>(s) * total + x];
        if (fused)
            adam_update(adam, x, v);
        else
            grad[x] = v;
    }
}

// ---------------------------------------------------------------------------------------
// Owner-computes backward of packed xy planes (the reference's grid_back,
// odie/native/runtime.cu:111-137, without atomics).  Workgroup b owns the parameters
// [b*cap, (b+1)*cap) -- whole levels or a part of one, in plane-offset order -- and walks the
// coordinates (a share of them when split) through every level whose parameters meet its
// slice, adding w_k * u (the fp32 product) as 64-bit fixed point in LDS.  One scale per
// upstream column (level, feature), from that column's largest |u| over all coordinates, so every
// slice and split of a level shares it; split slices write their raw sums and
// packed_reduce_kernel adds them exactly, so the gradient is the same however it is split.
// ---------------------------------------------------------------------------------------
struct PackedOwnerArgs {
    const float* coords;
    const uint16_t* upstream;     // fp16 [n][width]
    const int32_t* desc;
    const uint64_t* node_bitmap;
    const int32_t* prefix;
    const uint8_t* bitmap;
    const uint32_t* bounds;       // [width]: largest fp16 magnitude (bits) of each upstream column
    float* gradient;
    long long* partial;           // [splits][params] when splits > 1
    int64_t n;
    int64_t params;
    int levels;
    int width;
    int cap;                      // values per slice
    int splits;
};

constexpr int kBoundBlock = 256;

// Largest |u| of every upstream column, as fp16 magnitude bits (their unsigned order is the
// magnitude order, NaN above infinity).  Thread t takes column t % width of every
// (kBoundBlock / width)-th row.  bounds must be zero on entry; width <= kBoundBlock.
__global__ __launch_bounds__(kBoundBlock) void packed_bound_kernel(PackedOwnerArgs a, uint32_t* bounds) {
    __shared__ uint32_t peak[kBoundBlock];
    peak[threadIdx.x] = 0u;
    __syncthreads();
    const int per = kBoundBlock / a.width;
    const int column = threadIdx.x % a.width, first = threadIdx.x / a.width;
    uint32_t mine = 0u;
    if (first < per) {
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * per + first; i < a.n; i += static_cast<int64_t>(gridDim.x) * per) {
            const uint32_t m = a.upstream[static_cast<size_t>(i) * a.width + column] & 0x7fffu;
            mine = m > mine ? m : mine;
        }
    }
    if (mine) atomicMax(peak + column, mine);
    __syncthreads();
    if (threadIdx.x < a.width && peak[threadIdx.x]) atomicMax(bounds + threadIdx.x, peak[threadIdx.x]);
}

__device__ inline int64_t level_end(const PackedOwnerArgs& a, int l) {
    return l + 1 < a.levels ? static_cast<int64_t>(a.desc[8 * (l + 1) + 2]) : a.params;
}

// Fixed-point shift of feature c of the level with descriptor d (upstream column d[6] + c).
__device__ inline int32_t packed_shift(const PackedOwnerArgs& a, const int32_t* d, int c) {
    const int column = d[6] + c;
    const uint32_t m = column < a.width ? a.bounds[column] : 0u;
    return column_shift(__float_as_uint(__half2float(bits_to_half(static_cast<uint16_t>(m)))), a.n);
}

// Coordinates [b0, b1) against one level of F features (1, 2 or 4; direct or ranked rows):
// every stage issues the loads of all kPackedBatch coordinates of a thread before using any of them
// (positions, cell bits, upstream values, the rank words of the four corners).
constexpr int kPackedBatch = 2;   // coordinates per thread per iteration (fits 128 VGPRs with F = 4)

template <int F, bool DIRECT>
__device__ inline void packed_level(const PackedOwnerArgs& a, const int32_t* d, int64_t b0, int64_t b1, int64_t lo,
                                    int64_t hi, unsigned long long* acc) {
    const int r = d[0], points = d[1], column = d[6];
    const int64_t first = d[2];
    float scale[F];
#pragma unroll
    for (int c = 0; c < F; ++c) scale[c] = shift_scale(packed_shift(a, d, c));
    for (int64_t i0 = b0 + threadIdx.x; i0 < b1; i0 += kPackedBatch * kOwnerBlock) {
        float2 xy[kPackedBatch];
#pragma unroll
        for (int b = 0; b < kPackedBatch; ++b) {
            const int64_t i = i0 + b * kOwnerBlock;
            xy[b] = reinterpret_cast<const float2*>(a.coords)[i < b1 ? i : b0];
        }
        int cell[kPackedBatch];
        float w[kPackedBatch][4];
        uint8_t bits[kPackedBatch];
        float us[kPackedBatch][F];
#pragma unroll
        for (int b = 0; b < kPackedBatch; ++b) {
            plane_geometry(xy[b].x, xy[b].y, r, cell[b], w[b]);
            bits[b] = a.bitmap[d[4] + (cell[b] >> 3)];
            const int64_t i = i0 + b * kOwnerBlock;
            const uint16_t* row = a.upstream + static_cast<size_t>(i < b1 ? i : b0) * a.width;
#pragma unroll
            for (int c = 0; c < F; ++c)
                us[b][c] = column + c < a.width ? __half2float(bits_to_half(row[column + c])) * scale[c] : 0.0f;
        }
        int node[kPackedBatch][4];
        int32_t base[kPackedBatch][4];
        uint64_t word[kPackedBatch][4];
#pragma unroll
        for (int b = 0; b < kPackedBatch; ++b)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                node[b][k] = (cell[b] + (k & 1) + (k >> 1) * r) % points;
                if constexpr (!DIRECT) {
                    const int at = d[3] + (node[b][k] >> 6);
                    base[b][k] = a.prefix[at];
                    word[b][k] = a.node_bitmap[at];
                }
            }
#pragma unroll
        for (int b = 0; b < kPackedBatch; ++b) {
            const bool on = i0 + b * kOwnerBlock < b1 && ((bits[b] >> (cell[b] & 7)) & 1);
            if (!on) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                int rank = node[b][k];
                if constexpr (!DIRECT)
                    rank = base[b][k] + __popcll(word[b][k] & ((uint64_t{1} << (node[b][k] & 63)) - uint64_t{1}));
#pragma unroll
                for (int c = 0; c < F; ++c) {
                    int64_t p = first + static_cast<int64_t>(rank) * F + c;
                    p = p < 0 ? 0 : (p >= a.params ? a.params - 1 : p);
                    const int32_t q = round_to_int(w[b][k] * us[b][c]);
                    if (p >= lo && p < hi)
                        atomicAdd(acc + (p - lo), static_cast<unsigned long long>(static_cast<long long>(q)));
                }
            }
        }
    }
}

// Level of parameter p: the last level whose plane offset is <= p (levels in offset order).
__device__ inline int packed_level_of(const PackedOwnerArgs& a, int64_t p) {
    int lo = 0, hi = a.levels - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.desc[8 * mid + 2] <= p) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Shift of parameter p (feature (p - offset) % F of its level).
__device__ inline int32_t packed_param_shift(const PackedOwnerArgs& a, int64_t p) {
    const int32_t* d = a.desc + 8 * packed_level_of(a, p);
    const int features = d[5] > 0 ? d[5] : 1;
    return packed_shift(a, d, static_cast<int>((p - d[2]) % features));
}

__global__ __launch_bounds__(kOwnerBlock) void packed_owner_kernel(PackedOwnerArgs a) {
    extern __shared__ unsigned long long acc[];
    const int slice = blockIdx.x / a.splits, s = blockIdx.x % a.splits;
    const int64_t lo = static_cast<int64_t>(slice) * a.cap;
    const int64_t hi = lo + a.cap < a.params ? lo + a.cap : a.params;
    const uint32_t span = static_cast<uint32_t>(hi - lo);
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) acc[j] = 0ull;
    __syncthreads();
    const int64_t share = (a.n + a.splits - 1) / a.splits;
    const int64_t b0 = share * s < a.n ? share * s : a.n;
    const int64_t b1 = b0 + share < a.n ? b0 + share : a.n;
    for (int l = 0; l < a.levels; ++l) {
        if (level_end(a, l) <= lo || a.desc[8 * l + 2] >= hi) continue;
        const int32_t* d = a.desc + 8 * l;
        const bool direct = d[7] != 0;
        switch (d[5]) {
            case 1: direct ? packed_level<1, true>(a, d, b0, b1, lo, hi, acc)
                           : packed_level<1, false>(a, d, b0, b1, lo, hi, acc); break;
            case 2: direct ? packed_level<2, true>(a, d, b0, b1, lo, hi, acc)
                           : packed_level<2, false>(a, d, b0, b1, lo, hi, acc); break;
            default: direct ? packed_level<4, true>(a, d, b0, b1, lo, hi, acc)
                            : packed_level<4, false>(a, d, b0, b1, lo, hi, acc); break;
        }
    }
    __syncthreads();
    if (a.splits > 1) {
        long long* out = a.partial + static_cast<int64_t>(s) * a.params + lo;
        for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) out[j] = static_cast<long long>(acc[j]);
        return;
    }
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock)
        a.gradient[lo + j] = unscaled(static_cast<long long>(acc[j]), packed_param_shift(a, lo + j));
}

__global__ __launch_bounds__(256) void packed_reduce_kernel(PackedOwnerArgs a) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t x = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; x < a.params; x += stride) {
        long long sum = 0;
        for (int s = 0; s < a.splits; ++s) sum += a.partial[static_cast<int64_t>(s) * a.params + x];
        a.gradient[x] = unscaled(sum, packed_param_shift(a, x));
    }
}

template <typename Kernel>
int allow_lds(Kernel kernel, size_t bytes) {
    const hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (status != hipSuccess) return fail(std::string("LDS attribute: ") + hipGetErrorString(status));
    return 0;
}

// Expected fraction of an expert's coordinates listed in the band runs of one slice of level
// lv (uniform y), used only to size the splits: cell rows the slice's table rows are reached
// from, over all cell rows, plus a slot at either end of every run.
double band_coverage(const DevLevel& lv, int64_t entries, int64_t slices, int row_bits) {
    const double top = std::floor(std::fmaf(lv.scale, 1.0f, 0.5f));
    if (!(lv.scale >= 1.0f) || !(top < 16777216.0)) return 1.0;
    const double rows = top + 1.0;                                     // cell rows
    double share;
    if (!lv.hashed) share = (static_cast<double>(entries) / lv.res + 3.0) / rows + 2.0 / kBands;
    else if (row_bits > 0) share = (rows + 1.0) / slices * (std::floor((rows + 1.0) / std::ldexp(1.0, row_bits)) + 1.0) *
                                   (2.0 / rows + 2.0 / kBands);
    else share = 1.0;
    return share < 1.0 ? share : 1.0;
}

}  // namespace

// The band lists of every expert's coordinates (count, per-slot scan, starts, place) on in.stream.
int build_band_lists(const OwnerLaunch& in, int parts, int32_t* counts, int32_t* start, int32_t* list, float2* sorted,
                     int32_t* ordered) {
    BandArgs b{};
    b.coords = in.coords;
    b.offsets = in.offsets;
    b.n = in.n;
    b.experts = in.experts;
    b.parts = parts;
    b.counts = counts;
    b.start = start;
    b.list = list;
    b.sorted = sorted;
    b.ordered = ordered;
    const uint32_t blocks = round_up(static_cast<uint32_t>(in.experts) * parts, kXcds);
    int group = 1;
    while (group < parts && group < 64) group <<= 1;
    const int per = (parts + group - 1) / group;
    const int64_t column_waves = static_cast<int64_t>(in.experts) * kBandSlots / (64 / group);
    const uint32_t column_blocks = static_cast<uint32_t>((column_waves + kWaves - 1) / kWaves);
    hipStream_t s = in.stream;
    band_kernel<false><<<blocks, kBandBlock, 0, s>>>(b);
    band_columns_kernel<<<column_blocks, kBandBlock, 0, s>>>(b, group, per);
    band_start_kernel<<<static_cast<uint32_t>(in.experts), kBandBlock, 0, s>>>(b);
    band_kernel<true><<<blocks, kBandBlock, 0, s>>>(b);
    return check_launch("owner band lists");
}

int launch_owner_backward(const OwnerLaunch& in) {
    const int F = in.features;
    const int L = in.n_levels;
    const bool half = in.up_half != 0;
    const size_t elem = half ? 2 : 4;
    const int64_t lds_bytes = in.lds_bytes;
    // int64 accumulators per slice, minus entry rounding; the band workspace after them (kept in
    // both modes so that both slice alike and choose the same coarse group)
    const int64_t cap = (lds_bytes - kReserveBytes) / 8 - F;
    if (cap < 64) return fail("odie_grid_backward: LDS budget too small for the owner backward");
    if (L * F > kPeakBlock) return fail("odie_grid_backward: more than 256 (level, feature) columns");
    OwnerArgs o{};
    o.coords = in.coords;
    o.offsets = in.offsets;
    o.n = in.n;
    o.expert_params = in.expert_params;
    o.experts = in.experts;
    o.n_levels = L;
    o.features = F;
    o.accumulate = in.accumulate;
    o.fused = in.adam != nullptr;
    if (in.adam) o.adam = *in.adam;
    // XCD-major items only when every XCD's chunk holds whole experts: with fewer experts than
    // XCDs a chunk is a run of one expert's items, so the coarse-group splits (the heaviest,
    // numbered first) would all land on the first XCDs (measured, one expert of 2^19-entry levels
    // and 2^22 coordinates: 1.00 ms remapped against 0.80 ms in launch order, which deals the
    // items round-robin over the XCDs).
    o.remap = in.remap && in.experts >= kXcds;
    int group = 0;
    int64_t grouped = 0;
    // the coarse group: the leading levels whose values fit the slice
    while (group < L && grouped + static_cast<int64_t>(in.levels[group].size) * F <= cap) {
        grouped += static_cast<int64_t>(in.levels[group].size) * F;
        ++group;
    }
    int bits = 0;
    while ((int64_t{2} << bits) * F <= cap) ++bits;   // 2^bits entries: largest block that fits
    // Slices of the finer levels: as many equal parts as the LDS needs; banded, hashed levels
    // take aligned blocks of 2^bits entries (a block is reached from the rows whose hash selects it).
    // Masked levels take aligned blocks of 2^bits entries too (the last one short on a dense level).
    const auto slice_level = [&](int l, bool band, bool masked, int64_t& slices, int64_t& entries, int& row_bits) {
        const DevLevel& lv = in.levels[l];
        slices = (static_cast<int64_t>(lv.size) * F + cap - 1) / cap;
        entries = (lv.size + slices - 1) / slices;
        row_bits = 0;
        if (masked) {
            entries = int64_t{1} << bits;
            slices = (lv.size + entries - 1) / entries;
            row_bits = bits;
        } else if (band && lv.hashed && lv.mask && (int64_t{1} << bits) < lv.size) {
            entries = int64_t{1} << bits;
            slices = lv.size / entries;
            row_bits = bits;
        }
    };
    // Banded or not: band lists cost a pre-pass and make every listed visit a gather, so they
    // pay when they cut the visits (coordinates times passes) at least four times over, as with
    // few experts of large tables (measured on MI355X: 2.3x faster with one expert of 2^19-entry
    // levels, 1.07x slower with 64 experts of 2^16).  Band lists hold int32 coordinate indices.
    bool banded = in.banded == 1;
    if (in.banded == 2 && group < L && in.n < (int64_t{1} << 31) - 1) {
        double plain = group, listed = group;
        for (int l = group; l < L; ++l) {
            int64_t slices, entries;
            int row_bits;
            slice_level(l, false, false, slices, entries, row_bits);
            plain += slices;
            slice_level(l, true, false, slices, entries, row_bits);
            listed += slices * band_coverage(in.levels[l], entries, slices, row_bits);
        }
        banded = listed * 4.0 <= plain;
    }
    banded = banded && in.n < (int64_t{1} << 31) - 1;
    o.banded = banded;
    // Slice masks (unbanded): a level cut into 2..8 aligned blocks of 2^bits entries whose
    // accumulators leave room for the waves' rings in the dynamic LDS.
    const size_t shmem = static_cast<size_t>(cap + F) * 8 + kReserveBytes;
    MaskArgs mask_args{};
    for (int l = 0; l < L; ++l) o.mask_plane[l] = -1;
    for (int l = group; l < L && in.masks && !banded; ++l) {
        const DevLevel& lv = in.levels[l];
        const int64_t block = int64_t{1} << bits;
        const bool fits = static_cast<size_t>(block * F * 8 + kRingBytes) <= shmem;
        if (block < lv.size && (lv.size + block - 1) / block <= 8 && fits && mask_args.planes < kMaxMaskPlanes) {
            o.mask_plane[l] = mask_args.planes;
            mask_args.bits[mask_args.planes] = bits;
            mask_args.level[mask_args.planes] = lv;
            ++mask_args.planes;
        }
    }
    const int64_t mask_stride = (in.n + 255) / 256 * 256;
    o.ring_at = static_cast<int>(shmem - kRingBytes);
    int passes = group > 0 ? 1 : 0;
    for (int l = 0; l < L; ++l) {
        o.level[l] = in.levels[l];
        if (l < group) continue;
        int64_t slices, entries;
        slice_level(l, banded, o.mask_plane[l] >= 0, slices, entries, o.row_bits[l]);
        o.slices[l] = static_cast<int>(slices);
        o.slice_entries[l] = static_cast<int>(entries);
        passes += static_cast<int>(slices);
    }
    o.group = group;
    o.cap = static_cast<int>(cap + F);

    // Splits per pass.
    int group_splits = group > 0 ? 1 : 0;
    for (int l = group; l < L; ++l) o.splits[l] = 1;
    int64_t max_splits = 1;
    if (banded) {
        // Size every item near a target share of the estimated work (coordinate-level visits):
        // an eighth of a CU's share of the whole pass (less, below), at least 65536 visits (each item pays a
        // fixed set-up; measured best on MI355X for one expert of 2^19-entry levels and 2^22
        // coordinates).  A visit of the coarse group counts kGroupCost times: all of its
        // contributions land in its slice (measured).
        constexpr double kGroupCost = 2.5;
        const double per = static_cast<double>(in.n) / in.experts;
        double work = kGroupCost * group * per;
        for (int l = group; l < L; ++l)
            work += o.slices[l] * per * band_coverage(in.levels[l], o.slice_entries[l], o.slices[l], o.row_bits[l]);
        constexpr double kLeastItem = 65536.0;
        // With band-ordered planes (one expert, the backward's own transpose) a visit reads its
        // upstream value in order instead of gathering it, so the fixed cost of an item weighs
        // more: 1/2.8 of a CU's share there, ~195000 visits for the same single expert (measured
        // in launch order: 0.79 ms at fixed splits of 190000 and 200000 visits, 0.81-0.84 ms
        // from 100000 to 230000, 0.86 ms at an eighth, ~68000 -- the time moves in steps as the
        // ways per pass round up).
        const bool band_order = group < L && !in.planes && in.experts == 1;
        const double share = band_order ? 2.8 : 8.0;
        double target = in.split_target > 0 ? static_cast<double>(in.split_target) : work * in.experts / (share * kCus);
        if (in.split_target <= 0 && target < kLeastItem) target = kLeastItem;
        const auto ways = [&](double visits, double most) {
            const double w = std::ceil(visits / target);
            return static_cast<int>(w < 1.0 ? 1.0 : (w > most ? most : w));
        };
        if (group > 0) group_splits = ways(kGroupCost * group * per, 256.0);
        for (int l = group; l < L; ++l)
            o.splits[l] = ways(per * band_coverage(in.levels[l], o.slice_entries[l], o.slices[l], o.row_bits[l]), 64.0);
    } else {
        // Too few work items to fill the GPU: every pass is split over the coordinates (and the
        // partials summed by split_reduce_kernel).  Otherwise only the coarse-group pass may be:
        // it walks every coordinate through `group` fully landing levels, about group + 1 times
        // the work of a fine slice (measured: ~6x with 5 levels), and when that alone exceeds one
        // CU's share of the whole pass it would set the kernel's length, so it is cut into
        // pieces of about that share.
        const int64_t per_pass = static_cast<int64_t>(in.experts) * passes;
        int splits = 1;
        bool all = false;
        if (per_pass < 128) {
            const int64_t want = (512 + per_pass - 1) / per_pass;
            const int64_t most = in.n / (static_cast<int64_t>(in.experts) * 16384);
            splits = static_cast<int>(want < most ? want : (most > 1 ? most : 1));
            all = true;
        } else if (group > 0) {
            const double share = static_cast<double>(in.experts) * (passes + group) / kCus;   // fine-slice units
            if (group + 1 > share) {
                const int64_t want = static_cast<int64_t>(std::ceil((group + 1) / (share > 1.0 ? share : 1.0)));
                const int64_t most = in.n / (static_cast<int64_t>(in.experts) * 4096);
                splits = static_cast<int>(want < most ? want : (most > 1 ? most : 1));
            }
        }
        if (group > 0) group_splits = splits;
        if (all)
            for (int l = group; l < L; ++l) o.splits[l] = splits;
    }
    int items = group_splits;
    int heavy = group_splits;
    bool leading = banded;   // banded: the split levels' items (each about the target) come first
    int64_t split_floats = group_splits > 1 ? grouped : 0;   // values of the expert that splits cover
    for (int l = group; l < L; ++l) {
        o.first_item[l] = items;
        items += o.slices[l] * o.splits[l];
        if (o.splits[l] > 1) split_floats = static_cast<int64_t>(in.levels[l].offset + in.levels[l].size) * F;
        leading = leading && o.splits[l] > 1;
        if (leading) heavy = items;
        if (o.splits[l] > max_splits) max_splits = o.splits[l];
    }
    if (group_splits > max_splits) max_splits = group_splits;
    o.items = items;
    o.group_splits = group_splits;
    o.heavy = heavy;
    if (static_cast<int64_t>(in.experts) * items >= (int64_t{1} << 31))
        return fail("odie_grid_backward: too many owner work items");

    // Workspace: level-major planes, block maxima, split partials, band lists.
    const int64_t row_blocks = (in.n + kTransposeRows - 1) / kTransposeRows;
    const int64_t records = (in.n + kMaxRows - 1) / kMaxRows;
    const auto align = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const size_t planes_bytes = in.planes ? 0 : align(static_cast<size_t>(in.n) * L * F * elem);
    const size_t max_bytes = in.planes ? 0 : align(static_cast<size_t>(records) * L * F * 4);
    const size_t total_params = static_cast<size_t>(in.experts) * in.expert_params;
    const bool split = max_splits > 1;
    const size_t partial_bytes = split && !banded ? align(static_cast<size_t>(max_splits) * total_params * 4) : 0;
    const size_t partial64_bytes =
        split && banded ? align(static_cast<size_t>(max_splits) * in.experts * split_floats * 8) : 0;
    const size_t peak_bytes = align(static_cast<size_t>(in.experts) * L * F * 4);
    const bool lists = banded && group < L;
    const int parts = [&] {
        const int64_t want = (in.n / in.experts + kBandPart - 1) / kBandPart;
        return static_cast<int>(want < 1 ? 1 : (want > kMaxBandParts ? kMaxBandParts : want));
    }();
    const size_t count_bytes = lists ? align(static_cast<size_t>(in.experts) * parts * kBandSlots * 4) : 0;
    const size_t start_bytes = lists ? align(static_cast<size_t>(in.experts) * (kBandSlots + 1) * 4 + 4) : 0;
    const size_t list_bytes = lists ? align(static_cast<size_t>(in.n) * 4) : 0;
    const size_t sorted_bytes = lists ? align(static_cast<size_t>(in.n) * 8) : 0;
    // the handoff a forward can fill for this pass: the band lists (starts and the ordered word,
    // list, sorted), or the slice masks (masks are planned only for unbanded passes)
    const int64_t list_at = static_cast<int64_t>(start_bytes);
    const int64_t sorted_at = list_at + static_cast<int64_t>(list_bytes);
    const int64_t handoff_bytes = lists ? sorted_at + static_cast<int64_t>(sorted_bytes) : mask_stride * mask_args.planes;
    if (in.plan_out) {
        HandoffPlan& plan = *in.plan_out;
        plan = HandoffPlan{};
        plan.planes = mask_args.planes;
        plan.stride = mask_stride;
        for (int l = 0; l < L; ++l)
            if (o.mask_plane[l] >= 0) {
                plan.level[o.mask_plane[l]] = l;
                plan.bits[o.mask_plane[l]] = mask_args.bits[o.mask_plane[l]];
            }
        plan.lists = lists ? 1 : 0;
        plan.parts = parts;
        plan.ordered_at = static_cast<int64_t>(in.experts) * (kBandSlots + 1) * 4;
        plan.list_at = list_at;
        plan.sorted_at = sorted_at;
        plan.bytes = handoff_bytes;
        return 0;
    }
    const bool handed = in.handoff != nullptr && handoff_bytes > 0;
    if (handed && in.handoff_bytes < handoff_bytes)
        return fail("odie_grid_backward: the handoff buffer is shorter than the plan's (odie_grid_handoff_bytes)");
    const bool given_masks = handed && !lists;
    const bool given_lists = handed && lists;
    const size_t mask_bytes = given_masks ? 0 : static_cast<size_t>(mask_stride) * mask_args.planes;
    const size_t sizes[] = {planes_bytes, max_bytes, partial_bytes, partial64_bytes, peak_bytes,
                            given_lists ? 0 : count_bytes, given_lists ? 0 : start_bytes,
                            given_lists ? 0 : list_bytes, given_lists ? 0 : sorted_bytes, mask_bytes};
    constexpr int kParts = sizeof(sizes) / sizeof(sizes[0]);
    size_t at[kParts], sum = 0;
    for (int k = 0; k < kParts; ++k) {
        at[k] = sum;
        sum += sizes[k];
    }
    char* space = static_cast<char*>(workspace(sum, in.stream));
    if (!space) return -1;
    // upstream already level-major with its maxima (the caller wrote them): no transpose
    const bool given = in.planes != nullptr;
    o.planes = given ? in.planes : space + at[0];
    o.blockmax = given ? in.blockmax : reinterpret_cast<float*>(space + at[1]);
    o.partial = reinterpret_cast<float*>(space + at[2]);
    o.partial64 = reinterpret_cast<long long*>(space + at[3]);
    o.partial_floats = split_floats;
    uint32_t* peaks = reinterpret_cast<uint32_t*>(space + at[4]);
    o.peaks = peaks;
    const char* lists_at = given_lists ? reinterpret_cast<const char*>(in.handoff) : space + at[6];
    o.band_start = reinterpret_cast<const int32_t*>(lists_at);
    o.band_list = reinterpret_cast<const int32_t*>(given_lists ? lists_at + list_at : space + at[7]);
    o.band_sorted = reinterpret_cast<const float2*>(given_lists ? lists_at + sorted_at : space + at[8]);
    o.ordered = reinterpret_cast<const int32_t*>(lists_at + static_cast<size_t>(in.experts) * (kBandSlots + 1) * 4);
    o.masks = !mask_args.planes ? nullptr : given_masks ? in.handoff : reinterpret_cast<const uint8_t*>(space + at[9]);
    o.mask_stride = mask_stride;
    o.grad = in.grad;
    hipStream_t s = in.stream;

    if (lists && !given_lists &&
        build_band_lists(in, parts, reinterpret_cast<int32_t*>(space + at[5]), reinterpret_cast<int32_t*>(space + at[6]),
                         reinterpret_cast<int32_t*>(space + at[7]), reinterpret_cast<float2*>(space + at[8]),
                         const_cast<int32_t*>(o.ordered)))
        return -1;

    // the backward's own transpose writes the planes in band-list order (read in order by every
    // pass) for a single expert; planes the caller hands over stay in index order, and so do
    // several experts' (a 128-row record across two experts' ranges would hold other rows in list
    // order, and the column peaks it feeds, hence the fixed-point scales, would move)
    o.band_planes = lists && !given && in.experts == 1;
    TransposeArgs t{};
    t.list = o.band_planes ? o.band_list : nullptr;
    t.ordered = o.ordered;
    t.offsets = in.offsets;
    t.experts = in.experts;
    t.upstream = in.upstream;
    t.planes = space + at[0];
    t.blockmax = reinterpret_cast<float*>(space + at[1]);
    t.n = in.n;
    t.width = in.up_width;
    t.n_levels = L;
    t.vec_rows = (reinterpret_cast<uintptr_t>(in.upstream) % 16 == 0) && (in.up_width * elem) % 16 == 0 &&
                 (L * F * elem) % 16 == 0;
    const uint32_t tblocks = static_cast<uint32_t>(row_blocks);
    const uint32_t oblocks = round_up(static_cast<uint32_t>(static_cast<int64_t>(in.experts) * items), kXcds);

#define ODIE_TRANSPOSE(FF, HH)                                                                          \
    do {                                                                                                \
        if (FF == 2 && HH && t.vec_rows && L % 4 == 0) {                                                \
            if (L <= 16) transpose_half2_kernel<16><<<tblocks, kTransposeBlock, 0, s>>>(t);             \
            else transpose_half2_kernel<32><<<tblocks, kTransposeBlock, 0, s>>>(t);                     \
        } else if (L <= 16) transpose_kernel<FF, HH, 16><<<tblocks, kTransposeBlock, 0, s>>>(t);        \
        else transpose_kernel<FF, HH, 32><<<tblocks, kTransposeBlock, 0, s>>>(t);                       \
    } while (0)
    // every column's peak over each expert's records, the slice masks, then the owner pass
    const auto launch_peaks = [&]() {
        const int64_t peak_words = static_cast<int64_t>(in.experts) * L * F;
        if (mask_args.planes && !given_masks) {   // the mask launch clears the peaks as well
            mask_args.coords = in.coords;
            mask_args.masks = const_cast<uint8_t*>(o.masks);
            mask_args.peaks = peaks;
            mask_args.peak_words = peak_words;
            mask_args.n = in.n;
            mask_args.stride = mask_stride;
            slice_mask_kernel<<<static_cast<uint32_t>((in.n + 255) / 256), 256, 0, s>>>(mask_args);
        } else if (launch_fill_zero(reinterpret_cast<float*>(peaks), peak_words, s)) {
            return -1;
        }
        const int64_t runs = (records + static_cast<int64_t>(kPeakRecords) * in.experts - 1) /
                             (static_cast<int64_t>(kPeakRecords) * in.experts);
        const dim3 grid(static_cast<uint32_t>(runs < 1 ? 1 : runs), static_cast<uint32_t>(in.experts));
        column_peaks_kernel<<<grid, kPeakBlock, 0, s>>>(o, peaks);
        return 0;
    };
#define ODIE_OWNER(FF, HH)                                                                              \
    do {                                                                                                \
        if (launch_peaks()) return -1;                                                                  \
        if (allow_lds(owner_kernel<FF, HH>, shmem)) return -1;                                          \
        owner_kernel<FF, HH><<<oblocks, kOwnerBlock, shmem, s>>>(o);                                    \
    } while (0)
#define ODIE_BOTH(FF)                                                                                   \
    do {                                                                                                \
        if (half) { if (!given) ODIE_TRANSPOSE(FF, true); ODIE_OWNER(FF, true); }                      \
        else { if (!given) ODIE_TRANSPOSE(FF, false); ODIE_OWNER(FF, false); }                         \
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
    if (split && banded) {
        int64_t blocks = (static_cast<int64_t>(in.experts) * split_floats + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        banded_reduce_kernel<<<static_cast<uint32_t>(blocks), 256, 0, s>>>(o);
    } else if (split) {
        // the group pass alone split: the expert's first values; every pass split: all levels
        const int64_t levels_end = static_cast<int64_t>(in.levels[L - 1].offset + in.levels[L - 1].size) * F;
        const int64_t prefix = group == L || o.splits[L - 1] > 1 ? levels_end : grouped;
        int64_t blocks = (static_cast<int64_t>(in.experts) * prefix + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        split_reduce_kernel<<<static_cast<uint32_t>(blocks), 256, 0, s>>>(o.partial, in.grad,
                                                                          static_cast<int64_t>(total_params),
                                                                          static_cast<int>(max_splits),
                                                                          in.accumulate, o.fused, o.adam,
                                                                          in.expert_params, prefix);
    }
    return check_launch("odie_grid_backward");
}

int launch_band_lists(const OwnerLaunch& in, const HandoffPlan& plan, uint8_t* handoff) {
    if (!plan.lists) return 0;
    const size_t count_bytes = (static_cast<size_t>(in.experts) * plan.parts * kBandSlots * 4 + 255) / 256 * 256;
    int32_t* counts = static_cast<int32_t*>(workspace(count_bytes, in.stream));
    if (!counts) return -1;
    return build_band_lists(in, plan.parts, counts, reinterpret_cast<int32_t*>(handoff),
                            reinterpret_cast<int32_t*>(handoff + plan.list_at),
                            reinterpret_cast<float2*>(handoff + plan.sorted_at),
                            reinterpret_cast<int32_t*>(handoff + plan.ordered_at));
}

int launch_packed_owner(const float* coords, int64_t n, const uint16_t* upstream, int width, const int32_t* desc,
                        int levels, const uint64_t* node_bitmap, const int32_t* node_prefix, const uint8_t* bitmap,
                        float* gradient, int64_t params, int64_t lds_bytes, int64_t splits, hipStream_t stream) {
    const int64_t cap = lds_bytes / 8;
    if (cap < 1024) return fail("odie_packed_backward: LDS budget too small for the owner backward");
    const int64_t slices = (params + cap - 1) / cap;
    if (slices > (int64_t{1} << 24)) return fail("odie_packed_backward: too many parameters");
    // Split the coordinates when the slices alone leave CUs idle: about kCus workgroups, each
    // walking at least 4096 coordinates (splits > 0: that many).
    if (splits <= 0) {
        splits = (kCus + slices - 1) / slices;
        const int64_t most = n / 4096 > 1 ? n / 4096 : 1;
        if (splits > most) splits = most;
        if (splits > 64) splits = 64;
    }
    if (splits < 1) splits = 1;
    const auto align = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    if (width > kBoundBlock) return fail("odie_packed_backward: upstream width above 256");
    const size_t bound_bytes = align(static_cast<size_t>(width) * 4);
    const size_t partial_bytes = splits > 1 ? align(static_cast<size_t>(splits) * params * 8) : 0;
    char* space = static_cast<char*>(workspace(bound_bytes + partial_bytes, stream));
    if (!space) return -1;
    PackedOwnerArgs a{};
    a.coords = coords;
    a.upstream = upstream;
    a.desc = desc;
    a.node_bitmap = node_bitmap;
    a.prefix = node_prefix;
    a.bitmap = bitmap;
    a.bounds = reinterpret_cast<const uint32_t*>(space);
    a.gradient = gradient;
    a.partial = reinterpret_cast<long long*>(space + bound_bytes);
    a.n = n;
    a.params = params;
    a.levels = levels;
    a.width = width;
    a.cap = static_cast<int>(cap);
    a.splits = static_cast<int>(splits);
    uint32_t* bounds = reinterpret_cast<uint32_t*>(space);
    if (launch_fill_zero(reinterpret_cast<float*>(bounds), width, stream)) return -1;
    const int64_t rows_per_block = kBoundBlock / width;
    int64_t bound_blocks = (n + rows_per_block - 1) / rows_per_block;
    if (bound_blocks > 1024) bound_blocks = 1024;
    if (bound_blocks < 1) bound_blocks = 1;
    packed_bound_kernel<<<static_cast<uint32_t>(bound_blocks), kBoundBlock, 0, stream>>>(a, bounds);
    const size_t shmem = static_cast<size_t>(cap) * 8;
    if (allow_lds(packed_owner_kernel, shmem)) return -1;
    packed_owner_kernel<<<static_cast<uint32_t>(slices * splits), kOwnerBlock, shmem, stream>>>(a);
    if (splits > 1) {
        int64_t blocks = (params + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        packed_reduce_kernel<<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(a);
    }
    return check_launch("odie_packed_backward");
}

}  // namespace odie
