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
constexpr int kRing = 128;            // per-wave LDS queue of candidate coordinates (power of two)
constexpr int kRingBytes = kOwnerBlock / 64 * kRing * 4;

struct TransposeArgs {
    const void* upstream;
    void* planes;
    float* blockmax;
    int64_t n;
    int width;
    int n_levels;
    int vec_rows;
};

// Maximum of two |upstream| records; NaN wins, so the owner pass sees a non-finite bound.
__device__ inline float nan_max(float a, float b) { return (b > a || b != b) ? b : a; }

// Record q of the block (rows q*128.. of its 1024) is waves 2*(q%2) and 2*(q%2)+1 of pass q/2.
__device__ inline void write_records(const TransposeArgs& a, const float* waves, int lmax) {
    constexpr int kRecords = kTransposeRows / kMaxRows;
    for (int t = threadIdx.x; t < kRecords * a.n_levels; t += kTransposeBlock) {
        const int q = t / a.n_levels, l = t % a.n_levels;
        const int64_t record = static_cast<int64_t>(blockIdx.x) * kRecords + q;
        if (record * kMaxRows >= a.n) continue;
        const float* pass = waves + (q / 2) * (kTransposeBlock / 64) * lmax;
        const int w = 2 * (q % 2);
        a.blockmax[record * a.n_levels + l] = nan_max(pass[w * lmax + l], pass[(w + 1) * lmax + l]);
    }
}

template <int F, bool HALF, int LMAX>
__global__ __launch_bounds__(kTransposeBlock) void transpose_kernel(TransposeArgs a) {
    using U = Elem<HALF>;
    constexpr int kPasses = kTransposeRows / kTransposeBlock;
    __shared__ float waves[kPasses][kTransposeBlock / 64][LMAX];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int used = a.n_levels * F;
    for (int r = 0; r < kPasses; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        float peak[LMAX];
#pragma unroll
        for (int l = 0; l < LMAX; ++l) peak[l] = 0.0f;
        if (i < a.n) {
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
                    for (int c = 0; c < F; ++c) peak[l] = nan_max(peak[l], fabsf(static_cast<float>(vals[l * F + c])));
                }
            }
        }
        // the wave's 64 rows lie in one record of kMaxRows = 128 rows
#pragma unroll
        for (int l = 0; l < LMAX; ++l) {
            if (l < a.n_levels) {
                float m = peak[l];
                for (int step = 32; step; step >>= 1) m = nan_max(m, __shfl_xor(m, step));
                if (lane == 0) waves[r][wave][l] = m;
            }
        }
    }
    __syncthreads();
    write_records(a, &waves[0][0][0], LMAX);
}

// fp16 pairs (F = 2), levels a multiple of 4 and 16-byte rows: every thread loads its four
// rows first (16-byte loads), then writes one dword per level and row; |u| maxima are packed
// 16-bit magnitude maxima, two levels per dword, reduced over the wave's 64 rows (one half of
// a 128-row record).
template <int LMAX>
__global__ __launch_bounds__(kTransposeBlock) void transpose_half2_kernel(TransposeArgs a) {
    constexpr int kPasses = kTransposeRows / kTransposeBlock;
    constexpr int kChunks = LMAX / 4;  // 16-byte chunks per row (4 levels each)
    __shared__ uint32_t waves[kPasses][kTransposeBlock / 64][LMAX / 2];   // level pairs
    uint4 rows[kPasses][kChunks];
    const int chunks = a.n_levels / 4;
#pragma unroll
    for (int r = 0; r < kPasses; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        const uint4* row = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.upstream) +
                                                          static_cast<size_t>(i < a.n ? i : 0) * a.width);
#pragma unroll
        for (int j = 0; j < kChunks; ++j) rows[r][j] = j < chunks ? row[j] : make_uint4(0, 0, 0, 0);
    }
    uint32_t* planes = reinterpret_cast<uint32_t*>(a.planes);
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
#pragma unroll
    for (int r = 0; r < kPasses; ++r) {
        const int64_t i = static_cast<int64_t>(blockIdx.x) * kTransposeRows + r * kTransposeBlock + threadIdx.x;
        const bool valid = i < a.n;
        uint32_t peak[LMAX / 2];
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const uint32_t words[4] = {rows[r][j].x, rows[r][j].y, rows[r][j].z, rows[r][j].w};
            if (valid && j < chunks) {
#pragma unroll
                for (int q = 0; q < 4; ++q) planes[static_cast<size_t>(4 * j + q) * a.n + i] = words[q];
            }
            peak[2 * j] = valid ? pair_peak(words[0], words[1]) : 0u;
            peak[2 * j + 1] = valid ? pair_peak(words[2], words[3]) : 0u;
        }
#pragma unroll
        for (int p = 0; p < LMAX / 2; ++p) {
            if (2 * p < a.n_levels) {
                uint32_t m = peak[p];
                for (int step = 32; step; step >>= 1) m = pair_max(m, __shfl_xor(m, step));
                if (lane == 0) waves[r][wave][p] = m;
            }
        }
    }
    __syncthreads();
    constexpr int kRecords = kTransposeRows / kMaxRows;
    for (int t = threadIdx.x; t < kRecords * a.n_levels; t += kTransposeBlock) {
        const int q = t / a.n_levels, l = t % a.n_levels;
        const int64_t record = static_cast<int64_t>(blockIdx.x) * kRecords + q;
        if (record * kMaxRows >= a.n) continue;
        const uint32_t both = pair_max(waves[q / 2][2 * (q % 2)][l / 2], waves[q / 2][2 * (q % 2) + 1][l / 2]);
        a.blockmax[record * a.n_levels + l] = __half2float(bits_to_half(static_cast<uint16_t>(both >> (16 * (l % 2)))));
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
    int split_passes; // passes 0 .. split_passes-1 are split `splits` ways
    DevLevel level[ODIE_MAX_LEVELS];
    int first_pass[ODIE_MAX_LEVELS];
    int slices[ODIE_MAX_LEVELS];
    int slice_entries[ODIE_MAX_LEVELS];
    int row_bits[ODIE_MAX_LEVELS];   // > 0: slices are aligned 2^row_bits blocks screened by row
    int cap;                         // int64 accumulators in LDS; the candidate rings follow them
    int fused;                       // 1: apply the optimizer step instead of writing the gradient
    AdamStep adam;
    // Bucketed fine passes: pass p >= fine_first of expert e walks only the coordinates listed
    // in its bucket, list + start_e * fine_passes + (p - fine_first) * n_e, of length
    // bucket_count[e * fine_passes + p - fine_first] (start_e, n_e: the expert's coordinates).
    int bucketed;
    int fine_first;
    int fine_passes;
    const int32_t* bucket_count;
    const int32_t* bucket_list;
    int slice_bits[ODIE_MAX_LEVELS]; // bucketed: slice of entry j is j >> slice_bits
};

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
template <int F, int KIND>
__device__ inline void contribute(float x, float y, const float* us, const DevLevel& lv, uint32_t lo, uint32_t span,
                                  unsigned long long* acc) {
    const float px = __builtin_fmaf(lv.scale, x, 0.5f);
    const float py = __builtin_fmaf(lv.scale, y, 0.5f);
    const float flx = floorf(px), fly = floorf(py);
    const uint32_t gx = static_cast<uint32_t>(static_cast<int32_t>(flx));
    const uint32_t gy = static_cast<uint32_t>(static_cast<int32_t>(fly));
    const float fx = px - flx, fy = py - fly;
    float w[4];
    w[0] = (1.0f - fx) * (1.0f - fy);
    w[1] = fx * (1.0f - fy);
    w[2] = (1.0f - fx) * fy;
    w[3] = fx * fy;
    uint32_t idx[4];
    corner_index<KIND>(gx, gy, lv, idx);
    int32_t q[4][F];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int c = 0; c < F; ++c) q[k][c] = round_to_int(w[k] * us[c]);
    const uint32_t shift = lv.offset * F - lo;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t slot = idx[k] * F + shift;
        if (slot >= span) continue;
#pragma unroll
        for (int c = 0; c < F; ++c)
            atomicAdd(acc + slot + c, static_cast<unsigned long long>(static_cast<long long>(q[k][c])));
    }
}

template <int F, bool HALF>
__device__ inline void load_upstream(const Elem<HALF>* plane, int64_t at, float scale, bool valid, float* us) {
    if constexpr (HALF && F == 2) {
        const uint32_t word = *reinterpret_cast<const uint32_t*>(plane + at * F);
        us[0] = __half2float(bits_to_half(static_cast<uint16_t>(word & 0xffffu)));
        us[1] = __half2float(bits_to_half(static_cast<uint16_t>(word >> 16)));
    } else {
#pragma unroll
        for (int c = 0; c < F; ++c) us[c] = static_cast<float>(plane[at * F + c]);
    }
#pragma unroll
    for (int c = 0; c < F; ++c) us[c] = valid ? us[c] * scale : 0.0f;
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
template <int F, bool HALF, int KIND>
__device__ inline void accumulate_level(const float* coords, const Elem<HALF>* plane, const DevLevel lv, int64_t b0,
                                        int64_t b1, uint32_t lo, uint32_t span, float scale,
                                        unsigned long long* acc) {
    for (int64_t i = b0 + lane_offset<KIND>(); i < b1; i += kBatch * kOwnerBlock) {
        float2 xy[kBatch];
        float us[kBatch][F];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int64_t ii = i + b * kOwnerBlock;
            const int64_t at = ii < b1 ? ii : b0;
            xy[b] = reinterpret_cast<const float2*>(coords)[at];
            load_upstream<F, HALF>(plane, at, scale, ii < b1, us[b]);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) contribute<F, KIND>(xy[b].x, xy[b].y, us[b], lv, lo, span, acc);
    }
}

// The coordinates listed in list[k0, k1) against one level (a bucket of one slice).
template <int F, bool HALF, int KIND>
__device__ inline void accumulate_bucket(const float* coords, const Elem<HALF>* plane, const DevLevel lv,
                                         const int32_t* list, int64_t k0, int64_t k1, uint32_t lo, uint32_t span,
                                         float scale, unsigned long long* acc) {
    for (int64_t k = k0 + threadIdx.x; k < k1; k += kBatch * kOwnerBlock) {
        int32_t at[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int64_t kk = k + b * kOwnerBlock;
            at[b] = list[kk < k1 ? kk : k0];
        }
        float2 xy[kBatch];
        float us[kBatch][F];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            xy[b] = reinterpret_cast<const float2*>(coords)[at[b]];
            load_upstream<F, HALF>(plane, at[b], scale, k + b * kOwnerBlock < k1, us[b]);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) contribute<F, KIND>(xy[b].x, xy[b].y, us[b], lv, lo, span, acc);
    }
}

// A hashed level whose table slice is the aligned block of 2^row_bits entries number `slice`,
// with 2^row_bits above the level's resolution: corner (cx, cy) with cx <= res lands in slice
// ((cy * 2654435761) & mask) >> row_bits whatever cx is, so a coordinate can only touch the
// slice through its rows gy or gy+1.  Each wave screens its own contiguous share of the
// coordinates with that y-only test, queues the candidates in its private LDS ring and runs
// the full contribution only for them, 64 at a time.  Coordinates with x outside [0,1] are
// always queued (their corner columns are not bounded by the resolution).
template <int F, bool HALF>
__device__ inline void accumulate_rows(const float* coords, const Elem<HALF>* plane, const DevLevel lv, int64_t b0,
                                       int64_t b1, uint32_t lo, uint32_t span, float scale, unsigned long long* acc,
                                       int32_t* ring, uint32_t row_bits, uint32_t slice) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kWaves = kOwnerBlock / 64;
    const int64_t per = ((b1 - b0 + kWaves - 1) / kWaves + 63) / 64 * 64;
    const int64_t w0 = b0 + wave * per < b1 ? b0 + wave * per : b1;
    const int64_t w1 = w0 + per < b1 ? w0 + per : b1;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    const uint32_t row_mask = lv.mask >> row_bits;
    uint32_t head = 0, count = 0;
    auto drain = [&](uint32_t take) {
        const bool active = static_cast<uint32_t>(lane) < take;
        const int64_t i = active ? ring[(head + lane) & (kRing - 1)] : b0;
        const float2 xy = reinterpret_cast<const float2*>(coords)[i];
        float us[F];
        load_upstream<F, HALF>(plane, i, scale, active, us);
        if (lv.mask < (1u << 24)) contribute<F, kHashed24>(xy.x, xy.y, us, lv, lo, span, acc);
        else contribute<F, kHashedPow2>(xy.x, xy.y, us, lv, lo, span, acc);
        head += take;
        count -= take;
    };
    for (int64_t g = w0; g < w1; g += 64 * kBatch) {
        float2 xy[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int64_t i = g + b * 64 + lane;
            xy[b] = reinterpret_cast<const float2*>(coords)[i < w1 ? i : b0];
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int64_t i = g + b * 64 + lane;
            const float py = __builtin_fmaf(lv.scale, xy[b].y, 0.5f);
            const uint32_t gy = static_cast<uint32_t>(static_cast<int32_t>(floorf(py)));
            const uint32_t r0 = (hash_row(gy, lv) >> row_bits) & row_mask;
            const uint32_t r1 = (hash_row(gy + 1u, lv) >> row_bits) & row_mask;
            const bool inside = xy[b].x >= 0.0f && xy[b].x <= 1.0f;
            const bool pick = i < w1 && (r0 == slice || r1 == slice || !inside);
            const uint64_t picks = __ballot(pick);
            if (pick) ring[(head + count + __popcll(picks & below)) & (kRing - 1)] = static_cast<int32_t>(i);
            count += __popcll(picks);
            if (count >= 64) drain(64);
        }
    }
    while (count > 0) drain(count < 64 ? count : 64);
}

// Bucketing of the fine passes: for every coordinate of an expert and every fine level, the
// distinct slices its four corners fall in; each (expert, slice) bucket receives the
// coordinate's index once.  A workgroup counts its share of one expert's coordinates per bucket
// in LDS, reserves its run of every bucket with one global atomic, then writes the indices.
// The order inside a bucket does not matter: the owner's integer sums are order free.
constexpr int kBucketBlock = 256;

template <int KIND>
__device__ inline int slices_of(float x, float y, const DevLevel& lv, int bits, int slices[4]) {
    const float px = __builtin_fmaf(lv.scale, x, 0.5f);
    const float py = __builtin_fmaf(lv.scale, y, 0.5f);
    const uint32_t gx = static_cast<uint32_t>(static_cast<int32_t>(floorf(px)));
    const uint32_t gy = static_cast<uint32_t>(static_cast<int32_t>(floorf(py)));
    uint32_t idx[4];
    corner_index<KIND>(gx, gy, lv, idx);
    int count = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int slice = static_cast<int>(idx[k] >> bits);
        bool seen = false;
#pragma unroll
        for (int j = 0; j < k; ++j) seen |= j < count && slices[j] == slice;
        if (!seen) slices[count++] = slice;
    }
    return count;
}

template <bool PLACE>
__device__ inline void bucket_coordinate(const OwnerArgs& a, float x, float y, int32_t* bins, int32_t* list,
                                         int64_t list_base, int64_t stride, int32_t index) {
    for (int l = a.group; l < a.n_levels; ++l) {
        const DevLevel& lv = a.level[l];
        int slices[4];
        int count;
        switch (level_kind(lv)) {
            case kHashed24: count = slices_of<kHashed24>(x, y, lv, a.slice_bits[l], slices); break;
            case kHashedPow2: count = slices_of<kHashedPow2>(x, y, lv, a.slice_bits[l], slices); break;
            case kGeneric: count = slices_of<kGeneric>(x, y, lv, a.slice_bits[l], slices); break;
            default: count = slices_of<kDense>(x, y, lv, a.slice_bits[l], slices); break;
        }
        for (int j = 0; j < count; ++j) {
            const int q = a.first_pass[l] - a.fine_first + (slices[j] < a.slices[l] ? slices[j] : a.slices[l] - 1);
            const int32_t at = atomicAdd(bins + q, 1);
            if constexpr (PLACE) list[list_base + static_cast<int64_t>(q) * stride + bins[a.fine_passes + q] + at] = index;
        }
    }
}

__global__ __launch_bounds__(kBucketBlock) void bucket_kernel(OwnerArgs a, int bsplits, int32_t* counts,
                                                              int32_t* list) {
    extern __shared__ int32_t bins[];   // [fine_passes] counts / cursors, then [fine_passes] run starts
    const int e = blockIdx.x / bsplits, s = blockIdx.x % bsplits;
    int64_t base = 0, stop = a.n;
    if (a.offsets) {
        base = a.offsets[e];
        stop = a.offsets[e + 1];
        if (stop < base) stop = base;
        if (stop > a.n) stop = a.n;
        if (base > stop) base = stop;
    }
    const int64_t share = (stop - base + bsplits - 1) / bsplits;
    const int64_t b0 = base + share * s < stop ? base + share * s : stop;
    const int64_t b1 = b0 + share < stop ? b0 + share : stop;
    for (int q = threadIdx.x; q < a.fine_passes; q += kBucketBlock) bins[q] = 0;
    __syncthreads();
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kBucketBlock) {
        const float2 xy = reinterpret_cast<const float2*>(a.coords)[i];
        bucket_coordinate<false>(a, xy.x, xy.y, bins, nullptr, 0, 0, 0);
    }
    __syncthreads();
    int32_t* row = counts + static_cast<int64_t>(e) * a.fine_passes;
    for (int q = threadIdx.x; q < a.fine_passes; q += kBucketBlock) {
        const int32_t c = bins[q];
        bins[a.fine_passes + q] = c ? atomicAdd(row + q, c) : 0;
        bins[q] = 0;
    }
    __syncthreads();
    const int64_t list_base = base * a.fine_passes;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kBucketBlock) {
        const float2 xy = reinterpret_cast<const float2*>(a.coords)[i];
        bucket_coordinate<true>(a, xy.x, xy.y, bins, list, list_base, stop - base, static_cast<int32_t>(i));
    }
}

// Block -> work item.  Remapped, each XCD takes a contiguous chunk of the items (an expert's
// slices share its coordinates in that XCD's L2).  Inside a chunk the heavy items -- the
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

template <int F, bool HALF>
__global__ __launch_bounds__(kOwnerBlock) void owner_kernel(OwnerArgs a) {
    extern __shared__ unsigned long long acc[];
    __shared__ float reduce[kOwnerBlock / 64];
    using U = Elem<HALF>;
    // Work items per expert: the first split_passes passes split `splits` ways (all of them, or
    // only the coarse group pass), the others whole.
    const int split_passes = a.split_passes;
    const uint32_t per_expert = static_cast<uint32_t>(split_passes * a.splits + (a.passes - split_passes));
    const uint32_t total = static_cast<uint32_t>(a.experts) * per_expert;
    const uint32_t heavy = a.group > 0 && split_passes > 0 ? static_cast<uint32_t>(a.splits) : 0u;
    const uint32_t work = work_of(blockIdx.x, gridDim.x, a.remap, per_expert, heavy);
    if (work >= total) return;
    const int e = work / per_expert;
    const int r = work % per_expert;
    const int p = r < split_passes * a.splits ? r / a.splits : split_passes + (r - split_passes * a.splits);
    const int s = r < split_passes * a.splits ? r % a.splits : 0;
    const int splits = p < split_passes ? a.splits : 1;   // ways this pass is split

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
    const int64_t share = (stop - base + splits - 1) / splits;
    const int64_t b0 = base + share * s < stop ? base + share * s : stop;
    const int64_t b1 = b0 + share < stop ? b0 + share : stop;
    const bool bucket = a.bucketed && p >= a.fine_first;
    // a bucketed pass bounds its scale over all of the expert's coordinates (every split of the
    // pass then shares one scale); otherwise over this split's range
    const int64_t m0 = bucket ? base : b0, m1 = bucket ? stop : b1;

    // Fixed-point scale from the bound 4 * count * max|upstream| over this range and levels.
    float bound = 0.0f;
    if (m1 > m0) {
        const int64_t r0 = m0 / kMaxRows, r1 = (m1 - 1) / kMaxRows;
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
    const double limit = 4.0 * static_cast<double>(m1 - m0) * static_cast<double>(peak);
    int shift = 60;
    if (peak > 0.0f && limit <= 1.0e300) {
        const int by_value = 30 - ilogb(peak);
        const int by_sum = 61 - ilogb(limit);
        shift = by_value < by_sum ? by_value : by_sum;
    }
    if (shift > 120) shift = 120;
    const float scale = ldexpf(1.0f, shift);
    const bool finite = !(peak != peak) && peak <= 3.0e38f;

    int32_t* ring = reinterpret_cast<int32_t*>(acc + a.cap) + (threadIdx.x / 64) * kRing;
    for (int l = l0; l < l1; ++l) {
        const DevLevel lv = a.level[l];
        const U* plane = reinterpret_cast<const U*>(a.planes) + static_cast<size_t>(l) * a.n * F;
        if (bucket) {
            const int q = p - a.fine_first;
            const int64_t count = a.bucket_count[static_cast<int64_t>(e) * a.fine_passes + q];
            const int32_t* list = a.bucket_list + base * a.fine_passes + static_cast<int64_t>(q) * (stop - base);
            const int64_t k0 = 0, k1 = count;
            switch (level_kind(lv)) {
                case kHashed24: accumulate_bucket<F, HALF, kHashed24>(a.coords, plane, lv, list, k0, k1, lo, span, scale, acc); break;
                case kHashedPow2: accumulate_bucket<F, HALF, kHashedPow2>(a.coords, plane, lv, list, k0, k1, lo, span, scale, acc); break;
                case kGeneric: accumulate_bucket<F, HALF, kGeneric>(a.coords, plane, lv, list, k0, k1, lo, span, scale, acc); break;
                default: accumulate_bucket<F, HALF, kDense>(a.coords, plane, lv, list, k0, k1, lo, span, scale, acc); break;
            }
        } else if (a.row_bits[l] > 0 && !(a.group > 0 && p == 0))
            accumulate_rows<F, HALF>(a.coords, plane, lv, b0, b1, lo, span, scale, acc, ring, a.row_bits[l],
                                     static_cast<uint32_t>(p - a.first_pass[l]));
        else if (lv.hashed && lv.mask && lv.mask < (1u << 24))
            accumulate_level<F, HALF, kHashed24>(a.coords, plane, lv, b0, b1, lo, span, scale, acc);
        else if (lv.hashed && lv.mask)
            accumulate_level<F, HALF, kHashedPow2>(a.coords, plane, lv, b0, b1, lo, span, scale, acc);
        else if (lv.hashed)
            accumulate_level<F, HALF, kGeneric>(a.coords, plane, lv, b0, b1, lo, span, scale, acc);
        else
            accumulate_level<F, HALF, kDense>(a.coords, plane, lv, b0, b1, lo, span, scale, acc);
    }
    __syncthreads();
    const double unscale = ldexp(1.0, -shift);
    if (a.fused && splits == 1) {
        // The final gradient of these parameters is in LDS: update them right here.  One
        // workgroup holds the CU, so the loads of four elements per thread are issued before
        // any of them is used, to keep memory latency off the critical path.
        const AdamStep& o = a.adam;
        const int64_t first = static_cast<int64_t>(e) * a.expert_params + lo;
        constexpr int kBatch = 4;
        for (uint32_t j0 = threadIdx.x; j0 < span; j0 += kBatch * kOwnerBlock) {
            float g[kBatch], p[kBatch], m[kBatch], v[kBatch];
            uint32_t age[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const uint32_t j = j0 + k * kOwnerBlock;
                const int64_t i = first + (j < span ? j : 0);
                p[k] = o.master[i];
                m[k] = o.m[i];
                v[k] = o.v[i];
                age[k] = o.variant != 0 ? o.steps[i] : 0u;
                g[k] = static_cast<float>(static_cast<double>(static_cast<long long>(acc[j < span ? j : 0])) * unscale);
                if (!finite) g[k] = __builtin_nanf("");
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const uint32_t j = j0 + k * kOwnerBlock;
                if (j >= span) continue;
                const int64_t i = first + j;
                if (adam_math(o, g[k], p[k], m[k], v[k], age[k])) {
                    o.master[i] = p[k];
                    o.m[i] = m[k];
                    o.v[i] = v[k];
                    if (o.variant != 0) o.steps[i] = age[k];
                }
                if (o.half_copy) o.half_copy[i] = half_to_bits(__float2half_rn(p[k]));
            }
        }
        return;
    }
    float* out = splits == 1 ? a.grad + static_cast<size_t>(e) * a.expert_params + lo
                               : a.partial + static_cast<size_t>(s) * a.experts * a.expert_params +
                                     static_cast<size_t>(e) * a.expert_params + lo;
    for (uint32_t j = threadIdx.x; j < span; j += kOwnerBlock) {
        float v = static_cast<float>(static_cast<double>(static_cast<long long>(acc[j])) * unscale);
        if (!finite) v = __builtin_nanf("");
        if (splits == 1 && a.accumulate) v += out[j];
        out[j] = v;
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

template <typename Kernel>
int allow_lds(Kernel kernel, size_t bytes) {
    const hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (status != hipSuccess) return fail(std::string("LDS attribute: ") + hipGetErrorString(status));
    return 0;
}

// Clears the bucket counts and fills the buckets of every fine pass.
int launch_buckets(const OwnerArgs& o, int32_t* counts, int32_t* list, hipStream_t s) {
    if (launch_fill_zero(reinterpret_cast<float*>(counts), static_cast<int64_t>(o.experts) * o.fine_passes, s))
        return -1;
    int64_t bsplits = (2048 + o.experts - 1) / o.experts;
    const int64_t most = o.n / (static_cast<int64_t>(o.experts) * kBucketBlock);
    if (bsplits > most) bsplits = most > 1 ? most : 1;
    const size_t shmem = static_cast<size_t>(o.fine_passes) * 2 * sizeof(int32_t);
    bucket_kernel<<<static_cast<uint32_t>(o.experts * bsplits), kBucketBlock, shmem, s>>>(o, static_cast<int>(bsplits),
                                                                                           counts, list);
    return check_launch("owner buckets");
}

}  // namespace

int launch_owner_backward(const OwnerLaunch& in) {
    const int F = in.features;
    const int L = in.n_levels;
    const bool half = in.up_half != 0;
    const size_t elem = half ? 2 : 4;
    const int64_t lds_bytes = in.lds_bytes;
    const int64_t cap = (lds_bytes - kRingBytes) / 8 - F;  // int64 accumulators per slice, minus entry rounding
    if (cap < 64) return fail("odie_grid_backward: LDS budget too small for the owner backward");

    OwnerArgs o{};
    o.coords = in.coords;
    o.offsets = in.offsets;
    o.n = in.n;
    o.expert_params = in.expert_params;
    o.experts = in.experts;
    o.n_levels = L;
    o.accumulate = in.accumulate;
    o.fused = in.adam != nullptr;
    if (in.adam) o.adam = *in.adam;
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
        int64_t slices = (floats + cap - 1) / cap;
        int64_t entries = (in.levels[l].size + slices - 1) / slices;
        int bits = 0;
        while ((int64_t{2} << bits) * F <= cap) ++bits;   // 2^bits entries: largest block that fits
        if (in.bucketed) {
            // aligned power-of-two slices: the bucketing pass finds a corner's slice by a shift
            entries = int64_t{1} << bits;
            slices = (in.levels[l].size + entries - 1) / entries;
            o.slice_bits[l] = bits;
        } else if (in.row_screen && in.levels[l].hashed && in.levels[l].mask &&
                   (int64_t{1} << bits) > in.levels[l].res && (int64_t{1} << bits) < in.levels[l].size) {
            entries = int64_t{1} << bits;
            slices = in.levels[l].size / entries;
            o.row_bits[l] = bits;
        }
        o.slices[l] = static_cast<int>(slices);
        o.slice_entries[l] = static_cast<int>(entries);
        o.first_pass[l] = passes;
        passes += static_cast<int>(slices);
    }
    o.group = group;
    o.passes = passes;
    o.cap = static_cast<int>(cap + F);
    o.fine_first = group > 0 ? 1 : 0;
    o.fine_passes = passes - o.fine_first;
    o.bucketed = in.bucketed && o.fine_passes > 0 && static_cast<int64_t>(o.fine_passes) * 8 <= 64 * 1024 &&
                 static_cast<int64_t>(o.fine_passes) * in.n < (int64_t{1} << 31);
    // Splits.  Too few work items to fill the GPU: every pass is split over the coordinates (and
    // the partials summed by split_reduce_kernel).  Otherwise only the coarse-group pass may be:
    // it walks every coordinate through `group` fully landing levels, about group + 1 times the
    // work of a fine slice (measured: ~6x with 5 levels), and when that alone exceeds one CU's
    // share of the whole pass it would set the kernel's length (the native step's single-expert
    // batch), so it is cut into pieces of about that share.
    const int64_t per_pass = static_cast<int64_t>(in.experts) * passes;
    int splits = 1;
    int split_passes = passes;
    if (per_pass < 128) {
        const int64_t want = (512 + per_pass - 1) / per_pass;
        const int64_t most = in.n / (static_cast<int64_t>(in.experts) * 16384);
        splits = static_cast<int>(want < most ? want : (most > 1 ? most : 1));
    } else if (group > 0) {
        const double share = static_cast<double>(in.experts) * (passes + group) / kCus;   // fine-slice units
        if (group + 1 > share) {
            const int64_t want = static_cast<int64_t>(std::ceil((group + 1) / (share > 1.0 ? share : 1.0)));
            const int64_t most = in.n / (static_cast<int64_t>(in.experts) * 4096);
            splits = static_cast<int>(want < most ? want : (most > 1 ? most : 1));
        }
        split_passes = 1;
    }
    if (o.bucketed) split_passes = o.fine_first;   // a bucket is summed whole (its order varies)
    if (splits == 1) split_passes = passes;
    o.splits = splits;
    o.split_passes = split_passes;

    // Workspace: level-major planes, block maxima, split partials.
    const int64_t row_blocks = (in.n + kTransposeRows - 1) / kTransposeRows;
    const int64_t records = (in.n + kMaxRows - 1) / kMaxRows;
    const size_t planes_bytes = in.planes ? 0 : (static_cast<size_t>(in.n) * L * F * elem + 255) / 256 * 256;
    const size_t max_bytes = in.planes ? 0 : (static_cast<size_t>(records) * L * 4 + 255) / 256 * 256;
    const size_t total_params = static_cast<size_t>(in.experts) * in.expert_params;
    const size_t partial_bytes = (splits > 1 ? static_cast<size_t>(splits) * total_params * 4 + 255 : 0) / 256 * 256;
    const size_t count_bytes =
        o.bucketed ? (static_cast<size_t>(in.experts) * o.fine_passes * 4 + 255) / 256 * 256 : 0;
    const size_t list_bytes = o.bucketed ? static_cast<size_t>(in.n) * o.fine_passes * 4 : 0;
    char* space = static_cast<char*>(
        workspace(planes_bytes + max_bytes + partial_bytes + count_bytes + list_bytes, in.stream));
    if (!space) return -1;
    // upstream already level-major with its maxima (the caller wrote them): no transpose
    const bool given = in.planes != nullptr;
    o.planes = given ? in.planes : space;
    o.blockmax = given ? in.blockmax : reinterpret_cast<float*>(space + planes_bytes);
    o.partial = reinterpret_cast<float*>(space + planes_bytes + max_bytes);
    int32_t* bucket_count = reinterpret_cast<int32_t*>(space + planes_bytes + max_bytes + partial_bytes);
    int32_t* bucket_list = reinterpret_cast<int32_t*>(space + planes_bytes + max_bytes + partial_bytes + count_bytes);
    o.bucket_count = bucket_count;
    o.bucket_list = bucket_list;
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
    const size_t shmem = static_cast<size_t>(cap + F) * 8 + kRingBytes;
    const uint32_t total =
        static_cast<uint32_t>(in.experts * (static_cast<int64_t>(split_passes) * splits + (passes - split_passes)));
    const uint32_t oblocks = round_up(total, kXcds);
    hipStream_t s = in.stream;

#define ODIE_TRANSPOSE(FF, HH)                                                                          \
    do {                                                                                                \
        if (FF == 2 && HH && t.vec_rows && L % 4 == 0) {                                                \
            if (L <= 16) transpose_half2_kernel<16><<<tblocks, kTransposeBlock, 0, s>>>(t);             \
            else transpose_half2_kernel<32><<<tblocks, kTransposeBlock, 0, s>>>(t);                     \
        } else if (L <= 16) transpose_kernel<FF, HH, 16><<<tblocks, kTransposeBlock, 0, s>>>(t);        \
        else transpose_kernel<FF, HH, 32><<<tblocks, kTransposeBlock, 0, s>>>(t);                       \
    } while (0)
#define ODIE_OWNER(FF, HH)                                                                              \
    do {                                                                                                \
        if (o.bucketed && launch_buckets(o, bucket_count, bucket_list, s)) return -1;                  \
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
    if (splits > 1 && split_passes > 0) {
        // only the coarse group pass split: the expert's first values
        const int64_t prefix = split_passes < passes
            ? static_cast<int64_t>(in.levels[group - 1].offset + in.levels[group - 1].size) * F
            : in.expert_params;
        int64_t blocks = (static_cast<int64_t>(in.experts) * prefix + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        split_reduce_kernel<<<static_cast<uint32_t>(blocks), 256, 0, s>>>(o.partial, in.grad,
                                                                          static_cast<int64_t>(total_params), splits,
                                                                          in.accumulate, o.fused, o.adam,
                                                                          in.expert_params, prefix);
    }
    return check_launch("odie_grid_backward");
}

}  // namespace odie
