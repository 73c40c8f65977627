// Decoder MLP on MFMA: in -> 64 -> 64 -> 16 (in = align16 of the grid's feature count, 16..80),
// ReLU on the hidden layers, no bias, no output activation, fp16 weights and activations, fp32
// accumulation -- the decoder head of the reference (FullyFusedMLP with n_input_dims W,
// odie/native/runtime.cu:17,151-162,190; odie/hash_grid.py:32-34, odie/model.py:186-195; used
// by the native step at odie/native/runtime.cu:270,273), fused with the step's loss (loss_grad,
// odie/native/runtime.cu:53-63) and the grid-gradient unscale (half_unscale by 128,
// odie/native/runtime.cu:282).
//
// Weights: fp16 [64*in + 5120] = W1 [64][in] | W2 [64][64] | W3 [16][64], each row-major
// [out][in] (7168 at in = 32).
//
// Work split: one wave per tile of 32 samples; every product is a v_mfma_f32_32x32x16_f16
// with the samples as the 32 columns.  The transposed form H^T = W * X^T keeps each sample in
// one lane pair, and the accumulator layout of one layer (lane l: sample l%32, rows
// 8*(v/4) + 4*(l/32) + v%4) is exactly the B operand of the next layer once the weights' K
// columns are permuted the same way (slot_of below), so activations never leave registers.
// Weight gradients contract over samples: each round of 4 tiles is transposed through a
// workgroup LDS buffer and contracted by the waves, each owning a quarter of the gradient in
// registers across all rounds; partials per workgroup are reduced by a second kernel in a
// fixed order: deterministic.
#include "mlp.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

template <int KT> __device__ inline void load_x(const uint16_t* x, int64_t row, bool valid, int g, half8 xb[KT]) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
        xb[kt] = valid ? *reinterpret_cast<const half8*>(x + row * (16 * KT) + kt * 16 + 8 * g) : half8{};
}

// Output row o of accumulator element v (v < 8): 8*(v/4) + 4*g + v%4.
__device__ inline void store_out(uint16_t* out, int64_t row, int g, const half8& y) {
    const u32x4 bits = __builtin_bit_cast(u32x4, y);   // element 2i in the low half of dword i
    uint16_t* p = out + row * kOut;
    *reinterpret_cast<uint2*>(p + 4 * g) = make_uint2(bits.x, bits.y);
    *reinterpret_cast<uint2*>(p + 8 + 4 * g) = make_uint2(bits.z, bits.w);
}

template <int KT>
__global__ __launch_bounds__(kMlpBlock) void mlp_forward_kernel(const uint16_t* x, int64_t n, const uint16_t* weights,
                                                                uint16_t* out) {
    __shared__ _Float16 w[Shape<KT>::kWeightHalfs];
    stage_weights<KT>(weights, w);
    __syncthreads();
    const int lane = threadIdx.x % 64, g = lane / 32, s = lane % 32;
    const int64_t tiles = (n + 31) / 32;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kMlpWaves;
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kMlpWaves + threadIdx.x / 64; tile < tiles; tile += waves) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < n;
        half8 xb[KT], h1[4], h2[4];
        f32x16 acc3;
        load_x<KT>(x, row, valid, g, xb);
        forward_tile<KT>(w, g, s, xb, h1, h2, acc3);
        const half8 y = round8(acc3, 0);
        if (valid) store_out(out, row, g, y);
    }
}

// Loads of one tile, issued a tile ahead of their use.
template <int KT> struct TileInput {
    half8 xb[KT];
    int32_t input;    // kept 32-bit: widening here would wait for the load right away
    uint32_t color;
};

// The next tile's row of this lane, advanced by a fixed stride each round and kept in one
// pinned 32-bit register: every prefetch load then addresses base (a kernel argument, in
// scalar registers) + a 32-bit byte offset derived from it, with no temporary address
// register whose reuse could force an early wait on the loads in flight.
__device__ inline uint32_t pin(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <class T> __device__ inline T load_at(const T* base, uint32_t byte_offset) {
    return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_offset);
}

// Loop-carried row and byte offsets of the next tile's loads (each advanced by a constant).
struct TileCursor {
    uint32_t row;       // row index
    uint32_t off4;      // row * 4
    uint32_t offx;      // row * 2 * in + 16 * g
};

template <int KT> __device__ inline void advance(TileCursor& c, uint32_t rows) {
    c.row = pin(c.row + rows);
    c.off4 = pin(c.off4 + rows * 4u);
    c.offx = pin(c.offx + rows * (32u * KT));
}

template <int KT> __device__ inline void fetch_tile(const MlpArgs& a, const TileCursor& c, TileInput<KT>& in) {
    const bool valid = c.row < a.n;
    // the small loads first: memory counters drain in issue order, so an early wait on them
    // leaves the 64-byte x loads in flight
    in.input = valid ? (a.rows ? load_at(a.rows, c.off4) : static_cast<int32_t>(c.row)) : 0;
    in.color = valid && a.colors ? load_at(a.colors, c.off4) : 0u;
    const half8* x = reinterpret_cast<const half8*>(a.x);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)   // + 32 kt bytes on the base, not the offset
        in.xb[kt] = valid ? load_at(x + 2 * kt, c.offx) : half8{};
}

// Shared transposition buffer of one round (4 tiles = 128 samples): feature-major rows of
// 128 samples, padded so that 16-byte reads of 16 consecutive rows hit distinct banks.
constexpr int kRoundSamples = 32 * kMlpWaves;
constexpr int kRS = kRoundSamples + 8;
// phase 1 rows: dy outputs 0..2, h2 (64), dh1 (64), x (in); phase 2 rows: dh2 (64), h1 (64)
constexpr int kDyRow = 0, kH2Row = 3, kDh1Row = 67, kXRow = 131;
template <int KT> constexpr int round_rows() { return kXRow + 16 * KT; }

// Writes this wave's 32 samples of 32*blocks features held in accumulator-row order
// (h[t][e] = feature feature_of(t, g, e)) into rows first.. of the round buffer.
__device__ inline void put_features(_Float16* T, int first, int column, const half8* h, int blocks, int g) {
    for (int t = 0; t < 2 * blocks; ++t)
#pragma unroll
        for (int e = 0; e < 8; ++e) T[(first + feature_of(t, g, e)) * kRS + column] = h[t][e];
}

// One 32x32 block of a weight gradient: sum over the round's 128 samples of rows a0..
// (M side, rows a0 + s for lanes s < a_rows) times rows b0.. (N side, lanes s < b_rows) of the
// round buffer; DUAL alternates two accumulators so that consecutive MFMAs do not depend on
// each other (their sum is the block).
template <bool DUAL>
__device__ inline void round_block(const _Float16* T, int a0, int b0, int a_rows, int b_rows, int g, int s,
                                   f32x16& acc0, f32x16& acc1) {
#pragma unroll
    for (int kt = 0; kt < kRoundSamples / 16; kt += 2) {
        const half8 a0v = s < a_rows ? lds8(T + (a0 + s) * kRS + kt * 16 + 8 * g) : half8{};
        const half8 a1v = s < a_rows ? lds8(T + (a0 + s) * kRS + kt * 16 + 16 + 8 * g) : half8{};
        const half8 b0v = s < b_rows ? lds8(T + (b0 + s) * kRS + kt * 16 + 8 * g) : half8{};
        const half8 b1v = s < b_rows ? lds8(T + (b0 + s) * kRS + kt * 16 + 16 + 8 * g) : half8{};
        acc0 = mfma(a0v, b0v, acc0);
        if constexpr (DUAL) acc1 = mfma(a1v, b1v, acc1);
        else acc0 = mfma(a1v, b1v, acc0);
    }
}

// Phase-1 gradient blocks of the round: dW3 (dy x h2, two 32-column blocks) then dW1 (dh1 x x,
// two 32-row blocks times ceil(in/32) column blocks); wave w owns blocks w, w + 4, ...
template <int KT> struct Phase1 {
    static constexpr int kColumnBlocks = (KT + 1) / 2;
    static constexpr int kBlocks = 2 + 2 * kColumnBlocks;
    static constexpr int kSlots = (kBlocks + kMlpWaves - 1) / kMlpWaves;   // 1 (in <= 32) or 2
};

// Block b of phase 1: A rows, B rows and their counts; dW1 block (mb, nb) = b - 2 = mb * NB + nb.
template <int KT> __device__ inline void phase1_block(int b, int& a0, int& b0, int& a_rows, int& b_rows) {
    if (b < 2) {
        a0 = kDyRow, a_rows = 3, b0 = kH2Row + 32 * b, b_rows = 32;
    } else {
        const int mb = (b - 2) / Phase1<KT>::kColumnBlocks, nb = (b - 2) % Phase1<KT>::kColumnBlocks;
        a0 = kDh1Row + 32 * mb, a_rows = 32, b0 = kXRow + 32 * nb;
        b_rows = 16 * KT - 32 * nb < 32 ? 16 * KT - 32 * nb : 32;
    }
}

// Work split: each wave computes the forward, loss and input gradient of its own tile in
// registers; the weight gradients are contracted per round of 4 tiles through the shared
// buffer in two phases (1: dW3 = dy x h2 and dW1 = dh1 x x; 2: dW2 = dh2 x h1), each wave
// owning its own 32x32 gradient blocks (Phase1 above; phase 2: one dW2 block per wave), so no
// cross-wave reduction is needed.  PLANES (in = 32 only) writes dz as level-major planes.
template <int KT, bool PLANES>
__global__ __launch_bounds__(kMlpBlock) void mlp_train_kernel(MlpArgs a) {
    using S = Shape<KT>;
    using P1 = Phase1<KT>;
    static_assert(!PLANES || KT == 2, "the planes layout is built for 16 levels x 2 features");
    constexpr int kNB = P1::kColumnBlocks;   // 32-row blocks of dX
    __shared__ _Float16 w[S::kWeightHalfs];
    __shared__ __attribute__((aligned(16))) _Float16 T[round_rows<KT>() * kRS];
    __shared__ uint32_t records[kMlpWaves][2][8];   // per wave and lane group: per-feature |dz| maxima of 8 levels
    stage_weights<KT>(a.weights, w);
    __syncthreads();
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, g = lane / 32, s = lane % 32;
    const int column = 32 * wave + s;   // this lane's sample column in the round buffer
    f32x16 gA[P1::kSlots], gA1 = zero16(), gB = zero16(), gB1 = zero16();
#pragma unroll
    for (int k = 0; k < P1::kSlots; ++k) gA[k] = zero16();
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kMlpWaves;
    const float inv255 = 1.0f / 255.0f;
    const float denominator = static_cast<float>(3 * a.real);
    TileCursor cursor;
    {
        const uint32_t row0 = static_cast<uint32_t>((blockIdx.x * kMlpWaves + wave) * 32 + s);
        cursor = {pin(row0), pin(row0 * 4u), pin(row0 * (32u * KT) + 16u * g)};
    }
    const uint32_t row_stride = static_cast<uint32_t>(stride * 32);
    // One round on the tile whose inputs are in `current` (loaded a round earlier).
    auto round = [&](int64_t base, const TileInput<KT>& current) {
        const int64_t tile = base + wave;
        const int64_t row = tile * 32 + s;
        const bool valid = tile < tiles && row < a.n;
        half8 xb[KT], h1[4], h2[4];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) xb[kt] = current.xb[kt];
        f32x16 acc3;
        forward_tile<KT>(w, g, s, xb, h1, h2, acc3);
        const int64_t input = current.input;
        const half8 y = round8(acc3, 0);
        half8 dy{};
        if (valid && a.out) store_out(a.out, input, g, y);
        // loss (odie/native/runtime.cu:53-63): outputs 0..2 live in lane group 0, v = 0..2
        if (valid && g == 0) {
            float square = 0.0f;
            if (input < a.real) {
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const float t = a.colors ? __fmul_rn(static_cast<float>((current.color >> (8 * c)) & 0xffu), inv255)
                                  : a.rgb ? __fmul_rn(static_cast<float>(a.rgb[3 * a.ids[input] + c]), inv255)
                                          : a.target[3 * input + c];
                    const float d = static_cast<float>(y[c]) - t;
                    square = fmaf(d, d, square);
                    const _Float16 scaled = static_cast<_Float16>(__fdiv_rn(2.0f * d, denominator) * 128.0f);
                    dy[c] = static_cast<_Float16>(static_cast<float>(scaled) * 128.0f);
                }
            }
            if (a.squares) a.squares[input] = __fdiv_rn(square, 3.0f);
        }
        if (valid && a.hidden) {
            uint16_t* hrow = a.hidden + row * 128;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                // elements 0..3 and 4..7 are features feature_of(t, g, 0) + 0..3 and + 8..11
                const u32x4 b1 = __builtin_bit_cast(u32x4, h1[t]), b2 = __builtin_bit_cast(u32x4, h2[t]);
                *reinterpret_cast<uint2*>(hrow + feature_of(t, g, 0)) = make_uint2(b1.x, b1.y);
                *reinterpret_cast<uint2*>(hrow + feature_of(t, g, 4)) = make_uint2(b1.z, b1.w);
                *reinterpret_cast<uint2*>(hrow + 64 + feature_of(t, g, 0)) = make_uint2(b2.x, b2.y);
                *reinterpret_cast<uint2*>(hrow + 64 + feature_of(t, g, 4)) = make_uint2(b2.z, b2.w);
            }
        }
        // input gradients: dH2 = relu'(h2) * (W3^T dy), dH1 = relu'(h1) * (W2^T dH2), dX = W1^T dH1
        half8 dh2[4], dh1[4];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const f32x16 acc = mfma(lds8(w + S::kW3t + (mb * 32 + s) * kS16 + 8 * g), dy, zero16());
            dh2[2 * mb] = mask8(round8(acc, 0), h2[2 * mb]);
            dh2[2 * mb + 1] = mask8(round8(acc, 8), h2[2 * mb + 1]);
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            f32x16 acc = zero16();
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc = mfma(lds8(w + S::kW2t + (mb * 32 + s) * kS64 + 16 * t + 8 * g), dh2[t], acc);
            dh1[2 * mb] = mask8(round8(acc, 0), h1[2 * mb]);
            dh1[2 * mb + 1] = mask8(round8(acc, 8), h1[2 * mb + 1]);
        }
        {
            // fp16(fp16(dx) / 128): one fp16 multiply by 2^-7 rounds the same exact value.  K step
            // ks = 2b + q of dX is half q of block b; word .x/.y/.z/.w of bits[ks] holds columns
            // 16ks + 4g + 0..1, + 2..3, 16ks + 8 + 4g + 0..1, + 2..3 of the row (for in = 32: the
            // feature pairs of levels 8ks + 2g, 8ks + 2g + 1, 8ks + 4 + 2g, 8ks + 5 + 2g).
            u32x4 bits[KT];
#pragma unroll
            for (int b = 0; b < kNB; ++b) {
                f32x16 acc = zero16();
                const bool row_ok = 32 * b + s < S::kIn;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const half8 at = row_ok ? lds8(w + S::kW1t + (32 * b + s) * kS64 + 16 * t + 8 * g) : half8{};
                    acc = mfma(at, dh1[t], acc);
                }
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    if (2 * b + q < KT)
                        bits[2 * b + q] =
                            __builtin_bit_cast(u32x4, round8(acc, 8 * q) * (half8)(static_cast<_Float16>(0.0078125f)));
            }
            if constexpr (PLANES) {
                if (valid) {
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        a.planes[(8 * q + 2 * g) * a.n + row] = bits[q].x;
                        a.planes[(8 * q + 2 * g + 1) * a.n + row] = bits[q].y;
                        a.planes[(8 * q + 4 + 2 * g) * a.n + row] = bits[q].z;
                        a.planes[(8 * q + 5 + 2 * g) * a.n + row] = bits[q].w;
                    }
                }
                // this round's 128 rows are one record: per-feature maxima of the lane group's
                // eight levels over its 32 lanes (lane s < 8 ends with word s), then over the four
                // waves (after the barrier below)
                const uint32_t words[8] = {bits[0].x, bits[0].y, bits[0].z, bits[0].w,
                                           bits[1].x, bits[1].y, bits[1].z, bits[1].w};
                uint32_t peak[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) peak[j] = valid ? pair_magnitudes(words[j]) : 0u;
                const uint32_t mine = group_max8(peak, lane);
                if (s < 8) records[wave][g][s] = mine;
            } else if (valid) {
                uint16_t* p = a.dz + row * S::kIn;
#pragma unroll
                for (int ks = 0; ks < KT; ++ks) {
                    *reinterpret_cast<uint2*>(p + 16 * ks + 4 * g) = make_uint2(bits[ks].x, bits[ks].y);
                    *reinterpret_cast<uint2*>(p + 16 * ks + 8 + 4 * g) = make_uint2(bits[ks].z, bits[ks].w);
                }
            }
        }
        // phase 1: dW3 = sum dy (x) h2, dW1 = sum dh1 (x) x
        if (g == 0)
#pragma unroll
            for (int c = 0; c < 3; ++c) T[(kDyRow + c) * kRS + column] = dy[c];
        put_features(T, kH2Row, column, h2, 2, g);
        put_features(T, kDh1Row, column, dh1, 2, g);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int e = 0; e < 8; ++e) T[(kXRow + kt * 16 + 8 * g + e) * kRS + column] = xb[kt][e];
        __syncthreads();
        if (PLANES && threadIdx.x < 32) {
            // column 2L + f (level L, feature f); level L = 8q + 4h + 2g + b is word 4q + 2h + b
            // of lane group g
            const int level = threadIdx.x / 2, f = threadIdx.x % 2;
            const int q = level / 8, h = (level / 4) % 2, lg = (level / 2) % 2, b = level % 2;
            uint32_t m = 0;
#pragma unroll
            for (int v = 0; v < kMlpWaves; ++v) m = pair_max(m, records[v][lg][4 * q + 2 * h + b]);
            a.blockmax[(base / kMlpWaves) * 32 + threadIdx.x] =
                __half2float(bits_to_half(static_cast<uint16_t>(m >> (16 * f))));
        }
#pragma unroll
        for (int k = 0; k < P1::kSlots; ++k) {
            const int block = wave + kMlpWaves * k;
            if (block < P1::kBlocks) {
                int a0, b0, a_rows, b_rows;
                phase1_block<KT>(block, a0, b0, a_rows, b_rows);
                if constexpr (P1::kSlots == 1) round_block<true>(T, a0, b0, a_rows, b_rows, g, s, gA[k], gA1);
                else round_block<false>(T, a0, b0, a_rows, b_rows, g, s, gA[k], gA1);
            }
        }
        __syncthreads();
        // phase 2: dW2 = sum dh2 (x) h1; rows 0..63 = dh2, 64..127 = h1
        put_features(T, 0, column, dh2, 2, g);
        put_features(T, 64, column, h1, 2, g);
        __syncthreads();
        round_block<true>(T, 32 * (wave >> 1), 64 + 32 * (wave & 1), 32, 32, g, s, gB, gB1);
        __syncthreads();

    };
    // Unrolled by two with ping-pong input buffers, so that a round never copies the next
    // round's prefetch (a copy would have to wait for it).
    TileInput<KT> even, odd;
    fetch_tile<KT>(a, cursor, even);
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kMlpWaves; base < tiles; base += 2 * stride) {
        advance<KT>(cursor, row_stride);
        fetch_tile<KT>(a, cursor, odd);
        round(base, even);
        if (base + stride >= tiles) break;
        advance<KT>(cursor, row_stride);
        fetch_tile<KT>(a, cursor, even);
        round(base + stride, odd);
    }
    // This workgroup's partial: each wave writes its own blocks (accumulator element v of
    // lane (g, s) is row 8*(v/4) + 4g + v%4, column s of the block).
    if constexpr (P1::kSlots == 1) gA[0] += gA1;
    gB += gB1;
    float* out = a.partials + static_cast<int64_t>(blockIdx.x) * S::kParams;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int r = 8 * (v / 4) + 4 * g + v % 4;
        out[S::kW1 + (32 * (wave >> 1) + r) * kHid + 32 * (wave & 1) + s] = gB[v];
    }
#pragma unroll
    for (int k = 0; k < P1::kSlots; ++k) {
        const int block = wave + kMlpWaves * k;
        if (block >= P1::kBlocks) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = 8 * (v / 4) + 4 * g + v % 4;
            if (block < 2) {
                if (v < 8) out[S::kW1 + kW2 + r * kHid + 32 * block + s] = gA[k][v];
            } else {
                const int mb = (block - 2) / P1::kColumnBlocks, nb = (block - 2) % P1::kColumnBlocks;
                if (32 * nb + s < S::kIn) out[(32 * mb + r) * S::kIn + 32 * nb + s] = gA[k][v];
            }
        }
    }
}

// dweights[p] = sum over workgroups of partials[b][p] in a fixed order: the 16 lane groups of a
// 1024-thread block take the workgroups b = q, q+16, q+32, ... (q = group), eight loads in
// flight per step, and the sixteen group sums are added in group order.
constexpr int kReduceParams = 64;
constexpr int kReduceGroups = 16;
__global__ __launch_bounds__(kReduceParams * kReduceGroups) void mlp_reduce_kernel(const float* partials, int blocks,
                                                                                   int params, float* dweights) {
    __shared__ float group_sum[kReduceGroups][kReduceParams];
    const int local = threadIdx.x % kReduceParams, q = threadIdx.x / kReduceParams;
    const int p = blockIdx.x * kReduceParams + local;
    float total = 0.0f;
    if (p < params) {
        int b = q;
        for (; b + 7 * kReduceGroups < blocks; b += 8 * kReduceGroups) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = partials[static_cast<int64_t>(b + kReduceGroups * j) * params + p];
#pragma unroll
            for (int j = 0; j < 8; ++j) total += v[j];
        }
        for (; b < blocks; b += kReduceGroups) total += partials[static_cast<int64_t>(b) * params + p];
    }
    group_sum[q][local] = total;
    __syncthreads();
    if (q == 0 && p < params) {
        float sum = group_sum[0][local];
#pragma unroll
        for (int g = 1; g < kReduceGroups; ++g) sum += group_sum[g][local];
        dweights[p] = sum;
    }
}

int mlp_blocks(int64_t n) {
    const int64_t tiles = (n + 31) / 32;
    int64_t blocks = (tiles + kMlpWaves - 1) / kMlpWaves;
    return static_cast<int>(blocks < 512 ? (blocks < 1 ? 1 : blocks) : 512);
}

// Input widths the decoder is built for: 16, 32, 48, 64, 80 (align16 of 2..80 grid features).
int input_steps(int width) { return width >= 16 && width <= 16 * kMaxInputSteps && width % 16 == 0 ? width / 16 : 0; }
int64_t decoder_params(int width) { return int64_t{64} * width + kW2 + kW3; }

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_mlp_forward(const uint16_t* x, int64_t n, int width, const uint16_t* weights, uint16_t* out,
                              uint64_t stream) {
    const int kt = input_steps(width);
    if (!kt) return fail("odie_mlp_forward: width must be 16, 32, 48, 64 or 80");
    if (n < 0) return fail("odie_mlp_forward: n must be nonnegative");
    if (n == 0) return 0;
    if (!x || !weights || !out) return fail("odie_mlp_forward: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(out) % 8)
        return fail("odie_mlp_forward: x must be 16-byte and out 8-byte aligned");
    const hipStream_t s = as_stream(stream);
    const int blocks = mlp_blocks(n);
    switch (kt) {
        case 1: mlp_forward_kernel<1><<<blocks, kMlpBlock, 0, s>>>(x, n, weights, out); break;
        case 2: mlp_forward_kernel<2><<<blocks, kMlpBlock, 0, s>>>(x, n, weights, out); break;
        case 3: mlp_forward_kernel<3><<<blocks, kMlpBlock, 0, s>>>(x, n, weights, out); break;
        case 4: mlp_forward_kernel<4><<<blocks, kMlpBlock, 0, s>>>(x, n, weights, out); break;
        default: mlp_forward_kernel<5><<<blocks, kMlpBlock, 0, s>>>(x, n, weights, out); break;
    }
    return check_launch("odie_mlp_forward");
}

namespace {

int mlp_train(const char* name, const uint16_t* x, int64_t n, int width, int64_t real, const uint16_t* weights,
              const uint32_t* colors, const uint8_t* rgb, const int64_t* ids, const float* target, const int32_t* rows,
              uint16_t* out, uint16_t* hidden, float* squares, uint16_t* dz, uint32_t* planes, float* blockmax,
              float* dweights, uint64_t stream) {
    const std::string who(name);
    const int kt = input_steps(width);
    if (!kt) return fail(who + ": width must be 16, 32, 48, 64 or 80");
    if (planes && kt != 2) return fail(who + ": the planes layout is built for width 32");
    if (n < 0 || real < 1) return fail(who + ": need n >= 0 and real >= 1");
    if (n * 2 * width >= (int64_t{1} << 32)) return fail(who + ": n * width must stay below 2^31 (32-bit byte offsets)");
    if (!weights || !dweights || (n && !x)) return fail(who + ": null pointer");
    if (n && (planes ? !blockmax : !dz)) return fail(who + ": null pointer");
    if (n && !colors && !(rgb ? ids != nullptr : target != nullptr))
        return fail(who + ": need colors, rgb with ids, or target");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(dz) % 8 ||
        reinterpret_cast<uintptr_t>(planes) % 4 || (out && reinterpret_cast<uintptr_t>(out) % 8))
        return fail(who + ": x must be 16-byte, dz and out 8-byte, planes 4-byte aligned");
    const hipStream_t s = as_stream(stream);
    const int64_t params = decoder_params(width);
    if (n == 0) return launch_fill_zero(dweights, params, s);
    const int blocks = mlp_blocks(n);
    float* partials = static_cast<float*>(workspace(static_cast<size_t>(blocks) * params * sizeof(float), s));
    if (!partials) return -1;
    MlpArgs a{x, weights, n, real, colors, rgb, ids, target, rows, out, hidden, squares, planes ? nullptr : dz, partials,
              planes, planes ? blockmax : nullptr};
    if (planes) {
        mlp_train_kernel<2, true><<<blocks, kMlpBlock, 0, s>>>(a);
    } else {
        switch (kt) {
            case 1: mlp_train_kernel<1, false><<<blocks, kMlpBlock, 0, s>>>(a); break;
            case 2: mlp_train_kernel<2, false><<<blocks, kMlpBlock, 0, s>>>(a); break;
            case 3: mlp_train_kernel<3, false><<<blocks, kMlpBlock, 0, s>>>(a); break;
            case 4: mlp_train_kernel<4, false><<<blocks, kMlpBlock, 0, s>>>(a); break;
            default: mlp_train_kernel<5, false><<<blocks, kMlpBlock, 0, s>>>(a); break;
        }
    }
    if (check_launch(name)) return -1;
    mlp_reduce_kernel<<<static_cast<uint32_t>((params + kReduceParams - 1) / kReduceParams),
                        kReduceParams * kReduceGroups, 0, s>>>(
        partials, blocks, static_cast<int>(params), dweights);
    return check_launch((who + " reduce").c_str());
}

}  // namespace

ODIE_API int odie_mlp_train(const uint16_t* x, int64_t n, int width, int64_t real, const uint16_t* weights,
                            const uint32_t* colors, const uint8_t* rgb, const int64_t* ids, const float* target,
                            const int32_t* rows, uint16_t* out, uint16_t* hidden, float* squares, uint16_t* dz,
                            float* dweights, uint64_t stream) {
    return mlp_train("odie_mlp_train", x, n, width, real, weights, colors, rgb, ids, target, rows, out, hidden, squares,
                     dz, nullptr, nullptr, dweights, stream);
}

ODIE_API int odie_mlp_train_planes(const uint16_t* x, int64_t n, int64_t real, const uint16_t* weights,
                                   const uint32_t* colors, const uint8_t* rgb, const int64_t* ids, const float* target,
                                   const int32_t* rows, uint16_t* out, uint16_t* hidden, float* squares,
                                   uint32_t* planes, float* blockmax, float* dweights, uint64_t stream) {
    if (n > 0 && !planes) return fail("odie_mlp_train_planes: planes is null");
    return mlp_train("odie_mlp_train_planes", x, n, kIn, real, weights, colors, rgb, ids, target, rows, out, hidden,
                     squares, nullptr, planes, blockmax, dweights, stream);
}
