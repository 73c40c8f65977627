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
// Weight gradients contract over samples: each wave transposes its own tile through its own LDS
// region and accumulates every weight gradient in its registers with 16x16x32 products (no
// workgroup barrier in the loop); the four waves' gradients are summed in wave order at the end
// and the workgroups' partials by a second kernel in a fixed order: deterministic.
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

// Every load is issued unconditionally, from a row clamped into [0, n) and from x in place of
// a null rows or colors (the values are then replaced): straight-line loads let the compiler
// count the memory operations in flight exactly, where loads under branches made it wait for
// the next tile's prefetch at the first product of the current one.
template <int KT> __device__ inline void fetch_tile(const MlpArgs& a, int64_t row, int g, TileInput<KT>& in) {
    const bool valid = row < a.n;
    const int64_t r = valid ? row : a.n - 1;
    const int32_t* rows = a.rows ? a.rows : reinterpret_cast<const int32_t*>(a.x);
    const uint32_t* colors = a.colors ? a.colors : reinterpret_cast<const uint32_t*>(a.x);
    // the small loads first: memory counters drain in issue order, so an early wait on them
    // leaves the 64-byte x loads in flight
    const int32_t input = rows[r];
    const uint32_t color = colors[r];
    const half8* x = reinterpret_cast<const half8*>(a.x + r * (16 * KT) + 8 * g);
    half8 xb[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) xb[kt] = x[2 * kt];
    in.input = !valid ? 0 : a.rows ? input : static_cast<int32_t>(row);
    in.color = valid && a.colors ? color : 0u;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) in.xb[kt] = valid ? xb[kt] : half8{};
}

// Per-wave transposition region: two sample-major matrices of the wave's current 32 samples,
// A (dy, then dh2, then dh1) and B (h2, then h1, then x), each sample a 160-byte row of up to 80
// fp16 features in 8-byte chunks of 4.  Chunk q of sample s sits at byte
//   s * 160 + 32 * (q / 4) + 8 * ((q % 4) ^ ((s / 4) % 4)),
// so that every 16 lanes of both access patterns meet 16 distinct 8-byte slots of a 128-byte bank
// line (no bank conflict): a lane stores its sample's feature chunks with ds_write_b64 (16 consecutive samples, one
// chunk: slots 4 * ((s + q / 4) % 4) + (q % 4 ^ s / 4 % 4), all distinct), and a 16x16x32 operand
// comes back with two ds_read_b64_tr_b16 (within a 16-lane group lane j fetches chunk 4b + j % 4
// of sample k0 + j / 4, and the read hands lane 4a + e element e of the chunks fetched by lanes a,
// a + 4, a + 8, a + 12: feature 16b + 4a + e of samples k0 .. k0 + 3).  Phase 1 puts dy in chunk 0
// of A; chunks 1..3 hold stale values whose products fall in gradient rows that are never
// written out.
constexpr int kRowBytes = 160;
constexpr int kMatrixBytes = 32 * kRowBytes;
constexpr int kRegionBytes = 2 * kMatrixBytes;

typedef int16_t short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v* lds_short4;

// Byte offset, within a matrix, of chunk q (q % 4 == lo) of sample s: lo ^ the sample's swizzle.
__device__ inline int chunk_at(int s, int lo) { return s * kRowBytes + 8 * (lo ^ ((s >> 2) & 3)); }

// Stores this lane's sample (byte row `at_lo`/`at_hi`: chunks 4t + g and 4t + 2 + g, see chunk_at)
// of 16*halves features held in accumulator-row order (elements 0..3 of h[t] are features
// 16t + 4g + 0..3, elements 4..7 features 16t + 8 + 4g + 0..3).
__device__ inline void put_chunks(char* M, int at_lo, int at_hi, const half8* h, int halves) {
    for (int t = 0; t < halves; ++t) {
        const u32x4 d = __builtin_bit_cast(u32x4, h[t]);
        *reinterpret_cast<uint2*>(M + at_lo + 32 * t) = make_uint2(d.x, d.y);
        *reinterpret_cast<uint2*>(M + at_hi + 32 * t) = make_uint2(d.z, d.w);
    }
}

// 16x16x32 operand of features 16*block .. +15 of matrix M: lane l holds feature 16*block + l%16,
// samples 8*(l/16) .. +7.  at[h] is the lane's fetch address for samples 8*(l/16) + 4h .. +3.
__device__ inline half8 operand16(const char* M, const int at[2], int block) {
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4)(M + at[0] + 32 * block));
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4)(M + at[1] + 32 * block));
    return __builtin_bit_cast(half8, (short8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ inline f32x4 mfma16(half8 a, half8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// Orders this wave's LDS accesses: lanes read what other lanes of the same wave wrote (the LDS
// executes one wave's instructions in issue order; this keeps the compiler from moving them).
__device__ inline void wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Work split: each wave takes tiles of 32 samples in turn (below: how records of 128 rows are
// handed out) and computes, per tile, the forward, loss and input gradient in registers (the accumulator layout of one
// layer is the B operand of the next), then the tile's share of every weight gradient: the tile's
// activations and gradients pass through the wave's own LDS region (one fp16 per sample and
// feature) and come back with the samples in the K positions of 16x16x32 products accumulated in
// the wave's registers (dW3 4 blocks, dW2 16, dW1 4*KT).  No workgroup barrier inside the loop;
// at the end the four waves' gradients are summed in wave order through LDS, and the workgroups'
// partials by mlp_reduce_kernel in a fixed order: deterministic.  PLANES (in = 32 only) writes dz
// as level-major planes with each 128-row record's per-column maxima.
template <int KT, bool PLANES, bool WHOLE>
__global__ __launch_bounds__(kMlpBlock, KT <= 3 ? 2 : 1) void mlp_train_kernel(MlpArgs a) {
    using S = Shape<KT>;
    static_assert(!PLANES || KT == 2, "the planes layout is built for 16 levels x 2 features");
    constexpr int kNB = (KT + 1) / 2;   // 32-row blocks of dX
    static_assert(kMlpWaves * kRegionBytes >= S::kParams * 4, "the regions hold the workgroup's gradient");
    static_assert(16 * KT <= 80, "a matrix row holds at most 80 features");
    __shared__ _Float16 w[S::kWeightHalfs];
    __shared__ __attribute__((aligned(16))) char T[kMlpWaves * kRegionBytes];
    stage_weights<KT>(a.weights, w);
    __syncthreads();
    // wave: uniform over the wave, in a scalar register (so are the tile positions derived from it)
    const int lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int g = lane / 32, s = lane % 32;
    char* const MA = T + wave * kRegionBytes;
    char* const MB = MA + kMatrixBytes;
    // store addresses of this lane's sample: chunks 4t + g, 4t + 2 + g (hidden layers), 4kt + 2g,
    // 4kt + 2g + 1 (x); fetch addresses of its operand rows: samples 8 * (lane / 16) + 4h + j / 4,
    // chunk j % 4 (j = lane % 16)
    const int at_lo = chunk_at(s, g), at_hi = chunk_at(s, g ^ 2);
    const int at_x0 = chunk_at(s, 2 * g), at_x1 = chunk_at(s, 2 * g + 1);
    const int at_op[2] = {chunk_at(8 * (lane >> 4) + ((lane & 15) >> 2), lane & 3),
                          chunk_at(8 * (lane >> 4) + 4 + ((lane & 15) >> 2), lane & 3)};
    f32x4 gW3[4], gW2[4][4], gW1[4][KT];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        gW3[i] = f32x4{};
#pragma unroll
        for (int j = 0; j < 4; ++j) gW2[i][j] = f32x4{};
#pragma unroll
        for (int j = 0; j < KT; ++j) gW1[i][j] = f32x4{};
    }
    const int64_t tiles = (a.n + 31) / 32;
    const float inv255 = 1.0f / 255.0f;
    const float denominator = static_cast<float>(3 * a.real);
    // with PLANES: per-feature |dz| maxima of the lane group's 8 levels (lane i: word i % 8) over
    // the last tile processed, and over the current record
    uint32_t tile_peak = 0, record_peak = 0;
    // With colors and rgb together, colors holds the slot's pixel index: the tile's three target
    // bytes are loaded before the next tile's prefetch is issued, so that the loss waits for them
    // alone (memory counters drain in issue order: loaded after the prefetch, they would make the
    // loss wait for the whole prefetch as well), and kept apart until the loss reads them (joining
    // them at once would wait for the loads there).
    const bool gather = a.colors && a.rgb;
    auto gather_bytes = [&](const TileInput<KT>& current, uint32_t byte[3]) {
        byte[0] = byte[1] = byte[2] = 0u;
        if (gather) {   // every lane (both lane groups of a sample read the same bytes), no branch
            // three byte loads from addresses the compiler cannot see as adjacent (it would merge
            // them into a 16-bit load whose split waits for it at once)
            typedef const __attribute__((address_space(1))) uint8_t* global_bytes;
            global_bytes p[3];
            p[0] = (global_bytes)(a.rgb + 3 * static_cast<uint64_t>(current.color));   // generic -> global
#pragma unroll
            for (int c = 1; c < 3; ++c) {
                p[c] = p[0] + c;
                asm volatile("" : "+v"(p[c]));
            }
#pragma unroll
            for (int c = 0; c < 3; ++c) byte[c] = *p[c];
        }
    };
    auto process = [&](int64_t tile, const TileInput<KT>& current, const uint32_t byte[3]) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        half8 h1[4], h2[4];
        f32x16 acc3;
        forward_tile<KT>(w, g, s, current.xb, h1, h2, acc3);
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
                    const uint32_t value = gather ? byte[c] : (current.color >> (8 * c)) & 0xffu;
                    const float t = a.colors ? __fmul_rn(static_cast<float>(value), inv255)
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
        // Each phase stores a pair of layers into the region, computes the next input gradient
        // from registers (after which those layers' registers are free), then the weight
        // gradient from the region: dW3 += dy (x) h2 over the tile's samples
        if (g == 0) {   // dy: features 0..2 of chunk 0, feature 3 zero
            const u32x4 d = __builtin_bit_cast(u32x4, dy);
            *reinterpret_cast<uint2*>(MA + at_lo) = make_uint2(d.x, d.y);
        }
        put_chunks(MB, at_lo, at_hi, h2, 4);
        // input gradients: dH2 = relu'(h2) * (W3^T dy), dH1 = relu'(h1) * (W2^T dH2), dX = W1^T dH1
        half8 dh2[4], dh1[4];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const f32x16 acc = mfma(lds8(w + S::kW3t + (mb * 32 + s) * kS16 + 8 * g), dy, zero16());
            dh2[2 * mb] = mask8(round8(acc, 0), h2[2 * mb]);
            dh2[2 * mb + 1] = mask8(round8(acc, 8), h2[2 * mb + 1]);
        }
        wave_fence();
        {
            const half8 A = operand16(MA, at_op, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) gW3[j] = mfma16(A, operand16(MB, at_op, j), gW3[j]);
        }
        // dW2 += dh2 (x) h1
        wave_fence();
        put_chunks(MA, at_lo, at_hi, dh2, 4);
        put_chunks(MB, at_lo, at_hi, h1, 4);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            f32x16 acc = zero16();
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc = mfma(lds8(w + S::kW2t + (mb * 32 + s) * kS64 + 16 * t + 8 * g), dh2[t], acc);
            dh1[2 * mb] = mask8(round8(acc, 0), h1[2 * mb]);
            dh1[2 * mb + 1] = mask8(round8(acc, 8), h1[2 * mb + 1]);
        }
        wave_fence();
        {
            half8 B[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) B[j] = operand16(MB, at_op, j);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const half8 A = operand16(MA, at_op, i);
#pragma unroll
                for (int j = 0; j < 4; ++j) gW2[i][j] = mfma16(A, B[j], gW2[i][j]);
            }
        }
        // dW1 += dh1 (x) x
        wave_fence();
        put_chunks(MA, at_lo, at_hi, dh1, 4);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {   // x: features 16kt + 8g + 0..7 of the lane's sample
            const u32x4 d = __builtin_bit_cast(u32x4, current.xb[kt]);
            *reinterpret_cast<uint2*>(MB + at_x0 + 32 * kt) = make_uint2(d.x, d.y);
            *reinterpret_cast<uint2*>(MB + at_x1 + 32 * kt) = make_uint2(d.z, d.w);
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
                    // level 8q + 2g + c at planes + (8q + c) * n (uniform: a scalar base) + the lane's
                    // 32-bit offset of plane 2g, row `row` (below 12n bytes; the host keeps 64n < 2^32)
                    const uint32_t at = static_cast<uint32_t>(2 * g * a.n + row) * 4u;
                    const auto put = [&](int level, uint32_t v) {
                        char* const base = reinterpret_cast<char*>(a.planes) + static_cast<int64_t>(level) * a.n * 4;
                        *reinterpret_cast<uint32_t*>(base + at) = v;
                    };
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        put(8 * q, bits[q].x);
                        put(8 * q + 1, bits[q].y);
                        put(8 * q + 4, bits[q].z);
                        put(8 * q + 5, bits[q].w);
                    }
                }
                // per-feature maxima of the lane group's eight levels over its 32 lanes (every
                // lane i ends with word i % 8)
                const uint32_t words[8] = {bits[0].x, bits[0].y, bits[0].z, bits[0].w,
                                           bits[1].x, bits[1].y, bits[1].z, bits[1].w};
                uint32_t peak[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) peak[j] = valid ? pair_magnitudes(words[j]) : 0u;
                tile_peak = group_max8(peak, lane);
            } else if (valid) {
                uint16_t* p = a.dz + row * S::kIn;
#pragma unroll
                for (int ks = 0; ks < KT; ++ks) {
                    *reinterpret_cast<uint2*>(p + 16 * ks + 4 * g) = make_uint2(bits[ks].x, bits[ks].y);
                    *reinterpret_cast<uint2*>(p + 16 * ks + 8 + 4 * g) = make_uint2(bits[ks].z, bits[ks].w);
                }
            }
        }
        wave_fence();
        {
            half8 A[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) A[i] = operand16(MA, at_op, i);
#pragma unroll
            for (int j = 0; j < KT; ++j) {
                const half8 B = operand16(MB, at_op, j);
#pragma unroll
                for (int i = 0; i < 4; ++i) gW1[i][j] = mfma16(A[i], B, gW1[i][j]);
            }
        }
    };
    // Two ways to hand out the 128-row records (4 tiles), chosen from n alone, so that the row and
    // planes layouts give every wave the same tiles in the same order (bit-identical gradients):
    // whole records per wave when there are at least four per wave (WHOLE; no barrier at all), else a
    // record per workgroup, tile w to wave w (the record's maxima then meet through LDS, one
    // barrier pair per record).  Either way two tiles per step with ping-pong input buffers, so
    // that a tile never copies the next tile's prefetch (a copy would have to wait for it).
    const int64_t records = (tiles + 3) / 4;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kMlpWaves;
    constexpr bool whole = WHOLE;   // the host's choice: records >= 4 * waves
    // this wave's sequence of tiles: position i -> tile_of(i); in the shared mode every wave of a
    // workgroup has the same count, so the barriers below are uniform
    const int64_t first = whole ? static_cast<int64_t>(blockIdx.x) * kMlpWaves + wave : static_cast<int64_t>(blockIdx.x);
    const int64_t step = whole ? waves : static_cast<int64_t>(gridDim.x);
    const int64_t count = first < records ? ((records - 1 - first) / step + 1) * (whole ? 4 : 1) : 0;
    auto tile_of = [&](int64_t i) {
        return whole ? (first + (i / 4) * step) * 4 + i % 4 : (first + i * step) * 4 + wave;
    };
    // level L = 8q + 4h + 2g + b of column 2L + f is word 4q + 2h + b of lane group g
    __shared__ uint32_t pairs[kMlpWaves][32];
    auto finish = [&](int64_t i) {   // after the tile at position i
        if constexpr (PLANES) {
            record_peak = pair_max(record_peak, tile_peak);
            if (whole && i % 4 != 3) return;
            // lanes 0..31 hold the pair of their column 2L + f
            const int level = lane / 2, f = lane % 2;
            const int lg = (level / 2) % 2, word = 4 * (level / 8) + 2 * ((level / 4) % 2) + level % 2;
            const uint32_t m = static_cast<uint32_t>(__shfl(static_cast<int>(record_peak), 32 * lg + word));
            record_peak = 0;
            const int64_t record = tile_of(i) / 4;
            if constexpr (WHOLE) {
                if (lane < 32) a.blockmax[record * 32 + lane] = __half2float(bits_to_half(static_cast<uint16_t>(m >> (16 * f))));
                return;
            }
            // the four waves' tiles of the record meet in LDS
            if (lane < 32) pairs[wave][lane] = m;
            __syncthreads();
            if (threadIdx.x < 32) {
                uint32_t total = 0;
#pragma unroll
                for (int v = 0; v < kMlpWaves; ++v) total = pair_max(total, pairs[v][threadIdx.x]);
                a.blockmax[record * 32 + threadIdx.x] = __half2float(bits_to_half(static_cast<uint16_t>(total >> (16 * f))));
            }
            __syncthreads();
        }
    };
    TileInput<KT> even, odd;
    uint32_t bytes[3];
    if (count) fetch_tile<KT>(a, tile_of(0) * 32 + s, g, even);
    for (int64_t i = 0; i < count; i += 2) {
        gather_bytes(even, bytes);
        fetch_tile<KT>(a, tile_of(i + 1) * 32 + s, g, odd);
        tile_peak = 0;
        if (tile_of(i) < tiles) process(tile_of(i), even, bytes);
        finish(i);
        if (i + 1 >= count) break;
        gather_bytes(odd, bytes);
        fetch_tile<KT>(a, tile_of(i + 2) * 32 + s, g, even);
        tile_peak = 0;
        if (tile_of(i + 1) < tiles) process(tile_of(i + 1), odd, bytes);
        finish(i + 1);
    }
    // The workgroup's partial: the four waves' gradients summed in wave order in LDS (lane l holds
    // rows 4 * (l / 16) + v, column l % 16 of each 16x16 block), then written out.
    __syncthreads();
    float* P = reinterpret_cast<float*>(T);
    const int rq = 4 * (lane >> 4), cn = lane & 15;
    for (int turn = 0; turn < kMlpWaves; ++turn) {
        if (wave == turn) {
            auto put = [&](int p, float v) { P[p] = turn ? P[p] + v : v; };
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = 16 * i + rq + v;
#pragma unroll
                    for (int j = 0; j < KT; ++j) put(r * S::kIn + 16 * j + cn, gW1[i][j][v]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) put(S::kW1 + r * kHid + 16 * j + cn, gW2[i][j][v]);
                }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v)   // rows 3..15 of dW3 are zero: dy has three outputs
                    put(S::kW1 + kW2 + (rq + v) * kHid + 16 * j + cn, rq + v < 3 ? gW3[j][v] : 0.0f);
        }
        __syncthreads();
    }
    float* out = a.partials + static_cast<int64_t>(blockIdx.x) * S::kParams;
    for (int p = threadIdx.x; p < S::kParams; p += kMlpBlock) out[p] = P[p];
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
    // whole 128-row records per wave when there are at least four per wave (see the kernel)
    const int64_t records = ((n + 31) / 32 + 3) / 4;
    const bool whole = records >= int64_t{4} * blocks * kMlpWaves;
#define ODIE_TRAIN(KT, PLANES)                                                                      \
    (whole ? mlp_train_kernel<KT, PLANES, true><<<blocks, kMlpBlock, 0, s>>>(a)                    \
           : mlp_train_kernel<KT, PLANES, false><<<blocks, kMlpBlock, 0, s>>>(a))
    if (planes) {
        ODIE_TRAIN(2, true);
    } else {
        switch (kt) {
            case 1: ODIE_TRAIN(1, false); break;
            case 2: ODIE_TRAIN(2, false); break;
            case 3: ODIE_TRAIN(3, false); break;
            case 4: ODIE_TRAIN(4, false); break;
            default: ODIE_TRAIN(5, false); break;
        }
    }
#undef ODIE_TRAIN
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
