// Decoder MLP on MFMA: 32 -> 64 -> 64 -> 16, ReLU on the hidden layers, no bias, no output
// activation, fp16 weights and activations, fp32 accumulation -- the decoder head of the
// reference (FullyFusedMLP config at odie/hash_grid.py:32-34, odie/model.py:186-195; used by
// the native step at odie/native/runtime.cu:270,273), fused with the step's loss
// (loss_grad, odie/native/runtime.cu:53-63) and the grid-gradient unscale
// (half_unscale by 128, odie/native/runtime.cu:282).
//
// Weights: fp16 [7168] = W1 [64][32] | W2 [64][64] | W3 [16][64], each row-major [out][in].
//
// Work split: one wave per tile of 32 samples; every product is a v_mfma_f32_32x32x16_f16
// with the samples as the 32 columns.  The transposed form H^T = W * X^T keeps each sample in
// one lane pair, and the accumulator layout of one layer (lane l: sample l%32, rows
// 8*(v/4) + 4*(l/32) + v%4) is exactly the B operand of the next layer once the weights' K
// columns are permuted the same way (slot_of below), so activations never leave registers.
// Weight gradients contract over samples: the operands are transposed through a per-wave LDS
// buffer and accumulated in registers across all tiles of a wave, then reduced across waves
// (LDS, fixed order) and across workgroups (a second kernel, fixed order): deterministic.
#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kIn = 32, kHid = 64, kOut = 16;
constexpr int kW1 = kHid * kIn, kW2 = kHid * kHid, kW3 = kOut * kHid;
constexpr int kParams = kW1 + kW2 + kW3;
constexpr int kMlpBlock = 256;
constexpr int kMlpWaves = kMlpBlock / 64;

// LDS rows are padded so that 16-byte reads of 16 consecutive lanes hit distinct banks.
constexpr int kS32 = 40, kS64 = 72, kS16 = 24;
constexpr int kW1a = 0;                     // W1 [64][32]            (layer 1, A operand)
constexpr int kW2p = kW1a + 64 * kS32;      // W2 [64][slot(64)]      (layer 2)
constexpr int kW3p = kW2p + 64 * kS64;      // W3 [16][slot(64)]      (layer 3)
constexpr int kW3t = kW3p + 16 * kS64;      // W3^T [64][slot(16)]    (dH2 = W3^T dY)
constexpr int kW2t = kW3t + 64 * kS16;      // W2^T [64][slot(64)]    (dH1 = W2^T dH2)
constexpr int kW1t = kW2t + 64 * kS64;      // W1^T [32][slot(64)]    (dX = W1^T dH1)
constexpr int kWeightHalfs = kW1t + 32 * kS64;
constexpr int kTStride = 40;                // transposition rows: 32 samples + pad
constexpr int kTRows = 128;
constexpr int kWaveHalfs = kTRows * kTStride;

// K slot of feature k inside a 16-wide K step: the accumulator row order
// 16t + 8*(e/4) + 4*g + e%4 (lane group g, element e) flattened to 16t + 8g + e.
__device__ inline int slot_of(int k) {
    const int t = k >> 4, w = k & 15;
    return 16 * t + 8 * ((w >> 2) & 1) + 4 * (w >> 3) + (w & 3);
}
// Feature held by lane group g, element e of K step t (inverse of slot_of).
__device__ inline int feature_of(int t, int g, int e) { return 16 * t + 8 * (e >> 2) + 4 * g + (e & 3); }

__device__ inline f32x16 mfma(half8 a, half8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ inline half8 lds8(const _Float16* p) { return *reinterpret_cast<const half8*>(p); }
__device__ inline f32x16 zero16() { return f32x16{}; }

// Make LDS writes of every lane of this wave visible to reads of other lanes of the wave.
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline _Float16 relu_half(float x) { return static_cast<_Float16>(x > 0.0f ? x : 0.0f); }

// Weights into LDS in the six operand layouts (once per workgroup).
__device__ void stage_weights(const uint16_t* weights, _Float16* w) {
    for (int i = threadIdx.x; i < kParams; i += kMlpBlock) {
        const _Float16 v = __builtin_bit_cast(_Float16, weights[i]);
        if (i < kW1) {
            const int r = i / kIn, c = i % kIn;
            w[kW1a + r * kS32 + c] = v;
            w[kW1t + c * kS64 + slot_of(r)] = v;
        } else if (i < kW1 + kW2) {
            const int j = i - kW1, r = j / kHid, c = j % kHid;
            w[kW2p + r * kS64 + slot_of(c)] = v;
            w[kW2t + c * kS64 + slot_of(r)] = v;
        } else {
            const int j = i - kW1 - kW2, o = j / kHid, c = j % kHid;
            w[kW3p + o * kS64 + slot_of(c)] = v;
            w[kW3t + c * kS16 + slot_of(o)] = v;
        }
    }
}

struct MlpArgs {
    const uint16_t* x;        // [n][32] fp16
    const uint16_t* weights;  // [7168] fp16
    int64_t n;
    int64_t real;             // rows whose input index is >= real are padding (dy = 0)
    const uint8_t* rgb;       // image bytes [pixels][3] (target by pixel id), or null
    const int64_t* ids;       // pixel id per input row (with rgb)
    const float* target;      // fp32 [input rows][3] (without rgb)
    const int32_t* rows;      // input row of tile row j (null: identity)
    uint16_t* out;            // fp16 [input rows][16], or null
    uint16_t* hidden;         // fp16 [n][128] = h1 | h2 of tile row j, or null
    float* squares;           // fp32 [input rows], or null
    uint16_t* dz;             // fp16 [n][32] = fp16(fp16(dL/dx) / 128)
    float* partials;          // fp32 [blocks][7168]
};

// Forward of one tile: x (B operand of layer 1) -> h1, h2 (B operands of the next layers),
// y accumulator (rows 0..15 valid).
__device__ inline void forward_tile(const _Float16* w, int g, int s, const half8 xb[2], half8 h1[4], half8 h2[4],
                                    f32x16& acc3) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        f32x16 acc = zero16();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) acc = mfma(lds8(w + kW1a + (mb * 32 + s) * kS32 + kt * 16 + 8 * g), xb[kt], acc);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h1[2 * mb][e] = relu_half(acc[e]);
            h1[2 * mb + 1][e] = relu_half(acc[8 + e]);
        }
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        f32x16 acc = zero16();
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = mfma(lds8(w + kW2p + (mb * 32 + s) * kS64 + 16 * t + 8 * g), h1[t], acc);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h2[2 * mb][e] = relu_half(acc[e]);
            h2[2 * mb + 1][e] = relu_half(acc[8 + e]);
        }
    }
    acc3 = zero16();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const half8 a = s < kOut ? lds8(w + kW3p + s * kS64 + 16 * t + 8 * g) : half8{};
        acc3 = mfma(a, h2[t], acc3);
    }
}

__device__ inline void load_x(const uint16_t* x, int64_t row, bool valid, int g, half8 xb[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
        xb[kt] = valid ? *reinterpret_cast<const half8*>(x + row * kIn + kt * 16 + 8 * g) : half8{};
}

// Output row o of accumulator element v (v < 8): 8*(v/4) + 4*g + v%4.
__device__ inline void store_out(uint16_t* out, int64_t row, int g, const half8& y) {
    const u32x4 bits = __builtin_bit_cast(u32x4, y);   // element 2i in the low half of dword i
    uint16_t* p = out + row * kOut;
    *reinterpret_cast<uint2*>(p + 4 * g) = make_uint2(bits.x, bits.y);
    *reinterpret_cast<uint2*>(p + 8 + 4 * g) = make_uint2(bits.z, bits.w);
}

__global__ __launch_bounds__(kMlpBlock) void mlp_forward_kernel(const uint16_t* x, int64_t n, const uint16_t* weights,
                                                                uint16_t* out) {
    __shared__ _Float16 w[kWeightHalfs];
    stage_weights(weights, w);
    __syncthreads();
    const int lane = threadIdx.x % 64, g = lane / 32, s = lane % 32;
    const int64_t tiles = (n + 31) / 32;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kMlpWaves;
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kMlpWaves + threadIdx.x / 64; tile < tiles; tile += waves) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < n;
        half8 xb[2], h1[4], h2[4];
        f32x16 acc3;
        load_x(x, row, valid, g, xb);
        forward_tile(w, g, s, xb, h1, h2, acc3);
        half8 y;
#pragma unroll
        for (int v = 0; v < 8; ++v) y[v] = static_cast<_Float16>(acc3[v]);
        if (valid) store_out(out, row, g, y);
    }
}

__global__ __launch_bounds__(kMlpBlock) void mlp_train_kernel(MlpArgs a) {
    __shared__ _Float16 w[kWeightHalfs];
    __shared__ __attribute__((aligned(16))) _Float16 transposed[kMlpWaves * kWaveHalfs];
    stage_weights(a.weights, w);
    __syncthreads();
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, g = lane / 32, s = lane % 32;
    _Float16* T = transposed + wave * kWaveHalfs;
    f32x16 gw3[2], gw2[2][2], gw1[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        gw3[i] = zero16();
        gw1[i] = zero16();
        gw2[i][0] = zero16();
        gw2[i][1] = zero16();
    }
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kMlpWaves;
    const float inv255 = 1.0f / 255.0f;
    const float denominator = static_cast<float>(3 * a.real);
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kMlpWaves + wave; tile < tiles; tile += waves) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        const int64_t input = valid ? (a.rows ? a.rows[row] : row) : 0;
        half8 xb[2], h1[4], h2[4];
        f32x16 acc3;
        load_x(a.x, row, valid, g, xb);
        forward_tile(w, g, s, xb, h1, h2, acc3);
        half8 y, dy{};
#pragma unroll
        for (int v = 0; v < 8; ++v) y[v] = static_cast<_Float16>(acc3[v]);
        if (valid && a.out) store_out(a.out, input, g, y);
        // loss (odie/native/runtime.cu:53-63): outputs 0..2 live in lane group 0, v = 0..2
        if (valid && g == 0) {
            float square = 0.0f;
            if (input < a.real) {
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const float t = a.rgb ? __fmul_rn(static_cast<float>(a.rgb[3 * a.ids[input] + c]), inv255)
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
        // dW3 = sum_samples dy (x) h2: T rows 0..15 = dy, 16..79 = h2 (feature-major, samples contiguous)
#pragma unroll
        for (int v = 0; v < 8; ++v) T[(8 * (v / 4) + 4 * g + v % 4) * kTStride + s] = dy[v];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) T[(16 + feature_of(t, g, e)) * kTStride + s] = h2[t][e];
        wave_sync();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const half8 ay = s < kOut ? lds8(T + s * kTStride + kt * 16 + 8 * g) : half8{};
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
                gw3[nb] = mfma(ay, lds8(T + (16 + nb * 32 + s) * kTStride + kt * 16 + 8 * g), gw3[nb]);
        }
        // dH2 = relu'(h2) * (W3^T dy)
        half8 dh2[4];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            f32x16 acc = mfma(lds8(w + kW3t + (mb * 32 + s) * kS16 + 8 * g), dy, zero16());
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                dh2[2 * mb][e] = h2[2 * mb][e] > static_cast<_Float16>(0.0f) ? static_cast<_Float16>(acc[e]) : _Float16{};
                dh2[2 * mb + 1][e] =
                    h2[2 * mb + 1][e] > static_cast<_Float16>(0.0f) ? static_cast<_Float16>(acc[8 + e]) : _Float16{};
            }
        }
        wave_sync();
        // dW2 = sum dh2 (x) h1: T rows 0..63 = dh2, 64..127 = h1
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                T[feature_of(t, g, e) * kTStride + s] = dh2[t][e];
                T[(64 + feature_of(t, g, e)) * kTStride + s] = h1[t][e];
            }
        wave_sync();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                const half8 ad = lds8(T + (mb * 32 + s) * kTStride + kt * 16 + 8 * g);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    gw2[mb][nb] = mfma(ad, lds8(T + (64 + nb * 32 + s) * kTStride + kt * 16 + 8 * g), gw2[mb][nb]);
            }
        // dH1 = relu'(h1) * (W2^T dH2)
        half8 dh1[4];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            f32x16 acc = zero16();
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = mfma(lds8(w + kW2t + (mb * 32 + s) * kS64 + 16 * t + 8 * g), dh2[t], acc);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                dh1[2 * mb][e] = h1[2 * mb][e] > static_cast<_Float16>(0.0f) ? static_cast<_Float16>(acc[e]) : _Float16{};
                dh1[2 * mb + 1][e] =
                    h1[2 * mb + 1][e] > static_cast<_Float16>(0.0f) ? static_cast<_Float16>(acc[8 + e]) : _Float16{};
            }
        }
        wave_sync();
        // dW1 = sum dh1 (x) x: T rows 0..63 = dh1, 64..95 = x
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) T[feature_of(t, g, e) * kTStride + s] = dh1[t][e];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 8; ++e) T[(64 + kt * 16 + 8 * g + e) * kTStride + s] = xb[kt][e];
        wave_sync();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const half8 bx = lds8(T + (64 + s) * kTStride + kt * 16 + 8 * g);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) gw1[mb] = mfma(lds8(T + (mb * 32 + s) * kTStride + kt * 16 + 8 * g), bx, gw1[mb]);
        }
        wave_sync();
        // dX = W1^T dH1, then the grid's unscale: fp16(fp16(dx) / 128)
        f32x16 acc = zero16();
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = mfma(lds8(w + kW1t + s * kS64 + 16 * t + 8 * g), dh1[t], acc);
        if (valid) {
            uint16_t* p = a.dz + row * kIn;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                half8 h;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    h[j] = static_cast<_Float16>(static_cast<float>(static_cast<_Float16>(acc[8 * q + j])) * (1.0f / 128.0f));
                const u32x4 bits = __builtin_bit_cast(u32x4, h);
                *reinterpret_cast<uint2*>(p + 16 * q + 4 * g) = make_uint2(bits.x, bits.y);
                *reinterpret_cast<uint2*>(p + 16 * q + 8 + 4 * g) = make_uint2(bits.z, bits.w);
            }
        }
    }
    // Reduce the waves' weight gradients in a fixed order through LDS, then write this
    // workgroup's partial.
    __syncthreads();
    float* sum = reinterpret_cast<float*>(transposed);   // 7168 floats fit in the transposition buffers
    for (int turn = 0; turn < kMlpWaves; ++turn) {
        if (wave == turn) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = 8 * (v / 4) + 4 * g + v % 4;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    float* p1 = sum + (mb * 32 + r) * kIn + s;
                    *p1 = turn ? *p1 + gw1[mb][v] : gw1[mb][v];
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        float* p2 = sum + kW1 + (mb * 32 + r) * kHid + nb * 32 + s;
                        *p2 = turn ? *p2 + gw2[mb][nb][v] : gw2[mb][nb][v];
                    }
                }
                if (v < 8) {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        float* p3 = sum + kW1 + kW2 + r * kHid + nb * 32 + s;
                        *p3 = turn ? *p3 + gw3[nb][v] : gw3[nb][v];
                    }
                }
            }
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < kParams; i += kMlpBlock) a.partials[static_cast<int64_t>(blockIdx.x) * kParams + i] = sum[i];
}

// dweights[p] = sum over workgroups of partials[b][p], in workgroup order.
__global__ __launch_bounds__(256) void mlp_reduce_kernel(const float* partials, int blocks, float* dweights) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= kParams) return;
    float total = 0.0f;
    for (int b = 0; b < blocks; ++b) total += partials[static_cast<int64_t>(b) * kParams + p];
    dweights[p] = total;
}

int mlp_blocks(int64_t n) {
    const int64_t tiles = (n + 31) / 32;
    int64_t blocks = (tiles + kMlpWaves - 1) / kMlpWaves;
    return static_cast<int>(blocks < 512 ? (blocks < 1 ? 1 : blocks) : 512);
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_mlp_forward(const uint16_t* x, int64_t n, const uint16_t* weights, uint16_t* out, uint64_t stream) {
    if (n < 0) return fail("odie_mlp_forward: n must be nonnegative");
    if (n == 0) return 0;
    if (!x || !weights || !out) return fail("odie_mlp_forward: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(out) % 8)
        return fail("odie_mlp_forward: x must be 16-byte and out 8-byte aligned");
    mlp_forward_kernel<<<mlp_blocks(n), kMlpBlock, 0, as_stream(stream)>>>(x, n, weights, out);
    return check_launch("odie_mlp_forward");
}

ODIE_API int odie_mlp_train(const uint16_t* x, int64_t n, int64_t real, const uint16_t* weights, const uint8_t* rgb,
                            const int64_t* ids, const float* target, const int32_t* rows, uint16_t* out,
                            uint16_t* hidden, float* squares, uint16_t* dz, float* dweights, uint64_t stream) {
    if (n < 0 || real < 1) return fail("odie_mlp_train: need n >= 0 and real >= 1");
    if (!weights || !dweights || (n && (!x || !dz))) return fail("odie_mlp_train: null pointer");
    if (n && !(rgb ? ids != nullptr : target != nullptr)) return fail("odie_mlp_train: need rgb with ids, or target");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(dz) % 8 ||
        (out && reinterpret_cast<uintptr_t>(out) % 8))
        return fail("odie_mlp_train: x must be 16-byte, dz and out 8-byte aligned");
    const hipStream_t s = as_stream(stream);
    if (n == 0) return launch_fill_zero(dweights, kParams, s);
    const int blocks = mlp_blocks(n);
    float* partials = static_cast<float*>(workspace(static_cast<size_t>(blocks) * kParams * sizeof(float), s));
    if (!partials) return -1;
    MlpArgs a{x, weights, n, real, rgb, ids, target, rows, out, hidden, squares, dz, partials};
    mlp_train_kernel<<<blocks, kMlpBlock, 0, s>>>(a);
    if (check_launch("odie_mlp_train")) return -1;
    mlp_reduce_kernel<<<(kParams + 255) / 256, 256, 0, s>>>(partials, blocks, dweights);
    return check_launch("odie_mlp_train reduce");
}
