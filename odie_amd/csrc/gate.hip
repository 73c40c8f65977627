// Router gate of the hash-grid model (router_enabled): a 32 -> 32 -> 16 fp16 MLP (ReLU hidden
// layer, no bias, no output activation; TCNN FullyFusedMLP at odie/hash_grid.py:28-30) gives one
// logit per level, s = 1 for the first K levels and sigmoid / softplus of the logit above, and
// every level's features are scaled by fp16(s * visible) -- parallel_gate and
// parallel_gate_back of odie/native/runtime.cu:64-92, with hash_router_gradient (:99-103)
// forming the grid's upstream.
//
//   gate_forward:  raw x [n][32] fp16 -> weighted [n][32] fp16 (the decoder input), s [n][L] fp32
//   gate_backward: raw x, value = fp16(dL/dweighted / 128) [n][32] (odie_mlp_train's dz), s ->
//                  upstream [n][32] = fp16(direct + fp16(dL/draw_gate / 128)),
//                  dWgate fp32 [1536] (loss scale 16384)
//
// Gate weights: fp16 [1536] = Wg1 [32][32] | Wg2 [16][32], row-major [out][in].  16 levels x 2
// features (32 inputs, 16 logits) per sample.
//
// One wave per tile of 32 samples, v_mfma_f32_32x32x16_f16 with samples as columns (the layout
// scheme of mlp.hip).  Lane (g, s) holds features 16kt + 8g + e (kt = 0, 1; e = 0..7) of
// sample s, i.e. levels 8kt + 4g + e/2 -- exactly the levels whose logits the layer-2
// accumulator gives that lane (rows 8(v/4) + 4g + v%4), so the gate arithmetic is per lane.
// The input-gradient product uses Wg1^T with its rows stored in the same feature order, so
// its accumulator lands in that layout too.
#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef int16_t short8 __attribute__((ext_vector_type(8)));
typedef uint16_t ushort8 __attribute__((ext_vector_type(8)));

constexpr int kIn = 32, kHid = 32, kLevels = 16;
constexpr int kG1 = kHid * kIn, kG2 = kLevels * kHid, kGateParams = kG1 + kG2;
constexpr int kGateBlock = 256;
constexpr int kGateWaves = kGateBlock / 64;
constexpr int kS = 40;                      // LDS row stride (halfs) of 32-wide rows
constexpr int kA1 = 0;                      // Wg1 [32][32] rows, A operand of layer 1
constexpr int kA2 = kA1 + 32 * kS;          // Wg2 [16][slot(32)]
constexpr int kT2 = kA2 + 16 * kS;          // Wg2^T [32][slot(16)], dHg = Wg2^T da
constexpr int kT1 = kT2 + 32 * kS;          // Wg1^T rows in lane-feature order [32][slot(32)]
constexpr int kWeightHalfs = kT1 + 32 * kS;
constexpr int kTStride = 40;                // per-wave transposition rows: 32 samples + pad
constexpr int kTRows = 112;                 // da 16, hg 32, dhg 32, x 32
constexpr int kWaveHalfs = kTRows * kTStride;

__device__ inline int slot_of(int k) {
    const int t = k >> 4, w = k & 15;
    return 16 * t + 8 * ((w >> 2) & 1) + 4 * (w >> 3) + (w & 3);
}
__device__ inline int feature_of(int t, int g, int e) { return 16 * t + 8 * (e >> 2) + 4 * g + (e & 3); }
// Feature held by accumulator row r of a 32-row block in the lane-feature order (row
// 8(v/4) + 4g + v%4 holds feature 16(v/8) + 8g + v%8).
__device__ inline int lane_feature_of_row(int r) {
    const int q = r >> 3, g = (r >> 2) & 1, j = r & 3;   // r = 8q + 4g + j, v = 4q + j
    const int v = 4 * q + j;
    return 16 * (v >> 3) + 8 * g + (v & 7);
}

__device__ inline f32x16 mfma(half8 a, half8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
__device__ inline half8 lds8(const _Float16* p) { return *reinterpret_cast<const half8*>(p); }
__device__ inline half8 round8(const f32x16& acc, int base) {
    const half2v p0 = __builtin_convertvector((float2v){acc[base + 0], acc[base + 1]}, half2v);
    const half2v p1 = __builtin_convertvector((float2v){acc[base + 2], acc[base + 3]}, half2v);
    const half2v p2 = __builtin_convertvector((float2v){acc[base + 4], acc[base + 5]}, half2v);
    const half2v p3 = __builtin_convertvector((float2v){acc[base + 6], acc[base + 7]}, half2v);
    return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3), __builtin_shufflevector(p2, p3, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ inline half8 relu8(half8 x) {
    return __builtin_bit_cast(half8, __builtin_elementwise_max(__builtin_bit_cast(short8, x), short8{}));
}
__device__ inline half8 mask8(half8 dh, half8 h) {
    const ushort8 keep = __builtin_elementwise_min(__builtin_bit_cast(ushort8, h), (ushort8)(uint16_t{1}));
    return __builtin_bit_cast(half8, __builtin_bit_cast(ushort8, dh) * keep);
}

__device__ void stage_gate(const uint16_t* weights, _Float16* w) {
    for (int i = threadIdx.x; i < kGateParams; i += kGateBlock) {
        const _Float16 v = __builtin_bit_cast(_Float16, weights[i]);
        if (i < kG1) {
            const int r = i / kIn, c = i % kIn;     // Wg1[hidden r][input c]
            w[kA1 + r * kS + c] = v;
            // Wg1^T: row = input in lane-feature order, column = hidden in slot order
            for (int row = 0; row < 32; ++row)
                if (lane_feature_of_row(row) == c) w[kT1 + row * kS + slot_of(r)] = v;
        } else {
            const int j = i - kG1, o = j / kHid, c = j % kHid;   // Wg2[level o][hidden c]
            w[kA2 + o * kS + slot_of(c)] = v;
            w[kT2 + c * kS + slot_of(o)] = v;
        }
    }
}

struct GateArgs {
    const uint16_t* raw;       // [n][32]
    const uint16_t* value;     // [n][32] (backward)
    const uint8_t* visible;    // [n][16] or null (all visible)
    const uint16_t* weights;   // [1536]
    float* sigmoid;            // [n][16]
    uint16_t* out;             // weighted [n][32] (forward) / upstream [n][32] (backward)
    float* partials;           // [blocks][1536] (backward)
    int64_t n;
    int coarse;                // levels < coarse are not gated (s = 1, no gate gradient)
    int softplus;
};

__device__ inline void load_rows(const uint16_t* base, int64_t row, bool valid, int g, half8 v[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
        v[kt] = valid ? *reinterpret_cast<const half8*>(base + row * kIn + kt * 16 + 8 * g) : half8{};
}
__device__ inline void store_rows(uint16_t* base, int64_t row, int g, const half8 v[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) *reinterpret_cast<half8*>(base + row * kIn + kt * 16 + 8 * g) = v[kt];
}

// Hidden layer and logits of one tile: hg (B operand form), logits for this lane's 8 levels
// (element v: level 8(v/4) + 4g + v%4), rounded to fp16 as the network's output.
__device__ inline void gate_layers(const _Float16* w, int g, int s, const half8 x[2], half8 hg[2], float z[8]) {
    f32x16 acc{};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) acc = mfma(lds8(w + kA1 + s * kS + kt * 16 + 8 * g), x[kt], acc);
    hg[0] = relu8(round8(acc, 0));
    hg[1] = relu8(round8(acc, 8));
    f32x16 lg{};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const half8 a = s < kLevels ? lds8(w + kA2 + s * kS + 16 * t + 8 * g) : half8{};
        lg = mfma(a, hg[t], lg);
    }
    const half8 l16 = round8(lg, 0);
#pragma unroll
    for (int v = 0; v < 8; ++v) z[v] = static_cast<float>(l16[v]);
}

// s of level l from its fp16 logit (odie/native/runtime.cu:72).
__device__ inline float gate_value(float z, int level, const GateArgs& a) {
    if (level < a.coarse) return 1.0f;
    if (a.softplus) return z > 20.0f ? z : log1pf(expf(z));
    return 1.0f / (1.0f + expf(-z));
}

__device__ inline float visible_of(const GateArgs& a, int64_t row, int level) {
    return a.visible ? static_cast<float>(a.visible[row * kLevels + level]) : 1.0f;
}

__global__ __launch_bounds__(kGateBlock) void gate_forward_kernel(GateArgs a) {
    __shared__ _Float16 w[kWeightHalfs];
    stage_gate(a.weights, w);
    __syncthreads();
    const int lane = threadIdx.x % 64, g = lane / 32, s = lane % 32;
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kGateWaves;
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kGateWaves + threadIdx.x / 64; tile < tiles; tile += stride) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        half8 x[2], hg[2];
        float z[8];
        load_rows(a.raw, row, valid, g, x);
        gate_layers(w, g, s, x, hg, z);
        if (!valid) continue;
        // level of logit v = 8(v/4) + 4g + v%4; features 2*level, 2*level + 1 sit at x[v/4][2(v%4)], [+1]
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const int level = 8 * (v / 4) + 4 * g + v % 4;
            const float sv = gate_value(z[v], level, a);
            a.sigmoid[row * kLevels + level] = sv;
            const _Float16 weight = static_cast<_Float16>(sv * visible_of(a, row, level));
            const int kt = v / 4, e = 2 * (v % 4);
            x[kt][e] = x[kt][e] * weight;
            x[kt][e + 1] = x[kt][e + 1] * weight;
        }
        store_rows(a.out, row, g, x);
    }
}

__global__ __launch_bounds__(kGateBlock) void gate_backward_kernel(GateArgs a) {
    __shared__ _Float16 w[kWeightHalfs];
    __shared__ __attribute__((aligned(16))) _Float16 transposed[kGateWaves * kWaveHalfs];
    stage_gate(a.weights, w);
    __syncthreads();
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, g = lane / 32, s = lane % 32;
    _Float16* T = transposed + wave * kWaveHalfs;
    f32x16 g1{}, g2{};
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kGateWaves;
    const _Float16 half128 = static_cast<_Float16>(128.0f);
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kGateWaves + wave; tile < tiles; tile += stride) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        half8 x[2], value[2], hg[2], direct[2];
        float z[8];
        load_rows(a.raw, row, valid, g, x);
        load_rows(a.value, row, valid, g, value);
        gate_layers(w, g, s, x, hg, z);
        // parallel_gate_back (odie/native/runtime.cu:77-91) per level of this lane
        half8 da{};
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const int level = 8 * (v / 4) + 4 * g + v % 4;
            const int kt = v / 4, e = 2 * (v % 4);
            const float sv = valid ? a.sigmoid[row * kLevels + level] : 0.0f;
            const float vis = valid ? visible_of(a, row, level) : 0.0f;
            const _Float16 weight = static_cast<_Float16>(sv * vis);
            direct[kt][e] = value[kt][e] * weight;
            direct[kt][e + 1] = value[kt][e + 1] * weight;
            _Float16 reduced = static_cast<_Float16>(0.0f);
            reduced = reduced + value[kt][e] * x[kt][e];
            reduced = reduced + value[kt][e + 1] * x[kt][e + 1];
            const float incoming = static_cast<float>(reduced) * vis;
            float derivative = 0.0f;
            if (level >= a.coarse) derivative = a.softplus ? incoming * -expm1f(-sv) : incoming * (1.0f - sv) * sv;
            da[v] = static_cast<_Float16>(derivative) * half128;
        }
        // gate MLP backward: dHg = relu'(hg) * (Wg2^T da); d(raw) = Wg1^T dHg
        half8 dhg[2];
        {
            const f32x16 acc = mfma(lds8(w + kT2 + s * kS + 8 * g), da, f32x16{});
            dhg[0] = mask8(round8(acc, 0), hg[0]);
            dhg[1] = mask8(round8(acc, 8), hg[1]);
        }
        f32x16 acc{};
#pragma unroll
        for (int t = 0; t < 2; ++t) acc = mfma(lds8(w + kT1 + s * kS + 16 * t + 8 * g), dhg[t], acc);
        if (valid) {
            // hash_router_gradient (odie/native/runtime.cu:99-103): direct + fp16(dr / 128)
            const half8 scale = (half8)(static_cast<_Float16>(0.0078125f));
            half8 up[2] = {direct[0] + round8(acc, 0) * scale, direct[1] + round8(acc, 8) * scale};
            store_rows(a.out, row, g, up);
        }
        // weight gradients over this tile's samples: dWg2 = sum da (x) hg, dWg1 = sum dhg (x) x;
        // rows 0..15 da, 16..47 hg, 48..79 dhg, 80..111 x (feature-major, samples contiguous)
#pragma unroll
        for (int v = 0; v < 8; ++v) T[(8 * (v / 4) + 4 * g + v % 4) * kTStride + s] = da[v];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                T[(16 + feature_of(t, g, e)) * kTStride + s] = hg[t][e];
                T[(48 + feature_of(t, g, e)) * kTStride + s] = dhg[t][e];
                T[(80 + 16 * t + 8 * g + e) * kTStride + s] = x[t][e];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const half8 ada = s < kLevels ? lds8(T + s * kTStride + kt * 16 + 8 * g) : half8{};
            g2 = mfma(ada, lds8(T + (16 + s) * kTStride + kt * 16 + 8 * g), g2);
            g1 = mfma(lds8(T + (48 + s) * kTStride + kt * 16 + 8 * g), lds8(T + (80 + s) * kTStride + kt * 16 + 8 * g), g1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // reduce the waves' gradients in a fixed order through LDS, then write this workgroup's partial
    __syncthreads();
    float* sum = reinterpret_cast<float*>(transposed);
    for (int turn = 0; turn < kGateWaves; ++turn) {
        if (wave == turn) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = 8 * (v / 4) + 4 * g + v % 4;
                float* p1 = sum + r * kIn + s;                      // dWg1[hidden r][input s]
                *p1 = turn ? *p1 + g1[v] : g1[v];
                if (v < 8) {
                    float* p2 = sum + kG1 + r * kHid + s;           // dWg2[level r][hidden s]
                    *p2 = turn ? *p2 + g2[v] : g2[v];
                }
            }
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < kGateParams; i += kGateBlock)
        a.partials[static_cast<int64_t>(blockIdx.x) * kGateParams + i] = sum[i];
}

// dweights[p] = sum over workgroups of partials[b][p] in a fixed order: four lane groups of a
// 256-thread block take the workgroups b = q, q+4, q+8, ... (q = group), eight loads in flight
// per step, and the four group sums are added in group order.
constexpr int kReduceParams = 64;
__global__ __launch_bounds__(256) void gate_reduce_kernel(const float* partials, int blocks, float* dweights) {
    __shared__ float group_sum[4][kReduceParams];
    const int local = threadIdx.x % kReduceParams, q = threadIdx.x / kReduceParams;
    const int p = blockIdx.x * kReduceParams + local;
    float total = 0.0f;
    if (p < kGateParams) {
        int b = q;
        for (; b + 28 < blocks; b += 32) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = partials[static_cast<int64_t>(b + 4 * j) * kGateParams + p];
#pragma unroll
            for (int j = 0; j < 8; ++j) total += v[j];
        }
        for (; b < blocks; b += 4) total += partials[static_cast<int64_t>(b) * kGateParams + p];
    }
    group_sum[q][local] = total;
    __syncthreads();
    if (q == 0 && p < kGateParams)
        dweights[p] = ((group_sum[0][local] + group_sum[1][local]) + group_sum[2][local]) + group_sum[3][local];
}

int gate_blocks(int64_t n) {
    const int64_t tiles = (n + 31) / 32;
    const int64_t blocks = (tiles + kGateWaves - 1) / kGateWaves;
    return static_cast<int>(blocks < 256 ? (blocks < 1 ? 1 : blocks) : 256);
}

int check_gate(const char* what, int64_t n, int coarse, const void* raw, const void* weights) {
    const std::string w(what);
    if (n < 0 || n >= (int64_t{1} << 31)) return fail(w + ": n must be within [0, 2^31)");
    if (coarse < 0 || coarse > kLevels) return fail(w + ": coarse levels must be within [0, 16]");
    if (!weights || (n && !raw)) return fail(w + ": null pointer");
    if (reinterpret_cast<uintptr_t>(raw) % 16) return fail(w + ": rows must be 16-byte aligned");
    return 0;
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_gate_forward(const uint16_t* raw, int64_t n, const uint16_t* weights, const uint8_t* visible,
                               int coarse, int softplus, uint16_t* weighted, float* sigmoid, uint64_t stream) {
    if (check_gate("odie_gate_forward", n, coarse, raw, weights)) return -1;
    if (n == 0) return 0;
    if (!weighted || !sigmoid) return fail("odie_gate_forward: null pointer");
    if (reinterpret_cast<uintptr_t>(weighted) % 16) return fail("odie_gate_forward: rows must be 16-byte aligned");
    GateArgs a{raw, nullptr, visible, weights, sigmoid, weighted, nullptr, n, coarse, softplus ? 1 : 0};
    gate_forward_kernel<<<gate_blocks(n), kGateBlock, 0, as_stream(stream)>>>(a);
    return check_launch("odie_gate_forward");
}

ODIE_API int odie_gate_backward(const uint16_t* raw, const uint16_t* value, int64_t n, const uint16_t* weights,
                                const uint8_t* visible, const float* sigmoid, int coarse, int softplus,
                                uint16_t* upstream, float* dweights, uint64_t stream) {
    if (check_gate("odie_gate_backward", n, coarse, raw, weights)) return -1;
    if (!dweights) return fail("odie_gate_backward: null pointer");
    const hipStream_t s = as_stream(stream);
    if (n == 0) return launch_fill_zero(dweights, kGateParams, s);
    if (!value || !sigmoid || !upstream) return fail("odie_gate_backward: null pointer");
    if (reinterpret_cast<uintptr_t>(value) % 16 || reinterpret_cast<uintptr_t>(upstream) % 16)
        return fail("odie_gate_backward: rows must be 16-byte aligned");
    const int blocks = gate_blocks(n);
    float* partials = static_cast<float*>(workspace(static_cast<size_t>(blocks) * kGateParams * 4, s));
    if (!partials) return -1;
    GateArgs a{raw, value, visible, weights, const_cast<float*>(sigmoid), upstream, partials, n, coarse,
               softplus ? 1 : 0};
    gate_backward_kernel<<<blocks, kGateBlock, 0, s>>>(a);
    if (check_launch("odie_gate_backward")) return -1;
    gate_reduce_kernel<<<(kGateParams + kReduceParams - 1) / kReduceParams, 256, 0, s>>>(partials, blocks, dweights);
    return check_launch("odie_gate_backward reduce");
}
