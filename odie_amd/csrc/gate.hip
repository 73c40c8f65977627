// Router gate (router_enabled): a width -> 32 -> G fp16 MLP (ReLU hidden layer, no bias, no output
// activation; TCNN FullyFusedMLP at odie/native/runtime.cu:151-162,185, odie/hash_grid.py:28-30)
// gives one logit per level (G = align16(levels) outputs, odie/native/runtime.cu:17), s = 1 for the
// first K levels and sigmoid / softplus of the logit above, and every level's features are scaled
// by fp16(s * visible) -- parallel_gate and parallel_gate_back of odie/native/runtime.cu:64-92,
// with hash_router_gradient (:99-103) forming the grid's upstream.
//
//   gate_forward:  raw x [n][width] fp16 -> weighted [n][width] fp16 (the decoder input; columns
//                  past the levels' features are 1), s [n][L] fp32
//   gate_backward: raw x, value = fp16(dL/dweighted / 128) [n][width] (odie_mlp_train's dz), s ->
//                  upstream [n][width] = fp16(direct + fp16(dL/draw_gate / 128)),
//                  dWgate fp32 [32*width + 32*G] (loss scale 16384)
//
// Gate weights: fp16 [32*width + 32*G] = Wg1 [32][width] | Wg2 [G][32], row-major [out][in]
// (odie/config.py:176: width*32 + 32*align16(levels)).  Level l owns columns
// [offset_l, offset_l + F_l) of a row, F_l in {1, 2, 4}, offsets the running sum of F in level
// order (the descriptor's output feature offset, odie/model.py:100-101).
//
// One wave per tile of 32 samples, v_mfma_f32_32x32x16_f16 with samples as columns (the layout
// scheme of mlp.hip).  Lane (g, s) holds columns 16kt + 8g + e of sample s (B operand of layer
// 1) and the logits of levels 8(v/4) + 4g + v%4 (the layer-2 accumulator).  The per-level
// weights fp16(s * visible) and the per-column products value * x pass through a per-wave LDS
// table indexed by (sample, level) or (sample, column), so a level's columns may sit in any
// lanes.  The input gradient uses Wg1^T with its rows in the columns' lane order, so its
// accumulator lands in the layout of x.
#include <cstring>
#include <string>

#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef int16_t short8 __attribute__((ext_vector_type(8)));
typedef uint16_t ushort8 __attribute__((ext_vector_type(8)));

constexpr int kHid = 32;
constexpr int kMaxWidth = 80;              // align16(20 levels x 4 features)
constexpr int kMaxGateLevels = 32;
constexpr int kGateBlock = 256;
constexpr int kGateWaves = kGateBlock / 64;
constexpr int kS = 40;                      // LDS row stride (halfs) of 32-wide rows
constexpr int kTStride = 40;                // transposition rows: 32 samples + pad

// Operand layouts of the gate for width 16 * KT and G = 16 * GT outputs (halfs).
template <int KT, int GT> struct GateShape {
    static constexpr int kIn = 16 * KT, kG = 16 * GT;
    static constexpr int kBlocks = (KT + 1) / 2;           // 32-row blocks of the input gradient
    static constexpr int kG1 = kHid * kIn, kParams = kG1 + kG * kHid;
    static constexpr int kSIn = kIn + 8;
    static constexpr int kA1 = 0;                           // Wg1 [32][in], A operand of layer 1
    static constexpr int kA2 = kA1 + 32 * kSIn;             // Wg2 [G][slot(32)]
    static constexpr int kT2 = kA2 + kG * kS;               // Wg2^T [32][slot(G)], dHg = Wg2^T da
    static constexpr int kT1 = kT2 + 32 * kS;               // Wg1^T [blocks*32][slot(32)] in lane order
    static constexpr int kWeightHalfs = kT1 + kBlocks * 32 * kS;
    static constexpr int kTRows = kG + 2 * kHid + kIn;      // da G, hg 32, dhg 32, x in
    static constexpr int kWaveHalfs = kTRows * kTStride;
    static constexpr int kTableHalfs = 32 * kMaxGateLevels; // level weights [32 samples][32 levels]
    static_assert(kTableHalfs + 32 * kIn <= kWaveHalfs, "the level and product tables share a wave's buffer");
};

__device__ inline int slot_of(int k) {
    const int t = k >> 4, w = k & 15;
    return 16 * t + 8 * ((w >> 2) & 1) + 4 * (w >> 3) + (w & 3);
}
__device__ inline int feature_of(int t, int g, int e) { return 16 * t + 8 * (e >> 2) + 4 * g + (e & 3); }

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
// Orders this wave's LDS writes before its lanes read what other lanes wrote.
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Levels of the rows, passed by value to the kernels and copied to LDS there.
struct LevelTable {
    uint8_t level_of[kMaxWidth];       // level of column c (0xff: a padding column)
    uint8_t offset[kMaxGateLevels];    // first column of level l
    uint8_t features[kMaxGateLevels];  // columns of level l
};

struct GateArgs {
    const uint16_t* raw;       // [n][width]
    const uint16_t* value;     // [n][width] (backward)
    const uint8_t* visible;    // [n][L] or null (all visible)
    const uint16_t* weights;   // [32*width + 32*G]
    float* sigmoid;            // [n][L]
    uint16_t* out;             // weighted [n][width] (forward) / upstream [n][width] (backward)
    float* partials;           // [blocks][32*width + 32*G] (backward)
    int64_t n;
    int levels;                // L
    int coarse;                // levels < coarse are not gated (s = 1, no gate gradient)
    int softplus;
    LevelTable table;
};

struct SharedTable {
    uint8_t level_of[kMaxWidth];
    uint8_t offset[kMaxGateLevels];
    uint8_t features[kMaxGateLevels];
};

template <int KT, int GT> __device__ void stage_gate(const GateArgs& a, _Float16* w, SharedTable& t) {
    using S = GateShape<KT, GT>;
    for (int i = threadIdx.x; i < S::kBlocks * 32 * kS; i += kGateBlock) w[S::kT1 + i] = 0;   // rows past width
    for (int i = threadIdx.x; i < kMaxWidth; i += kGateBlock) t.level_of[i] = a.table.level_of[i];
    for (int i = threadIdx.x; i < kMaxGateLevels; i += kGateBlock) {
        t.offset[i] = a.table.offset[i];
        t.features[i] = a.table.features[i];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < S::kParams; i += kGateBlock) {
        const _Float16 v = __builtin_bit_cast(_Float16, a.weights[i]);
        if (i < S::kG1) {
            const int r = i / S::kIn, c = i % S::kIn;     // Wg1[hidden r][input c]
            w[S::kA1 + r * S::kSIn + c] = v;
            // Wg1^T: block c / 32, row slot_of(c % 32) (the lane order of column c), column = hidden in slot order
            w[S::kT1 + (32 * (c / 32) + slot_of(c % 32)) * kS + slot_of(r)] = v;
        } else {
            const int j = i - S::kG1, o = j / kHid, c = j % kHid;   // Wg2[level o][hidden c]
            w[S::kA2 + o * kS + slot_of(c)] = v;
            w[S::kT2 + c * kS + slot_of(o)] = v;
        }
    }
}

template <int KT> __device__ inline void load_rows(const uint16_t* base, int64_t row, bool valid, int g, half8 v[KT]) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
        v[kt] = valid ? *reinterpret_cast<const half8*>(base + row * (16 * KT) + kt * 16 + 8 * g) : half8{};
}
template <int KT> __device__ inline void store_rows(uint16_t* base, int64_t row, int g, const half8 v[KT]) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) *reinterpret_cast<half8*>(base + row * (16 * KT) + kt * 16 + 8 * g) = v[kt];
}

// Hidden layer and logits of one tile: hg (B operand form), logits for this lane's levels
// (element v: level 8(v/4) + 4g + v%4, v < 8 GT), rounded to fp16 as the network's output.
template <int KT, int GT>
__device__ inline void gate_layers(const _Float16* w, int g, int s, const half8 x[KT], half8 hg[2], half8 z[GT]) {
    using S = GateShape<KT, GT>;
    f32x16 acc{};
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) acc = mfma(lds8(w + S::kA1 + s * S::kSIn + kt * 16 + 8 * g), x[kt], acc);
    hg[0] = relu8(round8(acc, 0));
    hg[1] = relu8(round8(acc, 8));
    f32x16 lg{};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const half8 a = s < S::kG ? lds8(w + S::kA2 + s * kS + 16 * t + 8 * g) : half8{};
        lg = mfma(a, hg[t], lg);
    }
#pragma unroll
    for (int t = 0; t < GT; ++t) z[t] = round8(lg, 8 * t);
}

__device__ inline int level_of_element(int v, int g) { return 8 * (v / 4) + 4 * g + v % 4; }

// s of level l from its fp16 logit (odie/native/runtime.cu:72).
__device__ inline float gate_value(float z, int level, const GateArgs& a) {
    if (level < a.coarse) return 1.0f;
    if (a.softplus) return z > 20.0f ? z : log1pf(expf(z));
    return 1.0f / (1.0f + expf(-z));
}

__device__ inline float visible_of(const GateArgs& a, int64_t row, int level) {
    return a.visible ? static_cast<float>(a.visible[row * a.levels + level]) : 1.0f;
}

template <int KT, int GT> __global__ __launch_bounds__(kGateBlock) void gate_forward_kernel(GateArgs a) {
    using S = GateShape<KT, GT>;
    __shared__ _Float16 w[S::kWeightHalfs];
    __shared__ SharedTable table;
    __shared__ __attribute__((aligned(16))) _Float16 scratch[kGateWaves * S::kTableHalfs];
    stage_gate<KT, GT>(a, w, table);
    __syncthreads();
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, g = lane / 32, s = lane % 32;
    _Float16* weight_of = scratch + wave * S::kTableHalfs + s * kMaxGateLevels;   // this sample's level weights
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kGateWaves;
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kGateWaves + wave; tile < tiles; tile += stride) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        half8 x[KT], hg[2], z[GT];
        load_rows<KT>(a.raw, row, valid, g, x);
        gate_layers<KT, GT>(w, g, s, x, hg, z);
#pragma unroll
        for (int v = 0; v < 8 * GT; ++v) {
            const int level = level_of_element(v, g);
            if (level < a.levels) {
                const float sv = gate_value(static_cast<float>(z[v / 8][v % 8]), level, a);
                if (valid) a.sigmoid[row * a.levels + level] = sv;
                weight_of[level] = static_cast<_Float16>(sv * (valid ? visible_of(a, row, level) : 0.0f));
            }
        }
        wave_sync();
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int level = table.level_of[16 * kt + 8 * g + e];
                x[kt][e] = level != 0xff ? x[kt][e] * weight_of[level] : static_cast<_Float16>(1.0f);
            }
        if (valid) store_rows<KT>(a.out, row, g, x);
        wave_sync();
    }
}

template <int KT, int GT> __global__ __launch_bounds__(kGateBlock) void gate_backward_kernel(GateArgs a) {
    using S = GateShape<KT, GT>;
    __shared__ _Float16 w[S::kWeightHalfs];
    __shared__ SharedTable table;
    __shared__ __attribute__((aligned(16))) _Float16 transposed[kGateWaves * S::kWaveHalfs];
    stage_gate<KT, GT>(a, w, table);
    __syncthreads();
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, g = lane / 32, s = lane % 32;
    _Float16* T = transposed + wave * S::kWaveHalfs;
    // the level weights and the column products of this wave's samples share the wave's rows
    _Float16* weight_of = T + s * kMaxGateLevels;
    _Float16* product_of = T + S::kTableHalfs + s * S::kIn;
    f32x16 g1[S::kBlocks], g2{};
#pragma unroll
    for (int b = 0; b < S::kBlocks; ++b) g1[b] = f32x16{};
    const int64_t tiles = (a.n + 31) / 32;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kGateWaves;
    const _Float16 half128 = static_cast<_Float16>(128.0f);
    for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kGateWaves + wave; tile < tiles; tile += stride) {
        const int64_t row = tile * 32 + s;
        const bool valid = row < a.n;
        half8 x[KT], value[KT], hg[2], z[GT];
        load_rows<KT>(a.raw, row, valid, g, x);
        load_rows<KT>(a.value, row, valid, g, value);
        gate_layers<KT, GT>(w, g, s, x, hg, z);
        // parallel_gate_back (odie/native/runtime.cu:77-91): products value * raw per column,
        // weights fp16(s * visible) per level
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int e = 0; e < 8; ++e) product_of[16 * kt + 8 * g + e] = value[kt][e] * x[kt][e];
        float sv[8 * GT], vis[8 * GT];
#pragma unroll
        for (int v = 0; v < 8 * GT; ++v) {
            const int level = level_of_element(v, g);
            sv[v] = valid && level < a.levels ? a.sigmoid[row * a.levels + level] : 0.0f;
            vis[v] = valid && level < a.levels ? visible_of(a, row, level) : 0.0f;
            if (level < a.levels) weight_of[level] = static_cast<_Float16>(sv[v] * vis[v]);
        }
        wave_sync();
        half8 da[GT];
#pragma unroll
        for (int v = 0; v < 8 * GT; ++v) {
            const int level = level_of_element(v, g);
            _Float16 out = static_cast<_Float16>(0.0f);
            if (level < a.levels) {
                // the level's products summed in column order, one fp16 rounding per addition
                _Float16 reduced = static_cast<_Float16>(0.0f);
                const int first = table.offset[level], count = table.features[level];
                for (int c = 0; c < count; ++c) reduced = reduced + product_of[first + c];
                const float incoming = static_cast<float>(reduced) * vis[v];
                float derivative = 0.0f;
                if (level >= a.coarse)
                    derivative = a.softplus ? incoming * -expm1f(-sv[v]) : incoming * (1.0f - sv[v]) * sv[v];
                out = static_cast<_Float16>(derivative) * half128;
            }
            da[v / 8][v % 8] = out;
        }
        half8 direct[KT];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int level = table.level_of[16 * kt + 8 * g + e];
                direct[kt][e] = level != 0xff ? value[kt][e] * weight_of[level] : static_cast<_Float16>(0.0f);
            }
        wave_sync();   // the tables are dead; the rows below reuse their space
        // gate MLP backward: dHg = relu'(hg) * (Wg2^T da); d(raw) = Wg1^T dHg
        half8 dhg[2];
        {
            f32x16 acc{};
#pragma unroll
            for (int t = 0; t < GT; ++t) acc = mfma(lds8(w + S::kT2 + s * kS + 16 * t + 8 * g), da[t], acc);
            dhg[0] = mask8(round8(acc, 0), hg[0]);
            dhg[1] = mask8(round8(acc, 8), hg[1]);
        }
        // hash_router_gradient (odie/native/runtime.cu:99-103): direct + fp16(dr / 128); block b
        // of the input gradient holds K steps 2b, 2b + 1 of the row in x's lane layout
        const half8 scale = (half8)(static_cast<_Float16>(0.0078125f));
        half8 up[KT];
#pragma unroll
        for (int b = 0; b < S::kBlocks; ++b) {
            f32x16 acc{};
#pragma unroll
            for (int t = 0; t < 2; ++t) acc = mfma(lds8(w + S::kT1 + (32 * b + s) * kS + 16 * t + 8 * g), dhg[t], acc);
#pragma unroll
            for (int q = 0; q < 2; ++q)
                if (2 * b + q < KT) up[2 * b + q] = direct[2 * b + q] + round8(acc, 8 * q) * scale;
        }
        if (valid) store_rows<KT>(a.out, row, g, up);
        // weight gradients over this tile's samples: dWg2 = sum da (x) hg, dWg1 = sum dhg (x) x;
        // rows 0..G-1 da, G.. hg, G+32.. dhg, G+64.. x (feature-major, samples contiguous)
#pragma unroll
        for (int v = 0; v < 8 * GT; ++v) T[level_of_element(v, g) * kTStride + s] = da[v / 8][v % 8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                T[(S::kG + feature_of(t, g, e)) * kTStride + s] = hg[t][e];
                T[(S::kG + 32 + feature_of(t, g, e)) * kTStride + s] = dhg[t][e];
            }
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int e = 0; e < 8; ++e) T[(S::kG + 64 + 16 * kt + 8 * g + e) * kTStride + s] = x[kt][e];
        wave_sync();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const half8 ada = s < S::kG ? lds8(T + s * kTStride + kt * 16 + 8 * g) : half8{};
            g2 = mfma(ada, lds8(T + (S::kG + s) * kTStride + kt * 16 + 8 * g), g2);
            const half8 adh = lds8(T + (S::kG + 32 + s) * kTStride + kt * 16 + 8 * g);
#pragma unroll
            for (int b = 0; b < S::kBlocks; ++b) {
                const half8 bx = 32 * b + s < S::kIn ? lds8(T + (S::kG + 64 + 32 * b + s) * kTStride + kt * 16 + 8 * g)
                                                     : half8{};
                g1[b] = mfma(adh, bx, g1[b]);
            }
        }
        wave_sync();
    }
    // reduce the waves' gradients in a fixed order through LDS, then write this workgroup's partial
    __syncthreads();
    float* sum = reinterpret_cast<float*>(transposed);
    for (int turn = 0; turn < kGateWaves; ++turn) {
        if (wave == turn) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = 8 * (v / 4) + 4 * g + v % 4;
#pragma unroll
                for (int b = 0; b < S::kBlocks; ++b)
                    if (32 * b + s < S::kIn) {
                        float* p1 = sum + r * S::kIn + 32 * b + s;     // dWg1[hidden r][input 32b + s]
                        *p1 = turn ? *p1 + g1[b][v] : g1[b][v];
                    }
                if (r < S::kG) {
                    float* p2 = sum + S::kG1 + r * kHid + s;          // dWg2[level r][hidden s]
                    *p2 = turn ? *p2 + g2[v] : g2[v];
                }
            }
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < S::kParams; i += kGateBlock)
        a.partials[static_cast<int64_t>(blockIdx.x) * S::kParams + i] = sum[i];
}

// dweights[p] = sum over workgroups of partials[b][p] in a fixed order: four lane groups of a
// 256-thread block take the workgroups b = q, q+4, q+8, ... (q = group), eight loads in flight
// per step, and the four group sums are added in group order.
constexpr int kReduceParams = 64;
__global__ __launch_bounds__(256) void gate_reduce_kernel(const float* partials, int blocks, int params,
                                                          float* dweights) {
    __shared__ float group_sum[4][kReduceParams];
    const int local = threadIdx.x % kReduceParams, q = threadIdx.x / kReduceParams;
    const int p = blockIdx.x * kReduceParams + local;
    float total = 0.0f;
    if (p < params) {
        int b = q;
        for (; b + 28 < blocks; b += 32) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = partials[static_cast<int64_t>(b + 4 * j) * params + p];
#pragma unroll
            for (int j = 0; j < 8; ++j) total += v[j];
        }
        for (; b < blocks; b += 4) total += partials[static_cast<int64_t>(b) * params + p];
    }
    group_sum[q][local] = total;
    __syncthreads();
    if (q == 0 && p < params)
        dweights[p] = ((group_sum[0][local] + group_sum[1][local]) + group_sum[2][local]) + group_sum[3][local];
}

int gate_blocks(int64_t n) {
    const int64_t tiles = (n + 31) / 32;
    const int64_t blocks = (tiles + kGateWaves - 1) / kGateWaves;
    return static_cast<int>(blocks < 256 ? (blocks < 1 ? 1 : blocks) : 256);
}

// Validates the shape and fills the level table; returns the parameter count or -1.
int64_t gate_shape(const std::string& w, int64_t n, int width, int levels, const int32_t* features, int coarse,
                   const void* raw, const void* weights, LevelTable& table) {
    if (n < 0 || n >= (int64_t{1} << 31)) return fail(w + ": n must be within [0, 2^31)");
    if (width < 16 || width > kMaxWidth || width % 16) return fail(w + ": width must be 16, 32, 48, 64 or 80");
    if (levels < 1 || levels > kMaxGateLevels) return fail(w + ": levels must be within [1, 32]");
    if (coarse < 0 || coarse > levels) return fail(w + ": coarse levels must be within [0, levels]");
    if (!weights || (n && !raw)) return fail(w + ": null pointer");
    if (reinterpret_cast<uintptr_t>(raw) % 16) return fail(w + ": rows must be 16-byte aligned");
    std::memset(&table, 0xff, sizeof(table.level_of));
    int offset = 0;
    for (int l = 0; l < levels; ++l) {
        const int f = features ? features[l] : 2;
        if (f != 1 && f != 2 && f != 4) return fail(w + ": features per level must be 1, 2 or 4");
        if (offset + f > width) return fail(w + ": the levels' features exceed the row width");
        table.offset[l] = static_cast<uint8_t>(offset);
        table.features[l] = static_cast<uint8_t>(f);
        for (int c = 0; c < f; ++c) table.level_of[offset + c] = static_cast<uint8_t>(l);
        offset += f;
    }
    for (int l = levels; l < kMaxGateLevels; ++l) table.offset[l] = table.features[l] = 0;
    if ((offset + 15) / 16 * 16 != width) return fail(w + ": width must be align16 of the levels' features");
    const int g = (levels + 15) / 16 * 16;
    return int64_t{32} * width + int64_t{32} * g;
}

#define ODIE_GATE_SWITCH(KERNEL, kt, gt, blocks, stream, args)                                            \
    do {                                                                                                 \
        switch ((kt) * 4 + (gt)) {                                                                       \
            case 5: KERNEL<1, 1><<<blocks, kGateBlock, 0, stream>>>(args); break;                       \
            case 6: KERNEL<1, 2><<<blocks, kGateBlock, 0, stream>>>(args); break;                       \
            case 9: KERNEL<2, 1><<<blocks, kGateBlock, 0, stream>>>(args); break;                       \
            case 10: KERNEL<2, 2><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
            case 13: KERNEL<3, 1><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
            case 14: KERNEL<3, 2><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
            case 17: KERNEL<4, 1><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
            case 18: KERNEL<4, 2><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
            case 21: KERNEL<5, 1><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
            default: KERNEL<5, 2><<<blocks, kGateBlock, 0, stream>>>(args); break;                      \
        }                                                                                                \
    } while (0)

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_gate_forward(const uint16_t* raw, int64_t n, int width, int levels, const int32_t* features,
                               const uint16_t* weights, const uint8_t* visible, int coarse, int softplus,
                               uint16_t* weighted, float* sigmoid, uint64_t stream) {
    GateArgs a{};
    if (gate_shape("odie_gate_forward", n, width, levels, features, coarse, raw, weights, a.table) < 0) return -1;
    if (n == 0) return 0;
    if (!weighted || !sigmoid) return fail("odie_gate_forward: null pointer");
    if (reinterpret_cast<uintptr_t>(weighted) % 16) return fail("odie_gate_forward: rows must be 16-byte aligned");
    a.raw = raw;
    a.visible = visible;
    a.weights = weights;
    a.sigmoid = sigmoid;
    a.out = weighted;
    a.n = n;
    a.levels = levels;
    a.coarse = coarse;
    a.softplus = softplus ? 1 : 0;
    // one tile per wave (the forward has no per-block partials to bound the block count)
    const int64_t tiles = (n + 31) / 32;
    int64_t forward_blocks = (tiles + kGateWaves - 1) / kGateWaves;
    forward_blocks = forward_blocks < 1 ? 1 : (forward_blocks > 8192 ? 8192 : forward_blocks);
    const uint32_t blocks = static_cast<uint32_t>(forward_blocks);
    const hipStream_t s = as_stream(stream);
    ODIE_GATE_SWITCH(gate_forward_kernel, width / 16, (levels + 15) / 16, blocks, s, a);
    return check_launch("odie_gate_forward");
}

ODIE_API int odie_gate_backward(const uint16_t* raw, const uint16_t* value, int64_t n, int width, int levels,
                                const int32_t* features, const uint16_t* weights, const uint8_t* visible,
                                const float* sigmoid, int coarse, int softplus, uint16_t* upstream, float* dweights,
                                uint64_t stream) {
    GateArgs a{};
    const int64_t params = gate_shape("odie_gate_backward", n, width, levels, features, coarse, raw, weights, a.table);
    if (params < 0) return -1;
    if (!dweights) return fail("odie_gate_backward: null pointer");
    const hipStream_t s = as_stream(stream);
    if (n == 0) return launch_fill_zero(dweights, params, s);
    if (!value || !sigmoid || !upstream) return fail("odie_gate_backward: null pointer");
    if (reinterpret_cast<uintptr_t>(value) % 16 || reinterpret_cast<uintptr_t>(upstream) % 16)
        return fail("odie_gate_backward: rows must be 16-byte aligned");
    const int blocks = gate_blocks(n);
    float* partials = static_cast<float*>(workspace(static_cast<size_t>(blocks) * params * 4, s));
    if (!partials) return -1;
    a.raw = raw;
    a.value = value;
    a.visible = visible;
    a.weights = weights;
    a.sigmoid = const_cast<float*>(sigmoid);
    a.out = upstream;
    a.partials = partials;
    a.n = n;
    a.levels = levels;
    a.coarse = coarse;
    a.softplus = softplus ? 1 : 0;
    ODIE_GATE_SWITCH(gate_backward_kernel, width / 16, (levels + 15) / 16, static_cast<uint32_t>(blocks), s, a);
    if (check_launch("odie_gate_backward")) return -1;
    gate_reduce_kernel<<<static_cast<uint32_t>((params + kReduceParams - 1) / kReduceParams), 256, 0, s>>>(
        partials, blocks, static_cast<int>(params), dweights);
    return check_launch("odie_gate_backward reduce");
}
