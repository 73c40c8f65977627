// MFMA building blocks of the decoder MLP in -> 64 -> 64 -> 16 (in = 16..80 in steps of 16; ReLU
// hidden layers, no bias, fp16 weights and activations, fp32 accumulation), shared by the
// training kernel (mlp.hip) and the fused reconstruction (reconstruct.hip) so that both compute
// the same bits.
//
// One wave per tile of 32 samples; every product is a v_mfma_f32_32x32x16_f16 with the samples
// as the 32 columns.  Lane (g, s) = (lane / 32, lane % 32) holds, for sample s, input features
// 16*kt + 8*g + e (kt < in/16; e = 0..7) as the B operand of layer 1; the accumulator layout of
// one layer (rows 8*(v/4) + 4*g + v%4 of sample s) is the B operand of the next once the
// weights' K columns are permuted the same way (slot_of).
#pragma once
#include "common.h"

namespace odie {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef int16_t short8 __attribute__((ext_vector_type(8)));
typedef uint16_t ushort8 __attribute__((ext_vector_type(8)));

constexpr int kHid = 64, kOut = 16;
constexpr int kW2 = kHid * kHid, kW3 = kOut * kHid;
constexpr int kMlpBlock = 256;
constexpr int kMlpWaves = kMlpBlock / 64;
constexpr int kMaxInputSteps = 5;            // inputs up to 80 = align16(20 levels x 4 features)

// LDS rows are padded so that 16-byte reads of 16 consecutive lanes hit distinct banks (a row
// stride that is an odd multiple of 16 bytes).
constexpr int kS64 = 72, kS16 = 24;

// Shape of the decoder for an input width of 16 * KT features (KT K steps of layer 1):
// W1 [64][in] | W2 [64][64] | W3 [16][64], and the LDS offsets (halfs) of the six operand
// layouts the kernels read.
template <int KT> struct Shape {
    static constexpr int kIn = 16 * KT;
    static constexpr int kW1 = kHid * kIn;
    static constexpr int kParams = kW1 + kW2 + kW3;   // odie/config.py:176-177: W*64 + 64*64 + 64*16
    static constexpr int kSIn = kIn + 8;
    static constexpr int kW1a = 0;                      // W1 [64][in]            (layer 1, A operand)
    static constexpr int kW2p = kW1a + 64 * kSIn;       // W2 [64][slot(64)]      (layer 2)
    static constexpr int kW3p = kW2p + 64 * kS64;       // W3 [16][slot(64)]      (layer 3)
    static constexpr int kW3t = kW3p + 16 * kS64;       // W3^T [64][slot(16)]    (dH2 = W3^T dY)
    static constexpr int kW2t = kW3t + 64 * kS16;       // W2^T [64][slot(64)]    (dH1 = W2^T dH2)
    static constexpr int kW1t = kW2t + 64 * kS64;       // W1^T [in][slot(64)]    (dX = W1^T dH1)
    static constexpr int kWeightHalfs = kW1t + kIn * kS64;
    static constexpr int kForwardHalfs = kW3t;          // the three A-operand layouts of the forward
};

// The 16-level x 2-feature decoder of the multi-expert model and the fused reconstruction.
constexpr int kIn = 32;
constexpr int kParams = Shape<2>::kParams;
constexpr int kForwardHalfs = Shape<2>::kForwardHalfs;

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

// fp16 of acc[base .. base+7], two values per conversion (v_cvt_pk_f16_f32, round to nearest even).
__device__ inline half8 round8(const f32x16& acc, int base) {
    const half2v p0 = __builtin_convertvector((float2v){acc[base + 0], acc[base + 1]}, half2v);
    const half2v p1 = __builtin_convertvector((float2v){acc[base + 2], acc[base + 3]}, half2v);
    const half2v p2 = __builtin_convertvector((float2v){acc[base + 4], acc[base + 5]}, half2v);
    const half2v p3 = __builtin_convertvector((float2v){acc[base + 6], acc[base + 7]}, half2v);
    return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3), __builtin_shufflevector(p2, p3, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}

// ReLU of fp16 values on their bit patterns: a signed 16-bit max with 0 maps every negative
// value and -0 to +0 and keeps positive values (v_pk_max_i16), so relu(fp16(x)) equals
// fp16(x > 0 ? x : 0) bit for bit, and "h > 0" afterwards is "bits != 0".
__device__ inline half8 relu8(half8 x) {
    return __builtin_bit_cast(half8, __builtin_elementwise_max(__builtin_bit_cast(short8, x), short8{}));
}

// dh where the forward activation h is nonzero, +0 elsewhere: min(bits(h), 1) is 1 or 0 per
// value and multiplies the bit pattern of dh (v_pk_min_u16, v_pk_mul_lo_u16).
// dh where the forward activation h is nonzero, +0 elsewhere: min(bits(h), 1) is 1 or 0 per
// value and multiplies the bit pattern of dh (v_pk_min_u16, v_pk_mul_lo_u16).  Written as asm:
// from the ReLU before it the compiler would otherwise turn the two packed integer ops into
// per-half compares and selects, five times the work.
__device__ inline uint32_t mask_word(uint32_t dh, uint32_t h, uint32_t ones) {
    uint32_t r;
    asm("v_pk_min_u16 %0, %1, %3\n\tv_pk_mul_lo_u16 %0, %0, %2" : "=&v"(r) : "v"(h), "v"(dh), "v"(ones));
    return r;
}
__device__ inline half8 mask8(half8 dh, half8 h) {
    const u32x4 d = __builtin_bit_cast(u32x4, dh), m = __builtin_bit_cast(u32x4, h);
    const uint32_t ones = 0x00010001u;
    return __builtin_bit_cast(half8, (u32x4){mask_word(d.x, m.x, ones), mask_word(d.y, m.y, ones),
                                             mask_word(d.z, m.z, ones), mask_word(d.w, m.w, ones)});
}

// Weights into LDS in the six operand layouts (once per workgroup).
template <int KT> __device__ inline void stage_weights(const uint16_t* weights, _Float16* w) {
    using S = Shape<KT>;
    for (int i = threadIdx.x; i < S::kParams; i += kMlpBlock) {
        const _Float16 v = __builtin_bit_cast(_Float16, weights[i]);
        if (i < S::kW1) {
            const int r = i / S::kIn, c = i % S::kIn;
            w[S::kW1a + r * S::kSIn + c] = v;
            w[S::kW1t + c * kS64 + slot_of(r)] = v;
        } else if (i < S::kW1 + kW2) {
            const int j = i - S::kW1, r = j / kHid, c = j % kHid;
            w[S::kW2p + r * kS64 + slot_of(c)] = v;
            w[S::kW2t + c * kS64 + slot_of(r)] = v;
        } else {
            const int j = i - S::kW1 - kW2, o = j / kHid, c = j % kHid;
            w[S::kW3p + o * kS64 + slot_of(c)] = v;
            w[S::kW3t + c * kS16 + slot_of(o)] = v;
        }
    }
}

struct MlpArgs {
    const uint16_t* x;        // [n][in] fp16
    const uint16_t* weights;  // [64*in + 5120] fp16
    int64_t n;
    int64_t real;             // rows whose input index is >= real are padding (dy = 0)
    const uint32_t* colors;   // packed RGB8 target of tile row j, or null
    const uint8_t* rgb;       // image bytes [pixels][3] (target by pixel id), or null
    const int64_t* ids;       // pixel id per input row (with rgb)
    const float* target;      // fp32 [input rows][3] (without rgb)
    const int32_t* rows;      // input row of tile row j (null: identity)
    uint16_t* out;            // fp16 [input rows][16], or null
    uint16_t* hidden;         // fp16 [n][128] = h1 | h2 of tile row j, or null
    float* squares;           // fp32 [input rows], or null
    uint16_t* dz;             // fp16 [n][in] = fp16(fp16(dL/dx) / 128), or null with planes
    float* partials;          // fp32 [blocks][64*in + 5120]
    uint32_t* planes;         // dz as level-major fp16 pairs [16][n], or null
    float* blockmax;          // with planes: max |dz| per 128-row record and column [n/128][32] (column 2l + f)
};

// Forward of one tile: x (B operand of layer 1, KT K steps) -> h1, h2 (B operands of the next
// layers), y accumulator (rows 0..15 valid).
template <int KT>
__device__ inline void forward_tile(const _Float16* w, int g, int s, const half8 xb[KT], half8 h1[4], half8 h2[4],
                                    f32x16& acc3) {
    using S = Shape<KT>;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        f32x16 acc = zero16();
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
            acc = mfma(lds8(w + S::kW1a + (mb * 32 + s) * S::kSIn + kt * 16 + 8 * g), xb[kt], acc);
        h1[2 * mb] = relu8(round8(acc, 0));
        h1[2 * mb + 1] = relu8(round8(acc, 8));
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        f32x16 acc = zero16();
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = mfma(lds8(w + S::kW2p + (mb * 32 + s) * kS64 + 16 * t + 8 * g), h1[t], acc);
        h2[2 * mb] = relu8(round8(acc, 0));
        h2[2 * mb + 1] = relu8(round8(acc, 8));
    }
    acc3 = zero16();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const half8 a = s < kOut ? lds8(w + S::kW3p + s * kS64 + 16 * t + 8 * g) : half8{};
        acc3 = mfma(a, h2[t], acc3);
    }
}

// Forward-only copy of the weights: the three A-operand layouts forward_tile reads.
template <int KT> __device__ inline void stage_forward_weights(const uint16_t* weights, _Float16* w) {
    using S = Shape<KT>;
    for (int i = threadIdx.x; i < S::kParams; i += kMlpBlock) {
        const _Float16 v = __builtin_bit_cast(_Float16, weights[i]);
        if (i < S::kW1) {
            w[S::kW1a + (i / S::kIn) * S::kSIn + i % S::kIn] = v;
        } else if (i < S::kW1 + kW2) {
            const int j = i - S::kW1;
            w[S::kW2p + (j / kHid) * kS64 + slot_of(j % kHid)] = v;
        } else {
            const int j = i - S::kW1 - kW2;
            w[S::kW3p + (j / kHid) * kS64 + slot_of(j % kHid)] = v;
        }
    }
}

}  // namespace
}  // namespace odie
