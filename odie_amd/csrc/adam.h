// Adam update of one parameter, shared by the standalone optimizer kernel and the encode
// backward's fused flush so that both give the same bits for the same gradient.
//
// variant 0 (torch.optim.Adam as configured at odie/optimizer.py:33-44, gradients divided by
//   the loss scale first, odie/optimizer.py:77-84), with t the global step:
//     m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g^2;
//     p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps)
// variant 1 (the tiny-cuda-nn Adam the reference's native runtime uses for the grid,
//   odie/native/runtime.cu:212-215; semantics documented at odie/train.py:121-124): a
//   parameter whose gradient is exactly zero is skipped and keeps its age; otherwise its own
//   step counter t_i advances and
//     p -= lr*sqrt(1-b2^t_i)/(1-b1^t_i) * m / (sqrt(v) + eps)
//   with 1 - b^t evaluated as -expm1(t * ln b) (ln b from the host in double): no cancellation
//   for small t, where fp32 1 - powf(b, t) keeps only the bits of b^t beyond 1.
// variant 2 (the tiny-cuda-nn Adam of the MLP heads, odie/native/runtime.cu:159-160, whose
//   weights are matrix parameters and so never skipped): as variant 1, but every parameter's
//   age advances on every step, zero gradient included.
// half_divisor > 0 first stores the gradient as a half-precision gradient buffer would:
//   g = fp16(fp16(g) / half_divisor) (the tiny-cuda-nn optimizers of the native step take fp16
//   gradients, odie/native/runtime.cu:212-215,301-309; half_divisor 1 is the plain fp16 store,
//   128 the heads' half_unscale, odie/native/kernels.cuh:140-143).
#pragma once
#include "common.h"

namespace odie {

struct AdamStep {
    float* master;          // fp32 parameters (updated)
    uint16_t* half_copy;    // fp16 copy written with the update, or null
    float* m;
    float* v;
    uint32_t* steps;        // per-parameter ages (variants 1, 2)
    int variant;
    float lr;
    float beta1;
    float beta2;
    float eps;
    float inv_scale;        // 1 / loss scale
    float step_size;        // variant 0: lr / (1 - b1^t)
    float inv_bc2_sqrt;     // variant 0: 1 / sqrt(1 - b2^t)
    float log_beta1;        // variants 1, 2: ln b1, ln b2
    float log_beta2;
    uint32_t rate_first;    // variants 1, 2: the first age of a 256-entry rate table (ages <= the step)
    float half_divisor;     // > 0: gradient rounded through fp16 first (see above); 0: as given
};

// The step size of variants 1 and 2 at age t: lr * sqrt(1 - b2^t) / (1 - b1^t).
__device__ inline float adam_rate(const AdamStep& a, uint32_t t) {
    const float age_f = static_cast<float>(t);
    return a.lr * sqrtf(-expm1f(age_f * a.log_beta2)) / -expm1f(age_f * a.log_beta1);
}

// A caller may hold adam_rate of the kRateTable ages from rate_first on (a parameter's age never
// exceeds the step count, and those that moved on every recent step have the latest ones): a
// table entry is the function's own value, so the update is the same bit for bit with or without it.
constexpr int kRateTable = 256;

// Updates p, m, v (and the age) from gradient g (still carrying the loss scale); returns
// false when the parameter is skipped (variant 1, zero gradient).  rates: null, or adam_rate of
// the ages rate_first .. rate_first + kRateTable - 1.
__device__ inline bool adam_math(const AdamStep& a, float g, float& p, float& m, float& v, uint32_t& age,
                                 const float* rates = nullptr) {
    if (a.half_divisor > 0.0f)
        g = __half2float(__float2half_rn(__half2float(__float2half_rn(g)) / a.half_divisor));
    g = g * a.inv_scale;
    if (a.variant != 0) {
        if (a.variant == 1 && g == 0.0f) return false;
        m = a.beta1 * m + (1.0f - a.beta1) * g;
        v = a.beta2 * v + (1.0f - a.beta2) * (g * g);
        const uint32_t t = age + 1;
        age = t;
        const uint32_t slot = t - a.rate_first;   // wraps past the table for t < rate_first
        const float rate = rates && slot < kRateTable ? rates[slot] : adam_rate(a, t);
        p = p - rate * (m / (sqrtf(v) + a.eps));
    } else {
        m = a.beta1 * m + (1.0f - a.beta1) * g;
        v = a.beta2 * v + (1.0f - a.beta2) * (g * g);
        p = p - a.step_size * (m / (sqrtf(v) * a.inv_bc2_sqrt + a.eps));
    }
    return true;
}

// Full read-modify-write of parameter i.
__device__ inline void adam_update(const AdamStep& a, int64_t i, float g) {
    float p = a.master[i], m = a.m[i], v = a.v[i];
    uint32_t age = a.variant != 0 ? a.steps[i] : 0u;
    if (!adam_math(a, g, p, m, v, age)) {
        if (a.half_copy) a.half_copy[i] = half_to_bits(__float2half_rn(p));   // the copy always mirrors p
        return;
    }
    a.master[i] = p;
    a.m[i] = m;
    a.v[i] = v;
    if (a.variant != 0) a.steps[i] = age;
    if (a.half_copy) a.half_copy[i] = half_to_bits(__float2half_rn(p));
}

// Host: validates the optimizer arguments (the buffers too when check_pointers) and fills a
// (bias corrections of variant 0 in double).  Returns 0 or -1 with the error set.
int make_adam_step(const char* what, float* master, uint16_t* half_copy, float* m, float* v, uint32_t* steps,
                   int variant, int64_t step, float lr, float beta1, float beta2, float eps, float loss_scale,
                   bool check_pointers, AdamStep& a);

// Host: queues the standalone optimizer pass over n parameters with gradient grad (fp32, or
// fp16 when grad_half); buffers 16-byte aligned (fp16 ones 8-byte).
int launch_adam(const AdamStep& a, const void* grad, int grad_half, int64_t n, hipStream_t stream);

// One launch over up to kAdamSegments parameter sets (each its own step, gradient and count):
// the same per-parameter updates as launch_adam on each set.
constexpr int kAdamSegments = 3;
struct AdamSet {
    AdamStep step;
    const void* grad;
    int grad_half;
    int64_t n;
};
int launch_adam_sets(const AdamSet* sets, int count, hipStream_t stream);

}  // namespace odie
