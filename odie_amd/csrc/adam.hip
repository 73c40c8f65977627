// Fused Adam over a flat parameter range: fp32 master weights, optional fp16 copy written in
// the same pass, fp32 or fp16 gradients carrying a loss scale.  One streaming pass, four
// parameters per thread with 16-byte accesses where aligned.
//
// variant 0 (torch.optim.Adam as configured at odie/optimizer.py:324, gradients divided by
//   the loss scale first, odie/optimizer.py:365), with t the global step:
//     m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g^2;
//     p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps)
// variant 1 (the tiny-cuda-nn Adam the reference's native runtime uses for the grid,
//   odie/native/runtime.cu:212-215; semantics documented at odie/train.py:121-124): a
//   parameter whose gradient is exactly zero is skipped and keeps its age; otherwise its own
//   step counter t_i advances and
//     p -= lr*sqrt(1-b2^t_i)/(1-b1^t_i) * m / (sqrt(v) + eps)
// variant 2 (the tiny-cuda-nn Adam of the MLP heads, odie/native/runtime.cu:159-160, whose
//   weights are matrix parameters and so never skipped): as variant 1, but every parameter's
//   age advances on every step, zero gradient included.
// Bias corrections are computed per call on the host in double (variant 0) or per parameter
// on the device (variants 1 and 2, ages may differ between parameters).
#include <cmath>

#include "common.h"
#include "../../include/odie_amd.h"

namespace odie {
namespace {

constexpr int kAdamBlock = 256;

struct AdamArgs {
    float* master;
    uint16_t* half_copy;
    const void* grad;
    float* m;
    float* v;
    uint32_t* steps;
    int64_t n;
    int grad_half;
    int variant;
    float lr;
    float beta1;
    float beta2;
    float eps;
    float inv_scale;
    float step_size;      // variant 0: lr / (1 - b1^t)
    float inv_bc2_sqrt;   // variant 0: 1 / sqrt(1 - b2^t)
};

__device__ inline void adam_one(const AdamArgs& a, int64_t i, float g, float& p, float& m, float& v, bool& touched) {
    g = g * a.inv_scale;
    touched = true;
    if (a.variant != 0) {
        if (a.variant == 1 && g == 0.0f) {
            touched = false;
            return;
        }
        m = a.beta1 * m + (1.0f - a.beta1) * g;
        v = a.beta2 * v + (1.0f - a.beta2) * (g * g);
        const uint32_t t = a.steps[i] + 1;
        a.steps[i] = t;
        const float rate = a.lr * sqrtf(1.0f - powf(a.beta2, static_cast<float>(t))) /
                           (1.0f - powf(a.beta1, static_cast<float>(t)));
        p = p - rate * (m / (sqrtf(v) + a.eps));
    } else {
        m = a.beta1 * m + (1.0f - a.beta1) * g;
        v = a.beta2 * v + (1.0f - a.beta2) * (g * g);
        p = p - a.step_size * (m / (sqrtf(v) * a.inv_bc2_sqrt + a.eps));
    }
}

__global__ __launch_bounds__(kAdamBlock) void adam_kernel(AdamArgs a) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kAdamBlock * 4;
    for (int64_t base = (static_cast<int64_t>(blockIdx.x) * kAdamBlock + threadIdx.x) * 4; base < a.n; base += stride) {
        if (base + 4 <= a.n) {
            float4 p = *reinterpret_cast<float4*>(a.master + base);
            float4 m = *reinterpret_cast<float4*>(a.m + base);
            float4 v = *reinterpret_cast<float4*>(a.v + base);
            float g[4];
            if (a.grad_half) {
                const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.grad) + base);
                g[0] = __half2float(bits_to_half(static_cast<uint16_t>(raw.x & 0xffffu)));
                g[1] = __half2float(bits_to_half(static_cast<uint16_t>(raw.x >> 16)));
                g[2] = __half2float(bits_to_half(static_cast<uint16_t>(raw.y & 0xffffu)));
                g[3] = __half2float(bits_to_half(static_cast<uint16_t>(raw.y >> 16)));
            } else {
                const float4 raw = *reinterpret_cast<const float4*>(static_cast<const float*>(a.grad) + base);
                g[0] = raw.x; g[1] = raw.y; g[2] = raw.z; g[3] = raw.w;
            }
            float ps[4] = {p.x, p.y, p.z, p.w}, ms[4] = {m.x, m.y, m.z, m.w}, vs[4] = {v.x, v.y, v.z, v.w};
            bool touched[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) adam_one(a, base + j, g[j], ps[j], ms[j], vs[j], touched[j]);
            *reinterpret_cast<float4*>(a.master + base) = make_float4(ps[0], ps[1], ps[2], ps[3]);
            *reinterpret_cast<float4*>(a.m + base) = make_float4(ms[0], ms[1], ms[2], ms[3]);
            *reinterpret_cast<float4*>(a.v + base) = make_float4(vs[0], vs[1], vs[2], vs[3]);
            if (a.half_copy) {
                uint2 out;
                out.x = static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[0]))) |
                        (static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[1]))) << 16);
                out.y = static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[2]))) |
                        (static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[3]))) << 16);
                *reinterpret_cast<uint2*>(a.half_copy + base) = out;
            }
        } else {
            for (int64_t i = base; i < a.n; ++i) {
                float g = a.grad_half ? __half2float(bits_to_half(static_cast<const uint16_t*>(a.grad)[i]))
                                      : static_cast<const float*>(a.grad)[i];
                float p = a.master[i], m = a.m[i], v = a.v[i];
                bool touched;
                adam_one(a, i, g, p, m, v, touched);
                a.master[i] = p;
                a.m[i] = m;
                a.v[i] = v;
                if (a.half_copy) a.half_copy[i] = half_to_bits(__float2half_rn(p));
            }
        }
    }
}

}  // namespace
}  // namespace odie

using namespace odie;

ODIE_API int odie_adam_step(float* master, uint16_t* half_copy, const void* grad, int grad_dtype, float* m, float* v,
                            uint32_t* steps, int64_t n, int variant, int64_t step, float lr, float beta1, float beta2,
                            float eps, float loss_scale, uint64_t stream) {
    if (n < 0) return fail("odie_adam_step: n must be nonnegative");
    if (variant < 0 || variant > 2)
        return fail("odie_adam_step: variant must be 0 (torch), 1 (per-parameter age) or 2 (age, no skip)");
    if (grad_dtype != ODIE_F32 && grad_dtype != ODIE_F16) return fail("odie_adam_step: grad_dtype must be 0 or 1");
    if (variant == 0 && step < 1) return fail("odie_adam_step: step must be >= 1");
    if (!(loss_scale > 0.0f)) return fail("odie_adam_step: loss_scale must be positive");
    if (!(beta1 >= 0.0f && beta1 < 1.0f && beta2 >= 0.0f && beta2 < 1.0f)) return fail("odie_adam_step: betas must be in [0, 1)");
    if (n == 0) return 0;
    if (!master || !grad || !m || !v || (variant != 0 && !steps)) return fail("odie_adam_step: null pointer");
    const bool aligned = reinterpret_cast<uintptr_t>(master) % 16 == 0 && reinterpret_cast<uintptr_t>(m) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(grad) % (grad_dtype == ODIE_F16 ? 8 : 16) == 0 &&
                         (!half_copy || reinterpret_cast<uintptr_t>(half_copy) % 8 == 0);
    if (!aligned) return fail("odie_adam_step: buffers must be 16-byte aligned (fp16 buffers 8-byte)");
    AdamArgs a{};
    a.master = master;
    a.half_copy = half_copy;
    a.grad = grad;
    a.m = m;
    a.v = v;
    a.steps = steps;
    a.n = n;
    a.grad_half = grad_dtype == ODIE_F16;
    a.variant = variant;
    a.lr = lr;
    a.beta1 = beta1;
    a.beta2 = beta2;
    a.eps = eps;
    a.inv_scale = 1.0f / loss_scale;
    if (variant == 0) {
        const double bc1 = 1.0 - std::pow(static_cast<double>(beta1), static_cast<double>(step));
        const double bc2 = 1.0 - std::pow(static_cast<double>(beta2), static_cast<double>(step));
        a.step_size = static_cast<float>(static_cast<double>(lr) / bc1);
        a.inv_bc2_sqrt = static_cast<float>(1.0 / std::sqrt(bc2));
    }
    int64_t blocks = (n + kAdamBlock * 4 - 1) / (kAdamBlock * 4);
    if (blocks > 16384) blocks = 16384;
    adam_kernel<<<static_cast<uint32_t>(blocks), kAdamBlock, 0, as_stream(stream)>>>(a);
    return check_launch("odie_adam_step");
}
