// Fused Adam over a flat parameter range: fp32 master weights, optional fp16 copy written in
// the same pass, fp32 or fp16 gradients carrying a loss scale.  One streaming pass, four
// parameters per thread with 16-byte accesses where aligned.  The update rules (variants 0,
// 1, 2) are in adam.h, shared with the encode backward's fused flush.
#include <cmath>

#include "adam.h"
#include "../../include/odie_amd.h"

namespace odie {

int make_adam_step(const char* what, float* master, uint16_t* half_copy, float* m, float* v, uint32_t* steps,
                   int variant, int64_t step, float lr, float beta1, float beta2, float eps, float loss_scale,
                   bool check_pointers, AdamStep& a) {
    const std::string w(what);
    if (variant < 0 || variant > 2)
        return fail(w + ": variant must be 0 (torch), 1 (per-parameter age) or 2 (age, no skip)");
    if (variant == 0 && step < 1) return fail(w + ": step must be >= 1");
    if (!(loss_scale > 0.0f)) return fail(w + ": loss_scale must be positive");
    if (!(beta1 >= 0.0f && beta1 < 1.0f && beta2 >= 0.0f && beta2 < 1.0f)) return fail(w + ": betas must be in [0, 1)");
    if (check_pointers && (!master || !m || !v || (variant != 0 && !steps))) return fail(w + ": null pointer");
    a = AdamStep{};
    a.master = master;
    a.half_copy = half_copy;
    a.m = m;
    a.v = v;
    a.steps = steps;
    a.variant = variant;
    a.lr = lr;
    a.beta1 = beta1;
    a.beta2 = beta2;
    a.eps = eps;
    a.inv_scale = 1.0f / loss_scale;
    a.log_beta1 = static_cast<float>(std::log(static_cast<double>(beta1)));
    a.log_beta2 = static_cast<float>(std::log(static_cast<double>(beta2)));
    a.rate_first = step >= kRateTable ? static_cast<uint32_t>(step - kRateTable + 1) : 1u;
    if (variant == 0) {
        const double bc1 = 1.0 - std::pow(static_cast<double>(beta1), static_cast<double>(step));
        const double bc2 = 1.0 - std::pow(static_cast<double>(beta2), static_cast<double>(step));
        a.step_size = static_cast<float>(static_cast<double>(lr) / bc1);
        a.inv_bc2_sqrt = static_cast<float>(1.0 / std::sqrt(bc2));
    }
    return 0;
}

namespace {

constexpr int kAdamBlock = 256;

// The update of parameters [0, n) by block `block` of `blocks`: four per thread and step.
__device__ inline void adam_range(const AdamStep& a, const void* grad, int grad_half, int64_t n, int64_t block,
                                  int64_t blocks) {
    const int64_t stride = blocks * kAdamBlock * 4;
    for (int64_t base = (block * kAdamBlock + threadIdx.x) * 4; base < n; base += stride) {
        if (base + 4 <= n) {
            float g[4];
            if (grad_half) {
                const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(grad) + base);
                g[0] = __half2float(bits_to_half(static_cast<uint16_t>(raw.x & 0xffffu)));
                g[1] = __half2float(bits_to_half(static_cast<uint16_t>(raw.x >> 16)));
                g[2] = __half2float(bits_to_half(static_cast<uint16_t>(raw.y & 0xffffu)));
                g[3] = __half2float(bits_to_half(static_cast<uint16_t>(raw.y >> 16)));
            } else {
                const float4 raw = *reinterpret_cast<const float4*>(static_cast<const float*>(grad) + base);
                g[0] = raw.x; g[1] = raw.y; g[2] = raw.z; g[3] = raw.w;
            }
            // variant 1 leaves parameters with a zero gradient untouched: with no fp16 copy to
            // refresh, four of them need no further memory traffic (sparse updates stay cheap)
            if (a.variant == 1 && !a.half_copy && g[0] == 0.0f && g[1] == 0.0f && g[2] == 0.0f && g[3] == 0.0f)
                continue;
            const float4 p = *reinterpret_cast<float4*>(a.master + base);
            const float4 m = *reinterpret_cast<float4*>(a.m + base);
            const float4 v = *reinterpret_cast<float4*>(a.v + base);
            uint4 age = make_uint4(0, 0, 0, 0);
            if (a.variant != 0) age = *reinterpret_cast<const uint4*>(a.steps + base);
            float ps[4] = {p.x, p.y, p.z, p.w}, ms[4] = {m.x, m.y, m.z, m.w}, vs[4] = {v.x, v.y, v.z, v.w};
            uint32_t ts[4] = {age.x, age.y, age.z, age.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) adam_math(a, g[j], ps[j], ms[j], vs[j], ts[j]);
            *reinterpret_cast<float4*>(a.master + base) = make_float4(ps[0], ps[1], ps[2], ps[3]);
            *reinterpret_cast<float4*>(a.m + base) = make_float4(ms[0], ms[1], ms[2], ms[3]);
            *reinterpret_cast<float4*>(a.v + base) = make_float4(vs[0], vs[1], vs[2], vs[3]);
            if (a.variant != 0) *reinterpret_cast<uint4*>(a.steps + base) = make_uint4(ts[0], ts[1], ts[2], ts[3]);
            if (a.half_copy) {
                uint2 out;
                out.x = static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[0]))) |
                        (static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[1]))) << 16);
                out.y = static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[2]))) |
                        (static_cast<uint32_t>(half_to_bits(__float2half_rn(ps[3]))) << 16);
                *reinterpret_cast<uint2*>(a.half_copy + base) = out;
            }
        } else {
            for (int64_t i = base; i < n; ++i) {
                const float g = grad_half ? __half2float(bits_to_half(static_cast<const uint16_t*>(grad)[i]))
                                          : static_cast<const float*>(grad)[i];
                adam_update(a, i, g);
            }
        }
    }
}

__global__ __launch_bounds__(kAdamBlock) void adam_kernel(AdamStep a, const void* grad, int grad_half, int64_t n) {
    adam_range(a, grad, grad_half, n, blockIdx.x, gridDim.x);
}

// Several parameter sets in one launch: block b updates set k with first[k] <= b < first[k+1].
struct AdamSegments {
    AdamStep step[kAdamSegments];
    const void* grad[kAdamSegments];
    int grad_half[kAdamSegments];
    int64_t n[kAdamSegments];
    int64_t first[kAdamSegments + 1];
    int count;
};

__global__ __launch_bounds__(kAdamBlock) void adam_segments_kernel(AdamSegments s) {
    int k = 0;
    while (k + 1 < s.count && static_cast<int64_t>(blockIdx.x) >= s.first[k + 1]) ++k;
    adam_range(s.step[k], s.grad[k], s.grad_half[k], s.n[k], blockIdx.x - s.first[k], s.first[k + 1] - s.first[k]);
}

int64_t adam_blocks(int64_t n) {
    const int64_t blocks = (n + kAdamBlock * 4 - 1) / (kAdamBlock * 4);
    return blocks > 16384 ? 16384 : blocks;
}

}  // namespace

int launch_adam(const AdamStep& a, const void* grad, int grad_half, int64_t n, hipStream_t stream) {
    if (n == 0) return 0;
    adam_kernel<<<static_cast<uint32_t>(adam_blocks(n)), kAdamBlock, 0, stream>>>(a, grad, grad_half, n);
    return check_launch("adam step");
}

int launch_adam_sets(const AdamSet* sets, int count, hipStream_t stream) {
    if (count < 1 || count > kAdamSegments) return fail("adam step: 1 to 3 parameter sets per launch");
    AdamSegments s{};
    s.first[0] = 0;
    for (int k = 0; k < count; ++k) {
        s.step[k] = sets[k].step;
        s.grad[k] = sets[k].grad;
        s.grad_half[k] = sets[k].grad_half;
        s.n[k] = sets[k].n;
        s.first[k + 1] = s.first[k] + adam_blocks(sets[k].n);
    }
    s.count = count;
    if (s.first[count] == 0) return 0;
    adam_segments_kernel<<<static_cast<uint32_t>(s.first[count]), kAdamBlock, 0, stream>>>(s);
    return check_launch("adam step");
}

}  // namespace odie

using namespace odie;

ODIE_API int odie_adam_step(float* master, uint16_t* half_copy, const void* grad, int grad_dtype, float* m, float* v,
                            uint32_t* steps, int64_t n, int variant, int64_t step, float lr, float beta1, float beta2,
                            float eps, float loss_scale, uint64_t stream) {
    if (n < 0) return fail("odie_adam_step: n must be nonnegative");
    if (grad_dtype != ODIE_F32 && grad_dtype != ODIE_F16) return fail("odie_adam_step: grad_dtype must be 0 or 1");
    AdamStep a;
    if (make_adam_step("odie_adam_step", master, half_copy, m, v, steps, variant, step, lr, beta1, beta2, eps,
                       loss_scale, n > 0, a))
        return -1;
    if (n == 0) return 0;
    if (!grad) return fail("odie_adam_step: null pointer");
    const bool aligned = reinterpret_cast<uintptr_t>(master) % 16 == 0 && reinterpret_cast<uintptr_t>(m) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(grad) % (grad_dtype == ODIE_F16 ? 8 : 16) == 0 &&
                         (!half_copy || reinterpret_cast<uintptr_t>(half_copy) % 8 == 0) &&
                         (variant == 0 || reinterpret_cast<uintptr_t>(steps) % 16 == 0);
    if (!aligned) return fail("odie_adam_step: buffers must be 16-byte aligned (fp16 buffers 8-byte)");
    return launch_adam(a, grad, grad_dtype == ODIE_F16, n, as_stream(stream));
}
