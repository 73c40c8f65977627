/*
 * CPU oracle for the sparse grid-query hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the arithmetic of the
 * reference's grid encode, gradient scatter, residual accumulation and Adam update so
 * that the HIP kernels can be checked against it.  Only tests/, the smoke check and
 * bench.py's cpu_baseline leg load it, and only as the checker or as the timed CPU
 * baseline; the odie_amd package never does.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).  Contraction must stay
 * off: every fp32 multiply-add below is a separate IEEE multiply and add unless it is
 * written as fmaf(), exactly as the reference kernels do.
 *
 * Citations are to the reference repository (EternalRecurrence/ODIE).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------
 * IEEE binary16 helpers.  fp16 values travel as raw uint16 bit patterns.
 * ---------------------------------------------------------------------------- */

API float ora_h2f(uint16_t h) {
    const int sign = h >> 15, exponent = (h >> 10) & 31, mantissa = h & 1023;
    float value;
    if (exponent == 0) value = ldexpf((float)mantissa, -24);
    else if (exponent == 31) value = mantissa ? NAN : INFINITY;
    else value = ldexpf((float)(1024 + mantissa), exponent - 25);
    return sign ? -value : value;
}

/* Round a double to the nearest binary16, ties to even (subnormals kept). */
API uint16_t ora_d2h(double d) {
    uint16_t sign = signbit(d) ? 0x8000u : 0u;
    double a = fabs(d);
    if (isnan(d)) return 0x7e00u;
    if (a >= 65520.0) return sign | 0x7c00u;          /* rounds past 65504 */
    if (a < 0x1p-14) {                                  /* subnormal quantum 2^-24 */
        double q = rint(a * 0x1p24);                    /* exact scaling, RNE */
        return sign | (uint16_t)q;                      /* q == 1024 encodes 2^-14 */
    }
    int e2;
    frexp(a, &e2);                                      /* a in [2^(e2-1), 2^e2) */
    int e = e2 - 1;
    double q = rint(ldexp(a, 10 - e));                  /* in [1024, 2048] */
    if (q == 2048.0) { q = 1024.0; ++e; }
    if (e + 15 >= 31) return sign | 0x7c00u;
    return sign | (uint16_t)(((e + 15) << 10) | ((int)q - 1024));
}

API uint16_t ora_f2h(float f) { return ora_d2h((double)f); }

/* fp16 value as an exact integer multiple of 2^-24 (finite inputs only). */
static __int128 h_units(uint16_t h) {
    const int exponent = (h >> 10) & 31, mantissa = h & 1023;
    __int128 k = exponent == 0 ? (__int128)mantissa : ((__int128)(1024 + mantissa) << (exponent - 1));
    return (h >> 15) ? -k : k;
}

static int bitlen128(unsigned __int128 v) {
    uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
    if (hi) return 128 - __builtin_clzll(hi);
    if (lo) return 64 - __builtin_clzll(lo);
    return 0;
}

/* Fused fp16 multiply-add with one rounding (the semantics of __hfma / v_fma_f16):
 * a*b + c is formed exactly as an integer count of 2^-48 and rounded once. */
API uint16_t ora_hfma(uint16_t a, uint16_t b, uint16_t c) {
    if (((a >> 10) & 31) == 31 || ((b >> 10) & 31) == 31 || ((c >> 10) & 31) == 31)
        return ora_d2h((double)ora_h2f(a) * (double)ora_h2f(b) + (double)ora_h2f(c));
    __int128 s = h_units(a) * h_units(b) + (h_units(c) << 24);
    if (s == 0) {
        /* exact zero: +0 unless both the product and the addend are -0 or negative zero sums */
        int product_negative = ((a ^ b) >> 15) & 1;
        int both_negative = product_negative && (c >> 15);
        return both_negative ? 0x8000u : 0u;
    }
    uint16_t sign = s < 0 ? 0x8000u : 0u;
    unsigned __int128 m = (unsigned __int128)(s < 0 ? -s : s);    /* value = m * 2^-48 */
    /* quantum in units of 2^-48: subnormal range 2^24, otherwise 2^(E-10+48) */
    int bits = bitlen128(m);                                      /* m in [2^(bits-1), 2^bits) */
    int E = bits - 1 - 48;                                        /* value in [2^E, 2^(E+1)) */
    int shift = E < -14 ? 24 : E - 10 + 48;
    unsigned __int128 q = m >> shift, rem = m - (q << shift), half = (unsigned __int128)1 << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    if (E < -14) return sign | (uint16_t)q;                       /* q <= 1024 */
    if (q == 2048) { q = 1024; ++E; }
    if (E + 15 >= 31) return sign | 0x7c00u;
    return sign | (uint16_t)(((E + 15) << 10) | ((int)q - 1024));
}

/* Fast forms used inside the encode loops.  h2f_fast/d2h_fast are bit-level conversions
 * (same results as ora_h2f/ora_d2h); hfma_fast forms a*b + c in double, which is exact
 * unless the TwoSum error term is nonzero, and falls back to the exact integer path
 * otherwise -- so it returns ora_hfma's result for every input. */
static inline float h2f_fast(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0) { const float v = (float)m * 0x1p-24f; return sign ? -v : v; }
    uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

static inline uint16_t d2h_fast(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const uint64_t a = b & 0x7fffffffffffffffull;
    if (a >= 0x7ff0000000000000ull) return a > 0x7ff0000000000000ull ? 0x7e00u : (uint16_t)(sign | 0x7c00u);
    int e = (int)(a >> 52) - 1023;
    if (e >= 16) return sign | 0x7c00u;
    if (e < -25) return sign;
    const uint64_t m = (a & 0xfffffffffffffull) | (1ull << 52);
    const int shift = (e >= -14 ? e - 10 : -24) - (e - 52);
    uint64_t kept = m >> shift;
    const uint64_t rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (kept & 1))) ++kept;
    if (e >= -14) {
        if (kept == 2048) { kept = 1024; ++e; }
        if (e > 15) return sign | 0x7c00u;
        return (uint16_t)(sign | ((e + 15) << 10) | (kept - 1024));
    }
    return (uint16_t)(sign | kept);
}

static inline uint16_t hfma_fast(uint16_t a, uint16_t b, uint16_t c) {
    const double p = (double)h2f_fast(a) * (double)h2f_fast(b), q = (double)h2f_fast(c);
    const double s = p + q, v = s - p;
    const double err = (p - (s - v)) + (q - v);
    if (err != 0.0 || s == 0.0 || !isfinite(s)) return ora_hfma(a, b, c);
    return d2h_fast(s);
}

API uint16_t ora_hfma_fast(uint16_t a, uint16_t b, uint16_t c) { return hfma_fast(a, b, c); }
API uint16_t ora_d2h_fast(double d) { return d2h_fast(d); }

/* ------------------------------------------------------------------------------
 * Multiresolution hash grid (tiny-cuda-nn GridEncoding semantics, 2D).
 *
 * Level geometry follows odie/config.py:83-94 (hash_grid_layout): scale is the fp32
 * value 2^(l*log2 g)*base - 1 computed on the host, res = ceil(scale)+1, the table holds
 * min(align8(res^2), 2^log2T) entries and a level is hashed when res^2 exceeds it.
 * Position: p = fmaf(scale, x, 0.5), integer corner floor(p), fraction p - floor(p).
 * Index: dense x + y*res, hashed x ^ (y * 2654435761) (Instant-NGP Eq. 4), both mod size.
 * Corners are visited (0,0),(1,0),(0,1),(1,1) with weights (1-fx)(1-fy), fx(1-fy),
 * (1-fx)fy, fx*fy, the same order and products as odie/packed_kernels.cu:12-22.
 * ---------------------------------------------------------------------------- */

typedef struct {
    float scale;        /* fp32 grid scale */
    uint32_t res;       /* vertices per side */
    uint32_t size;      /* table entries */
    uint32_t offset;    /* entry offset of this level inside one expert's table */
    uint32_t hashed;    /* 1 when res^2 > size */
} ora_level;

static inline uint32_t hash_index(const ora_level* lv, uint32_t gx, uint32_t gy) {
    uint32_t index = lv->hashed ? (gx ^ (gy * 2654435761u)) : (gx + gy * lv->res);
    /* index mod size; the two shortcuts return the same value as the division */
    if ((lv->size & (lv->size - 1)) == 0) return index & (lv->size - 1);
    if (index < lv->size) return index;
    if (index - lv->size < lv->size) return index - lv->size;
    return index % lv->size;
}

static inline void hash_geometry(const ora_level* lv, float x, float y, uint32_t idx[4], float w[4]) {
    const float px = fmaf(lv->scale, x, 0.5f), py = fmaf(lv->scale, y, 0.5f);
    const float flx = floorf(px), fly = floorf(py);
    const uint32_t gx = (uint32_t)(int32_t)flx, gy = (uint32_t)(int32_t)fly;
    const float fx = px - flx, fy = py - fly;
    w[0] = (1.0f - fx) * (1.0f - fy);
    w[1] = fx * (1.0f - fy);
    w[2] = (1.0f - fx) * fy;
    w[3] = fx * fy;
    for (int k = 0; k < 4; ++k) idx[k] = hash_index(lv, gx + (uint32_t)(k & 1), gy + (uint32_t)(k >> 1));
}

/* Per-expert coordinate ranges: coordinates [offsets[e], offsets[e+1]) use the table at
 * e * expert_params.  A single grid is experts = 1, offsets = {0, n}. */
static int expert_of(const int64_t* offsets, int experts, int64_t i) {
    int lo = 0, hi = experts - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) / 2;
        if (offsets[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return lo;
}

/* Forward.  dtype 0: fp32 table, fp32 FMA chain, fp32 output.  dtype 1: fp16 table,
 * fp16 FMA chain (single rounding per step, starting at +0), fp16 output.
 * Output row i holds level l feature c at column l*F + c of `width` columns. */
API void ora_hash_forward(const float* xy, const int64_t* offsets, int experts, int64_t expert_params,
                          const void* table, int dtype, const ora_level* levels, int n_levels,
                          int features, int width, void* out, int threads) {
    const int64_t n = offsets[experts];
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
#endif
    for (int64_t i = 0; i < n; ++i) {
        const int e = expert_of(offsets, experts, i);
        const int64_t base = (int64_t)e * expert_params;
        uint32_t idx[4];
        float w[4];
        for (int l = 0; l < n_levels; ++l) {
            const ora_level* lv = levels + l;
            hash_geometry(lv, xy[2 * i], xy[2 * i + 1], idx, w);
            for (int c = 0; c < features; ++c) {
                if (dtype == 0) {
                    const float* t = (const float*)table;
                    float v = 0.0f;
                    for (int k = 0; k < 4; ++k)
                        v = fmaf(w[k], t[base + ((int64_t)lv->offset + idx[k]) * features + c], v);
                    ((float*)out)[i * width + l * features + c] = v;
                } else {
                    const uint16_t* t = (const uint16_t*)table;
                    uint16_t v = 0;
                    for (int k = 0; k < 4; ++k)
                        v = hfma_fast(d2h_fast((double)w[k]), t[base + ((int64_t)lv->offset + idx[k]) * features + c], v);
                    ((uint16_t*)out)[i * width + l * features + c] = v;
                }
            }
        }
    }
}

/* Backward checker: grad[param] = sum of w_k * upstream over every (coordinate, corner)
 * that reads it, in double, plus the sum of absolute contributions (the scale of the
 * allowed fp32 summation error) and, when count is not null, the number of contributions
 * (each one rounded once by a fixed-point sum).  Zero upstream values are skipped, as in
 * odie/packed_kernels.cu:79-80.  upstream is fp16 [n, width] (dtype 1) or fp32. */
API void ora_hash_backward(const float* xy, const int64_t* offsets, int experts, int64_t expert_params,
                           const void* upstream, int up_dtype, const ora_level* levels, int n_levels,
                           int features, int width, double* grad, double* magnitude, double* count) {
    const int64_t n = offsets[experts];
    for (int64_t i = 0; i < n; ++i) {
        const int e = expert_of(offsets, experts, i);
        const int64_t base = (int64_t)e * expert_params;
        uint32_t idx[4];
        float w[4];
        for (int l = 0; l < n_levels; ++l) {
            const ora_level* lv = levels + l;
            hash_geometry(lv, xy[2 * i], xy[2 * i + 1], idx, w);
            for (int c = 0; c < features; ++c) {
                const int64_t col = i * width + l * features + c;
                const float value = up_dtype ? h2f_fast(((const uint16_t*)upstream)[col]) : ((const float*)upstream)[col];
                if (value == 0.0f) continue;
                for (int k = 0; k < 4; ++k) {
                    const float add = w[k] * value;                     /* fp32 product */
                    const int64_t p = base + ((int64_t)lv->offset + idx[k]) * features + c;
                    grad[p] += (double)add;
                    if (magnitude) magnitude[p] += fabs((double)add);
                    if (count) count[p] += 1.0;
                }
            }
        }
    }
}

/* Backward as the CPU baseline runs it: fp32 accumulation, atomic adds across threads. */
API void ora_hash_backward_f32(const float* xy, const int64_t* offsets, int experts, int64_t expert_params,
                               const uint16_t* upstream, const ora_level* levels, int n_levels,
                               int features, int width, float* grad, int threads) {
    const int64_t n = offsets[experts];
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
#endif
    for (int64_t i = 0; i < n; ++i) {
        const int e = expert_of(offsets, experts, i);
        const int64_t base = (int64_t)e * expert_params;
        uint32_t idx[4];
        float w[4];
        for (int l = 0; l < n_levels; ++l) {
            const ora_level* lv = levels + l;
            hash_geometry(lv, xy[2 * i], xy[2 * i + 1], idx, w);
            for (int c = 0; c < features; ++c) {
                const float value = h2f_fast(upstream[i * width + l * features + c]);
                if (value == 0.0f) continue;
                for (int k = 0; k < 4; ++k) {
                    const float add = w[k] * value;
                    float* target = grad + base + ((int64_t)lv->offset + idx[k]) * features + c;
#ifdef _OPENMP
#pragma omp atomic
#endif
                    *target += add;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------------
 * Packed xy planes (odie/packed_kernels.cu:9-88, odie/model.py:64-118).
 * Descriptor row: R, points, plane offset, node-word offset, cell-bitmap byte offset,
 * F, output feature offset, direct.
 * ---------------------------------------------------------------------------- */

static inline void plane_geometry(float x, float y, int r, int* cell, float w[4]) {
    const float px = fmaf((float)(r - 1), x, 0.5f), py = fmaf((float)(r - 1), y, 0.5f);
    const int ix = (int)floorf(px), iy = (int)floorf(py);
    const float fx = px - (float)ix, fy = py - (float)iy;
    *cell = ix + iy * r;
    w[0] = (1.0f - fx) * (1.0f - fy);
    w[1] = fx * (1.0f - fy);
    w[2] = (1.0f - fx) * fy;
    w[3] = fx * fy;
}

static inline int plane_visible(const uint8_t* bitmap, const int32_t* d, int cell) {
    return (bitmap[d[4] + (cell >> 3)] >> (cell & 7)) & 1;
}

static inline int plane_row(const uint64_t* node_bitmap, const int32_t* prefix, const int32_t* d, int node) {
    if (d[7]) return node;
    const int word = d[3] + (node >> 6), bit = node & 63;
    const uint64_t mask = (((uint64_t)1) << bit) - 1u;
    return prefix[word] + __builtin_popcountll(node_bitmap[word] & mask);
}

/* features: fp16 [n, width]; columns no level writes are set to +0. visibility [n, L]. */
API void ora_packed_forward(const float* xy, int64_t n, const float* grid, const int32_t* descriptors, int n_levels,
                            const uint64_t* node_bitmap, const int32_t* prefix, const uint8_t* bitmap,
                            int width, uint16_t* features, uint8_t* visibility, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
#endif
    for (int64_t i = 0; i < n; ++i) {
        for (int c = 0; c < width; ++c) features[i * width + c] = 0;
        for (int l = 0; l < n_levels; ++l) {
            const int32_t* d = descriptors + 8 * l;
            int cell;
            float w[4];
            plane_geometry(xy[2 * i], xy[2 * i + 1], d[0], &cell, w);
            const int on = plane_visible(bitmap, d, cell);
            visibility[i * n_levels + l] = (uint8_t)on;
            for (int c = 0; c < d[5]; ++c) {
                uint16_t v = 0;
                if (on) {
                    for (int k = 0; k < 4; ++k) {
                        const int node = (cell + (k & 1) + (k >> 1) * d[0]) % d[1];
                        const int row = plane_row(node_bitmap, prefix, d, node);
                        v = hfma_fast(d2h_fast((double)w[k]), d2h_fast((double)grid[d[2] + (int64_t)row * d[5] + c]), v);
                    }
                }
                features[i * width + d[6] + c] = v;
            }
        }
    }
}

API void ora_packed_backward(const float* xy, int64_t n, const uint16_t* upstream, int width,
                             const int32_t* descriptors, int n_levels, const uint64_t* node_bitmap,
                             const int32_t* prefix, const uint8_t* bitmap, double* grad, double* magnitude,
                             double* count) {
    for (int64_t i = 0; i < n; ++i) {
        for (int l = 0; l < n_levels; ++l) {
            const int32_t* d = descriptors + 8 * l;
            int cell;
            float w[4];
            plane_geometry(xy[2 * i], xy[2 * i + 1], d[0], &cell, w);
            if (!plane_visible(bitmap, d, cell)) continue;
            for (int c = 0; c < d[5]; ++c) {
                const float value = h2f_fast(upstream[i * width + d[6] + c]);
                if (value == 0.0f) continue;
                for (int k = 0; k < 4; ++k) {
                    const int node = (cell + (k & 1) + (k >> 1) * d[0]) % d[1];
                    const int row = plane_row(node_bitmap, prefix, d, node);
                    const float add = w[k] * value;
                    const int64_t p = d[2] + (int64_t)row * d[5] + c;
                    grad[p] += (double)add;
                    if (magnitude) magnitude[p] += fabs((double)add);
                    if (count) count[p] += 1.0;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------------
 * Residual (odie/residual_cuda.cu:11-43, odie/selection.py:58-73): per pixel
 * t = byte/255 (correctly rounded fp32 division), d = p - t in fp32, d^2 in fp32,
 * rgb = (d0^2 + d1^2) + d2^2 in fp64, cell total += rgb / 3 in fp64, in raster order.
 * Cell of pixel (x, y) is (ymap[y], xmap[x]) from the column/row bounds xb, yb.
 * ---------------------------------------------------------------------------- */
API void ora_residual(const float* prediction, const void* target, int rgb8, int64_t begin, int64_t end,
                      int width, int resolution, const int32_t* xb, const int32_t* yb, double* totals) {
    int cx = 0, cy = 0;
    for (int64_t p = begin; p < end; ++p) {
        const int x = (int)(p % width), y = (int)(p / width);
        while (cy + 1 < resolution && yb[cy + 1] <= y) ++cy;
        while (cy > 0 && yb[cy] > y) --cy;
        cx = 0;
        while (cx + 1 < resolution && xb[cx + 1] <= x) ++cx;
        const int64_t q = (p - begin) * 3;
        float t[3];
        for (int c = 0; c < 3; ++c)
            t[c] = rgb8 ? (float)((const uint8_t*)target)[q + c] / 255.0f : ((const float*)target)[q + c];
        const float d0 = prediction[q] - t[0], d1 = prediction[q + 1] - t[1], d2 = prediction[q + 2] - t[2];
        double rgb = (double)(d0 * d0) + (double)(d1 * d1);
        rgb = rgb + (double)(d2 * d2);
        totals[(int64_t)cy * resolution + cx] += rgb / 3.0;
    }
}

/* ------------------------------------------------------------------------------
 * Adam, in double (the HIP update runs in fp32 and is compared with a tolerance).
 * variant 0, torch-style: torch.optim.Adam(betas, eps, weight_decay=0) as configured at
 *   odie/optimizer.py:33-44, gradient divided by the loss scale first (:77-84):
 *   m = b1*m + (1-b1)*g; v = b2*v + (1-b2)*g^2;
 *   p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps), t = the global step.
 * variant 1, tiny-cuda-nn style (odie/native/runtime.cu:212-215, documented at
 *   odie/train.py:121-124): a parameter whose gradient is exactly zero is skipped and keeps
 *   its age; otherwise its own counter t_i is incremented and
 *   p -= lr*sqrt(1-b2^t_i)/(1-b1^t_i) * m / (sqrt(v) + eps).
 * ---------------------------------------------------------------------------- */
API void ora_adam(int variant, double* param, const double* grad, double* m, double* v, uint32_t* steps,
                  int64_t n, int64_t step, double lr, double beta1, double beta2, double eps, double scale) {
    /* elementwise: the parallel loop gives the same result as a sequential one */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const double g = grad[i] / scale;
        if (variant == 1 && g == 0.0) continue;
        m[i] = beta1 * m[i] + (1.0 - beta1) * g;
        v[i] = beta2 * v[i] + (1.0 - beta2) * g * g;
        if (variant == 0) {
            const double bc1 = 1.0 - pow(beta1, (double)step), bc2 = 1.0 - pow(beta2, (double)step);
            param[i] -= lr / bc1 * m[i] / (sqrt(v[i]) / sqrt(bc2) + eps);
        } else {
            const uint32_t t = ++steps[i];
            const double rate = lr * sqrt(1.0 - pow(beta2, (double)t)) / (1.0 - pow(beta1, (double)t));
            param[i] -= rate * m[i] / (sqrt(v[i]) + eps);
        }
    }
}
