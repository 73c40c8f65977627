// Shared helpers for the gfx950 kernels and the C-ABI: error reporting, stream
// handles, launch-shape helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <string>

#define ODIE_API extern "C" __attribute__((visibility("default")))

namespace odie {

// Last error of the calling thread; the C-ABI returns -1 and leaves the message here,
// as the reference runtime does (odie/native/runtime.cu:318-331).
std::string& error_slot();
int fail(const std::string& message);
int check_launch(const char* what);
// Library-owned device scratch of at least `bytes`, one buffer per device, grown on demand (at
// least doubling; an outgrown buffer is kept until the process ends, so work already queued or
// captured in a graph keeps a valid address; steady-state calls allocate nothing).  Calls that
// use it must not overlap on one device.  Returns null and sets the error on failure.
void* workspace(size_t bytes, hipStream_t stream);
// Zero `count` floats (or any 4-byte words) with a fill kernel (graph-capturable).
int launch_fill_zero(float* data, int64_t count, hipStream_t stream);

inline hipStream_t as_stream(uint64_t bits) { return reinterpret_cast<hipStream_t>(bits); }

constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin across them
constexpr int kCus = 256; // MI355X: compute units (32 per XCD)

// Map a hardware block id onto a logical id so that consecutive logical ids run on the
// same XCD (and share its L2).  `blocks` must be a multiple of kXcds.
__device__ inline uint32_t xcd_major(uint32_t block, uint32_t blocks) {
    return (block % kXcds) * (blocks / kXcds) + block / kXcds;
}

inline uint32_t round_up(uint32_t value, uint32_t multiple) {
    return (value + multiple - 1) / multiple * multiple;
}

// Materialize an fp32 value before it is converted to fp16.  Without this the compiler
// folds fptrunc(a*b) into one v_fma_mixlo_f16, which rounds the exact product to fp16 once
// instead of rounding it to fp32 first and then to fp16 as the reference's
// __float2half_rn(weight) does (odie/packed_kernels.cu:58).
__device__ inline float keep_fp32(float value) {
    asm volatile("" : "+v"(value));
    return value;
}

// fp16 <-> 16-bit patterns without relying on __half's class layout.
__device__ inline __half bits_to_half(uint16_t bits) { return __ushort_as_half(bits); }

// Maxima of fp16 magnitudes on their bit patterns (|a| <= |b| iff the 15-bit magnitudes compare
// the same way, with Inf and NaN above every finite value), two 16-bit maxima per dword.
typedef uint16_t magnitude2 __attribute__((ext_vector_type(2)));

// {max |feature| of level A, max |feature| of level B} from the fp16 feature pairs of two levels.
__device__ inline uint32_t pair_peak(uint32_t level_a, uint32_t level_b) {
    const magnitude2 x = __builtin_bit_cast(magnitude2, level_a & 0x7fff7fffu);
    const magnitude2 y = __builtin_bit_cast(magnitude2, level_b & 0x7fff7fffu);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_shufflevector(x, y, 0, 2),
                                                                  __builtin_shufflevector(x, y, 1, 3)));
}

// Per-half maximum of two such dwords (v_pk_max_u16).
__device__ inline uint32_t pair_max(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(magnitude2, a),
                                                                  __builtin_bit_cast(magnitude2, b)));
}
__device__ inline uint16_t half_to_bits(__half value) { return __half_as_ushort(value); }

}  // namespace odie
