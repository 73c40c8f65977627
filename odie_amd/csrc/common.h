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
// For the entry points whose reference counterparts return the CUDA runtime's error code
// (selection_init, selection_chunk, score_chunk: `return int(cudaGetLastError())`, turned into a
// message by the caller through the runtime's error-string call): the HIP runtime's code instead
// of -1 -- hipErrorInvalidValue for a refused argument, the launch's own code for a failed
// launch -- with the message left in odie_error() as well.
int fail_code(const std::string& message, hipError_t code = hipErrorInvalidValue);
int launch_code(const char* what);
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

// Per-half maximum of two such dwords (v_pk_max_u16).
__device__ inline uint32_t pair_max(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(magnitude2, a),
                                                                  __builtin_bit_cast(magnitude2, b)));
}

// The two fp16 magnitudes of a feature pair (sign bits cleared): per-feature maxima of such
// words, taken with pair_max, are each feature's largest |value|.
__device__ inline uint32_t pair_magnitudes(uint32_t pair) { return pair & 0x7fff7fffu; }

template <int kControl> __device__ inline uint32_t dpp_move(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), kControl, 0xF, 0xF, false));
}

// Per-half maxima of eight dwords over the 32 lanes of a lane group (lanes 0-31 or 32-63; the
// whole wave active).  A reduction tree that halves the dwords a lane holds at every step: the
// half-row mirror (lane i <-> i ^ 7 within 8, which flips bit 2) trades dwords 0-3 against 4-7 by
// bit 2 of the lane, quad swaps by bits 1 and 0, so that lane i holds dword i % 8 over its 8
// lanes; a rotation by 8 within the row of 16 and a swizzle pairing i with i ^ 16 finish.  Lane i
// returns the maximum of dword i % 8 over the group (about 30 instructions where eight separate
// 32-lane reductions take 80).
__device__ inline uint32_t group_max8(const uint32_t d[8], int lane) {
    const bool b2 = (lane >> 2) & 1, b1 = (lane >> 1) & 1, b0 = lane & 1;
    uint32_t x4[4], x2[2];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t keep = b2 ? d[k + 4] : d[k], send = b2 ? d[k] : d[k + 4];
        x4[k] = pair_max(keep, dpp_move<0x141>(send));   // row_half_mirror
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t keep = b1 ? x4[k + 2] : x4[k], send = b1 ? x4[k] : x4[k + 2];
        x2[k] = pair_max(keep, dpp_move<0x4E>(send));    // quad_perm [2, 3, 0, 1]
    }
    const uint32_t keep = b0 ? x2[1] : x2[0], send = b0 ? x2[0] : x2[1];
    uint32_t x = pair_max(keep, dpp_move<0xB1>(send));  // quad_perm [1, 0, 3, 2]
    x = pair_max(x, dpp_move<0x128>(x));                  // row_ror:8
    return pair_max(x, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(x), 0x401F)));  // xor 16
}

// Route launch knobs (route.hip), set through odie_set_tuning's "route_" keys.
int set_route_tuning(const std::string& key, int value);

__device__ inline uint16_t half_to_bits(__half value) { return __half_as_ushort(value); }

}  // namespace odie
