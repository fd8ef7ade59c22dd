// ah_common.h — shared device/host helpers for the anneal MI355X (gfx950) backend.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half_t;
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace ah {

// ReLU outputs are stored with a sign-of-zero tag: Max(z, 0) for z < 0 is written as -0.0
// (numerically identical to the reference's +0.0 in every later product and sum), while
// z == ±0 is written as +0.0. The reference's ReLU backward mask Where(z == relu(z), adj, 0)
// (tensor/gradient_ruleset.go:153-161) is therefore recoverable from the stored activation
// alone: mask = !(bits == -0.0). This removes a separate pre-activation buffer.
__device__ __forceinline__ float relu_tag(float z) { return z < 0.0f ? -0.0f : z + 0.0f; }
__device__ __forceinline__ half_t relu_tag(half_t z) {
    return z < (half_t)0.0f ? (half_t)(-0.0f) : (half_t)(z + (half_t)0.0f);
}
__device__ __forceinline__ bool relu_dead(float h) { return __float_as_uint(h) == 0x80000000u; }
__device__ __forceinline__ bool relu_dead(half_t h) {
    return __builtin_bit_cast(uint16_t, h) == (uint16_t)0x8000u;
}

// f16 arithmetic as WGSL evaluates it: exact f32 op then round-to-nearest-even to f16.
__device__ __forceinline__ float q16(float v) { return (float)(half_t)v; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace ah
