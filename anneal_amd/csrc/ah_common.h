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

// Arrival ticket of the "last workgroup to arrive folds the partials" patterns (split-K contractions, the
// config-5 strip kernel's loss). Each workgroup stores its partial, passes a workgroup barrier, and then
// one thread takes a ticket; the workgroup that draws the last ticket reads every other partial.
// ticket_take is an acquire-release fetch_add at agent scope: its release orders the workgroup's partial
// stores (made the thread's own by the barrier) before the ticket, and its acquire orders the last
// arriver's reads (its other threads' through the barrier that follows) after every earlier release.
// On gfx950 the release writes back the XCD's L2 (buffer_wbl2 sc1) and the acquire invalidates it
// (buffer_inv sc1).
__device__ __forceinline__ int ticket_take(int *count) {
    return __hip_atomic_fetch_add(count, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
// The same ticket without the L2 write-back and invalidate, for a partial that travels entirely as
// agent-scope atomic stores and loads (which gfx950 performs at the cross-XCD coherence point, not in an
// XCD's L2): the wait for this wave's stores to complete stands in for the release. Used where the
// write-back's cost was measured: the config-5 strip kernel, whose workgroups each finish behind 512
// KiB of dX stores (64 us per launch with ticket_take against 54.5 us with this, MI355X).
__device__ __forceinline__ int ticket_take_atomic_partials(int *count) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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
