// Device helpers shared by the quantized-matmul kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vmhip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer access (gfx9 descriptor word 3 = 0x00020000): loads at or past
// `num_records` bytes return zeros instead of faulting, so tails need no
// branches.  Offsets are 32-bit: buffers must stay below 2 GiB.
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferFlags);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(offset), 0, 0));
}

__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b32(rsrc, static_cast<int>(offset), 0, 0);
}

// v_permlane16_swap_b32 exchanges the odd 16-lane rows of `a` with the even
// rows of `b`; the sum of the two results holds, in even rows, a's row pair
// sum and, in odd rows, b's.  v_permlane32_swap_b32: the upper 32 lanes of
// `a` trade places with the lower 32 lanes of `b`; the sum holds a's half
// sum in lanes 0..31 and b's in lanes 32..63.  (The results are read through
// memcpy: element access on the builtin's returned pair reads the first
// element twice with this compiler.)
__device__ __forceinline__ float swap_rows_add(float a, float b) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    unsigned q[2];
    __builtin_memcpy(q, &p, sizeof q);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ float swap_halves_add(float a, float b) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    unsigned q[2];
    __builtin_memcpy(q, &p, sizeof q);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Agent-scope relaxed accesses: coherent across the XCDs' L2s (sc1), used
// for split-K partials that another workgroup reads after a ticket.
__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), rsrc,
                                           static_cast<int>(offset), 0, 0);
}

// 16-byte forms of coherent_store / coherent_load: the sc1 cache-policy bit
// (16) on a buffer access is what the compiler emits for an agent-scope
// relaxed atomic store or load on gfx950 (written through to, or read from,
// the memory-side coherence point), for 16 bytes at a time.  Used for
// split-K partial tiles.
constexpr int kPolicySc1 = 16;

__device__ __forceinline__ void coherent_store16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), rsrc,
                                           static_cast<int>(offset), 0, kPolicySc1);
}

__device__ __forceinline__ u32x4 coherent_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(offset), 0,
                                                                          kPolicySc1));
}

// Split-K ticket hand-off.  Each workgroup stores its partials with
// agent-scope relaxed stores (coherent_store), every thread waits for its
// own stores to be acknowledged (publish_partials), the workgroup meets at
// __syncthreads(), and thread 0 draws a ticket with an agent-scope relaxed
// RMW; the workgroup that draws the last ticket reads the partials with
// agent-scope relaxed loads (coherent_load).
//
// The ordering between the partials and the ticket rests on gfx950, not on
// the language memory model (which would need a release RMW and an acquire
// fence, i.e. buffer_wbl2 sc1 and buffer_inv sc1: measured 11.1 -> 14.6 us
// at M = 16, K = 2048, N = 5632 INT8):
//   * a store with sc1 (agent scope) is written through the XCD's L2 to
//     the memory-side coherence point, and vmcnt counts it done only once
//     it is acknowledged from there, so after s_waitcnt vmcnt(0) it is
//     visible to every agent-scope access from any XCD;
//   * agent-scope atomics (the ticket) and sc1 loads are performed at or
//     re-fetched from that coherence point, never served from a stale L2
//     line;
//   * the compiler keeps the stores before the wait: the signal fences
//     around s_waitcnt forbid moving memory operations across it, and
//     __syncthreads() is a workgroup fence that the ticket cannot move above;
//   * the last arriver's loads are issued after the ticket's value arrives
//     (a data dependency through LDS and a barrier), and the hardware issues
//     them in order.
__device__ __forceinline__ void publish_partials() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Thread 0's ticket (after publish_partials() and __syncthreads()).
__device__ __forceinline__ unsigned ticket_take(unsigned* counter, unsigned /*count*/) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The reference LLaMA MLP's activation: Sigmoid(g), then Mul by g, then
// Mul by u (llama_graph.cpp:136), as the elementwise kernels round it.
// Every kernel that computes it in one pass uses this so that they agree
// bit for bit.
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float silu_mul_f32(float g, float u) { return (sigmoid_f32(g) * g) * u; }

}  // namespace vmhip
