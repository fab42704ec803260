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

// Agent-scope relaxed accesses: coherent across the XCDs' L2s (sc1), used
// for split-K partials that another workgroup reads after a ticket.
__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K ticket hand-off, ordered by the memory model rather than by
// hardware write-through alone.  Every thread of the workgroup stores its
// partials, then __syncthreads() makes those stores happen-before thread
// 0's ticket, an agent-scope release RMW.  The RMWs on one counter form a
// release sequence, so the thread that draws the last ticket and then
// issues an agent-scope acquire fence synchronizes with every earlier
// workgroup; its __syncthreads() passes that on to the rest of its
// workgroup before they load the partials.  Only the last arriver pays for
// the acquire.  On gfx950 the release is a buffer_wbl2 sc1 + vmcnt wait
// before the atomic, the acquire a buffer_inv sc1.
__device__ __forceinline__ unsigned ticket_release(unsigned* counter) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void ticket_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

// Thread 0's ticket with the acquire taken when it is the last of `count`.
__device__ __forceinline__ unsigned ticket_take(unsigned* counter, unsigned count) {
    const unsigned t = ticket_release(counter);
    if (t == count - 1u) ticket_acquire();
    return t;
}

}  // namespace vmhip
