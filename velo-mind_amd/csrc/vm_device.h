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

}  // namespace vmhip
