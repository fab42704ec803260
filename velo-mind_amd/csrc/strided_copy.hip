// Copies between strided layouts of one logical tensor (gather into a
// contiguous buffer, or scatter out of one), for operators whose HIP kernels
// take contiguous operands while their reference honours strides.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kT = 256;

struct StridedLayout {
    int64_t shape[VM_HIP_COPY_MAX_RANK];
    int64_t src[VM_HIP_COPY_MAX_RANK];   // element strides
    int64_t dst[VM_HIP_COPY_MAX_RANK];
    int rank;
};

// One element per thread (grid-stride): its row-major index over `shape`
// gives the coordinates, each layout's strides the two offsets.
template <typename T>
__global__ __launch_bounds__(kT) void copy_strided_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                          const StridedLayout L, int64_t total) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kT + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * kT) {
        int64_t rem = i, so = 0, dof = 0;
        for (int d = L.rank - 1; d >= 0; --d) {
            const int64_t c = rem % L.shape[d];
            rem /= L.shape[d];
            so += c * L.src[d];
            dof += c * L.dst[d];
        }
        dst[dof] = src[so];
    }
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

extern "C" int vm_hip_copy_strided(void* dst, const int64_t* dst_strides, const void* src, const int64_t* src_strides,
                                   const int64_t* shape, int rank, int elem_bytes, void* stream) {
    clear_error();
    if (rank < 1 || rank > VM_HIP_COPY_MAX_RANK || !shape || !dst_strides || !src_strides)
        return fail_inval("copy_strided: rank must be 1..8 with shape and strides");
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) return fail_inval("copy_strided: element size 1, 2 or 4");
    StridedLayout L{};
    L.rank = rank;
    int64_t total = 1;
    for (int d = 0; d < rank; ++d) {
        if (shape[d] < 0) return fail_inval("copy_strided: negative dimension");
        if (src_strides[d] < 0 || dst_strides[d] < 0) return fail_inval("copy_strided: negative stride");
        L.shape[d] = shape[d];
        L.src[d] = src_strides[d];
        L.dst[d] = dst_strides[d];
        if (shape[d] > 0 && total > INT64_MAX / shape[d]) return fail_inval("copy_strided: element count overflow");
        total *= shape[d];
    }
    if (total == 0) return 0;
    if (!dst || !src) return fail_inval("copy_strided: null pointer");
    const int64_t blocks = (total + kT - 1) / kT;
    const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (elem_bytes == 1)
        hipLaunchKernelGGL(copy_strided_kernel<uint8_t>, grid, dim3(kT), 0, s, static_cast<const uint8_t*>(src),
                           static_cast<uint8_t*>(dst), L, total);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(copy_strided_kernel<uint16_t>, grid, dim3(kT), 0, s, static_cast<const uint16_t*>(src),
                           static_cast<uint16_t*>(dst), L, total);
    else
        hipLaunchKernelGGL(copy_strided_kernel<uint32_t>, grid, dim3(kT), 0, s, static_cast<const uint32_t*>(src),
                           static_cast<uint32_t*>(dst), L, total);
    return check_launch("copy_strided", s);
}
