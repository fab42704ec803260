// Decode-shaped quantized matmul with fused extras: C = addend + A @ W,
// RMSNorm applied to A while it is staged, or A formed as the SwiGLU product
// of a gate and an up matrix while it is staged.  The same kernel as the
// plain launches (qmm_gemv_impl.h) with the extras compiled in; kept in its
// own translation unit so the plain kernels carry none of their code.
#include "qmm_gemv_impl.h"

namespace vmhip {

int gemv_qmm_fx_f32(const float* a, const uint8_t* const* wq, const float* const* scale, float* const* c,
                    const int* n, int count, int m, int k, int quant_type, int block_size, hipStream_t stream,
                    const float* addend, const float* norm_w, float norm_eps, const float* a_up) {
    if (count < 1 || count > kMaxMembers) return VM_HIP_EUNSUPPORTED;
    if (addend && count != 1) return VM_HIP_EUNSUPPORTED;  // the addend is [m, n] of one matrix
    if (norm_w && a_up) return VM_HIP_EUNSUPPORTED;
    Member members[kMaxMembers];
    for (int g = 0; g < count; ++g) members[g] = Member{wq[g], scale[g], c[g], n[g]};
    return gemv_group_f32<true>(a, members, count, m, k, quant_type, block_size,
                                GemvExtras{addend, norm_w, norm_eps, a_up}, stream);
}

}  // namespace vmhip
