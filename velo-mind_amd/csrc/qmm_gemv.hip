// Decode-shaped (rows_m <= 4) quantized matmul: the plain GEMV launches and
// the phase-trace reader.  The kernel and its launch configuration are in
// qmm_gemv_impl.h; launches with fused extras go to qmm_gemv_fx.hip.
#include "qmm_gemv_impl.h"

namespace vmhip {

int gemv_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int quant_type, int block_size, hipStream_t stream, const float* addend, const float* a_up) {
    if (addend || a_up)
        return gemv_qmm_fx_f32(a, &wq, &scale, &c, &n, 1, m, k, quant_type, block_size, stream, addend, nullptr,
                               0.0f, a_up);
    const Member one{wq, scale, c, n};
    return gemv_group_f32<false>(a, &one, 1, m, k, quant_type, block_size, GemvExtras{}, stream);
}

int gemv_qmm_group_f32(const float* a, const uint8_t* const* wq, const float* const* scale, float* const* c,
                       const int* n, int count, int m, int k, int quant_type, int block_size, hipStream_t stream,
                       const float* norm_w, float norm_eps) {
    if (norm_w)
        return gemv_qmm_fx_f32(a, wq, scale, c, n, count, m, k, quant_type, block_size, stream, nullptr, norm_w,
                               norm_eps, nullptr);
    if (count < 1 || count > kMaxMembers) return VM_HIP_EUNSUPPORTED;
    Member members[kMaxMembers];
    for (int g = 0; g < count; ++g) members[g] = Member{wq[g], scale[g], c[g], n[g]};
    return gemv_group_f32<false>(a, members, count, m, k, quant_type, block_size, GemvExtras{}, stream);
}

}  // namespace vmhip

using namespace vmhip;

extern "C" int vm_hip_gemv_trace_read(void* host, int64_t bytes) {
    clear_error();
#ifdef VM_GEMV_TRACE
    if (!host || bytes < 0) return fail_inval("vm_hip_gemv_trace_read: bad argument");
    const int64_t all = static_cast<int64_t>(sizeof(g_gemv_trace));
    VM_TRY_HIP(hipDeviceSynchronize(), "gemv_trace: sync");
    VM_TRY_HIP(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_gemv_trace), static_cast<size_t>(std::min(bytes, all))),
               "gemv_trace: copy");
    return 0;
#else
    (void)host;
    (void)bytes;
    set_error("vm_hip_gemv_trace_read: libvmhip was built without VM_GEMV_TRACE (VELOMIND_GEMV_TRACE=1)");
    return VM_HIP_EUNSUPPORTED;
#endif
}
