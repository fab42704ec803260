// Internal launchers shared between the libvmhip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vmhip {

// Decode-shaped GEMV for 1 <= m <= 4 rows (qmm_gemv.hip).  Returns
// VM_HIP_EUNSUPPORTED when the shape/alignment needs another kernel.  A
// non-null `addend` [m, n] is added to each output (addend + A x W, one fp32
// addition after the product's last rounding).  A non-null `a_up` [m, k]
// makes the activations the SwiGLU product silu_mul_f32(a, a_up).
int gemv_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int quant_type, int block_size, hipStream_t stream, const float* addend = nullptr,
                 const float* a_up = nullptr);

// The same GEMV for `count` (<= 4) matrices sharing the activations, in one
// launch (qmm_gemv.hip); VM_HIP_EUNSUPPORTED when a member needs another
// kernel.
// With a non-null norm_w, each row of A is first RMS-normalized (the
// separate RMSNorm kernel's arithmetic, bit for bit): C_g = RMSNorm(A) x W_g.
int gemv_qmm_group_f32(const float* a, const uint8_t* const* wq, const float* const* scale, float* const* c,
                       const int* n, int count, int m, int k, int quant_type, int block_size, hipStream_t stream,
                       const float* norm_w = nullptr, float norm_eps = 0.0f);

// The kernels with fused extras (qmm_gemv_fx.hip), reached through the two
// functions above when an extra is non-null: addend (one matrix only),
// norm_w or a_up (not both).
int gemv_qmm_fx_f32(const float* a, const uint8_t* const* wq, const float* const* scale, float* const* c,
                    const int* n, int count, int m, int k, int quant_type, int block_size, hipStream_t stream,
                    const float* addend, const float* norm_w, float norm_eps, const float* a_up);

// Prefill-shaped MFMA GEMM for m > 4 rows (qmm_gemm.hip).
int gemm_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int quant_type, int block_size, hipStream_t stream);

// How the GEMM takes a shape: kind 0 = INT8 per column, 1 = INT8 blockwise,
// 2 = INT4; `pieces`: A staged in the wide kernel's operand order (else
// row-major, a_split.h; blockwise scales always take the wide kernel).
// VM_HIP_EUNSUPPORTED when the GEMM does not take the shape (rows <= 4,
// K % 32, N % 16, sizes past 32-bit offsets).
struct GemmPlan {
    int kind = 0;
    bool pieces = false;
};
int gemm_plan(int m, int k, int n, int quant_type, int block_size, GemmPlan* plan);
// The GEMM on A staged by its producer (a_split.h layout for the plan).
int gemm_qmm_staged_f32(const GemmPlan& plan, const _Float16* ah, const int* row_exp, const uint8_t* wq,
                        const float* scale, float* c, int m, int k, int n, int block_size, hipStream_t stream);

// Any-shape reference-order kernel used for layouts the fast kernels do
// not cover (odd N, block sizes that are not multiples of 32).
int generic_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                    int n, int quant_type, int block_size, hipStream_t stream);

// Argument checks of vm_hip_qmm_f32 (0 or an error status).
int validate_qmm(const void* a, const int8_t* wq, const void* scale, const void* c, int64_t m, int64_t k,
                 int64_t n, int quant_type, int block_size);

// Routing behind vm_hip_qmm_f32 for validated arguments: GEMV (rows <= 4),
// MFMA GEMM (rows > 4) or the generic kernel.
int qmm_f32_impl(const float* a, const int8_t* wq, const float* scale, float* c, int64_t m, int64_t k,
                 int64_t n, int quant_type, int block_size, hipStream_t stream);

}  // namespace vmhip
