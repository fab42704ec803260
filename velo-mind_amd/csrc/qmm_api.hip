// C ABI entry points of the quantized matmul: argument validation,
// routing between the GEMV (rows_m <= 4), MFMA GEMM (rows_m > 4) and
// generic kernels, and the mixed-precision dtype keys.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "a_split.h"
#include "qmm_kernels.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

// Reference loop order (src/cpu/ops/quantized_matmul.cpp:48-141), one
// thread per output; used only for layouts the fast kernels do not cover.
__global__ __launch_bounds__(256) void generic_qmm_kernel(const float* __restrict__ a,
                                                          const uint8_t* __restrict__ wq,
                                                          const float* __restrict__ scale,
                                                          float* __restrict__ c, int m, int k,
                                                          int n, int int4, int bs) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= n || i >= m) return;
    const float* arow = a + static_cast<int64_t>(i) * k;
    float total = 0.0f;
    if (bs > 0) {
        for (int p0 = 0; p0 < k; p0 += bs) {
            const int p1 = p0 + bs < k ? p0 + bs : k;
            const float s = scale[static_cast<int64_t>(p0 / bs) * n + j];
            float part = 0.0f;
            for (int p = p0; p < p1; ++p) {
                float w;
                if (int4) {
                    const unsigned byte = wq[static_cast<int64_t>(p / 2) * n + j];
                    const unsigned v = (p & 1) ? (byte >> 4) & 0xFu : byte & 0xFu;
                    w = static_cast<float>((v & 8u) ? static_cast<int>(v) - 16 : static_cast<int>(v));
                } else {
                    w = static_cast<float>(static_cast<int8_t>(wq[static_cast<int64_t>(p) * n + j]));
                }
                part = fmaf(arow[p], w, part);
            }
            total = fmaf(part, s, total);
        }
    } else {
        for (int p = 0; p < k; ++p)
            total = fmaf(arow[p], static_cast<float>(static_cast<int8_t>(wq[static_cast<int64_t>(p) * n + j])), total);
        total *= scale[j];
    }
    c[static_cast<int64_t>(i) * n + j] = total;
}

__global__ void zero_kernel(float* __restrict__ c, int64_t count) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) c[i] = 0.0f;
}

// dtype.h:53-89 (fp16) and :97-107 (bf16), bit for bit.
__device__ uint16_t f32_to_f16_ref(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t raw_e = (x >> 23) & 0xFFu;
    const uint32_t mant = x & 0x7FFFFFu;
    if (raw_e == 0xFF) return static_cast<uint16_t>(sign | (mant ? 0x7E00u : 0x7C00u));
    int e = static_cast<int>(raw_e) - 112;
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        uint32_t m = (mant | 0x800000u) >> (1 - e);
        if ((m & 0x1000u) && (m & 0x2FFFu)) m += 0x2000u;
        return static_cast<uint16_t>(sign | (m >> 13));
    }
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7C00u);
    uint32_t m = mant;
    if ((m & 0x1000u) && (m & 0x2FFFu)) {
        m += 0x2000u;
        if (m & 0x800000u) {
            m = 0;
            if (++e >= 31) return static_cast<uint16_t>(sign | 0x7C00u);
        }
    }
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | (m >> 13));
}

__device__ uint16_t f32_to_bf16_ref(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu)) return static_cast<uint16_t>((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return static_cast<uint16_t>(x >> 16);
}

__global__ void f32_to_half_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                   int64_t count, int is_bf16) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    dst[i] = is_bf16 ? f32_to_bf16_ref(src[i]) : f32_to_f16_ref(src[i]);
}

unsigned blocks_for(int64_t count, int threads) {
    return static_cast<unsigned>((count + threads - 1) / threads);
}

}  // namespace

int generic_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                    int n, int quant_type, int block_size, hipStream_t stream) {
    const int int4 = quant_type == VM_HIP_QUANT_INT4;
    const int bs = int4 ? (block_size > 0 ? block_size : 32) : block_size;
    for (int i0 = 0; i0 < m; i0 += 65535) {
        const int rows = m - i0 < 65535 ? m - i0 : 65535;
        hipLaunchKernelGGL(generic_qmm_kernel, dim3(blocks_for(n, 256), rows), dim3(256), 0, stream,
                           a + static_cast<int64_t>(i0) * k, wq, scale, c + static_cast<int64_t>(i0) * n,
                           rows, k, n, int4, bs);
        VM_TRY(check_launch("QuantizedMatMul", stream));
    }
    return 0;
}

}  // namespace vmhip

namespace vmhip {

int validate_qmm(const void* a, const int8_t* wq, const void* scale, const void* c, int64_t m,
                 int64_t k, int64_t n, int quant_type, int block_size) {
    if (quant_type != VM_HIP_QUANT_INT8 && quant_type != VM_HIP_QUANT_INT4)
        return fail_inval("QuantizedMatMul: quant_type must be Int8 or Int4");
    if (m < 0 || k < 0 || n < 0) return fail_inval("QuantizedMatMul: negative shape");
    if (block_size < 0) return fail_inval("QuantizedMatMul: negative block_size");
    if (quant_type == VM_HIP_QUANT_INT4 && block_size > 0 && block_size % 2 != 0)
        return fail_inval("QuantizedMatMul: Int4 block_size must be even");
    if (m > INT32_MAX || k > INT32_MAX || n > INT32_MAX)
        return fail_inval("QuantizedMatMul: dimension exceeds the kernels' 32-bit index range");
    if (m == 0 || n == 0) return 0;
    if (!c) return fail_inval("QuantizedMatMul: null output");
    if (k > 0 && (!a || !wq || !scale)) return fail_inval("QuantizedMatMul: null input");
    return 0;
}

int qmm_f32_impl(const float* a, const int8_t* wq, const float* scale, float* c, int64_t m64,
                 int64_t k64, int64_t n64, int quant_type, int block_size, hipStream_t stream) {
    const int m = static_cast<int>(m64), k = static_cast<int>(k64), n = static_cast<int>(n64);
    if (m == 0 || n == 0) return 0;
    if (k == 0) {
        hipLaunchKernelGGL(zero_kernel, dim3(blocks_for(m64 * n64, 256)), dim3(256), 0, stream, c, m64 * n64);
        return check_launch("QuantizedMatMul", stream);
    }
    const auto* w = reinterpret_cast<const uint8_t*>(wq);
    // INT4 with block_size <= 0 uses 32-row blocks (quantized_matmul.cpp:67).
    if (quant_type == VM_HIP_QUANT_INT4 && block_size <= 0) block_size = 32;
    int rc = VM_HIP_EUNSUPPORTED;
    if (m <= 4) {
        rc = gemv_qmm_f32(a, w, scale, c, m, k, n, quant_type, block_size, stream);
    } else {
        rc = gemm_qmm_f32(a, w, scale, c, m, k, n, quant_type, block_size, stream);
    }
    if (rc == VM_HIP_EUNSUPPORTED) {
        rc = generic_qmm_f32(a, w, scale, c, m, k, n, quant_type, block_size, stream);
    }
    return rc;
}

}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_qmm_f32(const float* a, const int8_t* wq, const float* scale, float* c, int64_t rows_m,
                   int64_t k, int64_t n, int quant_type, int block_size, void* stream) {
    clear_error();
    VM_TRY(validate_qmm(a, wq, scale, c, rows_m, k, n, quant_type, block_size));
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    return qmm_f32_impl(a, wq, scale, c, rows_m, k, n, quant_type, block_size,
                        static_cast<hipStream_t>(stream));
}

int vm_hip_qmm_add_f32(const float* a, const int8_t* wq, const float* scale, const float* addend, float* c,
                       int64_t rows_m, int64_t k, int64_t n, int quant_type, int block_size, void* stream) {
    clear_error();
    VM_TRY(validate_qmm(a, wq, scale, c, rows_m, k, n, quant_type, block_size));
    if (rows_m == 0 || n == 0) return 0;
    if (!addend) return fail_inval("QuantizedMatMul+Add: null addend");
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    auto s = static_cast<hipStream_t>(stream);
    if (rows_m <= 4 && k > 0) {
        const int bs = (quant_type == VM_HIP_QUANT_INT4 && block_size <= 0) ? 32 : block_size;
        const int rc = gemv_qmm_f32(a, reinterpret_cast<const uint8_t*>(wq), scale, c, static_cast<int>(rows_m),
                                    static_cast<int>(k), static_cast<int>(n), quant_type, bs, s, addend);
        if (rc != VM_HIP_EUNSUPPORTED) return rc;
    }
    // Shapes the GEMV does not take: the product, then the addition.
    VM_TRY(qmm_f32_impl(a, wq, scale, c, rows_m, k, n, quant_type, block_size, s));
    return vm_hip_elementwise_f32(VM_HIP_EW_ADD, addend, c, c, rows_m * n, stream);
}

int vm_hip_qmm_swiglu_add_f32(const float* gate, const float* up, const int8_t* wq, const float* scale,
                              const float* addend, float* c, int64_t rows_m, int64_t k, int64_t n, int quant_type,
                              int block_size, void* stream) {
    clear_error();
    VM_TRY(validate_qmm(gate, wq, scale, c, rows_m, k, n, quant_type, block_size));
    if (rows_m == 0 || n == 0) return 0;
    if (k > 0 && !up) return fail_inval("QuantizedMatMul SwiGLU: null up");
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    auto s = static_cast<hipStream_t>(stream);
    if (rows_m <= 4 && k > 0) {
        const int bs = (quant_type == VM_HIP_QUANT_INT4 && block_size <= 0) ? 32 : block_size;
        const int rc = gemv_qmm_f32(gate, reinterpret_cast<const uint8_t*>(wq), scale, c, static_cast<int>(rows_m),
                                    static_cast<int>(k), static_cast<int>(n), quant_type, bs, s, addend, up);
        if (rc != VM_HIP_EUNSUPPORTED) return rc;
    }
    // Shapes the GEMV does not take: the SwiGLU product in the stream's
    // staging buffer, the product, then the addition.
    const float* x = gate;
    if (k > 0) {
        void* staged = nullptr;
        VM_TRY(get_staging(s, static_cast<std::size_t>(rows_m) * static_cast<std::size_t>(k) * sizeof(float), &staged));
        VM_TRY(vm_hip_elementwise_f32(VM_HIP_EW_SILU_MUL, gate, up, static_cast<float*>(staged), rows_m * k, stream));
        x = static_cast<const float*>(staged);
    }
    VM_TRY(qmm_f32_impl(x, wq, scale, c, rows_m, k, n, quant_type, block_size, s));
    return addend ? vm_hip_elementwise_f32(VM_HIP_EW_ADD, addend, c, c, rows_m * n, stream) : 0;
}

int vm_hip_qmm_a_layout(int64_t rows_m, int64_t k, int64_t n, int quant_type, int block_size, int* layout,
                        int64_t* bytes) {
    clear_error();
    if (!layout || !bytes) return fail_inval("vm_hip_qmm_a_layout: null argument");
    VM_TRY(validate_qmm(nullptr, nullptr, nullptr, nullptr, 0, k, n, quant_type, block_size));
    if (rows_m < 0) return fail_inval("vm_hip_qmm_a_layout: negative rows");
    *layout = VM_HIP_A_FP32;
    *bytes = 0;
    if (rows_m > INT32_MAX) return 0;
    // Staged layouts only for rows the staging producers take (the two
    // fp16 parts of a whole row held by one workgroup: k <= 6144).
    if (k > kStageMaxK) return 0;
    const int bs = (quant_type == VM_HIP_QUANT_INT4 && block_size <= 0) ? 32 : block_size;
    GemmPlan plan;
    if (gemm_plan(static_cast<int>(rows_m), static_cast<int>(k), static_cast<int>(n), quant_type, bs, &plan) != 0) {
        clear_error();
        return 0;
    }
    *layout = plan.pieces ? VM_HIP_A_PIECES : VM_HIP_A_ROWS;
    *bytes = static_cast<int64_t>(a_stage_bytes(rows_m, k, plan.pieces));
    return 0;
}

int vm_hip_qmm_staged_f32(const void* a_staged, const int8_t* wq, const float* scale, float* c, int64_t rows_m,
                          int64_t k, int64_t n, int quant_type, int block_size, void* stream) {
    clear_error();
    VM_TRY(validate_qmm(a_staged, wq, scale, c, rows_m, k, n, quant_type, block_size));
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    if (rows_m == 0 || n == 0) return 0;
    const int bs = (quant_type == VM_HIP_QUANT_INT4 && block_size <= 0) ? 32 : block_size;
    GemmPlan plan;
    if (gemm_plan(static_cast<int>(rows_m), static_cast<int>(k), static_cast<int>(n), quant_type, bs, &plan) != 0)
        return fail_inval("vm_hip_qmm_staged_f32: the shape does not take staged A (vm_hip_qmm_a_layout)");
    const auto* ah = static_cast<const _Float16*>(a_staged);
    const auto* row_exp = reinterpret_cast<const int*>(static_cast<const char*>(a_staged) +
                                                       a_stage_half_bytes(rows_m, k, plan.pieces));
    return gemm_qmm_staged_f32(plan, ah, row_exp, reinterpret_cast<const uint8_t*>(wq), scale, c, static_cast<int>(rows_m),
                               static_cast<int>(k), static_cast<int>(n), bs, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Sibling quantized matmuls sharing A, optionally RMS-normalizing A first
// (norm_w non-null): one GEMV launch for rows_m <= 4 where it covers every
// member; otherwise the normalized rows go to the stream's staging buffer
// (the separate RMSNorm kernel) and each member runs on its own.
int qmm_group_impl(const float* a, const float* norm_w, float norm_eps, int64_t rows_m, int64_t k,
                   const vm_hip_qmm_member* members, int count, int quant_type, int block_size, void* stream) {
    if (!members || count < 1 || count > VM_HIP_QMM_GROUP_MAX)
        return fail_inval("QuantizedMatMul group: 1 to VM_HIP_QMM_GROUP_MAX members");
    for (int g = 0; g < count; ++g)
        VM_TRY(validate_qmm(a, members[g].codes, members[g].scales, members[g].c, rows_m, k, members[g].n, quant_type,
                            block_size));
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    auto s = static_cast<hipStream_t>(stream);
    const int bs = (quant_type == VM_HIP_QUANT_INT4 && block_size <= 0) ? 32 : block_size;
    bool empty = rows_m == 0 || k == 0;
    for (int g = 0; g < count; ++g) empty = empty || members[g].n == 0;
    if (!empty && rows_m <= 4) {
        const uint8_t* wq[VM_HIP_QMM_GROUP_MAX];
        const float* sc[VM_HIP_QMM_GROUP_MAX];
        float* c[VM_HIP_QMM_GROUP_MAX];
        int n[VM_HIP_QMM_GROUP_MAX];
        for (int g = 0; g < count; ++g) {
            wq[g] = reinterpret_cast<const uint8_t*>(members[g].codes);
            sc[g] = members[g].scales;
            c[g] = members[g].c;
            n[g] = static_cast<int>(members[g].n);
        }
        const int rc = gemv_qmm_group_f32(a, wq, sc, c, n, count, static_cast<int>(rows_m), static_cast<int>(k),
                                          quant_type, bs, s, norm_w, norm_eps);
        if (rc != VM_HIP_EUNSUPPORTED) return rc;
        clear_error();
    }
    const float* x = a;
    if (norm_w && rows_m > 0 && k > 0) {
        void* staged = nullptr;
        VM_TRY(get_staging(s, static_cast<std::size_t>(rows_m) * static_cast<std::size_t>(k) * sizeof(float), &staged));
        VM_TRY(vm_hip_rmsnorm_f32(a, norm_w, static_cast<float*>(staged), rows_m, k, norm_eps, stream));
        x = static_cast<const float*>(staged);
    }
    // one launch per member (prefill rows, or a member the grouped GEMV
    // does not cover)
    for (int g = 0; g < count; ++g)
        VM_TRY(qmm_f32_impl(x, members[g].codes, members[g].scales, members[g].c, rows_m, k, members[g].n, quant_type,
                            block_size, s));
    return 0;
}

}  // namespace

extern "C" {

int vm_hip_qmm_group_f32(const float* a, int64_t rows_m, int64_t k, const vm_hip_qmm_member* members, int count,
                         int quant_type, int block_size, void* stream) {
    clear_error();
    return qmm_group_impl(a, nullptr, 0.0f, rows_m, k, members, count, quant_type, block_size, stream);
}

int vm_hip_qmm_norm_group_f32(const float* a, const float* norm_w, float eps, int64_t rows_m, int64_t k,
                              const vm_hip_qmm_member* members, int count, int quant_type, int block_size,
                              void* stream) {
    clear_error();
    if (!norm_w && rows_m > 0 && k > 0) return fail_inval("QuantizedMatMul group: null RMSNorm weight");
    return qmm_group_impl(a, norm_w, eps, rows_m, k, members, count, quant_type, block_size, stream);
}

int vm_hip_qmm(const void* a, int a_dtype, const int8_t* wq, const void* scale, int scale_dtype,
               void* c, int c_dtype, int64_t rows_m, int64_t k, int64_t n, int quant_type,
               int block_size, void* stream) {
    clear_error();
    const bool key_ok =
        (a_dtype == VM_HIP_DTYPE_F32 && scale_dtype == VM_HIP_DTYPE_F32 && c_dtype == VM_HIP_DTYPE_F32) ||
        (a_dtype == VM_HIP_DTYPE_F16 && c_dtype == VM_HIP_DTYPE_F16 &&
         (scale_dtype == VM_HIP_DTYPE_F16 || scale_dtype == VM_HIP_DTYPE_F32)) ||
        (a_dtype == VM_HIP_DTYPE_BF16 && c_dtype == VM_HIP_DTYPE_BF16 &&
         (scale_dtype == VM_HIP_DTYPE_BF16 || scale_dtype == VM_HIP_DTYPE_F32));
    if (!key_ok) return fail_inval("QuantizedMatMul: unsupported (activation, scale, output) dtype key");
    VM_TRY(validate_qmm(a, wq, scale, c, rows_m, k, n, quant_type, block_size));
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    auto s = static_cast<hipStream_t>(stream);
    if (a_dtype == VM_HIP_DTYPE_F32)
        return qmm_f32_impl(static_cast<const float*>(a), wq, static_cast<const float*>(scale),
                            static_cast<float*>(c), rows_m, k, n, quant_type, block_size, s);
    if (rows_m == 0 || n == 0) return 0;

    // Stage half operands as fp32: [A | scales | C] in the per-stream buffer.
    const int64_t nblk = quant_type == VM_HIP_QUANT_INT4
                             ? (k + (block_size > 0 ? block_size : 32) - 1) / (block_size > 0 ? block_size : 32)
                             : (block_size > 0 ? (k + block_size - 1) / block_size : 1);
    const int64_t a_elems = rows_m * k;
    const int64_t s_elems = (scale_dtype == VM_HIP_DTYPE_F32) ? 0 : nblk * n;
    const int64_t c_elems = rows_m * n;
    const auto align = [](int64_t e) { return (e + 63) & ~int64_t(63); };
    void* stage = nullptr;
    VM_TRY(get_staging(s, static_cast<std::size_t>(align(a_elems) + align(s_elems) + align(c_elems)) * 4, &stage));
    float* a32 = static_cast<float*>(stage);
    float* s32 = a32 + align(a_elems);
    float* c32 = s32 + align(s_elems);
    VM_TRY(vm_hip_half_to_f32(static_cast<const uint16_t*>(a), a_dtype, a32, a_elems, stream));
    const float* sc = static_cast<const float*>(scale);
    if (s_elems) {
        VM_TRY(vm_hip_half_to_f32(static_cast<const uint16_t*>(scale), scale_dtype, s32, s_elems, stream));
        sc = s32;
    }
    VM_TRY(qmm_f32_impl(a32, wq, sc, c32, rows_m, k, n, quant_type, block_size, s));
    hipLaunchKernelGGL(f32_to_half_kernel, dim3(blocks_for(c_elems, 256)), dim3(256), 0, s, c32,
                       static_cast<uint16_t*>(c), c_elems, c_dtype == VM_HIP_DTYPE_BF16 ? 1 : 0);
    return check_launch("QuantizedMatMul", s);
}

}  // extern "C"
