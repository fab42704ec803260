// Prefill-shaped (rows_m > 4) quantized matmul.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "qmm_kernels.h"
#include "vm_internal.h"

namespace vmhip {

int gemm_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int quant_type, int block_size, hipStream_t stream) {
    // Row panels of four through the GEMV kernel.
    for (int i0 = 0; i0 < m; i0 += 4) {
        const int rows = m - i0 < 4 ? m - i0 : 4;
        const int rc = gemv_qmm_f32(a + static_cast<int64_t>(i0) * k, wq, scale,
                                    c + static_cast<int64_t>(i0) * n, rows, k, n, quant_type,
                                    block_size, stream);
        if (rc != 0) return rc;
    }
    return 0;
}

}  // namespace vmhip
