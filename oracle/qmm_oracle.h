/*
 * qmm_oracle.h -- CPU restatement of VeloMind's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * product path and the timed CPU baseline in bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (velo-mind_amd) never links or calls it.
 *
 * Every function restates one reference function; the citation next to it
 * is the file:line under the reference tree (src/quant.cpp,
 * src/cpu/ops/quantized_matmul.cpp, include/velomind/dtype.h).
 *
 * Pinning (what checks each function, see tests/test_oracle_*.py):
 *   vmo_quantize_int8_per_channel  KAT (0.5-tie rounds away), invariants,
 *                                  reference roundtrip-metric thresholds
 *                                  on the reference test's own inputs.
 *   vmo_quantize_int4_block        KATs (tie, nibble order, odd-K tail),
 *                                  invariants, roundtrip thresholds.
 *   vmo_dequantize_*               exact code*scale identity, error bound.
 *   vmo_quant_metrics              closed forms (identical input, scaled
 *                                  input, orthogonal input).
 *   vmo_qmm_2d_f32 (INT8)          reference test: dequant + fp32 MatMul
 *                                  < 1e-4 on the reference test inputs.
 *   vmo_qmm_2d_f32 (INT4 / block)  closed forms with per-block scales
 *                                  (no reference test executes INT4).
 *   vmo_qmm_decode_int8            reference test: stream vs scalar < 1e-4.
 *   fp16/bf16 converters           exhaustive / special-value checks
 *                                  against numpy's IEEE conversions.
 */
#ifndef VELOMIND_QMM_ORACLE_H
#define VELOMIND_QMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantType values mirror include/velomind/quant.h:18-22. */
enum { VMO_QUANT_NONE = 0, VMO_QUANT_INT8 = 1, VMO_QUANT_INT4 = 2 };
/* DataType values mirror include/velomind/types.h:20-29. */
enum { VMO_F32 = 0, VMO_I32 = 1, VMO_I8 = 2, VMO_BOOL = 3, VMO_F16 = 4, VMO_BF16 = 5 };

/* src/quant.cpp:74-104 */
void vmo_quantize_int8_per_channel(const float* src, int8_t* dst_q, float* dst_scale,
                                   size_t rows, size_t cols);
/* src/quant.cpp:106-123 */
void vmo_dequantize_int8_per_channel(const int8_t* src_q, const float* scale, float* dst,
                                     size_t rows, size_t cols);
/* src/quant.cpp:125-175 */
void vmo_quantize_int4_block(const float* src, uint8_t* dst_packed, float* dst_scale,
                             size_t rows, size_t cols, size_t block_size);
/* src/quant.cpp:177-209 */
void vmo_dequantize_int4_block(const uint8_t* src_packed, const float* scale, float* dst,
                               size_t rows, size_t cols, size_t block_size);
/* src/quant.cpp:26-72; out = {max_diff, rmse, snr_db, cosine_sim} */
void vmo_quant_metrics(const float* original, const float* reconstructed, size_t count,
                       float out[4]);

/* src/cpu/ops/quantized_matmul.cpp:48-141 (fp32 instantiation). */
void vmo_qmm_scalar_f32(const float* a, const int8_t* b_q, const float* scale, float* c,
                        size_t m, size_t k, size_t n,
                        size_t a_row_stride, size_t a_col_stride,
                        size_t b_row_stride, size_t b_col_stride,
                        size_t c_row_stride, size_t c_col_stride,
                        int quant_type, int block_size);

/* src/cpu/ops/quantized_matmul.cpp:190-235 (+ AVX2 body :146-188).
 * Returns 1 when the streaming path applies, 0 otherwise. */
int vmo_qmm_decode_int8(const float* a, const int8_t* b_q, const float* scale, float* c,
                        size_t k, size_t n, size_t a_stride, size_t b_row_stride,
                        size_t b_col_stride, int quant_type, int block_size);

/* src/cpu/ops/quantized_matmul.cpp:237-267, contiguous operands:
 * a [m,k], b_q [k,n] or packed [(k+1)/2,n], c [m,n]. */
void vmo_qmm_2d_f32(const float* a, const int8_t* b_q, const float* scale, float* c,
                    size_t m, size_t k, size_t n, int quant_type, int block_size);

/* Mixed-precision instantiations (quantized_matmul.cpp:363-367): the
 * scalar reference with TAct/TScale/TOut in {f32, f16, bf16}; values are
 * raw 16-bit patterns for the half types, converted with the reference's
 * round-to-nearest-even helpers (dtype.h:21-107). */
void vmo_qmm_scalar_mixed(const void* a, int a_dtype, const int8_t* b_q, const void* scale,
                          int scale_dtype, void* c, int c_dtype, size_t m, size_t k, size_t n,
                          int quant_type, int block_size);

/* include/velomind/dtype.h:21-107 */
float    vmo_f16_to_f32(uint16_t h);
uint16_t vmo_f32_to_f16(float f);
float    vmo_bf16_to_f32(uint16_t b);
uint16_t vmo_f32_to_bf16(float f);


/* 1 when the running CPU has AVX2+FMA (quantized_matmul.cpp:36-43). */
int vmo_cpu_has_avx2_fma(void);

#ifdef __cplusplus
}
#endif

#endif
