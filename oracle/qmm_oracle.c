/*
 * qmm_oracle.c -- CPU restatement of VeloMind's quantize/pack routines and
 * its CPU QuantizedMatMul kernels.  TEST INFRASTRUCTURE ONLY (checker and
 * timed CPU baseline); see qmm_oracle.h for the pinning of each function.
 *
 * Build: oracle/build_oracle.py compiles this file with gcc -O2
 * -ffp-contract=off, so that scalar loops use a separate multiply and add
 * exactly like the reference build (no -march, hence no FMA contraction).
 */
#include "qmm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ---- helpers ----------------------------------------------------------- */

/* Two's-complement value of a 4-bit field (quant.cpp:17-22). */
static inline int nib_to_int(unsigned v) {
    v &= 0xFu;
    return (v & 0x8u) ? (int)v - 16 : (int)v;
}

/* std::clamp(v, lo, hi) for finite v (quant.cpp:100, :161). */
static inline float clampf(float v, float lo, float hi) {
    if (v < lo) return lo;
    if (hi < v) return hi;
    return v;
}

/* Largest |x| over rows [r0, r1) of column c of a row-major [rows, cols]
 * matrix; strict '>' keeps the first maximum (quant.cpp:86-92, :147-153). */
static float column_absmax(const float* src, size_t cols, size_t c, size_t r0, size_t r1) {
    float best = 0.0f;
    for (size_t r = r0; r < r1; ++r) {
        float v = fabsf(src[r * cols + c]);
        if (v > best) best = v;
    }
    return best;
}

/* ---- quant.cpp restatement --------------------------------------------- */

void vmo_quantize_int8_per_channel(const float* src, int8_t* dst_q, float* dst_scale,
                                   size_t rows, size_t cols) {
    /* quant.cpp:81-83: silently ignore empty / null requests. */
    if (!src || !dst_q || !dst_scale || rows == 0 || cols == 0) return;
    for (size_t c = 0; c < cols; ++c) {
        const float amax = column_absmax(src, cols, c, 0, rows);
        /* quant.cpp:94-96: correctly rounded division, then a reciprocal
         * that is multiplied (not divided) below. */
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        dst_scale[c] = s;
        for (size_t r = 0; r < rows; ++r) {
            /* quant.cpp:99-101: roundf is half-away-from-zero. */
            const float q = clampf(roundf(src[r * cols + c] * inv), -127.0f, 127.0f);
            dst_q[r * cols + c] = (int8_t)q;
        }
    }
}

void vmo_dequantize_int8_per_channel(const int8_t* src_q, const float* scale, float* dst,
                                     size_t rows, size_t cols) {
    if (!src_q || !scale || !dst || rows == 0 || cols == 0) return;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c)
            dst[r * cols + c] = (float)src_q[r * cols + c] * scale[c];
}

void vmo_quantize_int4_block(const float* src, uint8_t* dst_packed, float* dst_scale,
                             size_t rows, size_t cols, size_t block_size) {
    if (!src || !dst_packed || !dst_scale || rows == 0 || cols == 0 || block_size == 0) return;
    const size_t nblk = (rows + block_size - 1) / block_size;
    /* quant.cpp:140: bytes not written below (odd-K high nibble) stay 0. */
    memset(dst_packed, 0, ((rows + 1) / 2) * cols);
    for (size_t c = 0; c < cols; ++c) {
        for (size_t b = 0; b < nblk; ++b) {
            const size_t r0 = b * block_size;
            const size_t r1 = (r0 + block_size < rows) ? r0 + block_size : rows;
            const float amax = column_absmax(src, cols, c, r0, r1);
            const float s = amax > 0.0f ? amax / 7.0f : 1.0f;   /* quant.cpp:155 */
            const float inv = 1.0f / s;
            dst_scale[b * cols + c] = s;
            /* quant.cpp:159-171: row pairs (r, r+1) of the block share the
             * byte at packed row r/2; the even row is the low nibble. */
            for (size_t r = r0; r < r1; r += 2) {
                const int lo = (int8_t)clampf(roundf(src[r * cols + c] * inv), -8.0f, 7.0f);
                int hi = 0;
                if (r + 1 < r1)
                    hi = (int8_t)clampf(roundf(src[(r + 1) * cols + c] * inv), -8.0f, 7.0f);
                dst_packed[(r / 2) * cols + c] =
                    (uint8_t)(((unsigned)lo & 0xFu) | (((unsigned)hi & 0xFu) << 4));
            }
        }
    }
}

void vmo_dequantize_int4_block(const uint8_t* src_packed, const float* scale, float* dst,
                               size_t rows, size_t cols, size_t block_size) {
    if (!src_packed || !scale || !dst || rows == 0 || cols == 0 || block_size == 0) return;
    const size_t nblk = (rows + block_size - 1) / block_size;
    for (size_t b = 0; b < nblk; ++b) {
        const size_t r0 = b * block_size;
        const size_t r1 = (r0 + block_size < rows) ? r0 + block_size : rows;
        for (size_t r = r0; r < r1; r += 2) {
            for (size_t c = 0; c < cols; ++c) {
                const float s = scale[b * cols + c];
                const unsigned byte = src_packed[(r / 2) * cols + c];
                dst[r * cols + c] = (float)nib_to_int(byte) * s;
                if (r + 1 < r1) dst[(r + 1) * cols + c] = (float)nib_to_int(byte >> 4) * s;
            }
        }
    }
}

void vmo_quant_metrics(const float* original, const float* reconstructed, size_t count,
                       float out[4]) {
    /* quant.cpp:31-33: default metrics {0, 0, 0, 1}. */
    out[0] = 0.0f; out[1] = 0.0f; out[2] = 0.0f; out[3] = 1.0f;
    if (count == 0 || !original || !reconstructed) return;
    float max_diff = 0.0f;
    double sdd = 0.0, soo = 0.0, srr = 0.0, sor = 0.0;
    for (size_t i = 0; i < count; ++i) {
        const double o = original[i], r = reconstructed[i];
        const double d = fabs(o - r);
        if (d > max_diff) max_diff = (float)d;
        sdd += d * d; soo += o * o; srr += r * r; sor += o * r;
    }
    out[0] = max_diff;
    out[1] = (float)sqrt(sdd / (double)count);
    out[2] = sdd > 1e-15 ? (float)(10.0 * log10(soo / sdd)) : 100.0f;
    const double den = sqrt(soo) * sqrt(srr);
    out[3] = den > 1e-15 ? (float)(sor / den) : 1.0f;
}

/* ---- CPU QuantizedMatMul restatement ----------------------------------- */

/* Weight code at logical (row p, column j) as float: INT8 reads the byte
 * directly; INT4 selects the nibble of packed row p/2 by the parity of p
 * (quantized_matmul.cpp:83-85). */
static inline float code_at(const int8_t* b_q, int int4, size_t p, size_t j,
                            size_t b_row_stride, size_t b_col_stride) {
    if (int4) {
        const unsigned byte = (uint8_t)b_q[(p / 2) * b_row_stride + j * b_col_stride];
        return (float)nib_to_int((p & 1u) ? byte >> 4 : byte);
    }
    return (float)b_q[p * b_row_stride + j * b_col_stride];
}

/* Generic scalar loop over float operands; a_at/s_at read activations and
 * scales of any dtype as float and the result is returned through store. */
typedef float (*load_fn)(const void* base, size_t idx);
typedef void (*store_fn)(void* base, size_t idx, float v);

static float load_f32(const void* p, size_t i) { return ((const float*)p)[i]; }
static float load_f16(const void* p, size_t i) { return vmo_f16_to_f32(((const uint16_t*)p)[i]); }
static float load_bf16(const void* p, size_t i) { return vmo_bf16_to_f32(((const uint16_t*)p)[i]); }
static void store_f32(void* p, size_t i, float v) { ((float*)p)[i] = v; }
static void store_f16(void* p, size_t i, float v) { ((uint16_t*)p)[i] = vmo_f32_to_f16(v); }
static void store_bf16(void* p, size_t i, float v) { ((uint16_t*)p)[i] = vmo_f32_to_bf16(v); }

static void qmm_scalar_generic(const void* a, load_fn la, const int8_t* b_q, const void* scale,
                               load_fn ls, void* c, store_fn sc, size_t m, size_t k, size_t n,
                               size_t a_rs, size_t a_cs, size_t b_rs, size_t b_cs,
                               size_t c_rs, size_t c_cs, int quant_type, int block_size) {
    const int int4 = quant_type == VMO_QUANT_INT4;
    /* quantized_matmul.cpp:67: INT4 falls back to 32-row blocks when the
     * attribute is not positive; INT8 with block_size <= 0 is per-channel. */
    size_t bs = 0;
    if (int4) bs = block_size > 0 ? (size_t)block_size : 32;
    else if (block_size > 0) bs = (size_t)block_size;

    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            float total = 0.0f;
            if (bs) {
                /* quantized_matmul.cpp:76-90 / :107-119: per-block partial
                 * sum, then one multiply by the block scale. */
                for (size_t p0 = 0; p0 < k; p0 += bs) {
                    const size_t p1 = (p0 + bs < k) ? p0 + bs : k;
                    const float s = ls(scale, (p0 / bs) * n + j);
                    float part = 0.0f;
                    for (size_t p = p0; p < p1; ++p)
                        part += la(a, i * a_rs + p * a_cs) * code_at(b_q, int4, p, j, b_rs, b_cs);
                    total += part * s;
                }
            } else {
                /* quantized_matmul.cpp:129-137: full-K sum times scale[j]. */
                for (size_t p = 0; p < k; ++p)
                    total += la(a, i * a_rs + p * a_cs) * code_at(b_q, 0, p, j, b_rs, b_cs);
                total = total * ls(scale, j);
            }
            sc(c, i * c_rs + j * c_cs, total);
        }
    }
}

void vmo_qmm_scalar_f32(const float* a, const int8_t* b_q, const float* scale, float* c,
                        size_t m, size_t k, size_t n,
                        size_t a_row_stride, size_t a_col_stride,
                        size_t b_row_stride, size_t b_col_stride,
                        size_t c_row_stride, size_t c_col_stride,
                        int quant_type, int block_size) {
    qmm_scalar_generic(a, load_f32, b_q, scale, load_f32, c, store_f32, m, k, n,
                       a_row_stride, a_col_stride, b_row_stride, b_col_stride,
                       c_row_stride, c_col_stride, quant_type, block_size);
}

static load_fn loader_for(int dtype) {
    return dtype == VMO_F16 ? load_f16 : dtype == VMO_BF16 ? load_bf16 : load_f32;
}
static store_fn storer_for(int dtype) {
    return dtype == VMO_F16 ? store_f16 : dtype == VMO_BF16 ? store_bf16 : store_f32;
}

void vmo_qmm_scalar_mixed(const void* a, int a_dtype, const int8_t* b_q, const void* scale,
                          int scale_dtype, void* c, int c_dtype, size_t m, size_t k, size_t n,
                          int quant_type, int block_size) {
    qmm_scalar_generic(a, loader_for(a_dtype), b_q, scale, loader_for(scale_dtype), c,
                       storer_for(c_dtype), m, k, n, k, 1, n, 1, n, 1, quant_type, block_size);
}

#if defined(__x86_64__)
/* quantized_matmul.cpp:146-188: 64-column panels walked down K; eight
 * int8 codes widened to fp32 and fused-multiply-added per step, then one
 * multiply by the column scale. */
__attribute__((target("avx2,fma")))
static void decode_stream_int8_avx2(const float* a, const int8_t* b_q, const float* scale,
                                    float* c, size_t k, size_t n, size_t b_row_stride) {
    enum { PANEL = 64 };
    for (size_t n0 = 0; n0 < n; n0 += PANEL) {
        const size_t w = (n - n0 < PANEL) ? n - n0 : PANEL;
        float acc[PANEL] __attribute__((aligned(32)));
        for (size_t j = 0; j < PANEL; ++j) acc[j] = 0.0f;
        for (size_t p = 0; p < k; ++p) {
            const __m256 av = _mm256_set1_ps(a[p]);
            const int8_t* row = b_q + p * b_row_stride + n0;
            size_t j = 0;
            for (; j + 8 <= w; j += 8) {
                const __m256 wv = _mm256_cvtepi32_ps(
                    _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(row + j))));
                _mm256_storeu_ps(acc + j, _mm256_fmadd_ps(av, wv, _mm256_loadu_ps(acc + j)));
            }
            /* The reference's scalar tail sits in an avx2,fma function and
             * is contracted to an FMA by the compiler. */
            for (; j < w; ++j) acc[j] = fmaf(a[p], (float)row[j], acc[j]);
        }
        for (size_t j = 0; j < w; ++j) c[n0 + j] = acc[j] * scale[n0 + j];
    }
}
#endif

int vmo_cpu_has_avx2_fma(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

int vmo_qmm_decode_int8(const float* a, const int8_t* b_q, const float* scale, float* c,
                        size_t k, size_t n, size_t a_stride, size_t b_row_stride,
                        size_t b_col_stride, int quant_type, int block_size) {
    /* quantized_matmul.cpp:203-208: per-channel INT8 with unit strides only. */
    if (quant_type != VMO_QUANT_INT8 || block_size != 0) return 0;
    if (a_stride != 1 || b_col_stride != 1) return 0;
#if defined(__x86_64__)
    if (vmo_cpu_has_avx2_fma()) {
        decode_stream_int8_avx2(a, b_q, scale, c, k, n, b_row_stride);
        return 1;
    }
#endif
    /* quantized_matmul.cpp:218-233: portable panel loop (mul + add). */
    for (size_t n0 = 0; n0 < n; n0 += 64) {
        const size_t w = (n - n0 < 64) ? n - n0 : 64;
        float acc[64];
        for (size_t j = 0; j < w; ++j) acc[j] = 0.0f;
        for (size_t p = 0; p < k; ++p)
            for (size_t j = 0; j < w; ++j)
                acc[j] += a[p] * (float)b_q[p * b_row_stride + n0 + j];
        for (size_t j = 0; j < w; ++j) c[n0 + j] = acc[j] * scale[n0 + j];
    }
    return 1;
}

/* The scalar reference's arithmetic (quantized_matmul.cpp:48-141) for
 * contiguous fp32 operands, in row-major order: for each row of A (and each
 * block), the K loop runs outside the column loop, so every output element
 * sees exactly the sequence of fp32 operations of qmm_scalar_generic (a
 * block's products added in K order, times the block scale, added to the
 * element's total; per-channel INT8: products added in K order, then times
 * the column scale), with no contraction (-ffp-contract=off), while the
 * codes are read a row at a time and the column loop vectorizes.  Pinned
 * bit for bit against vmo_qmm_scalar_f32 (tests/test_oracle_qmm.py). */
__attribute__((optimize("O3")))
static void qmm_rows_f32(const float* a, const int8_t* b_q, const float* scale, float* c, size_t m, size_t k,
                         size_t n, int quant_type, int block_size) {
    const int int4 = quant_type == VMO_QUANT_INT4;
    size_t bs = 0;
    if (int4) bs = block_size > 0 ? (size_t)block_size : 32;
    else if (block_size > 0) bs = (size_t)block_size;
    float* code = (float*)malloc((n ? n : 1) * 3 * sizeof(float));
    if (!code) abort();
    float* part = code + n;
    float* total = part + n;
    for (size_t i = 0; i < m; ++i) {
        const float* ai = a + i * k;
        for (size_t j = 0; j < n; ++j) total[j] = 0.0f;
        const size_t step = bs ? bs : (k ? k : 1);
        for (size_t p0 = 0; p0 < k; p0 += step) {
            const size_t p1 = (p0 + step < k) ? p0 + step : k;
            float* acc = bs ? part : total;
            if (bs)
                for (size_t j = 0; j < n; ++j) part[j] = 0.0f;
            for (size_t p = p0; p < p1; ++p) {
                if (int4) {
                    const uint8_t* row = (const uint8_t*)b_q + (p / 2) * n;
                    if (p & 1u)
                        for (size_t j = 0; j < n; ++j) code[j] = (float)nib_to_int(row[j] >> 4);
                    else
                        for (size_t j = 0; j < n; ++j) code[j] = (float)nib_to_int(row[j]);
                } else {
                    const int8_t* row = b_q + p * n;
                    for (size_t j = 0; j < n; ++j) code[j] = (float)row[j];
                }
                const float av = ai[p];
                for (size_t j = 0; j < n; ++j) acc[j] += av * code[j];
            }
            if (bs) {
                const float* s = scale + (p0 / bs) * n;
                for (size_t j = 0; j < n; ++j) total[j] += part[j] * s[j];
            }
        }
        if (!bs)
            for (size_t j = 0; j < n; ++j) total[j] = total[j] * scale[j];
        for (size_t j = 0; j < n; ++j) c[i * n + j] = total[j];
    }
    free(code);
}

void vmo_qmm_2d_f32(const float* a, const int8_t* b_q, const float* scale, float* c,
                    size_t m, size_t k, size_t n, int quant_type, int block_size) {
    /* quantized_matmul.cpp:254-266: M=1 tries the streaming decode first. */
    if (m == 1 && vmo_qmm_decode_int8(a, b_q, scale, c, k, n, 1, n, 1, quant_type, block_size))
        return;
    qmm_rows_f32(a, b_q, scale, c, m, k, n, quant_type, block_size);
}

/* ---- dtype.h restatement: half-precision conversions -------------------- */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float vmo_f16_to_f32(uint16_t h) {
    /* dtype.h:21-51 */
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return bits_to_f32(sign);
        int exp = -14;                      /* subnormal: normalise mantissa */
        while (!(m & 0x400u)) { m <<= 1; --exp; }
        return bits_to_f32(sign | ((uint32_t)(exp + 127) << 23) | ((m & 0x3FFu) << 13));
    }
    if (e == 0x1F) return bits_to_f32(sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u));
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t vmo_f32_to_f16(float f) {
    /* dtype.h:53-89: round to nearest even, overflow to infinity, quiet NaN. */
    const uint32_t x = f32_to_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t raw_e = (x >> 23) & 0xFFu;
    const uint32_t mant = x & 0x7FFFFFu;
    if (raw_e == 0xFF) return (uint16_t)(sign | (mant ? 0x7E00u : 0x7C00u));
    int e = (int)raw_e - 112;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = (mant | 0x800000u) >> (1 - e);
        if ((m & 0x1000u) && (m & 0x2FFFu)) m += 0x2000u;
        return (uint16_t)(sign | (m >> 13));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t m = mant;
    if ((m & 0x1000u) && (m & 0x2FFFu)) {
        m += 0x2000u;
        if (m & 0x800000u) {
            m = 0;
            if (++e >= 31) return (uint16_t)(sign | 0x7C00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
}

float vmo_bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

uint16_t vmo_f32_to_bf16(float f) {
    /* dtype.h:97-107: NaN keeps its payload and is made quiet; everything
     * else rounds to nearest even on the upper half. */
    uint32_t x = f32_to_bits(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu)) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

