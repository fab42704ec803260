/*
 * vm_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul library
 * (libvmhip.so).
 *
 * Plain pointers and sizes only: no C++ or torch types cross this boundary.
 * The C++ VeloMind host layer (velo-mind_amd/core) registers
 * DeviceType::HIP kernels, storage and transfers on top of these entry
 * points, and ctypes/cgo/JNI callers can bind them directly.
 *
 * Conventions
 *   - Every function returns 0 on success.  A positive value is the
 *     hipError_t the runtime reported; a negative value is one of the
 *     VM_HIP_E* codes below.  vm_hip_last_error() returns the message of
 *     the last failure on the calling thread.
 *   - `stream` is a hipStream_t passed as void*; NULL is the device's
 *     default (null) stream.  Compute entry points only enqueue work and
 *     return; transfers named *_h2d / *_d2h are synchronous on return
 *     (the reference's MemoryTransfer contract).
 *   - Matrices use the reference layouts byte for byte (quant.cpp):
 *       INT8  codes  int8  [K, N]          scales f32 [N] (per column)
 *                                          or [ceil(K/B), N] (blockwise)
 *       INT4  codes  uint8 [(K+1)/2, N]    scales f32 [ceil(K/B), N]
 *             row pair (2r, 2r+1) shares byte row r; the even row is the
 *             low nibble; nibbles are two's complement.
 *     Activations A are row-major [M, K]; the output C is row-major [M, N].
 */
#ifndef VM_HIP_H
#define VM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VM_HIP_ABI_VERSION 1

/* Library status codes (negative; positive values are hipError_t). */
#define VM_HIP_OK           0
#define VM_HIP_EINVAL      (-1) /* invalid argument (shape, null pointer, dtype)      */
#define VM_HIP_EUNSUPPORTED (-2) /* valid request that this build does not implement  */
#define VM_HIP_EINJECTED   (-3) /* failure injected via VELOMIND_FAIL_BACKEND        */
#define VM_HIP_ENODEVICE   (-4) /* no gfx950 device visible                          */

/* QuantType values: include/velomind/quant.h:18-22. */
#define VM_HIP_QUANT_INT8 1
#define VM_HIP_QUANT_INT4 2

/* DataType values: include/velomind/types.h:20-29. */
#define VM_HIP_DTYPE_F32  0
#define VM_HIP_DTYPE_F16  4
#define VM_HIP_DTYPE_BF16 5

/* ---- library / device ------------------------------------------------ */

/* ABI version of the loaded library (VM_HIP_ABI_VERSION). */
int vm_hip_abi_version(void);

/* Message of the last failure on this thread ("" if none). */
const char* vm_hip_last_error(void);

/* Number of visible gfx950 devices.  Replaces the reference's
 * DeviceAvailabilityFn for CUDA (src/cuda/storage.cu:79-83). */
int vm_hip_device_count(int* count);

/* hipSetDevice / hipGetDevice. */
int vm_hip_set_device(int device);
int vm_hip_get_device(int* device);

/* Block until all work on the current device has finished. */
int vm_hip_device_synchronize(void);

/* ---- memory ------------------------------------------------------------ */

/* Device allocation; *ptr is NULL for bytes == 0.  Replaces the
 * reference's StorageCreatorFn for CUDA (src/cuda/storage.cu:17-41,
 * src/internal/registry/storage.h:13). */
int vm_hip_malloc(void** ptr, size_t bytes);
int vm_hip_free(void* ptr);

/* Synchronous copies (complete on return).  Replace the reference's
 * MemoryTransfer{copy_h2d, copy_d2h} (src/cuda/storage.cu:43-78,
 * src/internal/registry/memory_transfer.h:11-14). */
int vm_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int vm_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
/* Asynchronous device-to-device copy on `stream`. */
int vm_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);

/* ---- streams and events (the reference's per-thread CudaContext,
 *      src/cuda/cuda_context.h:16-74) -------------------------------- */
int vm_hip_stream_create(void** stream);
int vm_hip_stream_destroy(void* stream);
int vm_hip_stream_synchronize(void* stream);
int vm_hip_event_create(void** event);
int vm_hip_event_destroy(void* event);
int vm_hip_event_record(void* event, void* stream);
int vm_hip_event_synchronize(void* event);
int vm_hip_event_elapsed_ms(float* ms, void* start, void* end);

/* ---- HIP graphs (no counterpart in the reference, whose engine rebuilds
 *      and re-launches its graph every token): capture the launches one
 *      decode step makes on `stream` once and replay them with a single
 *      call.  Capture needs a non-null stream, and every quantized-matmul
 *      shape in the captured region must have run once on that stream
 *      before capture (the split-K workspace cannot grow while capturing).
 *      Eager calls after the capture may grow the stream's workspace; the
 *      graph keeps the buffers it captured, which stay allocated until the
 *      stream is destroyed (destroy graphs before their stream).
 *      The captured kernels reset their own counters, so the graph holds no
 *      memset nodes. ------------------------------------------------- */
int vm_hip_stream_begin_capture(void* stream);
int vm_hip_stream_end_capture(void* stream, void** graph_exec);
int vm_hip_graph_launch(void* graph_exec, void* stream);
int vm_hip_graph_destroy(void* graph_exec);

/* ---- the hot path ------------------------------------------------------ */

/*
 * C[m, n] = sum_k A[m, k] * W[k, n], W dequantized from `wq`/`scale`.
 *
 * Replaces the QuantizedMatMul kernels of the reference's CPU and CUDA
 * backends: src/cpu/ops/quantized_matmul.cpp:237-267 (dispatch) and
 * :48-141 (semantics), src/cuda/ops/quantized_matmul.cu:203-266 (launch).
 *
 *   quant_type  VM_HIP_QUANT_INT8 or VM_HIP_QUANT_INT4
 *   block_size  INT8: 0 = one scale per column, > 0 = blockwise scales
 *               [ceil(k/block_size), n].  INT4: > 0 and even; 0 means 32
 *               (quantized_matmul.cpp:67).
 *   rows_m      rows of A and C; batch dimensions of contiguous A/C fold
 *               into it (quantized_matmul.cu:262).
 *
 * Accumulation is fp32.  rows_m <= 4 runs the HBM-bound GEMV kernels;
 * larger rows_m runs the MFMA GEMM, which carries each row of A as two
 * fp16 parts under a power-of-two row scale (22 significant bits for any
 * finite fp32 A); codes are exact in fp16, per-column scales multiply each
 * fp32 result and blockwise scales each 32-row chunk's fp32 sum, as the
 * reference does (quantized_matmul.cpp:76-90).  k == 0 writes zeros;
 * rows_m == 0 or n == 0 is a no-op.
 */
int vm_hip_qmm_f32(const float* a, const int8_t* wq, const float* scale, float* c,
                   int64_t rows_m, int64_t k, int64_t n, int quant_type, int block_size,
                   void* stream);

/*
 * C = addend + A x W: a QuantizedMatMul followed by the residual Add that
 * consumes it (the reference LLaMA layer's h + o_proj(ctx) and
 * h + down(act), llama_graph.cpp:122, :139), with the Add's one fp32
 * addition applied to each output after the product's last rounding, so C
 * equals vm_hip_qmm_f32 then an elementwise Add bit for bit.  rows_m <= 4:
 * one GEMV launch; otherwise the product and the addition as two launches.
 * addend [rows_m, n] may not alias C's rows being written by another call.
 * No counterpart in the reference (the graph compiler on DeviceType::HIP
 * fuses such pairs).
 */
int vm_hip_qmm_add_f32(const float* a, const int8_t* wq, const float* scale, const float* addend,
                       float* c, int64_t rows_m, int64_t k, int64_t n, int quant_type,
                       int block_size, void* stream);

/*
 * C = addend + SwiGLU(gate, up) x W: the reference LLaMA MLP's
 * Mul(Mul(Sigmoid(gate), gate), up) (llama_graph.cpp:136) as the
 * activations of a QuantizedMatMul, and the residual Add after it
 * (:139); addend may be NULL (no Add).  Each activation is rounded as
 * vm_hip_elementwise_f32's VM_HIP_EW_SILU_MUL rounds it, so C equals the
 * separate launches bit for bit.  rows_m <= 4: one GEMV launch that forms
 * the activations while it stages them; otherwise they go to a per-stream
 * buffer first.  gate and up are [rows_m, k].  No counterpart in the
 * reference (the graph compiler on DeviceType::HIP fuses the chain).
 */
int vm_hip_qmm_swiglu_add_f32(const float* gate, const float* up, const int8_t* wq,
                              const float* scale, const float* addend, float* c, int64_t rows_m,
                              int64_t k, int64_t n, int quant_type, int block_size, void* stream);

/*
 * Sibling quantized matmuls sharing A: for every member g,
 * C_g[rows_m, n_g] = A[rows_m, k] x W_g (codes_g, scales_g), all with the
 * same quant_type and block_size.  No counterpart in the reference, whose
 * graph runs q, k, v (and gate, up) as separate QuantizedMatMul nodes
 * (examples/common/llama/llama_graph.cpp:118, :132-136); the graph compiler
 * on DeviceType::HIP groups such siblings into one call.
 *
 * rows_m <= 4: ONE GEMV launch covers the members' columns side by side
 * (weights read once each, one launch and one split-K tail instead of
 * count); the K split follows the combined width, so each C_g equals the
 * separate vm_hip_qmm_f32 result up to the grouping of its fp32 partial
 * sums.  Larger rows_m (or a member the GEMV does not cover): one
 * vm_hip_qmm_f32 per member.  Each member is checked as vm_hip_qmm_f32
 * checks its arguments.
 */
#define VM_HIP_QMM_GROUP_MAX 4
typedef struct vm_hip_qmm_member {
    const int8_t* codes;
    const float*  scales;
    float*        c;
    int64_t       n;
} vm_hip_qmm_member;
int vm_hip_qmm_group_f32(const float* a, int64_t rows_m, int64_t k, const vm_hip_qmm_member* members,
                         int count, int quant_type, int block_size, void* stream);

/*
 * vm_hip_qmm_group_f32 on RMSNorm(A): each row of A [rows_m, k] is first
 * normalized as RMSNorm over its k values with weight norm_w [k] and
 * epsilon eps (src/cpu/ops/rmsnorm.cpp:17-60; the same arithmetic as
 * vm_hip_rmsnorm_f32, bit for bit), then multiplied by every member.  The
 * reference LLaMA layer's RMSNorm feeding q | k | v and gate | up
 * (llama_graph.cpp:53-56, :125-136); the graph compiler on DeviceType::HIP
 * fuses the pair.  rows_m <= 4: one GEMV launch that normalizes while it
 * stages A; otherwise the normalized rows go to a per-stream buffer first.
 * No counterpart in the reference.
 */
int vm_hip_qmm_norm_group_f32(const float* a, const float* norm_w, float eps, int64_t rows_m,
                              int64_t k, const vm_hip_qmm_member* members, int count,
                              int quant_type, int block_size, void* stream);

/*
 * vm_hip_qmm_f32 without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, kernels and results as vm_hip_qmm_f32.  Its split-K
 * scratch is a static device array of VM_HIP_QMM_NOALLOC_SCRATCH_BYTES per
 * GPU (VM_HIP_QMM_NOALLOC_COUNTER_BYTES of counters, the rest fp32
 * partials), held until the process ends; a shape that needs more returns
 * VM_HIP_EINVAL before launching anything.  All calls on one GPU share that
 * array: calls that overlap on one GPU (other streams, other host threads)
 * race and must be serialized by the caller.
 */
#define VM_HIP_QMM_NOALLOC_SCRATCH_BYTES (16u << 20)
#define VM_HIP_QMM_NOALLOC_COUNTER_BYTES (2u << 20)
int vm_hip_qmm_f32_noalloc(const float* a, const int8_t* wq, const float* scale, float* c,
                           int64_t rows_m, int64_t k, int64_t n, int quant_type, int block_size,
                           void* stream);

/*
 * Same operation for the reference's mixed-precision dtype keys
 * (src/cpu/ops/quantized_matmul.cpp:363-367): (a, scale, c) dtypes in
 * {(F32,F32,F32), (F16,F16,F16), (F16,F32,F16), (BF16,BF16,BF16),
 * (BF16,F32,BF16)}.  Half inputs are widened to fp32, accumulation is fp32
 * and half outputs are rounded to nearest even (include/velomind/dtype.h:
 * 53-107).
 */
int vm_hip_qmm(const void* a, int a_dtype, const int8_t* wq, const void* scale,
               int scale_dtype, void* c, int c_dtype, int64_t rows_m, int64_t k, int64_t n,
               int quant_type, int block_size, void* stream);

/*
 * Per-column symmetric INT8 quantization of a device fp32 matrix
 * w[rows, cols] into codes q[rows, cols] and scales[cols], bit-exact with
 * quantize_weights_int8_per_channel (src/quant.cpp:74-104).
 */
int vm_hip_pack_int8(const float* w, int8_t* q, float* scale, int64_t rows, int64_t cols,
                     void* stream);

/*
 * Blockwise symmetric INT4 quantization of a device fp32 matrix
 * w[rows, cols] into packed[(rows+1)/2, cols] and scales[ceil(rows/block),
 * cols], bit-exact with quantize_weights_int4_block (src/quant.cpp:
 * 125-175).  `block` must be positive and even (odd blocks make the
 * reference's pair packing overwrite bytes across blocks; the graph
 * validation rejects them, src/internal/op_validation.h:180-182).
 */
int vm_hip_pack_int4(const float* w, uint8_t* packed, float* scale, int64_t rows,
                     int64_t cols, int64_t block, void* stream);

/* Inverse maps (src/quant.cpp:106-123 and :177-209). */
int vm_hip_dequant_int8(const int8_t* q, const float* scale, float* w, int64_t rows,
                        int64_t cols, void* stream);
int vm_hip_dequant_int4(const uint8_t* packed, const float* scale, float* w, int64_t rows,
                        int64_t cols, int64_t block, void* stream);

/* Widen a device fp16/bf16 buffer to fp32 (dtype.h:21-51, :91-95); the
 * device half of the reference's convert_dtype (src/dtype.cpp:74-95) used
 * by quantize_storage_int{8,4} for half-precision sources. */
int vm_hip_half_to_f32(const uint16_t* src, int src_dtype, float* dst, int64_t count,
                       void* stream);

/* ---- the rest of the LLaMA graph (fp32, contiguous row-major) ----------
 * Each entry point has the semantics of the reference CPU kernel it cites,
 * so a graph of these operators built on DeviceType::HIP computes what the
 * reference's graph (examples/common/llama/llama_graph.cpp:14-330)
 * computes on the CPU.  Shape validation beyond what the kernel needs to
 * stay in bounds is the graph layer's job (src/internal/op_validation.h). */

/* out[i, :] = table[idx[i], :]; table [vocab, hidden], idx int32 [count].
 * Replaces src/cpu/ops/embedding.cpp:16-33.  Indices outside [0, vocab)
 * produce zero rows; the executor rejects them before launch, as the
 * reference does (src/executable.cpp:54-66). */
int vm_hip_embedding_f32(const float* table, int64_t vocab, int64_t hidden, const int32_t* idx,
                         int64_t count, float* out, void* stream);

/* y[r, :] = x[r, :] / sqrt(mean(x[r, :]^2) + eps) * w, over the last axis
 * of length dim.  Replaces src/cpu/ops/rmsnorm.cpp:17-60. */
int vm_hip_rmsnorm_f32(const float* x, const float* w, float* y, int64_t rows, int64_t dim,
                       float eps, void* stream);

/* Rotary embedding of rows of head_dim values: with h = head_dim / 2 and
 * p = (cos_rows > 1 ? r % cos_rows : 0),
 *   y[r, j]     = x[r, j] * cos[p, j] - x[r, j + h] * sin[p, j]
 *   y[r, j + h] = x[r, j + h] * cos[p, j] + x[r, j] * sin[p, j].
 * Replaces src/cpu/ops/rotary_embedding.cpp:16-45. */
int vm_hip_rope_f32(const float* x, const float* cos_table, const float* sin_table, float* y,
                    int64_t rows, int64_t head_dim, int64_t cos_rows, void* stream);

/* y = x transposed by `perm` (rank 1..6; perm NULL reverses the axes).
 * Replaces src/cpu/ops/transpose.cpp:17-68. */
int vm_hip_transpose_f32(const float* x, float* y, int rank, const int64_t* in_shape,
                         const int* perm, void* stream);

/* Strided slice: y[o] = x[begins + o * steps] per axis, with begins and
 * out_shape already clamped as the reference's signature clamps them.
 * Replaces src/cpu/ops/slice.cpp:21-110. */
int vm_hip_slice_f32(const float* x, float* y, int rank, const int64_t* in_shape,
                     const int64_t* begins, const int64_t* steps, const int64_t* out_shape,
                     void* stream);

/* Concat of two tensors along one axis: for each of `outer` leading
 * indices, a's block of a_block elements then b's of b_block.  Replaces
 * src/cpu/ops/concat.cpp:19-72. */
int vm_hip_concat_f32(const float* a, const float* b, float* y, int64_t outer, int64_t a_block,
                      int64_t b_block, void* stream);

/* Repeat heads: x [outer, kv_heads, inner] -> y [outer, kv_heads * repeats,
 * inner], output head h copying input head h / repeats.  Replaces
 * src/cpu/ops/repeat_kv.cpp:20-62. */
int vm_hip_repeat_kv_f32(const float* x, float* y, int64_t outer, int64_t kv_heads,
                         int64_t repeats, int64_t inner, void* stream);

/* Elementwise y = a + b, a * b or sigmoid(a) over n elements.  Replace
 * src/cpu/ops/add.cpp:16-26, mul.cpp:16-26 and sigmoid.cpp:17-27.
 * VM_HIP_EW_SILU_MUL: y = (sigmoid(a) * a) * b, the reference LLaMA MLP's
 * Mul(Mul(Sigmoid(gate), gate), up) (llama_graph.cpp:136) with the same
 * roundings in the same order, in one pass (the graph compiler's fused
 * step on DeviceType::HIP). */
#define VM_HIP_EW_ADD      0
#define VM_HIP_EW_MUL      1
#define VM_HIP_EW_SIGMOID  2
#define VM_HIP_EW_SILU_MUL 3
int vm_hip_elementwise_f32(int op, const float* a, const float* b, float* y, int64_t n,
                           void* stream);

/* Softmax along one axis of a tensor viewed as [outer, cols, inner].
 * Replaces src/cpu/ops/softmax.cpp:18-48. */
int vm_hip_softmax_f32(const float* x, float* y, int64_t outer, int64_t cols, int64_t inner,
                       void* stream);

/* Batched matrix product C[b] = A[b] B[b], A [batch, m, k], B [batch, k, n],
 * C [batch, m, n], fp32 throughout.  Replaces the fp32 path of
 * src/cpu/ops/matmul.cpp (equal batch dimensions, shape_helpers.h:36-84). */
int vm_hip_matmul_f32(const float* a, const float* b, float* c, int64_t batch, int64_t m,
                      int64_t k, int64_t n, void* stream);

/* Attention with grouped KV heads: q [batch, hq, sq, d], k [batch, hk, sk,
 * d], v [batch, hk, sk, dv] -> o [batch, hq, sq, dv]; query head h reads KV
 * head h / (hq / hk).  scale <= 0 means 1/sqrt(d).  With `causal`, query
 * row i sees keys 0 .. sk - sq + i.  Replaces
 * src/cpu/ops/fused_attention.cpp:22-138. */
int vm_hip_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t batch,
                         int64_t hq, int64_t hk, int64_t sq, int64_t sk, int64_t d, int64_t dv,
                         float scale, int causal, void* stream);

/* One decode position's attention inputs of the reference LLaMA layer in one
 * launch (llama_graph.cpp:79-84, :296-305): q_out = RoPE(q) [hq, 1, d];
 * k_out = Concat(k_past, RoPE(k)) and v_out = Concat(v_past, v) on the
 * sequence axis, k [hkv, 1, d], v [hkv, 1, dv], the pasts [hkv, s_past, .],
 * the outputs [hkv, s_past + 1, .].  cos/sin [1, d / 2] (the position's
 * row).  Bit for bit what vm_hip_rope_f32 and vm_hip_concat_f32 produce.
 * No counterpart in the reference (the graph compiler on DeviceType::HIP
 * fuses these four nodes). */
int vm_hip_rope_append_f32(const float* q, const float* k, const float* v, const float* k_past,
                           const float* v_past, const float* cos_table, const float* sin_table,
                           float* q_out, float* k_out, float* v_out, int64_t hq, int64_t hkv,
                           int64_t s_past, int64_t d, int64_t dv, void* stream);

/* Decode attention of the reference LLaMA graph's unfused chain
 * (llama_graph.cpp:95-107: RepeatKV on K and V, Transpose of K, MatMul,
 * Softmax, MatMul) in one launch: q [hq, 1, d], k [hkv, s, d], v [hkv, s,
 * dv] -> o [hq, 1, dv]; query head h reads kv head h / (hq / hkv).  Bit for
 * bit the chain's result on this library's MatMul and Softmax kernels (the
 * same fp32 operations in the same order), without the repeated K/V, the
 * transposed K and the score rows.  No mask and no scale (the chain has
 * none at one query row).  s + d <= 16384.  The graph compiler on
 * DeviceType::HIP runs matching chains through it. */
int vm_hip_attention_decode_chain_f32(const float* q, const float* k, const float* v, float* o,
                                      int64_t hq, int64_t hkv, int64_t s, int64_t d, int64_t dv,
                                      void* stream);

/* ---- the resident decoder (velomind::examples::llama::HipLlamaDecoder) ---
 * Fused forms of reference graph nodes for a decoder that keeps its KV
 * cache resident ([Hkv, max_seq, D] per layer, appended in place) and reads
 * the current position from device memory (`pos`, one int32), so one
 * decode step is a fixed launch sequence a HIP graph can replay.  The
 * reference has no such entry points: its engine rebuilds the graph every
 * token (examples/common/llama/llama_engine.cpp:395-455); each one below
 * names the graph nodes it computes. */

/* dst[i] ~ N(mean, stddev^2): SplitMix64 counter hash + Box-Muller; the
 * same (seed, n) gives the same values on every call.  Synthetic weights
 * (the reference's FillSyntheticFn, llama_engine.h:56-57). */
int vm_hip_fill_normal_f32(float* dst, int64_t n, uint64_t seed, float mean, float stddev,
                           void* stream);

/* h[r] += delta[r] (skipped when delta is NULL), then
 * hn[r] = rmsnorm(h[r]) * w: the residual Add followed by the next RMSNorm
 * (llama_graph.cpp:121-127, add.cpp, rmsnorm.cpp:17-60). */
int vm_hip_add_rmsnorm_f32(float* h, const float* delta, const float* w, float* hn, int64_t rows,
                           int64_t dim, float eps, void* stream);

/* From the fused projection qkv [rows, (heads + 2 kv_heads) * head_dim]
 * (q heads, then k heads, then v heads) at positions p = *pos + r: RoPE on
 * q into q_out [heads, rows, head_dim] and on k into k_cache at row p, v
 * copied into v_cache at row p; caches [kv_heads, max_seq, head_dim];
 * cos/sin tables [max_seq, head_dim / 2].  Replaces Reshape + Transpose +
 * RotaryEmbedding + Concat of llama_graph.cpp:63-85, :296-300.  Rows with
 * p >= max_seq are not written. */
int vm_hip_rope_kv_append_f32(const float* qkv, int64_t rows, const float* cos_table,
                              const float* sin_table, const int32_t* pos, float* q_out,
                              float* k_cache, float* v_cache, int64_t heads, int64_t kv_heads,
                              int64_t head_dim, int64_t max_seq, void* stream);

/* One query row per head, q [heads, head_dim], at position *pos over keys
 * 0..*pos of the caches; out [heads * head_dim].  Grouped heads are read
 * directly (no RepeatKV); scale <= 0 means 1/sqrt(head_dim).  head_dim 64
 * or 128, at most 16 query heads per KV head, 16-byte aligned operands.  Replaces RepeatKV +
 * FusedAttention (or MatMul/Softmax/MatMul) + Transpose + Reshape of a
 * decode step (llama_graph.cpp:88-118, fused_attention.cpp:22-138). */
int vm_hip_attention_decode_f32(const float* q, const float* k_cache, const float* v_cache,
                                const int32_t* pos, float* out, int64_t heads, int64_t kv_heads,
                                int64_t head_dim, int64_t max_seq, float scale, void* stream);

/* Causal attention of q [heads, rows, head_dim] at positions *pos + i over
 * the caches; out [rows, heads * head_dim] (token-major).  head_dim 64.
 * The prefill counterpart of vm_hip_attention_decode_f32. */
int vm_hip_attention_prefill_f32(const float* q, const float* k_cache, const float* v_cache,
                                 const int32_t* pos, float* out, int64_t rows, int64_t heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t max_seq, float scale,
                                 void* stream);

/* out[r, j] = sigmoid(g) * g * u with g = gate_up[r, j] and
 * u = gate_up[r, inter + j]: Sigmoid + Mul + Mul of the SwiGLU block
 * (llama_graph.cpp:22-28) on the fused gate|up projection. */
int vm_hip_silu_mul_f32(const float* gate_up, float* out, int64_t rows, int64_t inter,
                        void* stream);

/* *token_out = first index of the maximum of x[0..n) (NaN skipped), the
 * reference's sample_argmax (examples/tinyllama/sample.cpp:18-38).  With
 * pos != NULL the token is also written to tokens[*pos + 1] (when that is
 * below max_seq and tokens != NULL) and *pos is incremented. */
int vm_hip_argmax_f32(const float* x, int64_t n, int32_t* token_out, int32_t* pos,
                      int32_t* tokens, int64_t max_seq, void* stream);

/* ---- Split-K decode GEMV with consumer-side reduction -------------------
 * No counterpart in the reference: the resident decoder's projections.
 * One activation row (M = 1) times a packed [k, n] matrix (quant.cpp
 * layout, as vm_hip_qmm_f32); split s of the K range writes its partial
 * sums to out[s * n + j] for s < slices, and the kernel that reads the
 * result adds the slices in order s = 0, 1, ...  The slice count is a
 * function of (k, n, quant_type, block_size, max_slices) only:
 * vm_hip_gemv_slices_count returns it.  INT4 blocks and INT8 blocks must
 * hold a multiple of 8 byte rows (INT8 per-column scales: block_size 0);
 * n % 16 == 0 and k % 4 == 0.  The activation row comes from
 *   VM_HIP_GEMV_SRC_PLAIN   act[k]
 *   VM_HIP_GEMV_SRC_SLICES  the sum of act_slices slices [act_slices][k]
 *   VM_HIP_GEMV_SRC_SWIGLU  silu(g) * u, g and u the sums of act_slices
 *                           slices [act_slices][2k] of a fused gate|up
 *                           projection (g = columns 0..k-1, u = k..2k-1),
 *                           the Sigmoid/Mul/Mul of llama_graph.cpp:22-28 */
#define VM_HIP_GEMV_SRC_PLAIN   0
#define VM_HIP_GEMV_SRC_SLICES  1
#define VM_HIP_GEMV_SRC_SWIGLU  2
/* NORMRES  residual Add + RMSNorm in front of the projection
 *          (llama_graph.cpp:118-136): h = act + sum of `slices` slices of
 *          delta [slices][k] (0 slices: h = act), x = h * norm_w.  The
 *          norm's 1/rms is left to the consumer (the projection is linear):
 *          split s writes sum(h^2) over its K range to ss_out[s]; h_out
 *          (optional) receives h.
 * ATTN     x = decode attention output merged from per-chunk partials
 *          act[(head * chunks + c) * (head_dim + 4)] = {m, l, -, -,
 *          o[head_dim]} (vm_hip_attention_decode_slices_f32), chunks c with
 *          c * chunk <= min(*pos, max_seq - 1), in chunk order.
 * SWIGLU with ss_in != NULL first multiplies g and u by
 *          1 / sqrt(sum(ss_in[0..ss_count)) / ss_dim + eps). */
#define VM_HIP_GEMV_SRC_NORMRES 3
#define VM_HIP_GEMV_SRC_ATTN    4
typedef struct vm_hip_gemv_src {
    int kind;               /* VM_HIP_GEMV_SRC_*                                   */
    int slices;             /* SLICES/SWIGLU: act slices; NORMRES: delta slices     */
    const float* act;       /* x, slices, residual h or attention partials          */
    const float* delta;     /* NORMRES                                             */
    const float* norm_w;    /* NORMRES                                             */
    float* h_out;           /* NORMRES, optional                                   */
    float* ss_out;          /* NORMRES, optional: [slices of this GEMV]             */
    const float* ss_in;     /* SWIGLU, optional                                    */
    int ss_count;
    float ss_dim;
    float eps;
    const int32_t* pos;     /* ATTN                                                */
    int head_dim, chunk, chunks, max_seq;   /* ATTN partial layout                 */
} vm_hip_gemv_src;
int vm_hip_qmm_gemv_slices_src_f32(const vm_hip_gemv_src* src, const int8_t* wq, const float* scale,
                                   float* out, int64_t k, int64_t n, int quant_type, int block_size,
                                   int max_slices, void* stream);
int vm_hip_gemv_slices_count(int64_t k, int64_t n, int quant_type, int block_size, int max_slices,
                             int* slices);
int vm_hip_qmm_gemv_slices_f32(const float* act, int act_kind, int64_t act_slices, const int8_t* wq,
                               const float* scale, float* out, int64_t k, int64_t n, int quant_type,
                               int block_size, int max_slices, void* stream);

/* Consumers of partial slices (no counterpart in the reference; the
 * decode step of the resident decoder):
 *   add_rmsnorm_slices  one row: h += sum of delta_slices slices
 *                       [delta_slices][dim] (in order; 0 = no residual),
 *                       hn = rmsnorm(h) * w; dim % 4 == 0, dim <= 8192,
 *                       16-byte aligned operands
 *   rope_kv_append_slices  vm_hip_rope_kv_append_f32 for one row whose
 *                       projection is qkv_slices slices [qkv_slices][width]
 *   argmax_slices       vm_hip_argmax_f32 of the sum of slices [slices][n]
 *   slices_sum          out[j] = sum over s of in[s * n + j] */
int vm_hip_add_rmsnorm_slices_f32(float* h, const float* delta, int64_t delta_slices, const float* w,
                                  float* hn, int64_t dim, float eps, void* stream);
int vm_hip_rope_kv_append_slices_f32(const float* qkv, int64_t qkv_slices, const float* cos_table,
                                     const float* sin_table, const int32_t* pos, float* q_out,
                                     float* k_cache, float* v_cache, int64_t heads, int64_t kv_heads,
                                     int64_t head_dim, int64_t max_seq, void* stream);
int vm_hip_argmax_slices_f32(const float* x, int64_t slices, int64_t n, int32_t* token_out,
                             int32_t* pos, int32_t* tokens, int64_t max_seq, void* stream);

/* vm_hip_argmax_slices_f32 across workgroups (each scans 1024 elements of
 * every slice; the last to finish reduces the candidates).  `workspace`:
 * at least vm_hip_argmax_workspace_bytes(n) bytes of device memory,
 * 16-byte aligned and zeroed before its first use; every call leaves it
 * zeroed again.  Calls that share a workspace must not overlap.  Falls back
 * to vm_hip_argmax_slices_f32 for unaligned x, n % 4 != 0 or more than 2^29
 * elements.  No counterpart in the reference (greedy sampling on the
 * device for the resident decoder). */
int64_t vm_hip_argmax_workspace_bytes(int64_t n);
int vm_hip_argmax_slices_ws_f32(const float* x, int64_t slices, int64_t n, int32_t* token_out,
                                int32_t* pos, int32_t* tokens, int64_t max_seq, void* workspace,
                                int64_t workspace_bytes, void* stream);
int vm_hip_slices_sum_f32(const float* in, int64_t slices, int64_t n, float* out, void* stream);

/* Decode attention fused with the split-K projection in front of it (no
 * counterpart in the reference; the resident decoder's one-token step):
 * q, the new key and the new value are the sums of qkv_slices slices
 * [qkv_slices][(heads + 2 kv_heads) head_dim] times the RMSNorm scale
 * 1 / sqrt(sum(ss[0..ss_count)) / ss_dim + eps) (ss_count 0: scale 1);
 * q and the key are rotated at p = *pos (tables as
 * vm_hip_rope_kv_append_f32), the key and value are written to the caches
 * at row p, and attention over keys 0..p leaves one record per (head,
 * chunk) in `partials` ([heads][chunks][head_dim + 4] = {m, l, -, -, o}),
 * merged by the consumer (VM_HIP_GEMV_SRC_ATTN).  vm_hip_attention_decode_
 * chunks gives the chunk length and count for (head_dim, max_seq).
 * slices_sum_scaled: slices_sum times the RMSNorm scale of ss. */
int vm_hip_attention_decode_chunks(int64_t head_dim, int64_t max_seq, int* chunk, int* chunks);
int vm_hip_attention_decode_slices_f32(const float* qkv, int64_t qkv_slices, const float* ss,
                                       int64_t ss_count, float ss_dim, float eps,
                                       const float* cos_table, const float* sin_table,
                                       const int32_t* pos, float* k_cache, float* v_cache,
                                       float* partials, int64_t heads, int64_t kv_heads,
                                       int64_t head_dim, int64_t max_seq, float scale, void* stream);
int vm_hip_slices_sum_scaled_f32(const float* in, int64_t slices, int64_t n, const float* ss,
                                 int64_t ss_count, float ss_dim, float eps, float* out, void* stream);

/* Up to four device regions (each below 2 GiB) that a launch reads into the
 * memory-side cache (MI355X Infinity Cache, 256 MB) with extra workgroups,
 * so that the launches after it find those bytes there instead of in HBM.
 * The loaded data is discarded; results do not depend on it. */
#define VM_HIP_PREFETCH_MAX 4
typedef struct vm_hip_prefetch {
    const void* ptr[VM_HIP_PREFETCH_MAX];
    uint64_t bytes[VM_HIP_PREFETCH_MAX];
    int count;
} vm_hip_prefetch;

/* vm_hip_attention_decode_slices_f32 whose launch also prefetches
 * `prefetch` (null or count 0: none) with otherwise idle CUs: the resident
 * decoder passes the next projections' weights. No counterpart in the
 * reference (a decode-step building block). */
int vm_hip_attention_decode_slices_prefetch_f32(const float* qkv, int64_t qkv_slices, const float* ss,
                                                int64_t ss_count, float ss_dim, float eps,
                                                const float* cos_table, const float* sin_table,
                                                const int32_t* pos, float* k_cache, float* v_cache,
                                                float* partials, int64_t heads, int64_t kv_heads,
                                                int64_t head_dim, int64_t max_seq, float scale,
                                                const vm_hip_prefetch* prefetch, void* stream);

/* Asynchronous strided copy of one logical tensor of `rank` (1..8)
 * dimensions `shape` whose elements are elem_bytes (1, 2 or 4) wide: the
 * element at coordinates x goes from src + sum(x[d] * src_strides[d]) to
 * dst + sum(x[d] * dst_strides[d]) (strides in elements, not negative).
 * Gathers a strided view into a contiguous buffer or scatters one back; the
 * caller guarantees both extents lie inside their allocations.  Backs the
 * HIP QuantizedMatMul on strided operands, which the reference's CPU kernel
 * honours (src/cpu/ops/quantized_matmul.cpp:306-315).  Overlapping
 * destinations (a zero stride over a dimension longer than one) are the
 * caller's to avoid. */
#define VM_HIP_COPY_MAX_RANK 8
int vm_hip_copy_strided(void* dst, const int64_t* dst_strides, const void* src, const int64_t* src_strides,
                        const int64_t* shape, int rank, int elem_bytes, void* stream);

/* Asynchronous 2-D device copy: `rows` rows of `width` bytes from src
 * (row pitch spitch) to dst (row pitch dpitch).  Used to assemble fused
 * weight matrices column block by column block. */
int vm_hip_memcpy_2d_d2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                         size_t rows, void* stream);

/* ---- Persistent decode step ---------------------------------------------
 * No counterpart in the reference, whose decode loop launches one graph of
 * ~155 QuantizedMatMul and ~250 other operators per token
 * (examples/common/llama/llama_engine.cpp:395-455, llama_graph.cpp:247-330).
 * One greedy LLaMA decode step (head_dim 64) as ONE cooperative launch: one
 * workgroup per compute unit walks every layer's QKV projection, fused
 * attention with in-place K/V append, output projection, gate|up and down
 * projections, the final norm, lm_head and argmax.  Workgroups exchange
 * data through 64-bit {epoch, value} words that consumers poll, so no
 * device-wide barrier separates the phases, and each workgroup has its
 * next projection's weights in flight while it waits.  (On an MI355X this
 * step is slower than the launch-per-projection step captured in a graph:
 * TinyLlama shapes ~930 us against ~710 us per token; the resident decoder
 * uses it only when VELOMIND_DECODE_PERSISTENT=1.)
 *
 * Weights are the quant.cpp layout (INT8 per column, or INT4 with blocks
 * of 32 * m rows): q|k|v fused as [hidden, (heads + 2 kv_heads) * 64] and
 * gate|up as [hidden, 2 * inter] (packed column by column, so the fused
 * matrix is byte for byte the parts side by side).  Positions: *pos is the
 * position of *token; keys 0 .. *pos are attended (the K/V of *pos is
 * appended first).  With logits_out == NULL the step writes argmax (first
 * maximum, NaN skipped) to *token and tokens[*pos + 1] (when below max_seq)
 * and increments *pos; with logits_out it writes the logits [vocab] and
 * leaves token and pos alone.  `step` must differ between consecutive calls
 * on one workspace (it tags the exchanged words); the workspace must be
 * zeroed once before the first step. */
typedef struct vm_hip_decode_layer {
    const int8_t* qkv_codes;
    const float*  qkv_scales;
    const int8_t* o_codes;
    const float*  o_scales;
    const int8_t* gate_up_codes;
    const float*  gate_up_scales;
    const int8_t* down_codes;
    const float*  down_scales;
    const float*  attn_norm;
    const float*  ffn_norm;
} vm_hip_decode_layer;

typedef struct vm_hip_decode_model {
    int64_t layers, hidden, inter, heads, kv_heads, head_dim, vocab, max_seq;
    int quant_type, block_size;
    float eps;
    const vm_hip_decode_layer* layer;   /* device array of `layers` records */
    const float*  embed;                /* [vocab, hidden]                  */
    const float*  final_norm;           /* [hidden]                         */
    const int8_t* lm_codes;             /* [hidden or (hidden+1)/2, vocab]  */
    const float*  lm_scales;
    const float*  cos_table;            /* [max_seq, head_dim / 2]          */
    const float*  sin_table;
    float*        k_cache;              /* [layers][kv_heads][max_seq][64]   */
    float*        v_cache;
    int32_t*      token;                /* device scalars and the sequence   */
    int32_t*      pos;
    int32_t*      tokens;               /* [max_seq]                         */
} vm_hip_decode_model;

/* Workspace bytes the step needs for this model on the current device
 * (VM_HIP_EUNSUPPORTED when the shape is outside the kernel's limits). */
int vm_hip_decode_workspace_bytes(const vm_hip_decode_model* model, int64_t* bytes);
int vm_hip_decode_step(const vm_hip_decode_model* model, void* workspace, int64_t workspace_bytes,
                       uint32_t step, float* logits_out, void* stream);
/* Nonzero when a step since the last call timed out waiting for another
 * workgroup (results of that step are invalid); clears the flag. */
int vm_hip_decode_status(void* workspace, int* failed, void* stream);
/* Phase timestamps of the last steps (u64, 100 MHz wall clock, laid out
 * [512 workgroups][34 slots][24 events]; see decode_persistent.hip), for
 * profiling: only in a library built with VELOMIND_DECODE_TRACE=1, which
 * compiles them in; VM_HIP_EUNSUPPORTED otherwise. */
int vm_hip_decode_trace_read(void* host, int64_t bytes);
/* Phase timestamps of the last decode GEMV launch (u64, 100 MHz wall clock,
 * laid out [4096 workgroups][8 events], workgroup y * gridDim.x + x; see
 * qmm_gemv.hip), for profiling: only in a library built with
 * VELOMIND_GEMV_TRACE=1; VM_HIP_EUNSUPPORTED otherwise. */
int vm_hip_gemv_trace_read(void* host, int64_t bytes);

/* ---- Prefill GEMM activations staged by their producer (no reference
 * counterpart; the resident decoder's prompts) ---------------------------
 * vm_hip_qmm_f32 with more than 4 rows first stages A in a pre-pass: each
 * row scaled by a power of two and split into two fp16 parts (22
 * significant bits), row-major or in the wide MFMA kernel's operand order.
 * A producer that holds whole rows can write that layout itself instead:
 * vm_hip_qmm_a_layout says which layout (VM_HIP_A_FP32: the shape takes
 * fp32 A only, as every row longer than 6144 does, the producers' limit)
 * and how many bytes the staged buffer needs for a call;
 * vm_hip_add_rmsnorm_stage_f32 (vm_hip_add_rmsnorm_f32's arithmetic) and
 * vm_hip_silu_mul_stage_f32 (vm_hip_silu_mul_f32's) write it, with the fp32
 * rows too when hn_out / out_f32 is given; vm_hip_qmm_staged_f32 runs the
 * GEMM on it, equal bit for bit to vm_hip_qmm_f32 on the fp32 rows. */
#define VM_HIP_A_FP32   0
#define VM_HIP_A_ROWS   1
#define VM_HIP_A_PIECES 2
int vm_hip_qmm_a_layout(int64_t rows_m, int64_t k, int64_t n, int quant_type, int block_size, int* layout,
                        int64_t* bytes);
int vm_hip_qmm_staged_f32(const void* a_staged, const int8_t* wq, const float* scale, float* c, int64_t rows_m,
                          int64_t k, int64_t n, int quant_type, int block_size, void* stream);
int vm_hip_add_rmsnorm_stage_f32(float* h, const float* delta, const float* w, void* a_staged, int layout,
                                 float* hn_out, int64_t rows, int64_t dim, float eps, void* stream);
int vm_hip_silu_mul_stage_f32(const float* gate_up, void* a_staged, int layout, float* out_f32, int64_t rows,
                              int64_t inter, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VM_HIP_H */
