/*
 * vm_llama.h -- C ABI of the LLaMA inference layer of libvelomind.so
 * (velo-mind_amd/core/include/velomind/llama/llama_hip.h), for callers that
 * bind C (ctypes, cgo, JNI) rather than the C++ classes.
 *
 * It mirrors the reference's LlamaEngine surface
 * (examples/common/llama/llama_engine.h:57-113): weights are loaded once,
 * prefill() runs a prompt and returns the last logits, forward_step() runs
 * one token at a position, generate() decodes greedily.  Two engines sit
 * behind it over the same weights:
 *   VM_LLAMA_ENGINE_GRAPH     the reference engine's loop: a Graph built
 *                             with build_forward_graph_{prefill,decode} on
 *                             DeviceType::HIP for every call
 *                             (llama_engine.cpp:333-455)
 *   VM_LLAMA_ENGINE_RESIDENT  the resident HIP decoder (fused weights,
 *                             in-place KV cache, HIP-graph decode steps);
 *                             no counterpart in the reference
 *
 * Weights are fp32 in the graph's [in, out] layout (HF [out, in] weights
 * transposed, q_proj pre-multiplied by 1/sqrt(head_dim), as the reference
 * loaders do: examples/tinyllama/model_loader.cpp:65-202).  Every function
 * returns 0 on success or -1 with the message in vm_llama_last_error().
 */
#ifndef VM_LLAMA_H
#define VM_LLAMA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* examples/common/llama/llama_config.h:7-24 */
typedef struct vm_llama_config {
    int64_t vocab_size;
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t num_layers;
    int64_t num_heads;
    int64_t num_kv_heads; /* 0 = num_heads */
    float rms_norm_eps;
    float rope_theta;
} vm_llama_config;

/* Weight kinds (LlamaWeight) and their shapes. */
#define VM_LLAMA_W_EMBED      0  /* [vocab, hidden]                  */
#define VM_LLAMA_W_FINAL_NORM 1  /* [hidden]                         */
#define VM_LLAMA_W_LM_HEAD    2  /* [hidden, vocab]                  */
#define VM_LLAMA_W_ATTN_NORM  3  /* per layer [hidden]               */
#define VM_LLAMA_W_FFN_NORM   4  /* per layer [hidden]               */
#define VM_LLAMA_W_Q          5  /* per layer [hidden, heads*D]      */
#define VM_LLAMA_W_K          6  /* per layer [hidden, kv_heads*D]   */
#define VM_LLAMA_W_V          7  /* per layer [hidden, kv_heads*D]   */
#define VM_LLAMA_W_O          8  /* per layer [hidden, hidden]       */
#define VM_LLAMA_W_GATE       9  /* per layer [hidden, intermediate] */
#define VM_LLAMA_W_UP        10  /* per layer [hidden, intermediate] */
#define VM_LLAMA_W_DOWN      11  /* per layer [intermediate, hidden] */

#define VM_LLAMA_ENGINE_GRAPH    0
#define VM_LLAMA_ENGINE_RESIDENT 1

typedef struct vm_llama_weights vm_llama_weights;
typedef struct vm_llama_session vm_llama_session;

const char* vm_llama_last_error(void);

/* fp32 weights resident on the GPU. */
int vm_llama_weights_create(const vm_llama_config* cfg, vm_llama_weights** out);
int vm_llama_weights_set(vm_llama_weights* w, int kind, int64_t layer, const float* host, int64_t numel);
/* Linears and embedding ~ N(0, stddev^2), norms ~ N(1, stddev^2), on the GPU. */
int vm_llama_weights_fill_synthetic(vm_llama_weights* w, uint64_t seed, float stddev);
/* Tied embeddings: lm_head := embedding^T on the GPU (the reference loaders'
 * fallback when tie_word_embeddings is set, model_loader.cpp:74-144). */
int vm_llama_weights_tie_lm_head(vm_llama_weights* w);
void vm_llama_weights_destroy(vm_llama_weights* w);

/* quant_type: 0 none (graph engine only), 1 INT8 per column, 2 INT4 with
 * blocks of block_size (0 = 32).  fused_attention selects FusedAttention
 * over MatMul/Softmax in the graph engine.  max_seq bounds prompt plus
 * generated tokens for the resident engine. */
int vm_llama_session_create(const vm_llama_weights* w, int engine, int quant_type, int block_size,
                            int fused_attention, int64_t max_seq, vm_llama_session** out);
void vm_llama_session_destroy(vm_llama_session* s);

/* logits_out: vocab floats (the last position's). */
int vm_llama_prefill(vm_llama_session* s, const int32_t* tokens, int64_t n, float* logits_out);
int vm_llama_forward_step(vm_llama_session* s, int32_t token, int64_t pos, float* logits_out);

/* Pre-packed weights (no counterpart in the reference, which packs at bind
 * time): every linear packed on the GPU once (quant.cpp layout, bit-exact),
 * saved to / loaded from a safetensors file of I8 codes and F32 scales
 * (names and metadata: velomind/llama/llama_packed.h).  A resident session
 * created from packed weights does no packing and keeps its own copy of the
 * linears (the packed handle may be destroyed after it is created). */
typedef struct vm_llama_packed vm_llama_packed;
int vm_llama_pack(const vm_llama_weights* w, int quant_type, int block_size, vm_llama_packed** out);
int vm_llama_packed_save(const vm_llama_packed* p, const char* path);
/* The model config recorded in a packed file. */
int vm_llama_packed_config(const char* path, vm_llama_config* out);
int vm_llama_packed_load(const char* path, const vm_llama_config* cfg, vm_llama_packed** out);
void vm_llama_packed_destroy(vm_llama_packed* p);
int vm_llama_session_create_packed(const vm_llama_packed* p, int64_t max_seq, vm_llama_session** out);

/* How the session runs a one-token decode step:
 *   VM_LLAMA_DECODE_GRAPH       a Graph per step (graph engine)
 *   VM_LLAMA_DECODE_PER_OP      resident: one launch per operation
 *   VM_LLAMA_DECODE_SLICES      resident: split-K slices GEMVs and their
 *                               consumers, five launches per layer
 *   VM_LLAMA_DECODE_PERSISTENT  resident: one launch per token
 *                               (vm_hip_decode_step, where the shape
 *                               allows and VELOMIND_DECODE_PERSISTENT=1 at
 *                               session creation) */
#define VM_LLAMA_DECODE_GRAPH      0
#define VM_LLAMA_DECODE_PER_OP     1
#define VM_LLAMA_DECODE_SLICES     2
#define VM_LLAMA_DECODE_PERSISTENT 3
int vm_llama_session_decode_path(const vm_llama_session* s, int* path);

/* Graph engine only: host seconds of the decode steps since the last
 * prefill, summed over steps -- out[0] building each step's Graph, out[1]
 * Graph::build on DeviceType::HIP, out[2] Executable::execute (launches and
 * the final drain), out[3] reading the logits back, out[5] destroying a
 * step's Executable and Graph, out[6] waiting for the helper thread that
 * builds the next step's Graph while a step runs (out[0], out[1] and out[5]
 * are then that thread's time, overlapped with out[2]) -- and out[4] the
 * number of steps.  No counterpart in the reference (its engine times whole
 * steps, llama_engine.cpp:395-455); -1 for a resident session. */
int vm_llama_session_step_timing(const vm_llama_session* s, double* out7);

/* Greedy decoding: prefill, then `steps` decode steps; out_tokens receives
 * steps + 1 tokens (the first from the prompt's logits).  timing (may be
 * NULL) receives {prefill seconds, decode seconds, decode steps timed}:
 * device-event time for the resident engine (decode time covers the
 * HIP-graph replays after the eager first step), host wall time for the
 * graph engine. */
int vm_llama_generate(vm_llama_session* s, const int32_t* prompt, int64_t n, int64_t steps,
                      int use_hip_graph, int32_t* out_tokens, double* timing);

#ifdef __cplusplus
}
#endif

#endif /* VM_LLAMA_H */
