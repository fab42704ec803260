// LLaMA decoder graphs on the VeloMind Graph API: the callers of
// QuantizedMatMul in the reference (examples/common/llama/llama_graph.h,
// llama_config.h, llama_rope_mask.h).  Same names, structures and graph
// shapes, so engine code written against the reference builds the same
// graphs here, and `g.build(DeviceType::HIP)` runs them on the GPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "velomind/graph.h"
#include "velomind/quant.h"
#include "velomind/tensor.h"
#include "velomind/types.h"
#include "velomind/velomind_core_export.h"

namespace velomind::examples::llama {

// examples/common/llama/llama_config.h:7-24
struct Config {
    std::size_t vocab_size = 0;
    std::size_t hidden_size = 0;
    std::size_t intermediate_size = 0;
    std::size_t num_layers = 0;
    std::size_t num_heads = 0;
    std::size_t num_kv_heads = 0;
    std::size_t effective_num_kv_heads() const noexcept { return num_kv_heads > 0 ? num_kv_heads : num_heads; }
    std::size_t head_dim() const noexcept { return num_heads == 0 ? 0 : hidden_size / num_heads; }
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    std::size_t max_seq_len = 2048;
    bool tie_word_embeddings = false;
};

// llama_graph.h:16-34.  Linear weights are [in, out] (K x N); with
// quant_type != None they are packed codes plus the *_scale tensors.
struct ForwardWeights {
    Graph* graph = nullptr;
    Tensor w_embed;
    Tensor w_lm_head;
    std::vector<Tensor> w_attn_norm;
    std::vector<Tensor> wq, wk, wv, wo;
    std::vector<Tensor> w_ffn_norm;
    std::vector<Tensor> w_gate, w_up, w_down;
    Tensor w_final_norm;
    Tensor cos_cache;
    Tensor sin_cache;
    Tensor causal_mask;
    bool use_fused_attention = false;
    QuantType quant_type = QuantType::None;
    int quant_block_size = 0;
    std::vector<Tensor> wq_scale, wk_scale, wv_scale, wo_scale;
    std::vector<Tensor> w_gate_scale, w_up_scale, w_down_scale;
    Tensor w_lm_head_scale;
};

// llama_graph.h:36-39: per-layer K and V, [Hkv, S, D] each.
struct KVCacheHandles {
    std::vector<Tensor> k;
    std::vector<Tensor> v;
};

// Last row of t ([S, ...] -> [1, ...]); t itself when S <= 1 (llama_graph.cpp:141-158).
VELOMIND_CORE_EXPORT auto slice_last_token(Graph& g, Tensor t) -> Tensor;

// Full-sequence prefill (llama_graph.cpp:162-245): tokens int32 [S];
// logits [S, vocab] or [1, vocab] with last_token_logits_only; kv_out, when
// given, receives the rotated K and the V of every layer.
VELOMIND_CORE_EXPORT auto build_forward_graph_prefill(Graph& g, const Config& cfg, Tensor tokens,
                                                      const ForwardWeights& w, KVCacheHandles* kv_out = nullptr,
                                                      bool last_token_logits_only = false) -> Tensor;

// One decode step (llama_graph.cpp:247-333): token int32 [1]; the cache of
// every layer is concatenated with the step's K/V on the sequence axis.
VELOMIND_CORE_EXPORT auto build_forward_graph_decode(Graph& g, const Config& cfg, Tensor token,
                                                     const ForwardWeights& w, const KVCacheHandles& kv_in,
                                                     KVCacheHandles* kv_out = nullptr) -> Tensor;

// Packs every linear and the lm_head of fp_weights (INT8 per column, or INT4
// blocks of block_size, 32 when 0) on `device` and binds the packed tensors
// into g; norms, embedding and positional caches are adopted as they are
// (llama_graph.cpp:336-425).
VELOMIND_CORE_EXPORT auto quantize_forward_weights(Graph& g, const ForwardWeights& fp_weights, QuantType type,
                                                   int block_size = 0, DeviceType device = DeviceType::CPU)
    -> ForwardWeights;

// RoPE tables [seq_len, head_dim/2] for positions pos_offset.. and the
// additive causal mask [num_heads, seq_len, seq_len] (llama_rope_mask.cpp:7-40).
VELOMIND_CORE_EXPORT void compute_rope_cache(std::size_t seq_len, std::size_t head_dim, float base,
                                             std::vector<float>& cos_out, std::vector<float>& sin_out,
                                             std::size_t pos_offset = 0);
VELOMIND_CORE_EXPORT void compute_causal_mask(std::size_t num_heads, std::size_t seq_len, std::vector<float>& mask_out);

}  // namespace velomind::examples::llama
