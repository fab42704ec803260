// LLaMA prefill/decode graphs (the reference's examples/common/llama/
// llama_graph.cpp and llama_rope_mask.cpp).  The operator sequence is the
// reference's, node for node, so a graph built here computes the same
// values on any device; the code is organised around one Layer builder.
#include "velomind/llama/llama_graph.h"

#include <cmath>
#include <stdexcept>
#include <string>
#include <utility>

#include "velomind/ops.h"

namespace velomind::examples::llama {

namespace {

struct Dims {
    dim_t heads, kv_heads, head_dim, hidden, group;
};

Dims dims_of(const Config& cfg, const char* who) {
    if (cfg.num_heads == 0 || cfg.hidden_size % cfg.num_heads != 0)
        throw std::runtime_error(std::string(who) + ": num_heads must be > 0 and divide hidden_size");
    const std::size_t hkv = cfg.effective_num_kv_heads();
    if (hkv == 0 || cfg.num_heads % hkv != 0)
        throw std::runtime_error(std::string(who) + ": num_heads must be divisible by num_kv_heads");
    return Dims{static_cast<dim_t>(cfg.num_heads), static_cast<dim_t>(hkv), static_cast<dim_t>(cfg.head_dim()),
                static_cast<dim_t>(cfg.hidden_size), static_cast<dim_t>(cfg.num_heads / hkv)};
}

Tensor scale_at(const std::vector<Tensor>& v, std::size_t i) { return i < v.size() ? v[i] : Tensor{}; }

// llama_graph.cpp:30-44: QuantizedMatMul when the weight carries scales.
Tensor linear(Graph& g, Tensor x, Tensor w, Tensor scale, const ForwardWeights& fw) {
    if (fw.quant_type != QuantType::None && scale)
        return g.op(OpDescriptor{Op::QuantizedMatMul,
                                 QuantizedMatMulAttrs{.quant_type = fw.quant_type, .block_size = fw.quant_block_size}},
                    x, w, scale);
    return g.op(Op::MatMul, x, w);
}

Tensor rmsnorm(Graph& g, Tensor x, Tensor w, const Config& cfg) {
    return g.op(OpDescriptor{Op::RMSNorm, RMSNormAttrs{cfg.rms_norm_eps, -1}}, x, w);
}

Tensor to_heads(Graph& g, Tensor x, dim_t seq, dim_t heads, dim_t d) {
    auto r = g.op(OpDescriptor{Op::Reshape, ReshapeAttrs{shape_t{seq, heads, d}}}, x);
    return g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{1, 0, 2}}}, r);
}

Tensor repeat_if_grouped(Graph& g, Tensor t, dim_t group) {
    if (group <= 1) return t;
    return g.op(OpDescriptor{Op::RepeatKV, RepeatKVAttrs{static_cast<int>(group), 0}}, t);
}

// One decoder layer.  `past` (decode) holds the cached K/V of the layer;
// the new K/V are what the caller records as the layer's cache output.
struct LayerOut {
    Tensor h, k, v;
};

LayerOut build_layer(Graph& g, const Config& cfg, const Dims& d, const ForwardWeights& w, std::size_t l, Tensor h,
                     dim_t seq, const KVCacheHandles* past) {
    auto hn = rmsnorm(g, h, w.w_attn_norm[l], cfg);
    // Q/K/V projections, [S, H*D] -> [H, S, D], RoPE on Q and K (llama_graph.cpp:53-85).
    auto q = to_heads(g, linear(g, hn, w.wq[l], scale_at(w.wq_scale, l), w), seq, d.heads, d.head_dim);
    auto k = to_heads(g, linear(g, hn, w.wk[l], scale_at(w.wk_scale, l), w), seq, d.kv_heads, d.head_dim);
    auto v = to_heads(g, linear(g, hn, w.wv[l], scale_at(w.wv_scale, l), w), seq, d.kv_heads, d.head_dim);
    if (w.cos_cache && w.sin_cache) {
        q = g.op(Op::RotaryEmbedding, q, w.cos_cache, w.sin_cache);
        k = g.op(Op::RotaryEmbedding, k, w.cos_cache, w.sin_cache);
    }
    if (past) {  // decode: append to the cache on the sequence axis (:296-305)
        k = g.op(OpDescriptor{Op::Concat, ConcatAttrs{1}}, past->k[l], k);
        v = g.op(OpDescriptor{Op::Concat, ConcatAttrs{1}}, past->v[l], v);
    }
    auto k_att = repeat_if_grouped(g, k, d.group);
    auto v_att = repeat_if_grouped(g, v, d.group);

    // Attention context (:88-107): fused, or MatMul / mask / Softmax / MatMul.
    Tensor ctx;
    if (w.use_fused_attention) {
        ctx = g.op(OpDescriptor{Op::FusedAttention, FusedAttentionAttrs{.scale = 1.0f, .is_causal = true}}, q, k_att,
                   v_att);
    } else {
        auto kt = g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{0, 2, 1}}}, k_att);
        auto scores = g.op(Op::MatMul, q, kt);
        if (w.causal_mask) scores = g.op(Op::Add, scores, w.causal_mask);
        ctx = g.op(Op::MatMul, g.op(Op::Softmax, scores), v_att);
    }
    // Back to [S, hidden] and the output projection (:110-122), residual.
    auto ctx_t = g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{1, 0, 2}}}, ctx);
    auto ctx2 = g.op(OpDescriptor{Op::Reshape, ReshapeAttrs{shape_t{seq, d.hidden}}}, ctx_t);
    h = g.op(Op::Add, h, linear(g, ctx2, w.wo[l], scale_at(w.wo_scale, l), w));

    // SwiGLU MLP with residual (:125-139).
    auto hn2 = rmsnorm(g, h, w.w_ffn_norm[l], cfg);
    auto gate = linear(g, hn2, w.w_gate[l], scale_at(w.w_gate_scale, l), w);
    auto up = linear(g, hn2, w.w_up[l], scale_at(w.w_up_scale, l), w);
    auto act = g.op(Op::Mul, g.op(Op::Mul, g.op(Op::Sigmoid, gate), gate), up);
    h = g.op(Op::Add, h, linear(g, act, w.w_down[l], scale_at(w.w_down_scale, l), w));
    return LayerOut{h, k, v};
}

Tensor head(Graph& g, const Config& cfg, const ForwardWeights& w, Tensor h, bool last_only, const char* who) {
    auto hn = rmsnorm(g, h, w.w_final_norm, cfg);
    if (!w.w_lm_head) throw std::runtime_error(std::string(who) + ": w_lm_head is required");
    if (last_only) hn = slice_last_token(g, hn);
    return linear(g, hn, w.w_lm_head, w.w_lm_head_scale, w);
}

}  // namespace

auto slice_last_token(Graph& g, Tensor t) -> Tensor {
    const auto& shape = t.shape();
    if (shape.empty()) throw std::invalid_argument("slice_last_token: empty shape");
    const int seq = static_cast<int>(shape[0]);
    if (seq <= 1) return t;
    SliceAttrs a;
    a.begins.push_back(seq - 1);
    a.ends.push_back(seq);
    a.strides.push_back(1);
    for (std::size_t i = 1; i < shape.size(); ++i) {
        a.begins.push_back(0);
        a.ends.push_back(static_cast<int>(shape[i]));
        a.strides.push_back(1);
    }
    return g.op(OpDescriptor{Op::Slice, std::move(a)}, t);
}

auto build_forward_graph_prefill(Graph& g, const Config& cfg, Tensor tokens, const ForwardWeights& w,
                                 KVCacheHandles* kv_out, bool last_token_logits_only) -> Tensor {
    const Dims d = dims_of(cfg, "llama prefill");
    if (tokens.shape().size() != 1) throw std::runtime_error("llama prefill: `tokens` must be a 1-D int32 tensor");
    const dim_t seq = tokens.shape()[0];
    const std::size_t nodes = cfg.num_layers * 28 + 10;
    g.reserve(nodes + cfg.num_layers * 12 + 20, nodes);
    if (kv_out) {
        kv_out->k.clear();
        kv_out->v.clear();
    }
    Tensor h = g.op(Op::Embedding, w.w_embed, tokens);
    for (std::size_t l = 0; l < cfg.num_layers; ++l) {
        auto out = build_layer(g, cfg, d, w, l, h, seq, nullptr);
        if (kv_out) {
            kv_out->k.push_back(out.k);
            kv_out->v.push_back(out.v);
            g.mark_output(out.k);
            g.mark_output(out.v);
        }
        h = out.h;
    }
    auto logits = head(g, cfg, w, h, last_token_logits_only, "llama prefill");
    if (kv_out) g.mark_output(logits);
    return logits;
}

auto build_forward_graph_decode(Graph& g, const Config& cfg, Tensor token, const ForwardWeights& w,
                                const KVCacheHandles& kv_in, KVCacheHandles* kv_out) -> Tensor {
    const Dims d = dims_of(cfg, "llama decode");
    if (token.shape().size() != 1 || token.shape()[0] != 1)
        throw std::runtime_error("llama decode: `token` must be a 1-D int32 tensor of length 1");
    if (kv_in.k.size() != cfg.num_layers || kv_in.v.size() != cfg.num_layers)
        throw std::runtime_error("llama decode: kv_in size must match num_layers");
    const std::size_t nodes = cfg.num_layers * 30 + 10;
    g.reserve(nodes + cfg.num_layers * 14 + 20, nodes);
    if (kv_out) {
        kv_out->k.clear();
        kv_out->v.clear();
    }
    Tensor h = g.op(Op::Embedding, w.w_embed, token);
    for (std::size_t l = 0; l < cfg.num_layers; ++l) {
        auto out = build_layer(g, cfg, d, w, l, h, 1, &kv_in);
        if (kv_out) {
            kv_out->k.push_back(out.k);
            kv_out->v.push_back(out.v);
            g.mark_output(out.k);
            g.mark_output(out.v);
        }
        h = out.h;
    }
    auto logits = head(g, cfg, w, h, false, "llama decode");
    if (kv_out) g.mark_output(logits);
    return logits;
}

auto quantize_forward_weights(Graph& g, const ForwardWeights& fp, QuantType type, int block_size, DeviceType device)
    -> ForwardWeights {
    if (type == QuantType::None) return fp;
    ForwardWeights qw = fp;
    qw.graph = &g;
    qw.quant_type = type;
    qw.quant_block_size = block_size;
    auto adopt = [&](const Tensor& t) -> Tensor {
        auto s = t ? t.shared_storage() : nullptr;
        return s ? g.input(s) : Tensor{};
    };
    qw.w_embed = adopt(fp.w_embed);
    qw.w_final_norm = adopt(fp.w_final_norm);
    qw.cos_cache = adopt(fp.cos_cache);
    qw.sin_cache = adopt(fp.sin_cache);
    qw.causal_mask = adopt(fp.causal_mask);
    const std::size_t layers = fp.wq.size();
    for (std::size_t l = 0; l < layers; ++l) {
        qw.w_attn_norm[l] = adopt(fp.w_attn_norm[l]);
        qw.w_ffn_norm[l] = adopt(fp.w_ffn_norm[l]);
    }
    auto pack = [&](const Tensor& src, Tensor& q, Tensor& s) {
        if (!src) return;
        auto st = src.shared_storage();
        if (!st) throw std::runtime_error("quantize_forward_weights: tensor storage is null");
        auto packed = type == QuantType::Int4
                          ? quantize_storage_int4(*st, block_size > 0 ? static_cast<std::size_t>(block_size) : 32,
                                                  device)
                          : quantize_storage_int8(*st, device);
        q = g.input(packed.first);
        s = g.input(packed.second);
    };
    std::vector<Tensor>* lin[] = {&qw.wq, &qw.wk, &qw.wv, &qw.wo, &qw.w_gate, &qw.w_up, &qw.w_down};
    std::vector<Tensor>* scl[] = {&qw.wq_scale,   &qw.wk_scale, &qw.wv_scale,    &qw.wo_scale,
                                  &qw.w_gate_scale, &qw.w_up_scale, &qw.w_down_scale};
    const std::vector<Tensor>* src[] = {&fp.wq, &fp.wk, &fp.wv, &fp.wo, &fp.w_gate, &fp.w_up, &fp.w_down};
    for (int i = 0; i < 7; ++i) {
        lin[i]->assign(layers, Tensor{});
        scl[i]->assign(layers, Tensor{});
        for (std::size_t l = 0; l < layers; ++l) pack((*src[i])[l], (*lin[i])[l], (*scl[i])[l]);
    }
    if (fp.w_lm_head) pack(fp.w_lm_head, qw.w_lm_head, qw.w_lm_head_scale);
    return qw;
}

void compute_rope_cache(std::size_t seq_len, std::size_t head_dim, float base, std::vector<float>& cos_out,
                        std::vector<float>& sin_out, std::size_t pos_offset) {
    const std::size_t half = head_dim / 2;
    cos_out.assign(seq_len * half, 0.0f);
    sin_out.assign(seq_len * half, 0.0f);
    for (std::size_t i = 0; i < half; ++i) {
        // inv_freq_i = base^(-2i/head_dim), evaluated in fp32 as 1 / pow.
        const float inv_freq = 1.0f / std::pow(base, static_cast<float>(2 * i) / static_cast<float>(head_dim));
        for (std::size_t t = 0; t < seq_len; ++t) {
            const float angle = static_cast<float>(t + pos_offset) * inv_freq;
            cos_out[t * half + i] = std::cos(angle);
            sin_out[t * half + i] = std::sin(angle);
        }
    }
}

void compute_causal_mask(std::size_t num_heads, std::size_t seq_len, std::vector<float>& mask_out) {
    mask_out.assign(num_heads * seq_len * seq_len, 0.0f);
    for (std::size_t h = 0; h < num_heads; ++h)
        for (std::size_t r = 0; r < seq_len; ++r)
            for (std::size_t c = r + 1; c < seq_len; ++c) mask_out[(h * seq_len + r) * seq_len + c] = -1e9f;
}

}  // namespace velomind::examples::llama
