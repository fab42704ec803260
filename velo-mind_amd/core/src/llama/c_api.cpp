// extern "C" surface of the LLaMA inference layer (include/vm_llama.h).
#include "vm_llama.h"

#include <algorithm>
#include <chrono>
#include <memory>
#include <stdexcept>
#include <string>

#include "velomind/llama/llama_hip.h"
#include "velomind/llama/llama_packed.h"

using namespace velomind;
using namespace velomind::examples::llama;

struct vm_llama_weights {
    std::shared_ptr<LlamaWeightSet> set;
};

struct vm_llama_packed {
    std::shared_ptr<PackedLlamaWeights> p;
};

struct vm_llama_session {
    std::shared_ptr<LlamaWeightSet> weights;  // keeps the fp32 weights alive
    std::unique_ptr<GraphLlamaSession> graph;
    std::unique_ptr<HipLlamaDecoder> resident;
};

namespace {

thread_local std::string t_error;

template <typename F>
int guarded(F&& f) {
    try {
        t_error.clear();
        f();
        return 0;
    } catch (const std::exception& e) {
        t_error = e.what();
    } catch (...) {
        t_error = "unknown error";
    }
    return -1;
}

Config to_config(const vm_llama_config& c) {
    if (c.vocab_size <= 0 || c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_layers <= 0 || c.num_heads <= 0 ||
        c.num_kv_heads < 0)
        throw std::invalid_argument("vm_llama_config: sizes must be positive");
    Config cfg;
    cfg.vocab_size = static_cast<std::size_t>(c.vocab_size);
    cfg.hidden_size = static_cast<std::size_t>(c.hidden_size);
    cfg.intermediate_size = static_cast<std::size_t>(c.intermediate_size);
    cfg.num_layers = static_cast<std::size_t>(c.num_layers);
    cfg.num_heads = static_cast<std::size_t>(c.num_heads);
    cfg.num_kv_heads = static_cast<std::size_t>(c.num_kv_heads);
    cfg.rms_norm_eps = c.rms_norm_eps;
    cfg.rope_theta = c.rope_theta;
    return cfg;
}

QuantType to_quant(int q) {
    switch (q) {
        case 0: return QuantType::None;
        case 1: return QuantType::Int8;
        case 2: return QuantType::Int4;
    }
    throw std::invalid_argument("vm_llama: quant_type must be 0, 1 or 2");
}

void copy_logits(const std::vector<float>& v, float* out) {
    if (out) std::copy(v.begin(), v.end(), out);
}

}  // namespace

extern "C" {

const char* vm_llama_last_error(void) { return t_error.c_str(); }

int vm_llama_weights_create(const vm_llama_config* cfg, vm_llama_weights** out) {
    return guarded([&] {
        if (!cfg || !out) throw std::invalid_argument("vm_llama_weights_create: null argument");
        *out = nullptr;
        auto w = std::make_unique<vm_llama_weights>();
        w->set = std::make_shared<LlamaWeightSet>(to_config(*cfg));
        *out = w.release();
    });
}

int vm_llama_weights_set(vm_llama_weights* w, int kind, int64_t layer, const float* host, int64_t numel) {
    return guarded([&] {
        if (!w || !host || numel < 0 || layer < 0) throw std::invalid_argument("vm_llama_weights_set: bad argument");
        if (kind < 0 || kind >= kLlamaWeightKinds) throw std::invalid_argument("vm_llama_weights_set: bad kind");
        w->set->set(static_cast<LlamaWeight>(kind), static_cast<std::size_t>(layer),
                    std::span<const float>(host, static_cast<std::size_t>(numel)));
    });
}

int vm_llama_weights_fill_synthetic(vm_llama_weights* w, uint64_t seed, float stddev) {
    return guarded([&] {
        if (!w) throw std::invalid_argument("vm_llama_weights_fill_synthetic: null weights");
        w->set->fill_synthetic(seed, stddev);
    });
}

int vm_llama_weights_tie_lm_head(vm_llama_weights* w) {
    return guarded([&] {
        if (!w) throw std::invalid_argument("vm_llama_weights_tie_lm_head: null weights");
        w->set->tie_lm_head_to_embedding();
    });
}

void vm_llama_weights_destroy(vm_llama_weights* w) { delete w; }

int vm_llama_session_create(const vm_llama_weights* w, int engine, int quant_type, int block_size, int fused_attention,
                            int64_t max_seq, vm_llama_session** out) {
    return guarded([&] {
        if (!w || !out) throw std::invalid_argument("vm_llama_session_create: null argument");
        *out = nullptr;
        auto s = std::make_unique<vm_llama_session>();
        s->weights = w->set;
        if (engine == VM_LLAMA_ENGINE_GRAPH) {
            s->graph = std::make_unique<GraphLlamaSession>(w->set, to_quant(quant_type), block_size, fused_attention != 0);
        } else if (engine == VM_LLAMA_ENGINE_RESIDENT) {
            if (max_seq <= 0) throw std::invalid_argument("vm_llama_session_create: max_seq must be positive");
            s->resident = std::make_unique<HipLlamaDecoder>(*w->set, to_quant(quant_type), block_size,
                                                            static_cast<std::size_t>(max_seq));
        } else {
            throw std::invalid_argument("vm_llama_session_create: unknown engine");
        }
        *out = s.release();
    });
}

void vm_llama_session_destroy(vm_llama_session* s) { delete s; }

int vm_llama_prefill(vm_llama_session* s, const int32_t* tokens, int64_t n, float* logits_out) {
    return guarded([&] {
        if (!s || !tokens || n <= 0) throw std::invalid_argument("vm_llama_prefill: bad argument");
        std::span<const std::int32_t> t(tokens, static_cast<std::size_t>(n));
        copy_logits(s->graph ? s->graph->prefill(t) : s->resident->prefill(t), logits_out);
    });
}

int vm_llama_forward_step(vm_llama_session* s, int32_t token, int64_t pos, float* logits_out) {
    return guarded([&] {
        if (!s || pos < 0) throw std::invalid_argument("vm_llama_forward_step: bad argument");
        const auto p = static_cast<std::size_t>(pos);
        copy_logits(s->graph ? s->graph->forward_step(token, p) : s->resident->forward_step(token, p), logits_out);
    });
}

int vm_llama_session_decode_path(const vm_llama_session* s, int* path) {
    return guarded([&] {
        if (!s || !path) throw std::invalid_argument("vm_llama_session_decode_path: null argument");
        *path = s->resident ? static_cast<int>(s->resident->decode_path()) : VM_LLAMA_DECODE_GRAPH;
    });
}

int vm_llama_session_step_timing(const vm_llama_session* s, double* out7) {
    return guarded([&] {
        if (!s || !out7) throw std::invalid_argument("vm_llama_session_step_timing: null argument");
        if (!s->graph) throw std::invalid_argument("vm_llama_session_step_timing: not a graph-engine session");
        const auto& t = s->graph->step_timing();
        std::copy(t.begin(), t.end(), out7);
    });
}

int vm_llama_generate(vm_llama_session* s, const int32_t* prompt, int64_t n, int64_t steps, int use_hip_graph,
                      int32_t* out_tokens, double* timing) {
    return guarded([&] {
        if (!s || !prompt || n <= 0 || steps < 0 || !out_tokens)
            throw std::invalid_argument("vm_llama_generate: bad argument");
        std::span<const std::int32_t> p(prompt, static_cast<std::size_t>(n));
        if (s->resident) {
            auto toks = s->resident->generate(p, static_cast<std::size_t>(steps), use_hip_graph != 0);
            std::copy(toks.begin(), toks.end(), out_tokens);
            if (timing) {
                timing[0] = s->resident->last_prefill_seconds();
                timing[1] = s->resident->last_decode_seconds();
                timing[2] = static_cast<double>(s->resident->last_decode_steps_timed());
            }
            return;
        }
        // Graph engine: the reference engine's generation loop (argmax sampling).
        auto argmax = [](const std::vector<float>& v) {
            std::int32_t best = -1;
            for (std::size_t i = 0; i < v.size(); ++i)
                if (v[i] == v[i] && (best < 0 || v[i] > v[static_cast<std::size_t>(best)]))
                    best = static_cast<std::int32_t>(i);
            return best;
        };
        const auto t0 = std::chrono::steady_clock::now();
        std::int32_t tok = argmax(s->graph->prefill(p));
        const auto t1 = std::chrono::steady_clock::now();
        out_tokens[0] = tok;
        std::size_t pos = p.size();
        for (int64_t i = 0; i < steps; ++i) {
            tok = argmax(s->graph->forward_step(tok, pos++));
            out_tokens[i + 1] = tok;
        }
        const auto t2 = std::chrono::steady_clock::now();
        if (timing) {
            timing[0] = std::chrono::duration<double>(t1 - t0).count();
            timing[1] = std::chrono::duration<double>(t2 - t1).count();
            timing[2] = static_cast<double>(steps);
        }
    });
}

int vm_llama_pack(const vm_llama_weights* w, int quant_type, int block_size, vm_llama_packed** out) {
    return guarded([&] {
        if (!w || !out) throw std::invalid_argument("vm_llama_pack: null pointer");
        auto p = std::make_unique<vm_llama_packed>();
        p->p = PackedLlamaWeights::pack(*w->set, to_quant(quant_type), block_size);
        *out = p.release();
    });
}

int vm_llama_packed_save(const vm_llama_packed* p, const char* path) {
    return guarded([&] {
        if (!p || !path) throw std::invalid_argument("vm_llama_packed_save: null pointer");
        p->p->save(path);
    });
}

int vm_llama_packed_config(const char* path, vm_llama_config* out) {
    return guarded([&] {
        if (!path || !out) throw std::invalid_argument("vm_llama_packed_config: null pointer");
        const Config c = llama_packed_config(path);
        out->vocab_size = static_cast<int64_t>(c.vocab_size);
        out->hidden_size = static_cast<int64_t>(c.hidden_size);
        out->intermediate_size = static_cast<int64_t>(c.intermediate_size);
        out->num_layers = static_cast<int64_t>(c.num_layers);
        out->num_heads = static_cast<int64_t>(c.num_heads);
        out->num_kv_heads = static_cast<int64_t>(c.num_kv_heads);
        out->rms_norm_eps = c.rms_norm_eps;
        out->rope_theta = c.rope_theta;
    });
}

int vm_llama_packed_load(const char* path, const vm_llama_config* cfg, vm_llama_packed** out) {
    return guarded([&] {
        if (!path || !cfg || !out) throw std::invalid_argument("vm_llama_packed_load: null pointer");
        auto p = std::make_unique<vm_llama_packed>();
        p->p = PackedLlamaWeights::load(path, to_config(*cfg));
        *out = p.release();
    });
}

void vm_llama_packed_destroy(vm_llama_packed* p) { delete p; }

int vm_llama_session_create_packed(const vm_llama_packed* p, int64_t max_seq, vm_llama_session** out) {
    return guarded([&] {
        if (!p || !out) throw std::invalid_argument("vm_llama_session_create_packed: null pointer");
        if (max_seq <= 0) throw std::invalid_argument("vm_llama_session_create_packed: max_seq must be positive");
        auto s = std::make_unique<vm_llama_session>();
        s->resident = std::make_unique<HipLlamaDecoder>(*p->p, static_cast<std::size_t>(max_seq));
        *out = s.release();
    });
}

}  // extern "C"
