// LlamaWeightSet and GraphLlamaSession (see velomind/llama/llama_hip.h).
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <stdexcept>
#include <string>

#include "backend_hip/hip_runtime.h"
#include "velomind/executable.h"
#include "velomind/llama/llama_hip.h"
#include "vm_hip.h"

namespace velomind::examples::llama {

namespace {

void check(int rc, const char* what) {
    if (rc != VM_HIP_OK) throw std::runtime_error(std::string(what) + ": " + vm_hip_last_error());
}

std::shared_ptr<TensorStorage> device_f32(const shape_t& shape) {
    TensorStorage meta;
    meta.shape = shape;
    meta.dtype = DataType::Float32;
    auto s = TensorStorage::allocate(storage_nbytes(meta), DeviceType::HIP);
    s->shape = shape;
    s->dtype = DataType::Float32;
    return s;
}

constexpr int kLinearKinds[] = {static_cast<int>(LlamaWeight::Wq),   static_cast<int>(LlamaWeight::Wk),
                                static_cast<int>(LlamaWeight::Wv),   static_cast<int>(LlamaWeight::Wo),
                                static_cast<int>(LlamaWeight::Gate), static_cast<int>(LlamaWeight::Up),
                                static_cast<int>(LlamaWeight::Down)};

}  // namespace

auto llama_weight_shape(const Config& c, LlamaWeight kind) -> shape_t {
    const auto h = static_cast<dim_t>(c.hidden_size);
    const auto kv = static_cast<dim_t>(c.effective_num_kv_heads() * c.head_dim());
    const auto i = static_cast<dim_t>(c.intermediate_size);
    const auto v = static_cast<dim_t>(c.vocab_size);
    switch (kind) {
        case LlamaWeight::Embed: return {v, h};
        case LlamaWeight::FinalNorm: return {h};
        case LlamaWeight::LmHead: return {h, v};
        case LlamaWeight::AttnNorm: return {h};
        case LlamaWeight::FfnNorm: return {h};
        case LlamaWeight::Wq: return {h, static_cast<dim_t>(c.num_heads * c.head_dim())};
        case LlamaWeight::Wk: return {h, kv};
        case LlamaWeight::Wv: return {h, kv};
        case LlamaWeight::Wo: return {h, h};
        case LlamaWeight::Gate: return {h, i};
        case LlamaWeight::Up: return {h, i};
        case LlamaWeight::Down: return {i, h};
    }
    throw std::invalid_argument("llama_weight_shape: unknown weight kind");
}

LlamaWeightSet::LlamaWeightSet(const Config& cfg) : _cfg(cfg) {
    if (cfg.num_heads == 0 || cfg.hidden_size % cfg.num_heads != 0 || cfg.num_layers == 0 || cfg.vocab_size == 0 ||
        cfg.intermediate_size == 0 || cfg.num_heads % cfg.effective_num_kv_heads() != 0)
        throw std::invalid_argument("LlamaWeightSet: inconsistent config");
    _w.resize(3 + (kLlamaWeightKinds - 3) * cfg.num_layers);
    for (int k = 0; k < kLlamaWeightKinds; ++k) {
        const auto kind = static_cast<LlamaWeight>(k);
        const std::size_t layers = llama_weight_per_layer(kind) ? cfg.num_layers : 1;
        for (std::size_t l = 0; l < layers; ++l) _w[slot(kind, l)] = device_f32(llama_weight_shape(cfg, kind));
    }
}

auto LlamaWeightSet::slot(LlamaWeight kind, std::size_t layer) const -> std::size_t {
    const int k = static_cast<int>(kind);
    if (k < 0 || k >= kLlamaWeightKinds) throw std::invalid_argument("LlamaWeightSet: unknown weight kind");
    if (!llama_weight_per_layer(kind)) return static_cast<std::size_t>(k);
    if (layer >= _cfg.num_layers) throw std::out_of_range("LlamaWeightSet: layer out of range");
    return 3 + static_cast<std::size_t>(k - 3) * _cfg.num_layers + layer;
}

void LlamaWeightSet::set(LlamaWeight kind, std::size_t layer, std::span<const float> host) {
    auto& s = _w[slot(kind, layer)];
    if (host.size() != storage_numel(*s))
        throw std::invalid_argument("LlamaWeightSet::set: expected " + std::to_string(storage_numel(*s)) +
                                    " values, got " + std::to_string(host.size()));
    check(vm_hip_memcpy_h2d(s->data, host.data(), host.size_bytes(), nullptr), "LlamaWeightSet::set");
}

void LlamaWeightSet::fill_synthetic(std::uint64_t seed, float stddev) {
    for (int k = 0; k < kLlamaWeightKinds; ++k) {
        const auto kind = static_cast<LlamaWeight>(k);
        const bool norm = kind == LlamaWeight::FinalNorm || kind == LlamaWeight::AttnNorm || kind == LlamaWeight::FfnNorm;
        const std::size_t layers = llama_weight_per_layer(kind) ? _cfg.num_layers : 1;
        for (std::size_t l = 0; l < layers; ++l) {
            auto& s = _w[slot(kind, l)];
            const std::uint64_t tseed = seed ^ (0x100000001B3ull * (static_cast<std::uint64_t>(k) * 4099 + l + 1));
            check(vm_hip_fill_normal_f32(static_cast<float*>(s->data), static_cast<std::int64_t>(storage_numel(*s)),
                                         tseed, norm ? 1.0f : 0.0f, stddev, nullptr),
                  "LlamaWeightSet::fill_synthetic");
        }
    }
    check(vm_hip_device_synchronize(), "LlamaWeightSet::fill_synthetic");
}

void LlamaWeightSet::tie_lm_head_to_embedding() {
    const auto& emb = _w[slot(LlamaWeight::Embed, 0)];
    auto& head = _w[slot(LlamaWeight::LmHead, 0)];
    const std::int64_t shape[2] = {emb->shape[0], emb->shape[1]};
    check(vm_hip_transpose_f32(static_cast<const float*>(emb->data), static_cast<float*>(head->data), 2, shape,
                               nullptr, nullptr),
          "LlamaWeightSet::tie_lm_head_to_embedding");
    check(vm_hip_device_synchronize(), "LlamaWeightSet::tie_lm_head_to_embedding");
}

auto LlamaWeightSet::storage(LlamaWeight kind, std::size_t layer) const -> std::shared_ptr<TensorStorage> {
    return _w[slot(kind, layer)];
}

// ------------------------------------------------------------ graph session

GraphLlamaSession::GraphLlamaSession(std::shared_ptr<const LlamaWeightSet> weights, QuantType quant_type,
                                     int block_size, bool use_fused_attention)
    : _weights(std::move(weights)), _qt(quant_type), _block(block_size), _fused(use_fused_attention) {
    if (!_weights) throw std::invalid_argument("GraphLlamaSession: null weights");
    if (_qt == QuantType::Int8 && _block > 0)
        throw std::invalid_argument("GraphLlamaSession: INT8 weights are packed per column (block_size 0)");
    if (_qt == QuantType::Int4 && _block <= 0) _block = 32;  // the packer's block (quant.h:89)
    const char* pipe = std::getenv("VELOMIND_GRAPH_PIPELINE");
    _pipeline = !(pipe && pipe[0] == '0');
    const auto& cfg = _weights->config();
    const std::size_t n = 7 * cfg.num_layers + 1;
    _lin.resize(n);
    _scale.resize(n);
    for (std::size_t i = 0; i < n; ++i) {
        const bool head = i + 1 == n;
        const auto kind = head ? LlamaWeight::LmHead : static_cast<LlamaWeight>(kLinearKinds[i % 7]);
        auto src = _weights->storage(kind, head ? 0 : i / 7);
        if (_qt == QuantType::None) {
            _lin[i] = src;
        } else {
            auto packed = _qt == QuantType::Int4 ? quantize_storage_int4(*src, static_cast<std::size_t>(_block),
                                                                         DeviceType::HIP)
                                                 : quantize_storage_int8(*src, DeviceType::HIP);
            _lin[i] = packed.first;
            _scale[i] = packed.second;
        }
    }
}

void GraphLlamaSession::bind(Graph& g, ForwardWeights& w) const {
    const auto& cfg = _weights->config();
    w.graph = &g;
    w.use_fused_attention = _fused;
    w.quant_type = _qt;
    w.quant_block_size = _block;
    w.w_embed = g.input(_weights->storage(LlamaWeight::Embed));
    w.w_final_norm = g.input(_weights->storage(LlamaWeight::FinalNorm));
    std::vector<Tensor>* lin[] = {&w.wq, &w.wk, &w.wv, &w.wo, &w.w_gate, &w.w_up, &w.w_down};
    std::vector<Tensor>* scl[] = {&w.wq_scale,     &w.wk_scale,   &w.wv_scale,    &w.wo_scale,
                                  &w.w_gate_scale, &w.w_up_scale, &w.w_down_scale};
    for (std::size_t l = 0; l < cfg.num_layers; ++l) {
        w.w_attn_norm.push_back(g.input(_weights->storage(LlamaWeight::AttnNorm, l)));
        w.w_ffn_norm.push_back(g.input(_weights->storage(LlamaWeight::FfnNorm, l)));
        for (int j = 0; j < 7; ++j) {
            lin[j]->push_back(g.input(_lin[l * 7 + j]));
            if (_qt != QuantType::None) scl[j]->push_back(g.input(_scale[l * 7 + j]));
        }
    }
    w.w_lm_head = g.input(_lin.back());
    if (_qt != QuantType::None) w.w_lm_head_scale = g.input(_scale.back());
}

auto GraphLlamaSession::prefill(std::span<const std::int32_t> tokens) -> std::vector<float> {
    if (tokens.empty()) throw std::invalid_argument("GraphLlamaSession::prefill: tokens is empty");
    drop_prebuilt();
    const auto& cfg = _weights->config();
    const auto s = static_cast<dim_t>(tokens.size());
    const auto half = static_cast<dim_t>(cfg.head_dim() / 2);
    Graph g;
    auto tok = g.input({s}, DataType::Int32);
    ForwardWeights w;
    bind(g, w);
    w.cos_cache = g.input({s, half}, DataType::Float32);
    w.sin_cache = g.input({s, half}, DataType::Float32);
    if (!_fused) w.causal_mask = g.input({static_cast<dim_t>(cfg.num_heads), s, s}, DataType::Float32);
    KVCacheHandles kv;
    auto logits = build_forward_graph_prefill(g, cfg, tok, w, &kv, true);
    auto exec = g.build(DeviceType::HIP);
    tok.copy_from_host(std::as_bytes(tokens));
    std::vector<float> c, sn, mask;
    compute_rope_cache(tokens.size(), cfg.head_dim(), cfg.rope_theta, c, sn, 0);
    w.cos_cache.copy_from_host(std::as_bytes(std::span(c)));
    w.sin_cache.copy_from_host(std::as_bytes(std::span(sn)));
    if (!_fused) {
        compute_causal_mask(cfg.num_heads, tokens.size(), mask);
        w.causal_mask.copy_from_host(std::as_bytes(std::span(mask)));
    }
    exec->execute();
    _k.clear();
    _v.clear();
    for (std::size_t l = 0; l < cfg.num_layers; ++l) {
        _k.push_back(kv.k[l].shared_storage());
        _v.push_back(kv.v[l].shared_storage());
    }
    _seq_len = tokens.size();
    _timing = {};
    std::vector<float> out(cfg.vocab_size);
    logits.copy_to_host(std::as_writable_bytes(std::span(out)));
    return out;
}

struct GraphLlamaSession::DecodeStep {
    std::size_t pos = 0;
    std::vector<std::shared_ptr<TensorStorage>> k_in, v_in;   // the K/V tensors the graph reads
    std::unique_ptr<Graph> graph;
    std::unique_ptr<Executable> exec;                          // destroyed before its graph
    Tensor tok, cos, sin, logits;
    KVCacheHandles kv_out;
    double construct_s = 0.0, build_s = 0.0;
    double teardown_s = 0.0;   // of the step the helper destroyed after building this one
};

auto GraphLlamaSession::make_step(std::size_t pos, std::vector<std::shared_ptr<TensorStorage>> k,
                                  std::vector<std::shared_ptr<TensorStorage>> v) const
    -> std::unique_ptr<DecodeStep> {
    using clock = std::chrono::steady_clock;
    const auto t0 = clock::now();
    const auto& cfg = _weights->config();
    const auto half = static_cast<dim_t>(cfg.head_dim() / 2);
    auto st = std::make_unique<DecodeStep>();
    st->pos = pos;
    st->graph = std::make_unique<Graph>();
    Graph& g = *st->graph;
    st->tok = g.input({1}, DataType::Int32);
    ForwardWeights w;
    bind(g, w);
    w.cos_cache = g.input({1, half}, DataType::Float32);
    w.sin_cache = g.input({1, half}, DataType::Float32);
    KVCacheHandles kv_in;
    for (std::size_t l = 0; l < cfg.num_layers; ++l) {
        kv_in.k.push_back(g.input(k[l]));
        kv_in.v.push_back(g.input(v[l]));
    }
    st->logits = build_forward_graph_decode(g, cfg, st->tok, w, kv_in, &st->kv_out);
    st->cos = w.cos_cache;
    st->sin = w.sin_cache;
    const auto t1 = clock::now();
    st->exec = g.build(DeviceType::HIP);
    const auto t2 = clock::now();
    st->construct_s = std::chrono::duration<double>(t1 - t0).count();
    st->build_s = std::chrono::duration<double>(t2 - t1).count();
    st->k_in = std::move(k);
    st->v_in = std::move(v);
    return st;
}

// The helper: one thread for the session's life, running one job at a
// time.  Every prebuilt step is built and destroyed on it, so its allocator
// state stays warm (a fresh thread per step made construction and teardown
// 2-2.5x slower).
struct GraphLlamaSession::Helper {
    using Job = std::packaged_task<std::unique_ptr<DecodeStep>()>;
    std::mutex mu;
    std::condition_variable cv;
    Job job;
    bool has_job = false, stop = false;
    std::thread th{[this] { run(); }};   // last: starts after the fields above exist

    ~Helper() {
        {
            std::lock_guard<std::mutex> lock(mu);
            stop = true;
        }
        cv.notify_one();
        th.join();
    }
    auto post(Job j) -> std::future<std::unique_ptr<DecodeStep>> {
        auto f = j.get_future();
        {
            std::lock_guard<std::mutex> lock(mu);
            job = std::move(j);
            has_job = true;
        }
        cv.notify_one();
        return f;
    }
    void run() {
        for (;;) {
            Job j;
            {
                std::unique_lock<std::mutex> lock(mu);
                cv.wait(lock, [&] { return has_job || stop; });
                if (!has_job) return;
                j = std::move(job);
                has_job = false;
            }
            j();
        }
    }
};

void GraphLlamaSession::drop_prebuilt() noexcept {
    if (_prebuilt.valid()) {
        try {
            (void)_prebuilt.get();
        } catch (...) {
            // a step nobody will run: its failure is nobody's to report
        }
    }
    _retired.reset();
}

GraphLlamaSession::~GraphLlamaSession() {
    drop_prebuilt();
    _helper.reset();
}

auto GraphLlamaSession::forward_step(std::int32_t token, std::size_t pos) -> std::vector<float> {
    if (_seq_len == 0) {
        const std::int32_t one[1] = {token};
        return prefill(one);
    }
    if (pos != _seq_len) throw std::invalid_argument("GraphLlamaSession::forward_step: pos must equal the cache length");
    using clock = std::chrono::steady_clock;
    auto sec = [](clock::time_point a, clock::time_point b) { return std::chrono::duration<double>(b - a).count(); };
    const auto t0 = clock::now();
    const auto& cfg = _weights->config();
    // The step prebuilt for this position over the current K/V, when there is
    // one (get() rethrows a failure of its build here, at its own step).
    std::unique_ptr<DecodeStep> step;
    if (_prebuilt.valid()) {
        step = _prebuilt.get();
        if (step && (step->pos != pos || step->k_in != _k || step->v_in != _v)) step.reset();
    }
    const auto t1 = clock::now();
    double teardown = 0.0;
    if (step) {
        teardown = step->teardown_s;
    } else {
        _retired.reset();
        step = make_step(pos, _k, _v);
    }
    if (_pipeline) {
        // The next position's graph reads this step's K/V outputs, which
        // exist from this build on.  The device is idle here, so blocks freed
        // by earlier steps become reusable now, without the helper having to
        // synchronize while this step runs.
        backend::hip::reclaim_freed_blocks();
        std::vector<std::shared_ptr<TensorStorage>> k_next, v_next;
        for (std::size_t l = 0; l < cfg.num_layers; ++l) {
            k_next.push_back(step->kv_out.k[l].shared_storage());
            v_next.push_back(step->kv_out.v[l].shared_storage());
        }
        int device = 0;
        check(vm_hip_get_device(&device), "GraphLlamaSession: current device");
        if (!_helper) _helper = std::make_unique<Helper>();
        _prebuilt = _helper->post(Helper::Job([this, pos, device, k = std::move(k_next), v = std::move(v_next),
                                               old = std::move(_retired)]() mutable {
            check(vm_hip_set_device(device), "GraphLlamaSession: helper device");
            auto next = make_step(pos + 1, std::move(k), std::move(v));
            const auto td = clock::now();
            old.reset();
            next->teardown_s = std::chrono::duration<double>(clock::now() - td).count();
            return next;
        }));
    }
    const std::int32_t one[1] = {token};
    step->tok.copy_from_host(std::as_bytes(std::span(one)));
    std::vector<float> c, sn;
    compute_rope_cache(1, cfg.head_dim(), cfg.rope_theta, c, sn, pos);
    step->cos.copy_from_host(std::as_bytes(std::span(c)));
    step->sin.copy_from_host(std::as_bytes(std::span(sn)));
    const auto t2 = clock::now();
    step->exec->execute();
    const auto t3 = clock::now();
    for (std::size_t l = 0; l < cfg.num_layers; ++l) {
        _k[l] = step->kv_out.k[l].shared_storage();
        _v[l] = step->kv_out.v[l].shared_storage();
    }
    _seq_len = pos + 1;
    std::vector<float> out(cfg.vocab_size);
    step->logits.copy_to_host(std::as_writable_bytes(std::span(out)));
    const auto t4 = clock::now();
    const double construct = step->construct_s, build = step->build_s;
    if (_pipeline) {
        _retired = std::move(step);   // destroyed by the helper while the next step runs
    } else {
        step.reset();
        teardown = sec(t4, clock::now());
    }
    _timing[0] += construct;
    _timing[1] += build;
    _timing[2] += sec(t2, t3);
    _timing[3] += sec(t3, t4);
    _timing[4] += 1.0;
    _timing[5] += teardown;
    _timing[6] += sec(t0, t1);
    return out;
}

}  // namespace velomind::examples::llama
