// PackedLlamaWeights (velomind/llama/llama_packed.h).
#include "velomind/llama/llama_packed.h"

#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "velomind/safetensors.h"
#include "vm_hip.h"

namespace velomind::examples::llama {

namespace {

void check(int rc, const char* what) {
    if (rc != VM_HIP_OK) throw std::runtime_error(std::string("PackedLlamaWeights: ") + what + ": " + vm_hip_last_error());
}

constexpr LlamaWeight kLayerLinears[] = {LlamaWeight::Wq, LlamaWeight::Wk,   LlamaWeight::Wv,  LlamaWeight::Wo,
                                         LlamaWeight::Gate, LlamaWeight::Up, LlamaWeight::Down};

std::shared_ptr<TensorStorage> device_alloc(std::size_t bytes, DataType dtype, const shape_t& shape) {
    auto s = TensorStorage::allocate(bytes, DeviceType::HIP);
    if (!s) throw std::runtime_error("PackedLlamaWeights: no HIP storage creator");
    s->dtype = dtype;
    s->shape = shape;
    s->size_bytes = bytes;
    return s;
}

std::vector<std::byte> download(const TensorStorage& s) {
    std::vector<std::byte> h(s.size_bytes);
    if (!h.empty()) check(vm_hip_memcpy_d2h(h.data(), s.data, h.size(), nullptr), "download");
    return h;
}

std::shared_ptr<TensorStorage> upload(const TensorStorage& host) {
    auto d = device_alloc(host.size_bytes, host.dtype, host.shape);
    if (host.size_bytes) check(vm_hip_memcpy_h2d(d->data, host.data, host.size_bytes, nullptr), "upload");
    return d;
}

// Shortest decimal that reads back as the same float.
std::string float_text(float v) {
    char buf[32];
    std::snprintf(buf, sizeof buf, "%.9g", static_cast<double>(v));
    return buf;
}

std::unordered_map<std::string, std::string> config_metadata(const Config& c) {
    return {{"velomind.vocab_size", std::to_string(c.vocab_size)},
            {"velomind.hidden_size", std::to_string(c.hidden_size)},
            {"velomind.intermediate_size", std::to_string(c.intermediate_size)},
            {"velomind.num_layers", std::to_string(c.num_layers)},
            {"velomind.num_heads", std::to_string(c.num_heads)},
            {"velomind.num_kv_heads", std::to_string(c.effective_num_kv_heads())},
            {"velomind.rms_norm_eps", float_text(c.rms_norm_eps)},
            {"velomind.rope_theta", float_text(c.rope_theta)}};
}

const std::string& meta_str(const std::unordered_map<std::string, std::string>& m, const char* key) {
    auto it = m.find(key);
    if (it == m.end()) throw std::runtime_error(std::string("packed weights: metadata '") + key + "' missing");
    return it->second;
}

std::size_t meta_size(const std::unordered_map<std::string, std::string>& m, const char* key) {
    const std::string& v = meta_str(m, key);
    std::size_t used = 0;
    unsigned long long x = 0;
    try {
        x = std::stoull(v, &used);
    } catch (const std::exception&) {
        used = 0;
    }
    if (used == 0 || used != v.size() || v[0] == '-')
        throw std::runtime_error(std::string("packed weights: metadata '") + key + "' is not a count: '" + v + "'");
    return static_cast<std::size_t>(x);
}

float meta_float(const std::unordered_map<std::string, std::string>& m, const char* key) {
    const std::string& v = meta_str(m, key);
    std::size_t used = 0;
    float x = 0.0f;
    try {
        x = std::stof(v, &used);
    } catch (const std::exception&) {
        used = 0;
    }
    if (used == 0 || used != v.size())
        throw std::runtime_error(std::string("packed weights: metadata '") + key + "' is not a number: '" + v + "'");
    return x;
}

Config config_from(const std::unordered_map<std::string, std::string>& m) {
    auto f = m.find("velomind.format");
    if (f == m.end() || f->second != "packed-linear-v1")
        throw std::runtime_error("packed weights: not a velomind packed-linear-v1 file");
    Config c;
    c.vocab_size = meta_size(m, "velomind.vocab_size");
    c.hidden_size = meta_size(m, "velomind.hidden_size");
    c.intermediate_size = meta_size(m, "velomind.intermediate_size");
    c.num_layers = meta_size(m, "velomind.num_layers");
    c.num_heads = meta_size(m, "velomind.num_heads");
    c.num_kv_heads = meta_size(m, "velomind.num_kv_heads");
    c.rms_norm_eps = meta_float(m, "velomind.rms_norm_eps");
    c.rope_theta = meta_float(m, "velomind.rope_theta");
    return c;
}

}  // namespace

auto llama_weight_name(LlamaWeight kind, std::size_t layer) -> std::string {
    const std::string l = "model.layers." + std::to_string(layer) + ".";
    switch (kind) {
        case LlamaWeight::Embed: return "model.embed_tokens.weight";
        case LlamaWeight::FinalNorm: return "model.norm.weight";
        case LlamaWeight::LmHead: return "lm_head.weight";
        case LlamaWeight::AttnNorm: return l + "input_layernorm.weight";
        case LlamaWeight::FfnNorm: return l + "post_attention_layernorm.weight";
        case LlamaWeight::Wq: return l + "self_attn.q_proj.weight";
        case LlamaWeight::Wk: return l + "self_attn.k_proj.weight";
        case LlamaWeight::Wv: return l + "self_attn.v_proj.weight";
        case LlamaWeight::Wo: return l + "self_attn.o_proj.weight";
        case LlamaWeight::Gate: return l + "mlp.gate_proj.weight";
        case LlamaWeight::Up: return l + "mlp.up_proj.weight";
        case LlamaWeight::Down: return l + "mlp.down_proj.weight";
    }
    throw std::invalid_argument("llama_weight_name: unknown weight kind");
}

auto PackedLlamaWeights::lin_slot(LlamaWeight kind, std::size_t layer) const -> std::size_t {
    if (kind == LlamaWeight::LmHead) return 7 * _cfg.num_layers;
    if (static_cast<int>(kind) < static_cast<int>(LlamaWeight::Wq) || layer >= _cfg.num_layers)
        throw std::invalid_argument("PackedLlamaWeights: not a linear or layer out of range");
    return 7 * layer + static_cast<std::size_t>(static_cast<int>(kind) - static_cast<int>(LlamaWeight::Wq));
}

auto PackedLlamaWeights::dense_slot(LlamaWeight kind, std::size_t layer) const -> std::size_t {
    switch (kind) {
        case LlamaWeight::Embed: return 0;
        case LlamaWeight::FinalNorm: return 1;
        case LlamaWeight::AttnNorm:
        case LlamaWeight::FfnNorm:
            if (layer >= _cfg.num_layers) throw std::invalid_argument("PackedLlamaWeights: layer out of range");
            return 2 + 2 * layer + (kind == LlamaWeight::FfnNorm ? 1 : 0);
        default: throw std::invalid_argument("PackedLlamaWeights: not an embedding or norm weight");
    }
}

auto PackedLlamaWeights::linear(LlamaWeight kind, std::size_t layer) const -> const PackedLinear& {
    return _lin[lin_slot(kind, layer)];
}

auto PackedLlamaWeights::dense(LlamaWeight kind, std::size_t layer) const -> std::shared_ptr<TensorStorage> {
    return _dense[dense_slot(kind, layer)];
}

auto PackedLlamaWeights::pack(const LlamaWeightSet& w, QuantType quant_type, int block_size)
    -> std::shared_ptr<PackedLlamaWeights> {
    if (quant_type == QuantType::None) throw std::invalid_argument("PackedLlamaWeights: quant_type must be Int8 or Int4");
    std::shared_ptr<PackedLlamaWeights> p(new PackedLlamaWeights());
    p->_cfg = w.config();
    p->_qt = quant_type;
    if (quant_type == QuantType::Int4) {
        p->_block = block_size > 0 ? block_size : 32;
        if (p->_block % 2) throw std::invalid_argument("PackedLlamaWeights: INT4 block must be even");
    } else {
        if (block_size > 0) throw std::invalid_argument("PackedLlamaWeights: INT8 weights are packed per column (block 0)");
        p->_block = 0;
    }
    const std::size_t L = p->_cfg.num_layers;
    p->_lin.resize(7 * L + 1);
    p->_dense.resize(2 + 2 * L);
    auto pack_one = [&](LlamaWeight kind, std::size_t layer) {
        auto src = w.storage(kind, layer);
        const auto k = static_cast<std::int64_t>(src->shape[0]), n = static_cast<std::int64_t>(src->shape[1]);
        PackedLinear& d = p->_lin[p->lin_slot(kind, layer)];
        d.k = k;
        d.n = n;
        if (quant_type == QuantType::Int4) {
            const std::int64_t nb = (k + p->_block - 1) / p->_block;
            d.codes = device_alloc(static_cast<std::size_t>((k + 1) / 2 * n), DataType::Int8, {(k + 1) / 2, n});
            d.scales = device_alloc(static_cast<std::size_t>(nb * n * 4), DataType::Float32, {nb, n});
            check(vm_hip_pack_int4(static_cast<const float*>(src->data), static_cast<std::uint8_t*>(d.codes->data),
                                   static_cast<float*>(d.scales->data), k, n, p->_block, nullptr),
                  "pack_int4");
        } else {
            d.codes = device_alloc(static_cast<std::size_t>(k * n), DataType::Int8, {k, n});
            d.scales = device_alloc(static_cast<std::size_t>(n * 4), DataType::Float32, {n});
            check(vm_hip_pack_int8(static_cast<const float*>(src->data), static_cast<std::int8_t*>(d.codes->data),
                                   static_cast<float*>(d.scales->data), k, n, nullptr),
                  "pack_int8");
        }
    };
    for (std::size_t l = 0; l < L; ++l) {
        for (LlamaWeight k : kLayerLinears) pack_one(k, l);
        p->_dense[p->dense_slot(LlamaWeight::AttnNorm, l)] = w.storage(LlamaWeight::AttnNorm, l);
        p->_dense[p->dense_slot(LlamaWeight::FfnNorm, l)] = w.storage(LlamaWeight::FfnNorm, l);
    }
    pack_one(LlamaWeight::LmHead, 0);
    p->_dense[0] = w.storage(LlamaWeight::Embed);
    p->_dense[1] = w.storage(LlamaWeight::FinalNorm);
    check(vm_hip_device_synchronize(), "pack");
    return p;
}

void PackedLlamaWeights::save(const std::filesystem::path& path) const {
    std::vector<std::vector<std::byte>> keep;
    std::vector<SafetensorsTensorView> views;
    const std::size_t L = _cfg.num_layers;
    keep.reserve(2 * _lin.size() + _dense.size());
    auto add = [&](const std::string& name, const TensorStorage& s) {
        keep.push_back(download(s));
        views.push_back({name, s.dtype, s.shape, std::span<const std::byte>(keep.back())});
    };
    auto add_dense = [&](LlamaWeight kind, std::size_t layer) { add(llama_weight_name(kind, layer), *dense(kind, layer)); };
    auto add_lin = [&](LlamaWeight kind, std::size_t layer) {
        const auto& pl = linear(kind, layer);
        const std::string nm = llama_weight_name(kind, layer);
        add(nm + ".codes", *pl.codes);
        add(nm + ".scales", *pl.scales);
    };
    add_dense(LlamaWeight::Embed, 0);
    for (std::size_t l = 0; l < L; ++l) {
        add_dense(LlamaWeight::AttnNorm, l);
        for (LlamaWeight k : kLayerLinears) add_lin(k, l);
        add_dense(LlamaWeight::FfnNorm, l);
    }
    add_dense(LlamaWeight::FinalNorm, 0);
    add_lin(LlamaWeight::LmHead, 0);
    auto meta = config_metadata(_cfg);
    meta["velomind.format"] = "packed-linear-v1";
    meta["velomind.quant_type"] = _qt == QuantType::Int4 ? "int4" : "int8";
    meta["velomind.block_size"] = std::to_string(_block);
    save_safetensors(path, views, meta);
}

auto llama_packed_config(const std::filesystem::path& path) -> Config {
    auto f = load_safetensors(path);
    if (!f) throw std::runtime_error("llama_packed_config: cannot read '" + path.string() + "' as safetensors");
    return config_from(f->metadata);
}

auto PackedLlamaWeights::load(const std::filesystem::path& path, const Config& cfg)
    -> std::shared_ptr<PackedLlamaWeights> {
    auto f = load_safetensors(path);
    if (!f) throw std::runtime_error("PackedLlamaWeights::load: cannot read '" + path.string() + "' as safetensors");
    const Config fc = config_from(f->metadata);
    if (fc.vocab_size != cfg.vocab_size || fc.hidden_size != cfg.hidden_size ||
        fc.intermediate_size != cfg.intermediate_size || fc.num_layers != cfg.num_layers ||
        fc.num_heads != cfg.num_heads || fc.num_kv_heads != cfg.effective_num_kv_heads())
        throw std::invalid_argument("PackedLlamaWeights::load: the file's model config differs from the requested one");
    std::shared_ptr<PackedLlamaWeights> p(new PackedLlamaWeights());
    p->_cfg = cfg;
    const std::string qt = f->metadata.count("velomind.quant_type") ? f->metadata.at("velomind.quant_type") : "";
    if (qt == "int4") p->_qt = QuantType::Int4;
    else if (qt == "int8") p->_qt = QuantType::Int8;
    else throw std::runtime_error("PackedLlamaWeights::load: unknown velomind.quant_type '" + qt + "'");
    p->_block = static_cast<int>(meta_size(f->metadata, "velomind.block_size"));
    if (p->_qt == QuantType::Int4 && (p->_block <= 0 || p->_block % 2))
        throw std::runtime_error("PackedLlamaWeights::load: INT4 block size must be even and positive");
    if (p->_qt == QuantType::Int8 && p->_block != 0)
        throw std::runtime_error("PackedLlamaWeights::load: INT8 weights are packed per column (block 0)");
    const std::size_t L = cfg.num_layers;
    p->_lin.resize(7 * L + 1);
    p->_dense.resize(2 + 2 * L);
    auto take = [&](const std::string& name, DataType dtype, const shape_t& shape) {
        auto it = f->tensors.find(name);
        if (it == f->tensors.end()) throw std::runtime_error("PackedLlamaWeights::load: tensor '" + name + "' missing");
        if (it->second->dtype != dtype || it->second->shape != shape)
            throw std::runtime_error("PackedLlamaWeights::load: tensor '" + name + "' has the wrong dtype or shape");
        return upload(*it->second);
    };
    auto load_lin = [&](LlamaWeight kind, std::size_t layer) {
        const shape_t ws = llama_weight_shape(cfg, kind);
        const std::int64_t k = ws[0], n = ws[1];
        PackedLinear& d = p->_lin[p->lin_slot(kind, layer)];
        d.k = k;
        d.n = n;
        const std::string nm = llama_weight_name(kind, layer);
        if (p->_qt == QuantType::Int4) {
            d.codes = take(nm + ".codes", DataType::Int8, {(k + 1) / 2, n});
            d.scales = take(nm + ".scales", DataType::Float32, {(k + p->_block - 1) / p->_block, n});
        } else {
            d.codes = take(nm + ".codes", DataType::Int8, {k, n});
            d.scales = take(nm + ".scales", DataType::Float32, {n});
        }
    };
    auto load_dense = [&](LlamaWeight kind, std::size_t layer) {
        p->_dense[p->dense_slot(kind, layer)] = take(llama_weight_name(kind, layer), DataType::Float32,
                                                     llama_weight_shape(cfg, kind));
    };
    load_dense(LlamaWeight::Embed, 0);
    load_dense(LlamaWeight::FinalNorm, 0);
    for (std::size_t l = 0; l < L; ++l) {
        load_dense(LlamaWeight::AttnNorm, l);
        load_dense(LlamaWeight::FfnNorm, l);
        for (LlamaWeight k : kLayerLinears) load_lin(k, l);
    }
    load_lin(LlamaWeight::LmHead, 0);
    return p;
}

}  // namespace velomind::examples::llama
