// Pre-packed LLaMA weights: every linear as quant.cpp's codes and scales on
// the GPU, saved to / loaded from a safetensors file, so a quantized model
// loads without packing (the reference packs at bind time,
// examples/common/llama/llama_graph.cpp:336-425, and has no on-disk form).
//
// File layout (safetensors, HF tensor names):
//   <linear>.codes    I8  [K, N] (INT8) or [(K+1)/2, N] (INT4: even K row in
//                         the low nibble), the graph's [in, out] orientation
//   <linear>.scales   F32 [N] (INT8 per column) or [ceil(K/block), N]
//   model.embed_tokens.weight, model.norm.weight, model.layers.{l}.
//   {input,post_attention}_layernorm.weight  F32, unchanged
// with <linear> = model.layers.{l}.self_attn.{q,k,v,o}_proj.weight,
// model.layers.{l}.mlp.{gate,up,down}_proj.weight and lm_head.weight, and
// __metadata__ keys "velomind.format" = "packed-linear-v1",
// "velomind.quant_type" ("int8" | "int4"), "velomind.block_size" and the
// model config ("velomind.vocab_size", ...).  Linears hold the graph's
// weights: the reference loaders' transposed HF weights, q_proj already
// scaled by 1/sqrt(head_dim) (examples/tinyllama/model_loader.cpp:65-202).
#pragma once

#include <cstdint>
#include <filesystem>
#include <memory>
#include <string>
#include <vector>

#include "velomind/llama/llama_hip.h"
#include "velomind/quant.h"
#include "velomind/tensor_storage.h"
#include "velomind/velomind_core_export.h"

namespace velomind::examples::llama {

struct PackedLinear {
    std::shared_ptr<TensorStorage> codes;    // Int8, on the GPU
    std::shared_ptr<TensorStorage> scales;   // Float32, on the GPU
    std::int64_t k = 0, n = 0;
};

// HF name of a weight kind ("model.layers.3.self_attn.q_proj.weight", ...).
VELOMIND_CORE_EXPORT auto llama_weight_name(LlamaWeight kind, std::size_t layer) -> std::string;

class VELOMIND_CORE_EXPORT PackedLlamaWeights {
public:
    // Packs every linear of `w` on the GPU (vm_hip_pack_int8 / _int4,
    // bit-exact with quant.cpp); the embedding and norms are shared.
    static auto pack(const LlamaWeightSet& w, QuantType quant_type, int block_size)
        -> std::shared_ptr<PackedLlamaWeights>;
    // Reads a file written by save() and uploads it.  The file's config
    // must equal `cfg` (llama_packed_config reads it from the file).
    static auto load(const std::filesystem::path& path, const Config& cfg) -> std::shared_ptr<PackedLlamaWeights>;
    void save(const std::filesystem::path& path) const;

    const Config& config() const noexcept { return _cfg; }
    QuantType quant_type() const noexcept { return _qt; }
    int block_size() const noexcept { return _block; }
    // Linears: Wq..Down per layer, LmHead (layer 0).
    auto linear(LlamaWeight kind, std::size_t layer = 0) const -> const PackedLinear&;
    // Embed, FinalNorm, AttnNorm, FfnNorm (fp32 on the GPU).
    auto dense(LlamaWeight kind, std::size_t layer = 0) const -> std::shared_ptr<TensorStorage>;

private:
    PackedLlamaWeights() = default;
    Config _cfg;
    QuantType _qt = QuantType::Int4;
    int _block = 32;
    std::vector<PackedLinear> _lin;                       // [7 * layers + 1]
    std::vector<std::shared_ptr<TensorStorage>> _dense;   // [2 + 2 * layers]
    auto lin_slot(LlamaWeight kind, std::size_t layer) const -> std::size_t;
    auto dense_slot(LlamaWeight kind, std::size_t layer) const -> std::size_t;
};

// The model config recorded in a packed file's metadata.
VELOMIND_CORE_EXPORT auto llama_packed_config(const std::filesystem::path& path) -> Config;

}  // namespace velomind::examples::llama
