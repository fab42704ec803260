// LLaMA inference on DeviceType::HIP, two ways over one set of weights:
//
//  * GraphLlamaSession -- the reference engine's loop
//    (examples/common/llama/llama_engine.cpp:333-455): every prefill and
//    every decode step builds a fresh Graph with build_forward_graph_*, binds
//    the resident weights and the previous step's KV tensors, builds it on
//    DeviceType::HIP and executes it.  This is the drop-in: the same graphs
//    the reference runs on CPU/CUDA run through the HIP kernels.
//
//  * HipLlamaDecoder -- the same model as a resident decoder: fused QKV and
//    gate|up weights packed once, a resident KV cache appended in place,
//    device-side position and greedy sampling, and a decode step captured
//    once as a HIP graph and replayed per token.
//
// Both take their fp32 weights from a LlamaWeightSet: device tensors in the
// graph's [in, out] layout (the reference loaders' layout after transposing
// HF [out, in] weights and pre-scaling Q by 1/sqrt(head_dim),
// examples/tinyllama/model_loader.cpp:65-202).
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <future>
#include <memory>
#include <span>
#include <vector>

#include "velomind/llama/llama_graph.h"
#include "velomind/tensor_storage.h"
#include "velomind/velomind_core_export.h"

namespace velomind::examples::llama {

enum class LlamaWeight : int {
    Embed = 0,      // [vocab, hidden]
    FinalNorm = 1,  // [hidden]
    LmHead = 2,     // [hidden, vocab]
    AttnNorm = 3,   // [hidden] per layer
    FfnNorm = 4,    // [hidden] per layer
    Wq = 5,         // [hidden, heads * head_dim]
    Wk = 6,         // [hidden, kv_heads * head_dim]
    Wv = 7,         // [hidden, kv_heads * head_dim]
    Wo = 8,         // [hidden, hidden]
    Gate = 9,       // [hidden, intermediate]
    Up = 10,        // [hidden, intermediate]
    Down = 11,      // [intermediate, hidden]
};
inline constexpr int kLlamaWeightKinds = 12;
VELOMIND_CORE_EXPORT auto llama_weight_shape(const Config& cfg, LlamaWeight kind) -> shape_t;
inline bool llama_weight_per_layer(LlamaWeight k) { return static_cast<int>(k) >= static_cast<int>(LlamaWeight::AttnNorm); }

// fp32 weights resident on the GPU.
class VELOMIND_CORE_EXPORT LlamaWeightSet {
public:
    explicit LlamaWeightSet(const Config& cfg);
    const Config& config() const noexcept { return _cfg; }
    // Copies host data (numel must match the weight's shape).
    void set(LlamaWeight kind, std::size_t layer, std::span<const float> host);
    // Synthetic weights: linears and the embedding ~ N(0, stddev^2), norms
    // ~ N(1, stddev^2), each tensor from its own seed derived from (seed,
    // kind, layer), generated on the GPU.
    void fill_synthetic(std::uint64_t seed, float stddev);
    // Tied embeddings: lm_head [hidden, vocab] becomes the embedding's
    // transpose, as the reference loaders do when tie_word_embeddings is set
    // (examples/tinyllama/model_loader.cpp:74-144, "lm_head falls back to
    // the embedding").
    void tie_lm_head_to_embedding();
    auto storage(LlamaWeight kind, std::size_t layer = 0) const -> std::shared_ptr<TensorStorage>;

private:
    Config _cfg;
    std::vector<std::shared_ptr<TensorStorage>> _w;  // [kind][layer]
    auto slot(LlamaWeight kind, std::size_t layer) const -> std::size_t;
};

// Decode steps overlap host and device work: while step t's graph runs,
// a helper thread builds the graph of position t + 1 (it depends on the
// position and on step t's K/V tensors, not on the next token's value) and
// destroys step t - 1's.  Every step still builds, runs and destroys its
// own Graph, with the same results as one after another;
// VELOMIND_GRAPH_PIPELINE=0 runs them one after another.
class VELOMIND_CORE_EXPORT GraphLlamaSession {
public:
    GraphLlamaSession(std::shared_ptr<const LlamaWeightSet> weights, QuantType quant_type, int block_size,
                      bool use_fused_attention);
    ~GraphLlamaSession();
    GraphLlamaSession(const GraphLlamaSession&) = delete;
    GraphLlamaSession& operator=(const GraphLlamaSession&) = delete;
    // Prompt at positions 0..n-1; returns the last position's logits.
    auto prefill(std::span<const std::int32_t> tokens) -> std::vector<float>;
    // One token at position `pos` (== tokens processed so far).
    auto forward_step(std::int32_t token, std::size_t pos) -> std::vector<float>;
    auto seq_len() const noexcept -> std::size_t { return _seq_len; }
    // Host seconds spent by the decode steps since the last prefill, summed:
    // [0] building each step's Graph (nodes, shapes, bound weights), [1]
    // Graph::build on HIP, [2] Executable::execute (launches and the final
    // drain), [3] reading the logits back, [5] destroying a step's
    // Executable and Graph, [6] waiting for the helper thread to finish the
    // step's Graph; [4] the number of steps.  With the helper thread, [0],
    // [1] and [5] are its time, overlapped with [2].
    auto step_timing() const noexcept -> const std::array<double, 7>& { return _timing; }

private:
    struct DecodeStep;
    struct Helper;
    void bind(Graph& g, ForwardWeights& w) const;
    // The graph of the decode step at `pos` reading K/V `k`, `v`, built on HIP.
    auto make_step(std::size_t pos, std::vector<std::shared_ptr<TensorStorage>> k,
                   std::vector<std::shared_ptr<TensorStorage>> v) const -> std::unique_ptr<DecodeStep>;
    // Waits for the helper thread and discards what it built.
    void drop_prebuilt() noexcept;
    std::shared_ptr<const LlamaWeightSet> _weights;
    QuantType _qt;
    int _block;
    bool _fused;
    bool _pipeline = true;
    // Packed linears (or the fp32 ones when unquantized), shared by every step's graph.
    std::vector<std::shared_ptr<TensorStorage>> _lin, _scale;  // [7 * layers + 1]
    std::vector<std::shared_ptr<TensorStorage>> _k, _v;        // per layer, [Hkv, S, D]
    std::size_t _seq_len = 0;
    std::array<double, 7> _timing{};
    std::unique_ptr<DecodeStep> _retired;                  // the last step run, destroyed by the helper
    std::future<std::unique_ptr<DecodeStep>> _prebuilt;    // the next position's step, from the helper
    std::unique_ptr<Helper> _helper;                       // the helper thread (started on first use)
};

class PackedLlamaWeights;

class VELOMIND_CORE_EXPORT HipLlamaDecoder {
public:
    HipLlamaDecoder(const LlamaWeightSet& weights, QuantType quant_type, int block_size, std::size_t max_seq);
    // From pre-packed weights (velomind/llama/llama_packed.h): no packing.
    HipLlamaDecoder(const PackedLlamaWeights& packed, std::size_t max_seq);
    ~HipLlamaDecoder();
    HipLlamaDecoder(const HipLlamaDecoder&) = delete;
    HipLlamaDecoder& operator=(const HipLlamaDecoder&) = delete;

    // Prompt at positions 0..n-1 (n <= max_seq); returns the last logits.
    auto prefill(std::span<const std::int32_t> tokens) -> std::vector<float>;
    // One token at position `pos` (<= tokens processed so far); returns logits.
    auto forward_step(std::int32_t token, std::size_t pos) -> std::vector<float>;
    // Greedy generation: prefill, then `steps` decode steps replayed from a
    // HIP graph (or launched eagerly with use_graph = false).  Returns the
    // steps + 1 generated tokens (the first comes from the prompt's logits).
    auto generate(std::span<const std::int32_t> prompt, std::size_t steps, bool use_graph = true)
        -> std::vector<std::int32_t>;
    // Device time of the last generate()'s prefill (with the first argmax)
    // and of its timed decode steps: every step with use_graph = false; with
    // graphs, the replays after the eager first step and the capture.
    auto last_prefill_seconds() const noexcept -> double { return _prefill_s; }
    auto last_decode_seconds() const noexcept -> double { return _decode_s; }
    auto last_decode_steps_timed() const noexcept -> std::size_t { return _decode_steps_timed; }
    auto max_seq() const noexcept -> std::size_t { return _max_seq; }
    // Logits of the most recent step or prefill.
    auto logits() const -> std::vector<float>;
    // How a one-token step runs: one launch per operation, split-K slices
    // with their consumers (five launches per layer), or one persistent
    // launch per token (vm_hip_decode_step).
    enum class DecodePath { PerOperation = 1, Slices = 2, Persistent = 3 };
    auto decode_path() const noexcept -> DecodePath;

private:
    struct Impl;
    std::unique_ptr<Impl> _impl;
    std::size_t _max_seq;
    double _prefill_s = 0.0, _decode_s = 0.0;
    std::size_t _decode_steps_timed = 0;
};

}  // namespace velomind::examples::llama
