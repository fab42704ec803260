// HipLlamaDecoder: the LLaMA forward pass of the reference graph
// (examples/common/llama/llama_graph.cpp:14-330) as a resident decoder.
//
// Weights.  Q|K|V and gate|up are packed as single matrices
// ([hidden, (H + 2 Hkv) D] and [hidden, 2 I]): quant.cpp packs every
// column independently (per-column INT8 scales, per-column INT4 blocks), so
// the packed fused matrix is byte for byte the three (two) packed matrices
// side by side, and one GEMV reads all of them.
//
// Step.  One token (or a prompt) runs as
//   embedding -> per layer [add+rmsnorm, QKV, rope+append, attention, O,
//   add+rmsnorm, gate|up, silu*mul, down] -> add+rmsnorm -> lm_head -> argmax
// with every position read from a device int32, so a decode step is a
// fixed launch sequence that is captured once as a HIP graph and replayed
// per token; the argmax writes the next token where the embedding reads it
// and advances the position.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "velomind/llama/llama_hip.h"
#include "velomind/llama/llama_packed.h"
#include "vm_hip.h"

namespace velomind::examples::llama {

namespace {

void check(int rc, const char* what) {
    if (rc != VM_HIP_OK) throw std::runtime_error(std::string("HipLlamaDecoder: ") + what + ": " + vm_hip_last_error());
}

struct DevBuf {
    void* p = nullptr;
    std::size_t bytes = 0;
    DevBuf() = default;
    explicit DevBuf(std::size_t n) : bytes(n) {
        if (n) check(vm_hip_malloc(&p, n), "allocation");
    }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        std::swap(p, o.p);
        std::swap(bytes, o.bytes);
        return *this;
    }
    ~DevBuf() {
        if (p) (void)vm_hip_free(p);
    }
    template <typename T>
    T* as() const { return static_cast<T*>(p); }
};

// One packed linear [k, n].
struct Packed {
    DevBuf codes, scales;
    std::int64_t k = 0, n = 0;
};

}  // namespace

struct HipLlamaDecoder::Impl {
    // Slice limits per projection: what each consumer reads with few
    // memory round trips (the residual norm and the SwiGLU staging add the
    // slices of a whole row; argmax scans the vocabulary once per slice).
    // lm_head: up to 16 slices (narrower workgroups on more CUs; SmolLM2-360M
    // INT8 decode 893.6 -> 864.9 us/token against 4, TinyLlama unchanged).
    static constexpr int kMaxQkv = 16, kMaxO = 16, kMaxGu = 16, kMaxDown = 22, kMaxLm = 16;
    // Prefetch of the next projections' weights by the attention launch
    // (VELOMIND_DECODE_PREFETCH=0 turns it off).
    bool prefetch = true;
    Config cfg;
    int qt = VM_HIP_QUANT_INT4;
    int block = 32;
    std::int64_t H = 0, Hk = 0, D = 0, hidden = 0, inter = 0, vocab = 0, qkv_n = 0;
    std::size_t max_seq = 0;
    void* stream = nullptr;
    void* graph = nullptr;
    void* ev0 = nullptr;
    void* ev1 = nullptr;

    // Weights.
    std::vector<Packed> qkv, o, gate_up, down;
    Packed lm_head;
    std::shared_ptr<TensorStorage> embed, final_norm;
    std::vector<std::shared_ptr<TensorStorage>> attn_norm, ffn_norm;
    // KV cache [layers][Hkv][max_seq][D] for K, then V; RoPE tables [max_seq][D/2].
    DevBuf kcache, vcache, cos_t, sin_t;
    // Activations sized for max_seq rows.
    DevBuf h, hn, qkv_out, q, ctx, attn_out, gu, act, down_out, logits;
    DevBuf idx, token, pos, tokens;
    DevBuf am_ws;   // argmax workspace
    std::size_t seq = 0;  // positions filled in the cache
    // One-token steps: projections leave split-K partial slices that their
    // consumers add (vm_hip_qmm_gemv_slices_f32); counts per projection.
    bool sliced = false;
    int s_qkv = 0, s_o = 0, s_gu = 0, s_down = 0, s_lm = 0;
    // slice limits of q|k|v, o, gate|up, down, lm_head (the kMax* values;
    // VELOMIND_SLICES_MAX="qkv,o,gu,down,lm" overrides them for sweeps)
    int qkv_max = kMaxQkv, o_max = kMaxO, gu_max = kMaxGu, down_max = kMaxDown, lm_max = kMaxLm;
    DevBuf qkv_sl, o_sl, gu_sl, down_sl, lm_sl;
    DevBuf h2, ss_attn, ss_ffn, ss_final, att_part;   // second residual buffer, norm partials, attention records
    int att_chunk = 0, att_chunks = 0;
    // One-launch decode steps (vm_hip_decode_step), opted into with
    // VELOMIND_DECODE_PERSISTENT=1: the model description, its per-layer
    // weight table on the device and the step's workspace.  Off by default:
    // on an MI355X the captured launch-per-projection step is faster
    // (TinyLlama shapes: ~710 us against ~930 us per token).
    bool persistent = false;
    vm_hip_decode_model pmodel{};
    DevBuf player, pws;
    std::uint32_t pstep = 0;

    float* kc(std::size_t l) const { return kcache.as<float>() + l * Hk * max_seq * D; }
    float* vc(std::size_t l) const { return vcache.as<float>() + l * Hk * max_seq * D; }

    void pack(Packed& dst, const float* w, std::int64_t k, std::int64_t n) {
        dst.k = k;
        dst.n = n;
        if (qt == VM_HIP_QUANT_INT4) {
            const std::int64_t nb = (k + block - 1) / block;
            dst.codes = DevBuf(static_cast<std::size_t>((k + 1) / 2 * n));
            dst.scales = DevBuf(static_cast<std::size_t>(nb * n * 4));
            check(vm_hip_pack_int4(w, dst.codes.as<std::uint8_t>(), dst.scales.as<float>(), k, n, block, stream),
                  "pack_int4");
        } else {
            dst.codes = DevBuf(static_cast<std::size_t>(k * n));
            dst.scales = DevBuf(static_cast<std::size_t>(n * 4));
            check(vm_hip_pack_int8(w, dst.codes.as<std::int8_t>(), dst.scales.as<float>(), k, n, stream),
                  "pack_int8");
        }
    }

    // Packs [k, n_1 + n_2 + ...] assembled column block by column block.
    void pack_fused(Packed& dst, std::initializer_list<std::shared_ptr<TensorStorage>> parts, std::int64_t k) {
        std::int64_t n = 0;
        for (auto& p : parts) n += p->shape[1];
        DevBuf tmp(static_cast<std::size_t>(k * n * 4));
        std::int64_t col = 0;
        for (auto& p : parts) {
            const std::int64_t w = p->shape[1];
            check(vm_hip_memcpy_2d_d2d(tmp.as<float>() + col, static_cast<std::size_t>(n * 4), p->data,
                                       static_cast<std::size_t>(w * 4), static_cast<std::size_t>(w * 4),
                                       static_cast<std::size_t>(k), stream),
                  "fuse weights");
            col += w;
        }
        pack(dst, tmp.as<float>(), k, n);
        check(vm_hip_stream_synchronize(stream), "pack");  // tmp is freed on return
    }

    int block_arg() const { return qt == VM_HIP_QUANT_INT4 ? block : 0; }

    // Slice count of the split-K GEMV for `w`, or 0 when the shape or block
    // size needs the final-output kernel.
    int slices_for(const Packed& w, int max_slices) const {
        int sl = 0;
        if (vm_hip_gemv_slices_count(w.k, w.n, qt, block_arg(), max_slices, &sl) != VM_HIP_OK) return 0;
        return sl;
    }

    void gemv_slices(const float* act, int kind, int act_slices, const Packed& w, float* out, int max_slices) {
        check(vm_hip_qmm_gemv_slices_f32(act, kind, act_slices, static_cast<const std::int8_t*>(w.codes.p),
                                         w.scales.as<float>(), out, w.k, w.n, qt, block_arg(), max_slices, stream),
              "quantized matmul (slices)");
    }

    void gemv_src(const vm_hip_gemv_src& src, const Packed& w, float* out, int max_slices) {
        check(vm_hip_qmm_gemv_slices_src_f32(&src, static_cast<const std::int8_t*>(w.codes.p), w.scales.as<float>(), out,
                                             w.k, w.n, qt, block_arg(), max_slices, stream),
              "quantized matmul (slices)");
    }

    // Residual + RMSNorm staged in front of a projection: x = (h + sum of
    // delta slices) * w; the projection's consumer applies 1/rms from ss.
    static vm_hip_gemv_src normres(const float* h_in, const float* delta, int delta_slices, const void* norm_w,
                                   float* h_out, float* ss_out) {
        vm_hip_gemv_src src{};
        src.kind = VM_HIP_GEMV_SRC_NORMRES;
        src.act = h_in;
        src.delta = delta_slices > 0 ? delta : nullptr;
        src.slices = delta_slices;
        src.norm_w = static_cast<const float*>(norm_w);
        src.h_out = h_out;
        src.ss_out = ss_out;
        return src;
    }

    // One token at *pos, five launches per layer:
    //   QKV (residual + RMSNorm staged)  ->  attention (slice sums, 1/rms,
    //   RoPE, in-place K/V append, chunk partials)  ->  O (partials merged
    //   while staging)  ->  gate|up (residual + RMSNorm staged)  ->  down
    //   (SwiGLU with 1/rms staged from the gate|up slices)
    // then the final norm staged in front of lm_head, whose slices stay in
    // lm_sl (greedy argmax does not need the positive 1/rms scale).  The
    // residual stream alternates between h (embedding, after each layer)
    // and h2 (after attention).
    void forward_one_sliced() {
        const float eps = cfg.rms_norm_eps;
        float* ha = h.as<float>();
        float* hb = h2.as<float>();
        const auto* posp = pos.as<std::int32_t>();
        const float dim = static_cast<float>(hidden);
        check(vm_hip_embedding_f32(static_cast<const float*>(embed->data), vocab, hidden, token.as<std::int32_t>(), 1,
                                   ha, stream),
              "embedding");
        vm_hip_gemv_src attn_src{};
        attn_src.kind = VM_HIP_GEMV_SRC_ATTN;
        attn_src.act = att_part.as<float>();
        attn_src.pos = posp;
        attn_src.head_dim = static_cast<int>(D);
        attn_src.chunk = att_chunk;
        attn_src.chunks = att_chunks;
        attn_src.max_seq = static_cast<int>(max_seq);
        for (std::size_t l = 0; l < cfg.num_layers; ++l) {
            gemv_src(normres(ha, down_sl.as<float>(), l == 0 ? 0 : s_down, attn_norm[l]->data, hb, ss_attn.as<float>()),
                     qkv[l], qkv_sl.as<float>(), qkv_max);
            // Attention leaves most CUs idle: its extra workgroups read the
            // output and gate|up projections' weights into the Infinity
            // Cache for the two launches after it (measured on MI355X:
            // TinyLlama INT4 decode 730 -> 714 us per token; prefetching
            // more, or with fewer workgroups, lengthens the attention launch
            // by more than the next launches gain).
            vm_hip_prefetch pf{};
            if (prefetch) {
                for (const Packed* pp : {&o[l], &gate_up[l]}) {
                    pf.ptr[pf.count] = pp->codes.p;
                    pf.bytes[pf.count++] = pp->codes.bytes;
                    pf.ptr[pf.count] = pp->scales.p;
                    pf.bytes[pf.count++] = pp->scales.bytes;
                }
            }
            check(vm_hip_attention_decode_slices_prefetch_f32(
                      qkv_sl.as<float>(), s_qkv, ss_attn.as<float>(), s_qkv, dim, eps, cos_t.as<float>(),
                      sin_t.as<float>(), posp, kc(l), vc(l), att_part.as<float>(), H, Hk, D,
                      static_cast<std::int64_t>(max_seq), 1.0f, &pf, stream),
                  "attention_decode");
            gemv_src(attn_src, o[l], o_sl.as<float>(), o_max);
            gemv_src(normres(hb, o_sl.as<float>(), s_o, ffn_norm[l]->data, ha, ss_ffn.as<float>()), gate_up[l],
                     gu_sl.as<float>(), gu_max);
            vm_hip_gemv_src sw{};
            sw.kind = VM_HIP_GEMV_SRC_SWIGLU;
            sw.act = gu_sl.as<float>();
            sw.slices = s_gu;
            sw.ss_in = ss_ffn.as<float>();
            sw.ss_count = s_gu;
            sw.ss_dim = dim;
            sw.eps = eps;
            gemv_src(sw, down[l], down_sl.as<float>(), down_max);
        }
        gemv_src(normres(ha, down_sl.as<float>(), s_down, final_norm->data, nullptr, ss_final.as<float>()), lm_head,
                 lm_sl.as<float>(), lm_max);
    }

    // One decode step as a single launch; logits (when given) instead of
    // the greedy token.
    void persistent_step(float* logits_out) {
        pstep = pstep + 1 >= (1u << 23) ? 1u : pstep + 1;
        check(vm_hip_decode_step(&pmodel, pws.p, static_cast<std::int64_t>(pws.bytes), pstep, logits_out, stream),
              "decode step");
    }

    void persistent_check() {
        int failed = 0;
        check(vm_hip_decode_status(pws.p, &failed, stream), "decode status");
        if (failed) throw std::runtime_error("HipLlamaDecoder: a decode step timed out waiting for a workgroup");
    }

    void setup_persistent();

    // Logits of the last sliced step (the final norm's 1/rms applied).
    void sliced_logits() {
        check(vm_hip_slices_sum_scaled_f32(lm_sl.as<float>(), s_lm, vocab, ss_final.as<float>(), s_lm,
                                           static_cast<float>(hidden), cfg.rms_norm_eps, logits.as<float>(), stream),
              "logits");
    }

    void setup(const Config& config, QuantType quant_type, int block_size, std::size_t max_seq_len);
    void allocate();

    // A packed linear assembled from already packed parts placed side by
    // side (columns of each part in order): quant.cpp packs every column on
    // its own, so this is byte for byte the packing of the concatenated
    // fp32 matrix.
    void assemble(Packed& dst, std::initializer_list<const PackedLinear*> parts) {
        const std::int64_t k = (*parts.begin())->k;
        std::int64_t n = 0;
        for (const auto* p : parts) {
            if (p->k != k) throw std::invalid_argument("HipLlamaDecoder: fused parts differ in K");
            n += p->n;
        }
        const bool int4 = qt == VM_HIP_QUANT_INT4;
        const std::int64_t code_rows = int4 ? (k + 1) / 2 : k;
        const std::int64_t scale_rows = int4 ? (k + block - 1) / block : 1;
        dst.k = k;
        dst.n = n;
        dst.codes = DevBuf(static_cast<std::size_t>(code_rows * n));
        dst.scales = DevBuf(static_cast<std::size_t>(scale_rows * n * 4));
        std::int64_t col = 0;
        for (const auto* p : parts) {
            if (p->codes->size_bytes != static_cast<std::size_t>(code_rows * p->n) ||
                p->scales->size_bytes != static_cast<std::size_t>(scale_rows * p->n * 4))
                throw std::invalid_argument("HipLlamaDecoder: packed part has the wrong size for its quantization");
            check(vm_hip_memcpy_2d_d2d(dst.codes.as<std::uint8_t>() + col, static_cast<std::size_t>(n), p->codes->data,
                                       static_cast<std::size_t>(p->n), static_cast<std::size_t>(p->n),
                                       static_cast<std::size_t>(code_rows), stream),
                  "assemble codes");
            check(vm_hip_memcpy_2d_d2d(dst.scales.as<float>() + col, static_cast<std::size_t>(n * 4), p->scales->data,
                                       static_cast<std::size_t>(p->n * 4), static_cast<std::size_t>(p->n * 4),
                                       static_cast<std::size_t>(scale_rows), stream),
                  "assemble scales");
            col += p->n;
        }
    }

    void qmm(const float* a, const Packed& w, float* c, std::int64_t rows) {
        check(vm_hip_qmm_f32(a, static_cast<const std::int8_t*>(w.codes.p), w.scales.as<float>(), c, rows, w.k, w.n,
                             qt, qt == VM_HIP_QUANT_INT4 ? block : 0, stream),
              "quantized matmul");
    }

    // ---- prompts: activations staged for the GEMM by their producer
    // (vm_hip_qmm_a_layout), instead of a pre-pass inside every GEMM call.
    // VELOMIND_STAGE_A=0 keeps the fp32 hand-over (comparisons).
    bool stage_a = true;
    DevBuf a_stage;

    void prepare_staging() {
        const char* env = std::getenv("VELOMIND_STAGE_A");
        stage_a = !(env && env[0] == '0');
    }

    // The layout the GEMM of `w` takes its `rows`-row activations in
    // (VM_HIP_A_FP32 when staging is off or does not apply).
    int stage_layout(const Packed& w, std::int64_t rows) {
        int lay = VM_HIP_A_FP32;
        std::int64_t bytes = 0;
        if (!stage_a || rows <= 4) return lay;
        check(vm_hip_qmm_a_layout(rows, w.k, w.n, qt, block_arg(), &lay, &bytes), "activation layout");
        if (lay != VM_HIP_A_FP32 && a_stage.bytes < static_cast<std::size_t>(bytes)) {
            check(vm_hip_stream_synchronize(stream), "staging buffer");
            a_stage = DevBuf(static_cast<std::size_t>(bytes));
        }
        return lay;
    }

    void qmm_staged(const Packed& w, float* c, std::int64_t rows) {
        check(vm_hip_qmm_staged_f32(a_stage.p, static_cast<const std::int8_t*>(w.codes.p), w.scales.as<float>(), c,
                                    rows, w.k, w.n, qt, block_arg(), stream),
              "quantized matmul (staged activations)");
    }

    // h += delta, RMSNorm with weight nw, then the projection `w` of it.
    void norm_qmm(float* hp, const float* delta, const float* nw, const Packed& w, float* out, std::int64_t rows) {
        const float eps = cfg.rms_norm_eps;
        const int lay = stage_layout(w, rows);
        if (lay == VM_HIP_A_FP32) {
            check(vm_hip_add_rmsnorm_f32(hp, delta, nw, hn.as<float>(), rows, hidden, eps, stream), "add_rmsnorm");
            qmm(hn.as<float>(), w, out, rows);
            return;
        }
        check(vm_hip_add_rmsnorm_stage_f32(hp, delta, nw, a_stage.p, lay, nullptr, rows, hidden, eps, stream),
              "add_rmsnorm (staged)");
        qmm_staged(w, out, rows);
    }

    // SiLU(gate) * up of the gate|up output, then the down projection.
    void silu_qmm(const float* gate_up_out, const Packed& w, float* out, std::int64_t rows) {
        const int lay = stage_layout(w, rows);
        if (lay == VM_HIP_A_FP32) {
            check(vm_hip_silu_mul_f32(gate_up_out, act.as<float>(), rows, inter, stream), "silu_mul");
            qmm(act.as<float>(), w, out, rows);
            return;
        }
        check(vm_hip_silu_mul_stage_f32(gate_up_out, a_stage.p, lay, nullptr, rows, inter, stream),
              "silu_mul (staged)");
        qmm_staged(w, out, rows);
    }

    // Layers over `rows` tokens whose first position is *pos; leaves the
    // last row's logits in `logits`.
    void forward(std::int64_t rows) {
        const float eps = cfg.rms_norm_eps;
        float* hp = h.as<float>();
        float* hnp = hn.as<float>();
        const auto* posp = pos.as<std::int32_t>();
        check(vm_hip_embedding_f32(static_cast<const float*>(embed->data), vocab, hidden,
                                   rows == 1 ? token.as<std::int32_t>() : idx.as<std::int32_t>(), rows, hp, stream),
              "embedding");
        for (std::size_t l = 0; l < cfg.num_layers; ++l) {
            norm_qmm(hp, l == 0 ? nullptr : down_out.as<float>(), static_cast<const float*>(attn_norm[l]->data),
                     qkv[l], qkv_out.as<float>(), rows);
            check(vm_hip_rope_kv_append_f32(qkv_out.as<float>(), rows, cos_t.as<float>(), sin_t.as<float>(), posp,
                                            q.as<float>(), kc(l), vc(l), H, Hk, D,
                                            static_cast<std::int64_t>(max_seq), stream),
                  "rope_kv_append");
            if (rows == 1)
                check(vm_hip_attention_decode_f32(q.as<float>(), kc(l), vc(l), posp, ctx.as<float>(), H, Hk, D,
                                                  static_cast<std::int64_t>(max_seq), 1.0f, stream),
                      "attention_decode");
            else
                check(vm_hip_attention_prefill_f32(q.as<float>(), kc(l), vc(l), posp, ctx.as<float>(), rows, H, Hk, D,
                                                   static_cast<std::int64_t>(max_seq), 1.0f, stream),
                      "attention_prefill");
            qmm(ctx.as<float>(), o[l], attn_out.as<float>(), rows);
            norm_qmm(hp, attn_out.as<float>(), static_cast<const float*>(ffn_norm[l]->data), gate_up[l],
                     gu.as<float>(), rows);
            silu_qmm(gu.as<float>(), down[l], down_out.as<float>(), rows);
        }
        // Only the last row reaches the head (slice_last_token, llama_graph.cpp:141-158).
        const std::int64_t last = (rows - 1) * hidden;
        check(vm_hip_add_rmsnorm_f32(hp + last, down_out.as<float>() + last,
                                     static_cast<const float*>(final_norm->data), hnp, 1, hidden, eps, stream),
              "add_rmsnorm");
        qmm(hnp, lm_head, logits.as<float>(), 1);
    }

    void set_pos(std::int64_t p) {
        const std::int32_t v = static_cast<std::int32_t>(p);
        check(vm_hip_memcpy_h2d(pos.p, &v, 4, stream), "position upload");
    }
};

void HipLlamaDecoder::Impl::setup(const Config& config, QuantType quant_type, int block_size, std::size_t max_seq_len) {
    auto& m = *this;
    m.cfg = config;
    const Config& c = m.cfg;
    if (const char* e = std::getenv("VELOMIND_DECODE_PREFETCH")) m.prefetch = std::string(e) != "0";
    if (quant_type == QuantType::None) throw std::invalid_argument("HipLlamaDecoder: weights must be quantized");
    m.qt = quant_type == QuantType::Int4 ? VM_HIP_QUANT_INT4 : VM_HIP_QUANT_INT8;
    if (m.qt == VM_HIP_QUANT_INT8 && block_size > 0)
        throw std::invalid_argument("HipLlamaDecoder: INT8 weights are packed per column (block_size 0)");
    m.block = m.qt == VM_HIP_QUANT_INT4 ? (block_size > 0 ? block_size : 32) : 0;
    if (m.qt == VM_HIP_QUANT_INT4 && m.block % 2) throw std::invalid_argument("HipLlamaDecoder: INT4 block must be even");
    m.H = static_cast<std::int64_t>(c.num_heads);
    m.Hk = static_cast<std::int64_t>(c.effective_num_kv_heads());
    m.D = static_cast<std::int64_t>(c.head_dim());
    m.hidden = static_cast<std::int64_t>(c.hidden_size);
    m.inter = static_cast<std::int64_t>(c.intermediate_size);
    m.vocab = static_cast<std::int64_t>(c.vocab_size);
    m.qkv_n = (m.H + 2 * m.Hk) * m.D;
    m.max_seq = max_seq_len;
    if (max_seq_len == 0 || max_seq_len > (1u << 20)) throw std::invalid_argument("HipLlamaDecoder: max_seq out of range");
    if (m.D != 64 && m.D != 128) throw std::invalid_argument("HipLlamaDecoder: head_dim must be 64 or 128");
    if (m.H / m.Hk > 16) throw std::invalid_argument("HipLlamaDecoder: at most 16 query heads per KV head");
    check(vm_hip_stream_create(&m.stream), "stream");
    check(vm_hip_event_create(&m.ev0), "event");
    check(vm_hip_event_create(&m.ev1), "event");
}

void HipLlamaDecoder::Impl::allocate() {
    auto& m = *this;
    const Config& c = m.cfg;
    const std::size_t max_seq = m.max_seq;
    const std::size_t kv = c.num_layers * m.Hk * max_seq * m.D * 4;
    m.kcache = DevBuf(kv);
    m.vcache = DevBuf(kv);
    std::vector<float> cs, sn;
    compute_rope_cache(max_seq, c.head_dim(), c.rope_theta, cs, sn, 0);
    m.cos_t = DevBuf(cs.size() * 4);
    m.sin_t = DevBuf(sn.size() * 4);
    check(vm_hip_memcpy_h2d(m.cos_t.p, cs.data(), cs.size() * 4, m.stream), "rope tables");
    check(vm_hip_memcpy_h2d(m.sin_t.p, sn.data(), sn.size() * 4, m.stream), "rope tables");

    const std::size_t rows = max_seq;
    m.h = DevBuf(rows * m.hidden * 4);
    m.hn = DevBuf(rows * m.hidden * 4);
    m.qkv_out = DevBuf(rows * m.qkv_n * 4);
    m.q = DevBuf(rows * m.H * m.D * 4);
    m.ctx = DevBuf(rows * m.hidden * 4);
    m.attn_out = DevBuf(rows * m.hidden * 4);
    m.gu = DevBuf(rows * 2 * m.inter * 4);
    m.act = DevBuf(rows * m.inter * 4);
    m.down_out = DevBuf(rows * m.hidden * 4);
    m.logits = DevBuf(m.vocab * 4);
    m.idx = DevBuf(rows * 4);
    m.token = DevBuf(4);
    m.pos = DevBuf(4);
    m.tokens = DevBuf(rows * 4);
    if (const char* e = std::getenv("VELOMIND_SLICES_MAX")) {
        int v[5] = {m.qkv_max, m.o_max, m.gu_max, m.down_max, m.lm_max};
        if (std::sscanf(e, "%d,%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4]) == 5 &&
            std::all_of(v, v + 5, [](int x) { return x >= 1 && x <= 64; })) {
            m.qkv_max = v[0];
            m.o_max = v[1];
            m.gu_max = v[2];
            m.down_max = v[3];
            m.lm_max = v[4];
        }
    }
    m.s_qkv = m.slices_for(m.qkv[0], m.qkv_max);
    m.s_o = m.slices_for(m.o[0], m.o_max);
    m.s_gu = m.slices_for(m.gate_up[0], m.gu_max);
    // down: twice the slices (four-wave workgroups instead of eight) while
    // the grid stays within one workgroup per CU (SmolLM2-360M, N = 960: 80
    // -> 160 workgroups, decode 891.7 -> 850.2 us/token; TinyLlama's 176
    // would become 352 and slow down, 687.8 -> 699.6).
    if (!std::getenv("VELOMIND_SLICES_MAX")) {
        const int wide = m.slices_for(m.down[0], 2 * m.down_max);
        if (wide > 0 && static_cast<std::int64_t>(wide) * ((m.down[0].n + 255) / 256) <= 256) m.down_max *= 2;
    }
    m.s_down = m.slices_for(m.down[0], m.down_max);
    m.s_lm = m.slices_for(m.lm_head, m.lm_max);
    m.sliced = m.s_qkv && m.s_o && m.s_gu && m.s_down && m.s_lm && m.hidden % 4 == 0 && m.inter % 4 == 0 &&
               m.H * m.D == m.hidden &&
               vm_hip_attention_decode_chunks(m.D, static_cast<std::int64_t>(max_seq), &m.att_chunk, &m.att_chunks) ==
                   VM_HIP_OK;
    if (m.sliced) {
        m.h2 = DevBuf(static_cast<std::size_t>(m.hidden * 4));
        m.ss_attn = DevBuf(static_cast<std::size_t>(m.s_qkv * 4));
        m.ss_ffn = DevBuf(static_cast<std::size_t>(m.s_gu * 4));
        m.ss_final = DevBuf(static_cast<std::size_t>(m.s_lm * 4));
        m.att_part = DevBuf(static_cast<std::size_t>(m.H * m.att_chunks * (m.D + 4) * 4));
        // the multi-workgroup argmax's ticket and candidates (zeroed once)
        m.am_ws = DevBuf(static_cast<std::size_t>(vm_hip_argmax_workspace_bytes(m.vocab)));
        const std::vector<unsigned char> zeros(m.am_ws.bytes, 0);
        check(vm_hip_memcpy_h2d(m.am_ws.p, zeros.data(), zeros.size(), m.stream), "argmax workspace");
        m.qkv_sl = DevBuf(static_cast<std::size_t>(m.s_qkv * m.qkv_n * 4));
        m.o_sl = DevBuf(static_cast<std::size_t>(m.s_o * m.hidden * 4));
        m.gu_sl = DevBuf(static_cast<std::size_t>(m.s_gu * 2 * m.inter * 4));
        m.down_sl = DevBuf(static_cast<std::size_t>(m.s_down * m.hidden * 4));
        m.lm_sl = DevBuf(static_cast<std::size_t>(m.s_lm * m.vocab * 4));
    }
    check(vm_hip_stream_synchronize(m.stream), "setup");
}

void HipLlamaDecoder::Impl::setup_persistent() {
    auto& m = *this;
    const char* env = std::getenv("VELOMIND_DECODE_PERSISTENT");
    if (!env || env[0] != '1') return;
    vm_hip_decode_model& d = m.pmodel;
    d.layers = static_cast<std::int64_t>(m.cfg.num_layers);
    d.hidden = m.hidden;
    d.inter = m.inter;
    d.heads = m.H;
    d.kv_heads = m.Hk;
    d.head_dim = m.D;
    d.vocab = m.vocab;
    d.max_seq = static_cast<std::int64_t>(m.max_seq);
    d.quant_type = m.qt;
    d.block_size = m.block_arg();
    d.eps = m.cfg.rms_norm_eps;
    std::int64_t bytes = 0;
    if (vm_hip_decode_workspace_bytes(&d, &bytes) != VM_HIP_OK) return;   // shape outside the kernel: per-launch path
    std::vector<vm_hip_decode_layer> table(m.cfg.num_layers);
    for (std::size_t l = 0; l < m.cfg.num_layers; ++l) {
        auto& t = table[l];
        t.qkv_codes = m.qkv[l].codes.as<std::int8_t>();
        t.qkv_scales = m.qkv[l].scales.as<float>();
        t.o_codes = m.o[l].codes.as<std::int8_t>();
        t.o_scales = m.o[l].scales.as<float>();
        t.gate_up_codes = m.gate_up[l].codes.as<std::int8_t>();
        t.gate_up_scales = m.gate_up[l].scales.as<float>();
        t.down_codes = m.down[l].codes.as<std::int8_t>();
        t.down_scales = m.down[l].scales.as<float>();
        t.attn_norm = static_cast<const float*>(m.attn_norm[l]->data);
        t.ffn_norm = static_cast<const float*>(m.ffn_norm[l]->data);
    }
    m.player = DevBuf(table.size() * sizeof(vm_hip_decode_layer));
    check(vm_hip_memcpy_h2d(m.player.p, table.data(), m.player.bytes, m.stream), "decode layer table");
    m.pws = DevBuf(static_cast<std::size_t>(bytes));
    const std::vector<unsigned char> zeros(m.pws.bytes, 0);
    check(vm_hip_memcpy_h2d(m.pws.p, zeros.data(), zeros.size(), m.stream), "decode workspace");
    d.layer = m.player.as<vm_hip_decode_layer>();
    d.embed = static_cast<const float*>(m.embed->data);
    d.final_norm = static_cast<const float*>(m.final_norm->data);
    d.lm_codes = m.lm_head.codes.as<std::int8_t>();
    d.lm_scales = m.lm_head.scales.as<float>();
    d.cos_table = m.cos_t.as<float>();
    d.sin_table = m.sin_t.as<float>();
    d.k_cache = m.kcache.as<float>();
    d.v_cache = m.vcache.as<float>();
    d.token = m.token.as<std::int32_t>();
    d.pos = m.pos.as<std::int32_t>();
    d.tokens = m.tokens.as<std::int32_t>();
    m.persistent = true;
}

HipLlamaDecoder::HipLlamaDecoder(const LlamaWeightSet& weights, QuantType quant_type, int block_size,
                                 std::size_t max_seq)
    : _impl(std::make_unique<Impl>()), _max_seq(max_seq) {
    auto& m = *_impl;
    m.setup(weights.config(), quant_type, block_size, max_seq);
    const Config& c = m.cfg;
    using W = LlamaWeight;
    m.embed = weights.storage(W::Embed);
    m.final_norm = weights.storage(W::FinalNorm);
    m.qkv.resize(c.num_layers);
    m.o.resize(c.num_layers);
    m.gate_up.resize(c.num_layers);
    m.down.resize(c.num_layers);
    for (std::size_t l = 0; l < c.num_layers; ++l) {
        m.attn_norm.push_back(weights.storage(W::AttnNorm, l));
        m.ffn_norm.push_back(weights.storage(W::FfnNorm, l));
        m.pack_fused(m.qkv[l], {weights.storage(W::Wq, l), weights.storage(W::Wk, l), weights.storage(W::Wv, l)},
                     m.hidden);
        m.pack(m.o[l], static_cast<const float*>(weights.storage(W::Wo, l)->data), m.hidden, m.hidden);
        m.pack_fused(m.gate_up[l], {weights.storage(W::Gate, l), weights.storage(W::Up, l)}, m.hidden);
        m.pack(m.down[l], static_cast<const float*>(weights.storage(W::Down, l)->data), m.inter, m.hidden);
    }
    m.pack(m.lm_head, static_cast<const float*>(weights.storage(W::LmHead)->data), m.hidden, m.vocab);

    m.allocate();
    m.prepare_staging();
    m.setup_persistent();
}

HipLlamaDecoder::HipLlamaDecoder(const PackedLlamaWeights& packed, std::size_t max_seq)
    : _impl(std::make_unique<Impl>()), _max_seq(max_seq) {
    auto& m = *_impl;
    m.setup(packed.config(), packed.quant_type(), packed.block_size(), max_seq);
    const Config& c = m.cfg;
    using W = LlamaWeight;
    m.embed = packed.dense(W::Embed);
    m.final_norm = packed.dense(W::FinalNorm);
    m.qkv.resize(c.num_layers);
    m.o.resize(c.num_layers);
    m.gate_up.resize(c.num_layers);
    m.down.resize(c.num_layers);
    for (std::size_t l = 0; l < c.num_layers; ++l) {
        m.attn_norm.push_back(packed.dense(W::AttnNorm, l));
        m.ffn_norm.push_back(packed.dense(W::FfnNorm, l));
        m.assemble(m.qkv[l], {&packed.linear(W::Wq, l), &packed.linear(W::Wk, l), &packed.linear(W::Wv, l)});
        m.assemble(m.o[l], {&packed.linear(W::Wo, l)});
        m.assemble(m.gate_up[l], {&packed.linear(W::Gate, l), &packed.linear(W::Up, l)});
        m.assemble(m.down[l], {&packed.linear(W::Down, l)});
    }
    m.assemble(m.lm_head, {&packed.linear(W::LmHead)});
    check(vm_hip_stream_synchronize(m.stream), "assemble");
    m.allocate();
    m.prepare_staging();
    m.setup_persistent();
}

HipLlamaDecoder::~HipLlamaDecoder() {
    if (!_impl) return;
    auto& m = *_impl;
    if (m.stream) (void)vm_hip_stream_synchronize(m.stream);
    if (m.graph) (void)vm_hip_graph_destroy(m.graph);
    if (m.ev0) (void)vm_hip_event_destroy(m.ev0);
    if (m.ev1) (void)vm_hip_event_destroy(m.ev1);
    // Buffers are freed by their destructors after the stream is idle.
    void* s = m.stream;
    _impl.reset();
    if (s) (void)vm_hip_stream_destroy(s);
}

auto HipLlamaDecoder::logits() const -> std::vector<float> {
    auto& m = *_impl;
    std::vector<float> out(static_cast<std::size_t>(m.vocab));
    check(vm_hip_memcpy_d2h(out.data(), m.logits.p, out.size() * 4, m.stream), "logits download");
    return out;
}

auto HipLlamaDecoder::decode_path() const noexcept -> DecodePath {
    if (_impl->persistent) return DecodePath::Persistent;
    return _impl->sliced ? DecodePath::Slices : DecodePath::PerOperation;
}

auto HipLlamaDecoder::prefill(std::span<const std::int32_t> tokens) -> std::vector<float> {
    auto& m = *_impl;
    if (tokens.empty() || tokens.size() > _max_seq)
        throw std::invalid_argument("HipLlamaDecoder::prefill: prompt length must be in [1, max_seq]");
    check(vm_hip_memcpy_h2d(m.idx.p, tokens.data(), tokens.size_bytes(), m.stream), "token upload");
    check(vm_hip_memcpy_h2d(m.tokens.p, tokens.data(), tokens.size_bytes(), m.stream), "token upload");
    if (tokens.size() == 1) check(vm_hip_memcpy_h2d(m.token.p, tokens.data(), 4, m.stream), "token upload");
    m.set_pos(0);
    m.forward(static_cast<std::int64_t>(tokens.size()));
    m.seq = tokens.size();
    m.set_pos(static_cast<std::int64_t>(m.seq) - 1);  // position of the last processed token
    return logits();
}

auto HipLlamaDecoder::forward_step(std::int32_t token, std::size_t pos) -> std::vector<float> {
    auto& m = *_impl;
    if (pos > m.seq || pos >= _max_seq) throw std::invalid_argument("HipLlamaDecoder::forward_step: bad position");
    check(vm_hip_memcpy_h2d(m.token.p, &token, 4, m.stream), "token upload");
    m.set_pos(static_cast<std::int64_t>(pos));
    if (m.persistent) {
        m.persistent_step(m.logits.as<float>());
        m.persistent_check();
    } else if (m.sliced) {
        m.forward_one_sliced();
        m.sliced_logits();
    } else {
        m.forward(1);
    }
    m.seq = pos + 1;
    return logits();
}

auto HipLlamaDecoder::generate(std::span<const std::int32_t> prompt, std::size_t steps, bool use_graph)
    -> std::vector<std::int32_t> {
    auto& m = *_impl;
    if (prompt.empty() || prompt.size() + steps + 1 > _max_seq)
        throw std::invalid_argument("HipLlamaDecoder::generate: prompt + steps + 1 must fit in max_seq");
    check(vm_hip_event_record(m.ev0, m.stream), "event");
    check(vm_hip_memcpy_h2d(m.idx.p, prompt.data(), prompt.size_bytes(), m.stream), "token upload");
    check(vm_hip_memcpy_h2d(m.tokens.p, prompt.data(), prompt.size_bytes(), m.stream), "token upload");
    if (prompt.size() == 1) check(vm_hip_memcpy_h2d(m.token.p, prompt.data(), 4, m.stream), "token upload");
    m.set_pos(0);
    m.forward(static_cast<std::int64_t>(prompt.size()));
    m.set_pos(static_cast<std::int64_t>(prompt.size()) - 1);
    // First generated token from the prompt's logits; *pos becomes its position.
    auto* tok = m.token.as<std::int32_t>();
    auto* posp = m.pos.as<std::int32_t>();
    auto* seqp = m.tokens.as<std::int32_t>();
    const auto ms = static_cast<std::int64_t>(_max_seq);
    check(vm_hip_argmax_f32(m.logits.as<float>(), m.vocab, tok, posp, seqp, ms, m.stream), "argmax");
    check(vm_hip_event_record(m.ev1, m.stream), "event");
    check(vm_hip_event_synchronize(m.ev1), "prefill");
    float ms_prefill = 0.0f;
    check(vm_hip_event_elapsed_ms(&ms_prefill, m.ev0, m.ev1), "event");
    _prefill_s = ms_prefill * 1e-3;

    auto step = [&] {
        if (m.persistent) {
            m.persistent_step(nullptr);
        } else if (m.sliced) {
            m.forward_one_sliced();
            check(vm_hip_argmax_slices_ws_f32(m.lm_sl.as<float>(), m.s_lm, m.vocab, tok, posp, seqp, ms, m.am_ws.p,
                                              static_cast<std::int64_t>(m.am_ws.bytes), m.stream),
                  "argmax");
        } else {
            m.forward(1);
            check(vm_hip_argmax_f32(m.logits.as<float>(), m.vocab, tok, posp, seqp, ms, m.stream), "argmax");
        }
    };
    std::size_t done = 0;
    _decode_steps_timed = 0;
    // A persistent step is one cooperative launch per token (not captured).
    if (steps > 0 && use_graph && !m.persistent) {
        // The first step runs eagerly: it sizes the per-stream split-K
        // workspaces (the prefill above may have regrown them), then the
        // step is captured against those buffers and replayed.  The graph is
        // captured again on every call, so it never holds a buffer that a
        // later prefill has reallocated.
        step();
        done = 1;
        if (m.graph) {
            check(vm_hip_graph_destroy(m.graph), "graph destroy");
            m.graph = nullptr;
        }
        if (steps > 1) {
            check(vm_hip_stream_begin_capture(m.stream), "graph capture");
            try {
                step();
            } catch (...) {
                void* g = nullptr;
                (void)vm_hip_stream_end_capture(m.stream, &g);
                if (g) (void)vm_hip_graph_destroy(g);
                throw;
            }
            check(vm_hip_stream_end_capture(m.stream, &m.graph), "graph capture");
        }
    }
    check(vm_hip_event_record(m.ev0, m.stream), "event");
    _decode_steps_timed = steps - done;
    if (m.graph && use_graph)
        for (; done < steps; ++done) check(vm_hip_graph_launch(m.graph, m.stream), "graph launch");
    else
        for (; done < steps; ++done) step();
    check(vm_hip_event_record(m.ev1, m.stream), "event");
    check(vm_hip_event_synchronize(m.ev1), "decode");
    if (m.persistent) m.persistent_check();
    float ms_decode = 0.0f;
    check(vm_hip_event_elapsed_ms(&ms_decode, m.ev0, m.ev1), "event");
    _decode_s = ms_decode * 1e-3;
    m.seq = prompt.size() + steps;

    std::vector<std::int32_t> out(steps + 1);
    check(vm_hip_memcpy_d2h(out.data(), seqp + prompt.size(), out.size() * 4, m.stream), "token download");
    return out;
}

}  // namespace velomind::examples::llama
