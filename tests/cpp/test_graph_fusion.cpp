// The graph compiler's fused chains (graph_compiler.cpp fuse_steps), checked
// on the CPU: host kernels for the chain's operators and host fused kernels
// that keep the same arithmetic order are registered for DeviceType::CPU in
// this binary, so the pass itself -- which chains it takes, what it leaves
// unallocated, what it refuses -- is exercised without a GPU.  The HIP
// fused kernels are checked against the unfused chains on the GPU
// (tests/test_hip_graph_fusion.py).
#include <cmath>
#include <cstring>
#include <memory>
#include <variant>

#include "internal/registry/kernel.h"
#include "test_helpers.h"

using namespace velomind;
using namespace vmtest;

namespace {

const float* cin(const pConstTensorStorage* in, int i) { return static_cast<const float*>(in[i]->data); }
float* cout0(const pTensorStorage* out) { return static_cast<float*>(out[0]->data); }
std::size_t numel(const TensorStorage& t) { return storage_numel(t); }

float sigmoid_host(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// element e (row-major order of its shape) of an operand that may be strided
float elem(const TensorStorage& t, std::size_t e) {
    const auto st = t.effective_strides();
    std::size_t off = 0;
    for (std::size_t d = t.shape.size(); d-- > 0;) {
        const auto extent = static_cast<std::size_t>(t.shape[d]);
        off += (e % extent) * static_cast<std::size_t>(st[d]);
        e /= extent;
    }
    return static_cast<const float*>(t.data)[off];
}

void add_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    for (std::size_t e = 0; e < numel(*out[0]); ++e) cout0(out)[e] = elem(*in[0], e) + elem(*in[1], e);
}
void mul_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    for (std::size_t e = 0; e < numel(*out[0]); ++e) cout0(out)[e] = cin(in, 0)[e] * cin(in, 1)[e];
}
void sigmoid_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    for (std::size_t e = 0; e < numel(*out[0]); ++e) cout0(out)[e] = sigmoid_host(cin(in, 0)[e]);
}
// [B, M, K] x [B, K, N], each output an fma chain over k from 0.
void matmul_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const auto& a = in[0]->shape;
    const auto& c = out[0]->shape;
    const std::size_t b = static_cast<std::size_t>(c[0]), m = static_cast<std::size_t>(a[1]),
                      k = static_cast<std::size_t>(a[2]), n = static_cast<std::size_t>(c[2]);
    for (std::size_t z = 0; z < b; ++z)
        for (std::size_t i = 0; i < m; ++i)
            for (std::size_t j = 0; j < n; ++j) {
                float acc = 0.0f;
                for (std::size_t t = 0; t < k; ++t)
                    acc = std::fma(cin(in, 0)[(z * m + i) * k + t], cin(in, 1)[(z * k + t) * n + j], acc);
                cout0(out)[(z * m + i) * n + j] = acc;
            }
}
// last axis
void softmax_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const std::size_t cols = static_cast<std::size_t>(in[0]->shape.back());
    const std::size_t rows = numel(*in[0]) / cols;
    for (std::size_t r = 0; r < rows; ++r) {
        const float* x = cin(in, 0) + r * cols;
        float mx = -INFINITY, sum = 0.0f;
        for (std::size_t j = 0; j < cols; ++j) mx = std::fmax(mx, x[j]);
        for (std::size_t j = 0; j < cols; ++j) sum += std::exp(x[j] - mx);
        for (std::size_t j = 0; j < cols; ++j) cout0(out)[r * cols + j] = std::exp(x[j] - mx) / sum;
    }
}
// [A, B, C] -> [A, C, B] (the only permutation these tests use)
void transpose_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const auto& s = in[0]->shape;
    for (dim_t a = 0; a < s[0]; ++a)
        for (dim_t b = 0; b < s[1]; ++b)
            for (dim_t c = 0; c < s[2]; ++c) cout0(out)[(a * s[2] + c) * s[1] + b] = cin(in, 0)[(a * s[1] + b) * s[2] + c];
}
// axis 0: head h of the output is head h / repeats of the input
void repeat_kv_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const int r = std::get<RepeatKVAttrs>(static_cast<const OpDescriptor*>(attrs)->attrs).repeats;
    const auto& s = in[0]->shape;
    const std::size_t inner = static_cast<std::size_t>(s[1] * s[2]);
    for (std::size_t h = 0; h < static_cast<std::size_t>(s[0]) * r; ++h)
        std::memcpy(cout0(out) + h * inner, cin(in, 0) + (h / r) * inner, inner * 4);
}

// RoPE over rows of the last axis with one cos/sin row
void rope_rotate(float a, float b, float c, float s, float* y0, float* y1) {
    *y0 = a * c - b * s;
    *y1 = b * c + a * s;
}
void rope_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const std::size_t d = static_cast<std::size_t>(in[0]->shape.back()), half = d / 2, rows = numel(*in[0]) / d;
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t j = 0; j < half; ++j)
            rope_rotate(cin(in, 0)[r * d + j], cin(in, 0)[r * d + j + half], cin(in, 1)[j], cin(in, 2)[j],
                        cout0(out) + r * d + j, cout0(out) + r * d + j + half);
}
// axis 1 of rank-3 tensors
void concat_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const auto& a = in[0]->shape;
    const std::size_t ab = static_cast<std::size_t>(a[1] * a[2]), bb = numel(*in[1]) / static_cast<std::size_t>(a[0]);
    for (std::size_t o = 0; o < static_cast<std::size_t>(a[0]); ++o) {
        std::memcpy(cout0(out) + o * (ab + bb), cin(in, 0) + o * ab, ab * 4);
        std::memcpy(cout0(out) + o * (ab + bb) + ab, cin(in, 1) + o * bb, bb * 4);
    }
}

// RMSNorm over the last axis
void rmsnorm_rows(const float* x, const float* w, float* y, std::size_t rows, std::size_t d, float eps) {
    for (std::size_t r = 0; r < rows; ++r) {
        float ss = 0.0f;
        for (std::size_t i = 0; i < d; ++i) ss = std::fma(x[r * d + i], x[r * d + i], ss);
        const float inv = 1.0f / std::sqrt(ss / static_cast<float>(d) + eps);
        for (std::size_t i = 0; i < d; ++i) y[r * d + i] = (x[r * d + i] * inv) * w[i];
    }
}
void rmsnorm_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const float eps = std::get<RMSNormAttrs>(static_cast<const OpDescriptor*>(attrs)->attrs).epsilon;
    const std::size_t d = static_cast<std::size_t>(in[0]->shape.back());
    rmsnorm_rows(cin(in, 0), cin(in, 1), cout0(out), numel(*in[0]) / d, d, eps);
}

// fused: the same operations in the same order as the chains above
void silu_mul_fused_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    for (std::size_t e = 0; e < numel(*out[0]); ++e) {
        const float g = cin(in, 0)[e];
        cout0(out)[e] = (sigmoid_host(g) * g) * cin(in, 1)[e];
    }
}
void qmm_add_fused_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto& qa = std::get<QuantizedMatMulAttrs>(static_cast<const OpDescriptor*>(attrs)->attrs);
    const std::size_t k = static_cast<std::size_t>(in[0]->shape.back()), n = static_cast<std::size_t>(in[1]->shape[1]);
    const std::size_t rows = numel(*out[0]) / n;
    vmo_qmm_2d_f32(cin(in, 0), static_cast<const std::int8_t*>(in[1]->data), cin(in, 2), cout0(out), rows, k, n,
                   static_cast<int>(qa.quant_type), qa.block_size);
    for (std::size_t e = 0; e < rows * n; ++e) cout0(out)[e] = cin(in, 3)[e] + cout0(out)[e];
}
void attention_decode_fused_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const auto& q = in[0]->shape;
    const auto& k = in[1]->shape;
    const std::size_t H = q[0], D = q[2], Hkv = k[0], S = k[1], Dv = in[2]->shape[2];
    std::vector<float> p(S);
    for (std::size_t h = 0; h < H; ++h) {
        const std::size_t kv = h / (H / Hkv);
        float mx = -INFINITY, sum = 0.0f;
        for (std::size_t s = 0; s < S; ++s) {
            float acc = 0.0f;
            for (std::size_t t = 0; t < D; ++t) acc = std::fma(cin(in, 0)[h * D + t], cin(in, 1)[(kv * S + s) * D + t], acc);
            p[s] = acc;
        }
        for (std::size_t s = 0; s < S; ++s) mx = std::fmax(mx, p[s]);
        for (std::size_t s = 0; s < S; ++s) sum += std::exp(p[s] - mx);
        for (std::size_t s = 0; s < S; ++s) p[s] = std::exp(p[s] - mx) / sum;
        for (std::size_t t = 0; t < Dv; ++t) {
            float acc = 0.0f;
            for (std::size_t s = 0; s < S; ++s) acc = std::fma(p[s], cin(in, 2)[(kv * S + s) * Dv + t], acc);
            cout0(out)[h * Dv + t] = acc;
        }
    }
}

// inputs [q, k, v, K_past, V_past, cos, sin], outputs [q', K, V]
void rope_append_fused_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const pConstTensorStorage rq[3] = {in[0], in[5], in[6]};
    const pConstTensorStorage rk[3] = {in[1], in[5], in[6]};
    rope_cpu(rq, out, nullptr);
    std::vector<float> kr(numel(*in[1]));
    TensorStorage tmp = *in[1];
    tmp.data = kr.data();
    const pTensorStorage ko[1] = {&tmp};
    rope_cpu(rk, ko, nullptr);
    const pConstTensorStorage ck[2] = {in[3], &tmp};
    const pConstTensorStorage cv[2] = {in[4], in[2]};
    concat_cpu(ck, out + 1, nullptr);
    concat_cpu(cv, out + 2, nullptr);
}

// inputs [g, u, B, S, h], outputs [C]
void swiglu_qmm_add_fused_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto& qa = std::get<QuantizedMatMulAttrs>(static_cast<const OpDescriptor*>(attrs)->attrs);
    const std::size_t k = static_cast<std::size_t>(in[0]->shape.back()), n = static_cast<std::size_t>(in[2]->shape[1]);
    const std::size_t rows = numel(*in[0]) / k;
    std::vector<float> act(rows * k);
    for (std::size_t e = 0; e < act.size(); ++e) act[e] = (sigmoid_host(cin(in, 0)[e]) * cin(in, 0)[e]) * cin(in, 1)[e];
    vmo_qmm_2d_f32(act.data(), static_cast<const std::int8_t*>(in[2]->data), cin(in, 3), cout0(out), rows, k, n,
                   static_cast<int>(qa.quant_type), qa.block_size);
    for (std::size_t e = 0; e < rows * n; ++e) cout0(out)[e] = cin(in, 4)[e] + cout0(out)[e];
}

// inputs [x, w, B_1, S_1, ..], outputs [C_1, ..]
void norm_qmm_fused_cpu(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto& na = *static_cast<const internal::NormQmmAttrs*>(attrs);
    const auto& qa = std::get<QuantizedMatMulAttrs>(na.desc.attrs);
    const std::size_t k = static_cast<std::size_t>(in[0]->shape.back()), rows = numel(*in[0]) / k;
    std::vector<float> hn(rows * k);
    rmsnorm_rows(cin(in, 0), cin(in, 1), hn.data(), rows, k, na.epsilon);
    for (std::size_t g = 0; g < na.members; ++g)
        vmo_qmm_2d_f32(hn.data(), static_cast<const std::int8_t*>(in[2 + 2 * g]->data), cin(in, 3 + 2 * g),
                       static_cast<float*>(out[g]->data), rows, k, static_cast<std::size_t>(in[2 + 2 * g]->shape[1]),
                       static_cast<int>(qa.quant_type), qa.block_size);
}

constexpr DataType F32 = DataType::Float32;
#define CPU_F32(OP, N, FN) \
    VELOMIND_REGISTER_OP_KERNEL(DeviceType::CPU, OP, (internal::KernelDtypeKey{{F32, F32, F32, F32}, N, F32}), &FN)
CPU_F32(Op::Add, 2, add_cpu)
CPU_F32(Op::Mul, 2, mul_cpu)
CPU_F32(Op::Sigmoid, 1, sigmoid_cpu)
CPU_F32(Op::MatMul, 2, matmul_cpu)
CPU_F32(Op::Softmax, 1, softmax_cpu)
CPU_F32(Op::Transpose, 1, transpose_cpu)
CPU_F32(Op::RepeatKV, 1, repeat_kv_cpu)
CPU_F32(Op::RotaryEmbedding, 3, rope_cpu)
CPU_F32(Op::Concat, 2, concat_cpu)
CPU_F32(Op::RMSNorm, 2, rmsnorm_cpu)
VELOMIND_REGISTER_FUSED(DeviceType::CPU, internal::FusedKind::SiluMul, &silu_mul_fused_cpu)
VELOMIND_REGISTER_FUSED(DeviceType::CPU, internal::FusedKind::QmmAdd, &qmm_add_fused_cpu)
VELOMIND_REGISTER_FUSED(DeviceType::CPU, internal::FusedKind::AttentionDecode, &attention_decode_fused_cpu)
VELOMIND_REGISTER_FUSED(DeviceType::CPU, internal::FusedKind::RopeAppend, &rope_append_fused_cpu)
VELOMIND_REGISTER_FUSED(DeviceType::CPU, internal::FusedKind::NormQmm, &norm_qmm_fused_cpu)
VELOMIND_REGISTER_FUSED(DeviceType::CPU, internal::FusedKind::SwigluQmmAdd, &swiglu_qmm_add_fused_cpu)

struct QmmWeights {
    std::vector<std::int8_t> q;
    std::vector<float> s;
};
QmmWeights int8_weights(std::size_t k, std::size_t n, unsigned seed) {
    const auto w = normal(k * n, seed, 0.05f);
    QmmWeights r{std::vector<std::int8_t>(k * n), std::vector<float>(n)};
    vmo_quantize_int8_per_channel(w.data(), r.q.data(), r.s.data(), k, n);
    return r;
}

// An MLP block with its residual: out = h + down(silu(gate(x)) * up(x)).
struct MlpRun {
    std::vector<float> out;
    std::size_t steps = 0, nodes = 0;
    bool inner_unallocated = false;
};
// strided_h: the residual is every other float of a host buffer (a view
// input, as the reference's strided TensorStorage views are).
MlpRun run_mlp(bool fuse, bool keep_sigmoid, bool keep_act = false, bool strided_h = false) {
    const std::size_t d = 64, f = 96;
    static const auto wg = int8_weights(d, f, 61), wu = int8_weights(d, f, 62), wd = int8_weights(f, d, 63);
    static const auto x = normal(d, 64), h = normal(d, 65);
    ScopedEnv env("VELOMIND_GRAPH_FUSE", fuse ? "1" : "0");
    Graph g;
    std::vector<float> h_pitched(2 * d, -1.0f);
    for (std::size_t j = 0; j < d; ++j) h_pitched[2 * j] = h[j];
    auto h_view = std::make_shared<TensorStorage>();
    h_view->shape = {1, (dim_t)d};
    h_view->strides = {(dim_t)(2 * d), 2};
    h_view->dtype = F32;
    h_view->data = h_pitched.data();
    h_view->size_bytes = d * 4;
    h_view->capacity_bytes = h_pitched.size() * 4;
    auto tx = g.input({1, (dim_t)d}, F32);
    auto th = strided_h ? g.input(h_view) : g.input({1, (dim_t)d}, F32);
    auto tg = g.input({(dim_t)d, (dim_t)f}, DataType::Int8), tgs = g.input({(dim_t)f}, F32);
    auto tu = g.input({(dim_t)d, (dim_t)f}, DataType::Int8), tus = g.input({(dim_t)f}, F32);
    auto td = g.input({(dim_t)f, (dim_t)d}, DataType::Int8), tds = g.input({(dim_t)d}, F32);
    auto gate = g.op(Op::QuantizedMatMul, tx, tg, tgs);
    auto up = g.op(Op::QuantizedMatMul, tx, tu, tus);
    auto sg = g.op(Op::Sigmoid, gate);
    auto t = g.op(Op::Mul, sg, gate);
    auto act = g.op(Op::Mul, t, up);
    auto y = g.op(Op::QuantizedMatMul, act, td, tds);
    auto out = g.op(Op::Add, th, y);
    g.mark_output(out);
    if (keep_sigmoid) g.mark_output(sg);
    if (keep_act) g.mark_output(act);
    auto exec = g.build(DeviceType::CPU);
    MlpRun r;
    r.steps = exec->num_steps();
    r.nodes = exec->num_nodes();
    r.inner_unallocated = g.tensor_storage_at(t.index())->data == nullptr &&
                          g.tensor_storage_at(y.index())->data == nullptr &&
                          (keep_act || g.tensor_storage_at(act.index())->data == nullptr);
    tx.copy_from_host(as_bytes(x));
    if (!strided_h) th.copy_from_host(as_bytes(h));
    tg.copy_from_host(as_bytes(wg.q));
    tgs.copy_from_host(as_bytes(wg.s));
    tu.copy_from_host(as_bytes(wu.q));
    tus.copy_from_host(as_bytes(wu.s));
    td.copy_from_host(as_bytes(wd.q));
    tds.copy_from_host(as_bytes(wd.s));
    exec->execute();
    r.out.resize(d);
    out.copy_to_host(as_writeable_bytes(r.out));
    return r;
}

// Decode attention of the reference layer at one query row.
struct AttnRun {
    std::vector<float> ctx;
    std::size_t steps = 0;
};
AttnRun run_attention(bool fuse, bool keep_scores, std::size_t hq, std::size_t hkv) {
    const std::size_t s = 37, dh = 16;
    const auto q = normal(hq * dh, 71), k = normal(hkv * s * dh, 72), v = normal(hkv * s * dh, 73);
    ScopedEnv env("VELOMIND_GRAPH_FUSE", fuse ? "1" : "0");
    Graph g;
    auto tq = g.input({(dim_t)hq, 1, (dim_t)dh}, F32);
    auto tk = g.input({(dim_t)hkv, (dim_t)s, (dim_t)dh}, F32);
    auto tv = g.input({(dim_t)hkv, (dim_t)s, (dim_t)dh}, F32);
    Tensor ka = tk, va = tv;
    if (hq != hkv) {
        const int rep = static_cast<int>(hq / hkv);
        ka = g.op(OpDescriptor{Op::RepeatKV, RepeatKVAttrs{rep, 0}}, tk);
        va = g.op(OpDescriptor{Op::RepeatKV, RepeatKVAttrs{rep, 0}}, tv);
    }
    auto kt = g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{0, 2, 1}}}, ka);
    auto scores = g.op(Op::MatMul, tq, kt);
    auto ctx = g.op(Op::MatMul, g.op(Op::Softmax, scores), va);
    g.mark_output(ctx);
    if (keep_scores) g.mark_output(scores);
    auto exec = g.build(DeviceType::CPU);
    AttnRun r;
    r.steps = exec->num_steps();
    tq.copy_from_host(as_bytes(q));
    tk.copy_from_host(as_bytes(k));
    tv.copy_from_host(as_bytes(v));
    exec->execute();
    r.ctx.resize(hq * dh);
    ctx.copy_to_host(as_writeable_bytes(r.ctx));
    return r;
}

}  // namespace

TEST_CASE("fusion: SwiGLU chain, its QuantizedMatMul and the residual Add run as one step", "[core][fusion]") {
    const auto off = run_mlp(false, false);
    const auto on = run_mlp(true, false);
    REQUIRE(off.nodes == 7);
    REQUIRE(off.steps == 7);
    // gate, up, SwigluQmmAdd (5 nodes)
    REQUIRE(on.nodes == 7);
    REQUIRE(on.steps == 3);
    REQUIRE(on.inner_unallocated);
    REQUIRE(!off.inner_unallocated);
    REQUIRE(std::memcmp(on.out.data(), off.out.data(), on.out.size() * 4) == 0);
    // the SwiGLU output requested: SiluMul and QmmAdd form apart
    const auto kept = run_mlp(true, false, true);
    REQUIRE(kept.steps == 4);
    REQUIRE(kept.inner_unallocated);
    REQUIRE(std::memcmp(kept.out.data(), off.out.data(), off.out.size() * 4) == 0);
}

TEST_CASE("fusion: a chain with a strided external operand runs node by node", "[core][fusion]") {
    // The fused kernels take dense operands: with the residual a strided
    // view, SwigluQmmAdd splits back into its five nodes, with the same result.
    const auto off = run_mlp(false, false);
    const auto on = run_mlp(true, false, false, true);
    REQUIRE(on.nodes == 7);
    REQUIRE(on.steps == 7);
    REQUIRE(!on.inner_unallocated);
    REQUIRE(std::memcmp(on.out.data(), off.out.data(), on.out.size() * 4) == 0);
}

TEST_CASE("fusion: a kept inner tensor keeps its chain unfused", "[core][fusion]") {
    // the Sigmoid's output is requested: SiluMul is not formed, QmmAdd still is
    const auto on = run_mlp(true, true);
    const auto off = run_mlp(false, true);
    REQUIRE(on.steps == 6);
    REQUIRE(std::memcmp(on.out.data(), off.out.data(), on.out.size() * 4) == 0);
}

TEST_CASE("fusion: decode attention chain runs as one step, with and without RepeatKV", "[core][fusion]") {
    for (auto [hq, hkv] : {std::pair<std::size_t, std::size_t>{6, 2}, {4, 4}}) {
        const auto off = run_attention(false, false, hq, hkv);
        const auto on = run_attention(true, false, hq, hkv);
        REQUIRE(off.steps == (hq != hkv ? 6u : 4u));
        REQUIRE(on.steps == 1);
        REQUIRE(std::memcmp(on.ctx.data(), off.ctx.data(), on.ctx.size() * 4) == 0);
        // scores requested: the chain is kept
        const auto kept = run_attention(true, true, hq, hkv);
        REQUIRE(kept.steps == off.steps);
        REQUIRE(std::memcmp(kept.ctx.data(), off.ctx.data(), off.ctx.size() * 4) == 0);
    }
}

namespace {
// One decode position of the reference layer's attention: RoPE on q and k,
// the KV caches grown by Concat, then the attention chain; K and V kept.
struct LayerAttnRun {
    std::vector<float> ctx, kc, vc;
    std::size_t steps = 0;
};
LayerAttnRun run_layer_attention(bool fuse, bool keep_rotated_q) {
    const std::size_t hq = 6, hkv = 2, s = 9, dh = 8, half = dh / 2;
    const auto q = normal(hq * dh, 81), k = normal(hkv * dh, 82), v = normal(hkv * dh, 83);
    const auto pk = normal(hkv * s * dh, 84), pv = normal(hkv * s * dh, 85), c = normal(half, 86), sn = normal(half, 87);
    ScopedEnv env("VELOMIND_GRAPH_FUSE", fuse ? "1" : "0");
    Graph g;
    auto tq = g.input({(dim_t)hq, 1, (dim_t)dh}, F32), tk = g.input({(dim_t)hkv, 1, (dim_t)dh}, F32);
    auto tv = g.input({(dim_t)hkv, 1, (dim_t)dh}, F32);
    auto tpk = g.input({(dim_t)hkv, (dim_t)s, (dim_t)dh}, F32), tpv = g.input({(dim_t)hkv, (dim_t)s, (dim_t)dh}, F32);
    auto tc = g.input({1, (dim_t)half}, F32), ts = g.input({1, (dim_t)half}, F32);
    auto qr = g.op(Op::RotaryEmbedding, tq, tc, ts);
    auto kr = g.op(Op::RotaryEmbedding, tk, tc, ts);
    auto kc = g.op(OpDescriptor{Op::Concat, ConcatAttrs{1}}, tpk, kr);
    auto vc = g.op(OpDescriptor{Op::Concat, ConcatAttrs{1}}, tpv, tv);
    auto ka = g.op(OpDescriptor{Op::RepeatKV, RepeatKVAttrs{3, 0}}, kc);
    auto va = g.op(OpDescriptor{Op::RepeatKV, RepeatKVAttrs{3, 0}}, vc);
    auto kt = g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{0, 2, 1}}}, ka);
    auto ctx = g.op(Op::MatMul, g.op(Op::Softmax, g.op(Op::MatMul, qr, kt)), va);
    g.mark_output(ctx);
    g.mark_output(kc);
    g.mark_output(vc);
    if (keep_rotated_q) g.mark_output(qr);
    auto exec = g.build(DeviceType::CPU);
    LayerAttnRun r;
    r.steps = exec->num_steps();
    tq.copy_from_host(as_bytes(q));
    tk.copy_from_host(as_bytes(k));
    tv.copy_from_host(as_bytes(v));
    tpk.copy_from_host(as_bytes(pk));
    tpv.copy_from_host(as_bytes(pv));
    tc.copy_from_host(as_bytes(c));
    ts.copy_from_host(as_bytes(sn));
    exec->execute();
    r.ctx.resize(hq * dh);
    r.kc.resize(hkv * (s + 1) * dh);
    r.vc.resize(hkv * (s + 1) * dh);
    ctx.copy_to_host(as_writeable_bytes(r.ctx));
    kc.copy_to_host(as_writeable_bytes(r.kc));
    vc.copy_to_host(as_writeable_bytes(r.vc));
    return r;
}
}  // namespace

TEST_CASE("fusion: RoPE on q and k with the KV appends run as one step", "[core][fusion]") {
    const auto off = run_layer_attention(false, false);
    const auto on = run_layer_attention(true, false);
    REQUIRE(off.steps == 10);
    REQUIRE(on.steps == 2);   // RopeAppend, AttentionDecode
    REQUIRE(std::memcmp(on.ctx.data(), off.ctx.data(), on.ctx.size() * 4) == 0);
    REQUIRE(std::memcmp(on.kc.data(), off.kc.data(), on.kc.size() * 4) == 0);
    REQUIRE(std::memcmp(on.vc.data(), off.vc.data(), on.vc.size() * 4) == 0);
    // a requested rotated q is an output of the fused step, which still forms
    const auto kept = run_layer_attention(true, true);
    REQUIRE(kept.steps == 2);
    REQUIRE(std::memcmp(kept.ctx.data(), off.ctx.data(), off.ctx.size() * 4) == 0);
}

namespace {
// y = QMM(RMSNorm(x)); with `second`, another QMM reads the norm too.
struct NormRun {
    std::vector<float> y;
    std::size_t steps = 0;
};
NormRun run_norm_qmm(bool fuse, bool second) {
    const std::size_t d = 64, n = 48;
    static const auto w1 = int8_weights(d, n, 91), w2 = int8_weights(d, n, 92);
    static const auto x = normal(2 * d, 93), nw = normal(d, 94);
    ScopedEnv env("VELOMIND_GRAPH_FUSE", fuse ? "1" : "0");
    Graph g;
    auto tx = g.input({2, (dim_t)d}, F32), tw = g.input({(dim_t)d}, F32);
    auto b1 = g.input({(dim_t)d, (dim_t)n}, DataType::Int8), s1 = g.input({(dim_t)n}, F32);
    auto b2 = g.input({(dim_t)d, (dim_t)n}, DataType::Int8), s2 = g.input({(dim_t)n}, F32);
    auto hn = g.op(OpDescriptor{Op::RMSNorm, RMSNormAttrs{1e-5f, -1}}, tx, tw);
    auto y = g.op(Op::QuantizedMatMul, hn, b1, s1);
    g.mark_output(y);
    if (second) g.mark_output(g.op(Op::QuantizedMatMul, hn, b2, s2));
    auto exec = g.build(DeviceType::CPU);
    NormRun r;
    r.steps = exec->num_steps();
    tx.copy_from_host(as_bytes(x));
    tw.copy_from_host(as_bytes(nw));
    b1.copy_from_host(as_bytes(w1.q));
    s1.copy_from_host(as_bytes(w1.s));
    if (second) {
        b2.copy_from_host(as_bytes(w2.q));
        s2.copy_from_host(as_bytes(w2.s));
    }
    exec->execute();
    r.y.resize(2 * n);
    y.copy_to_host(as_writeable_bytes(r.y));
    return r;
}
}  // namespace

TEST_CASE("fusion: RMSNorm read only by a QuantizedMatMul step runs inside it", "[core][fusion]") {
    const auto off = run_norm_qmm(false, false);
    const auto on = run_norm_qmm(true, false);
    REQUIRE(off.steps == 2);
    REQUIRE(on.steps == 1);
    REQUIRE(std::memcmp(on.y.data(), off.y.data(), on.y.size() * 4) == 0);
    // read by two separate steps (no group kernel here): the norm stays its own step
    const auto two = run_norm_qmm(true, true);
    REQUIRE(two.steps == 3);
    REQUIRE(std::memcmp(two.y.data(), off.y.data(), off.y.size() * 4) == 0);
}
