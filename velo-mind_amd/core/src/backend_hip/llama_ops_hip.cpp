// DeviceType::HIP kernels for the operators of the LLaMA graph other than
// QuantizedMatMul: KernelFn adapters from the VeloMind operator ABI to
// libvmhip's entry points.  Sizes come from the storages exactly as the
// reference's CPU kernels derive them (src/cpu/ops/*.cpp, cited per
// adapter); every operand must be contiguous (graph tensors are), and one
// launch goes on the executing thread's stream.  Float32 keys, plus the
// (Float32 table, Int32 index) key of Embedding.
#include <cstdint>
#include <string>
#include <variant>
#include <vector>

#include "backend_hip/hip_runtime.h"
#include "internal/op_contract.h"
#include "internal/registry/kernel.h"

namespace velomind::backend::hip {

namespace {

using internal::KernelDtypeKey;
constexpr DataType F32 = DataType::Float32;

const OpDescriptor& desc_of(const void* attrs) { return *static_cast<const OpDescriptor*>(attrs); }

void require_contiguous(Op op, const pConstTensorStorage* in, std::size_t n_in, const TensorStorage& out) {
    for (std::size_t i = 0; i < n_in; ++i)
        if (!in[i] || !in[i]->is_contiguous())
            throw std::invalid_argument(error_context(op, out, "launch") + ": strided operands are not supported on HIP");
    if (!out.is_contiguous())
        throw std::invalid_argument(error_context(op, out, "launch") + ": strided output is not supported on HIP");
}

std::int64_t prod(const shape_t& s, std::size_t from, std::size_t to) {
    std::int64_t p = 1;
    for (std::size_t i = from; i < to; ++i) p *= s[i];
    return p;
}

const float* fin(const pConstTensorStorage* in, int i) { return static_cast<const float*>(in[i]->data); }
float* fout(const pTensorStorage* out) { return static_cast<float*>(out[0]->data); }

void finish(Op op, const TensorStorage& out, int status) {
    if (status != VM_HIP_OK) throw_status(status, error_context(op, out, "launch"));
}

// embedding.cpp:16-33
void embedding_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::Embedding, in, 2, *out[0]);
    finish(Op::Embedding, *out[0],
           vm_hip_embedding_f32(fin(in, 0), in[0]->shape[0], in[0]->shape[1],
                                static_cast<const std::int32_t*>(in[1]->data),
                                static_cast<std::int64_t>(storage_numel(*in[1])), fout(out), current_stream()));
}

// rmsnorm.cpp:17-60 (last axis)
void rmsnorm_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::RMSNorm, in, 2, *out[0]);
    const auto& a = std::get<RMSNormAttrs>(desc_of(attrs).attrs);
    const std::int64_t dim = in[0]->shape.back();
    const auto rows = static_cast<std::int64_t>(storage_numel(*in[0])) / dim;
    finish(Op::RMSNorm, *out[0],
           vm_hip_rmsnorm_f32(fin(in, 0), fin(in, 1), fout(out), rows, dim, a.epsilon, current_stream()));
}

// rotary_embedding.cpp:16-45
void rope_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::RotaryEmbedding, in, 3, *out[0]);
    const std::int64_t d = in[0]->shape.back();
    const std::int64_t rows = static_cast<std::int64_t>(storage_numel(*in[0])) / d;
    const std::int64_t cos_rows = in[1]->shape.size() >= 2 ? in[1]->shape[0] : 1;
    finish(Op::RotaryEmbedding, *out[0],
           vm_hip_rope_f32(fin(in, 0), fin(in, 1), fin(in, 2), fout(out), rows, d, cos_rows, current_stream()));
}

// reshape.cpp: a byte copy into the output's shape.
void reshape_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::Reshape, in, 1, *out[0]);
    finish(Op::Reshape, *out[0],
           vm_hip_memcpy_d2d(out[0]->data, in[0]->data, storage_nbytes(*in[0]), current_stream()));
}

// transpose.cpp:17-68
void transpose_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::Transpose, in, 1, *out[0]);
    const auto& perm = std::get<TransposeAttrs>(desc_of(attrs).attrs).perm;
    const auto& s = in[0]->shape;
    std::vector<std::int64_t> shape(s.begin(), s.end());
    std::vector<int> p(perm.begin(), perm.end());
    finish(Op::Transpose, *out[0],
           vm_hip_transpose_f32(fin(in, 0), fout(out), static_cast<int>(s.size()), shape.data(),
                                p.empty() ? nullptr : p.data(), current_stream()));
}

// slice.cpp:21-110 with the signature's clamping (shape_helpers.h:178-211)
void slice_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::Slice, in, 1, *out[0]);
    const auto& a = std::get<SliceAttrs>(desc_of(attrs).attrs);
    const auto& s = in[0]->shape;
    std::vector<std::int64_t> shape(s.begin(), s.end()), begins(s.size(), 0), steps(s.size(), 1),
        oshape(out[0]->shape.begin(), out[0]->shape.end());
    for (std::size_t i = 0; i < a.begins.size() && i < s.size(); ++i) {
        begins[i] = internal::clamp_slice_bounds(a.begins[i], a.ends[i], s[i]).first;
        if (i < a.strides.size() && a.strides[i] > 0) steps[i] = a.strides[i];
    }
    finish(Op::Slice, *out[0],
           vm_hip_slice_f32(fin(in, 0), fout(out), static_cast<int>(s.size()), shape.data(), begins.data(),
                            steps.data(), oshape.data(), current_stream()));
}

// concat.cpp:19-72
void concat_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::Concat, in, 2, *out[0]);
    int axis = std::get<ConcatAttrs>(desc_of(attrs).attrs).axis;
    const auto& s = in[0]->shape;
    if (axis < 0) axis += static_cast<int>(s.size());
    const auto ax = static_cast<std::size_t>(axis);
    finish(Op::Concat, *out[0],
           vm_hip_concat_f32(fin(in, 0), fin(in, 1), fout(out), prod(s, 0, ax), prod(s, ax, s.size()),
                             prod(in[1]->shape, ax, s.size()), current_stream()));
}

// repeat_kv.cpp:20-62
void repeat_kv_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::RepeatKV, in, 1, *out[0]);
    const auto& a = std::get<RepeatKVAttrs>(desc_of(attrs).attrs);
    const auto& s = in[0]->shape;
    int axis = a.axis < 0 ? a.axis + static_cast<int>(s.size()) : a.axis;
    const auto ax = static_cast<std::size_t>(axis);
    finish(Op::RepeatKV, *out[0],
           vm_hip_repeat_kv_f32(fin(in, 0), fout(out), prod(s, 0, ax), s[ax], a.repeats, prod(s, ax + 1, s.size()),
                                current_stream()));
}

template <int EW, Op OP>
void elementwise_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    const std::size_t n_in = EW == VM_HIP_EW_SIGMOID ? 1 : 2;
    require_contiguous(OP, in, n_in, *out[0]);
    finish(OP, *out[0],
           vm_hip_elementwise_f32(EW, fin(in, 0), n_in == 2 ? fin(in, 1) : nullptr, fout(out),
                                  static_cast<std::int64_t>(storage_numel(*out[0])), current_stream()));
}

// softmax.cpp:18-48
void softmax_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::Softmax, in, 1, *out[0]);
    const auto& s = in[0]->shape;
    int axis = std::get<SoftmaxAttrs>(desc_of(attrs).attrs).axis;
    if (axis < 0) axis += static_cast<int>(s.size());
    const auto ax = static_cast<std::size_t>(axis);
    finish(Op::Softmax, *out[0],
           vm_hip_softmax_f32(fin(in, 0), fout(out), prod(s, 0, ax), s[ax], prod(s, ax + 1, s.size()),
                              current_stream()));
}

// matmul.cpp (fp32, equal batch dimensions)
void matmul_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::MatMul, in, 2, *out[0]);
    const auto& a = in[0]->shape;
    const auto& c = out[0]->shape;
    const std::int64_t m = a[a.size() - 2], k = a.back(), n = c.back();
    finish(Op::MatMul, *out[0],
           vm_hip_matmul_f32(fin(in, 0), fin(in, 1), fout(out), prod(c, 0, c.size() - 2), m, k, n,
                             current_stream()));
}

// fused_attention.cpp:22-138
void fused_attention_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    require_contiguous(Op::FusedAttention, in, 3, *out[0]);
    const auto& a = std::get<FusedAttentionAttrs>(desc_of(attrs).attrs);
    const auto& q = in[0]->shape;
    const auto& k = in[1]->shape;
    const std::size_t r = q.size();
    finish(Op::FusedAttention, *out[0],
           vm_hip_attention_f32(fin(in, 0), fin(in, 1), fin(in, 2), fout(out), prod(q, 0, r - 3), q[r - 3], k[r - 3],
                                q[r - 2], k[r - 2], q[r - 1], in[2]->shape.back(), a.scale, a.is_causal ? 1 : 0,
                                current_stream()));
}

// ---- fused steps (kernel.h FusedKind; the graph compiler checks shapes
// and dtypes before it forms one)

// Mul(Mul(Sigmoid(g), g), u): inputs [g, u].
void silu_mul_fused_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::Mul, in, 2, *out[0]);
    finish(Op::Mul, *out[0],
           vm_hip_elementwise_f32(VM_HIP_EW_SILU_MUL, fin(in, 0), fin(in, 1), fout(out),
                                  static_cast<std::int64_t>(storage_numel(*out[0])), current_stream()));
}

// RepeatKV / Transpose / MatMul / Softmax / MatMul at one query row:
// inputs [q [H, 1, D], K [Hkv, S, D], V [Hkv, S, Dv]], outputs [ctx [H, 1, Dv]].
void attention_decode_fused_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::MatMul, in, 3, *out[0]);
    const auto& q = in[0]->shape;
    const auto& k = in[1]->shape;
    finish(Op::MatMul, *out[0],
           vm_hip_attention_decode_chain_f32(fin(in, 0), fin(in, 1), fin(in, 2), fout(out), q[0], k[0], k[1], q[2],
                                             in[2]->shape[2], current_stream()));
}

// RoPE(q), Concat(K_past, RoPE(k)), Concat(V_past, v) at one position:
// inputs [q [H, 1, D], k [Hkv, 1, D], v [Hkv, 1, Dv], K_past [Hkv, S, D],
// V_past [Hkv, S, Dv], cos, sin], outputs [q', K [Hkv, S + 1, D], V].
void rope_append_fused_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void*) {
    require_contiguous(Op::Concat, in, 7, *out[1]);
    for (int i = 0; i < 3; ++i)
        if (!out[i]->is_contiguous())
            throw std::invalid_argument(error_context(Op::Concat, *out[i], "launch") + ": strided output is not supported on HIP");
    const auto& q = in[0]->shape;
    const auto& kp = in[3]->shape;
    finish(Op::Concat, *out[1],
           vm_hip_rope_append_f32(fin(in, 0), fin(in, 1), fin(in, 2), fin(in, 3), fin(in, 4), fin(in, 5), fin(in, 6),
                                  static_cast<float*>(out[0]->data), static_cast<float*>(out[1]->data),
                                  static_cast<float*>(out[2]->data), q[0], kp[0], kp[1], q[2], in[4]->shape[2],
                                  current_stream()));
}

}  // namespace

#define VM_HIP_F32_KERNEL(OP, N_IN, FN)                                                                  \
    VELOMIND_REGISTER_OP_KERNEL(::velomind::DeviceType::HIP, OP,                                         \
                                (KernelDtypeKey{{F32, F32, F32, F32}, N_IN, F32}), &FN)

VELOMIND_REGISTER_OP_KERNEL(::velomind::DeviceType::HIP, Op::Embedding,
                            (KernelDtypeKey{{F32, DataType::Int32}, 2, F32}), &embedding_hip)
VM_HIP_F32_KERNEL(Op::RMSNorm, 2, rmsnorm_hip)
VM_HIP_F32_KERNEL(Op::RotaryEmbedding, 3, rope_hip)
VM_HIP_F32_KERNEL(Op::Reshape, 1, reshape_hip)
VM_HIP_F32_KERNEL(Op::Transpose, 1, transpose_hip)
VM_HIP_F32_KERNEL(Op::Slice, 1, slice_hip)
VM_HIP_F32_KERNEL(Op::Concat, 2, concat_hip)
VM_HIP_F32_KERNEL(Op::RepeatKV, 1, repeat_kv_hip)
VM_HIP_F32_KERNEL(Op::Add, 2, (elementwise_hip<VM_HIP_EW_ADD, Op::Add>))
VM_HIP_F32_KERNEL(Op::Mul, 2, (elementwise_hip<VM_HIP_EW_MUL, Op::Mul>))
VM_HIP_F32_KERNEL(Op::Sigmoid, 1, (elementwise_hip<VM_HIP_EW_SIGMOID, Op::Sigmoid>))
VM_HIP_F32_KERNEL(Op::Softmax, 1, softmax_hip)
VM_HIP_F32_KERNEL(Op::MatMul, 2, matmul_hip)
VM_HIP_F32_KERNEL(Op::FusedAttention, 3, fused_attention_hip)

VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, internal::FusedKind::SiluMul, &silu_mul_fused_hip)
VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, internal::FusedKind::AttentionDecode, &attention_decode_fused_hip)
VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, internal::FusedKind::RopeAppend, &rope_append_fused_hip)
// vm_hip_attention_f32 maps query head h to kv head h / (hq / hk) itself,
// so FusedAttention reads K/V as they were before RepeatKV.
VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, internal::FusedKind::AttentionGqa, &fused_attention_hip)

}  // namespace velomind::backend::hip
