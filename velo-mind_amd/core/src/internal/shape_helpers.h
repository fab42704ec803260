// Output dtype/shape of the LLaMA-graph operators, evaluated after
// validate_op_metadata has checked the inputs.  Each mirrors the
// reference's signature of the same name (src/internal/shape_helpers.h:
// 15-262) so graphs infer the same shapes on every device.
#pragma once

#include <span>
#include <stdexcept>
#include <string>
#include <variant>

#include "internal/op_contract.h"
#include "internal/registry/shape.h"
#include "velomind/ops.h"
#include "velomind/tensor_storage.h"

namespace velomind::internal {

inline std::size_t resolve_axis(int axis, std::size_t rank, const char* op) {
    const std::int64_t a = axis < 0 ? axis + static_cast<std::int64_t>(rank) : axis;
    if (a < 0 || a >= static_cast<std::int64_t>(rank)) throw std::invalid_argument(std::string(op) + ": axis out of range");
    return static_cast<std::size_t>(a);
}

// Elementwise (Add/Sub/Mul/Div, unary activations): shape and dtype of the
// first input (:28-34).
inline auto signature_elementwise(std::span<const pConstTensorStorage> in, const OpAttrs&) -> OpSignature {
    if (in.empty()) return OpSignature{DataType::Float32, {}};
    return OpSignature{in[0]->dtype, in[0]->shape};
}

// Softmax keeps the input's shape and dtype; the axis must exist (:15-26).
inline auto signature_softmax(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    const auto* sm = std::get_if<SoftmaxAttrs>(&attrs);
    if (!sm) throw std::invalid_argument("Softmax: invalid attributes");
    resolve_axis(sm->axis, in[0]->shape.size(), "Softmax");
    return OpSignature{in[0]->dtype, in[0]->shape};
}

// MatMul [..., m, k] x [..., k, n] with equal batch dimensions after
// left-padding with ones; fp32 wins over a half operand (:36-84).
inline auto signature_matmul(std::span<const pConstTensorStorage> in, const OpAttrs&) -> OpSignature {
    const auto& a = in[0]->shape;
    const auto& b = in[1]->shape;
    if (a.size() < 2 || b.size() < 2) throw std::invalid_argument("velomind::MatMul signature: inputs must be rank >= 2");
    const std::size_t rank = std::max(a.size(), b.size());
    shape_t ap(rank - a.size(), 1), bp(rank - b.size(), 1);
    ap.insert(ap.end(), a.begin(), a.end());
    bp.insert(bp.end(), b.begin(), b.end());
    shape_t out;
    for (std::size_t i = 0; i + 2 < rank; ++i) {
        if (ap[i] != bp[i]) throw std::invalid_argument("velomind::MatMul signature: batch dim mismatch");
        out.push_back(ap[i]);
    }
    if (ap[rank - 1] != bp[rank - 2]) throw std::invalid_argument("velomind::MatMul signature: K dimension mismatch");
    out.push_back(ap[rank - 2]);
    out.push_back(bp[rank - 1]);
    DataType dt = in[0]->dtype;
    if ((in[0]->dtype == DataType::Float32) != (in[1]->dtype == DataType::Float32)) dt = DataType::Float32;
    return OpSignature{dt, std::move(out)};
}

// RMSNorm and RotaryEmbedding keep the input's shape and dtype (:86-92, :106-112).
inline auto signature_same_as_input(std::span<const pConstTensorStorage> in, const OpAttrs&) -> OpSignature {
    return OpSignature{in[0]->dtype, in[0]->shape};
}

// Embedding: indices' shape plus the table's row length, table dtype (:94-104).
inline auto signature_embedding(std::span<const pConstTensorStorage> in, const OpAttrs&) -> OpSignature {
    shape_t out = in[1]->shape;
    out.push_back(in[0]->shape.back());
    return OpSignature{in[0]->dtype, std::move(out)};
}

// Reshape to the attribute shape (:114-123).
inline auto signature_reshape(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    return OpSignature{in[0]->dtype, std::get<ReshapeAttrs>(attrs).shape};
}

// Transpose by perm; an empty perm reverses the axes (:125-146).
inline auto signature_transpose(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    const auto& perm = std::get<TransposeAttrs>(attrs).perm;
    const auto& s = in[0]->shape;
    shape_t out(s.size());
    for (std::size_t i = 0; i < s.size(); ++i) out[i] = perm.empty() ? s[s.size() - 1 - i] : s[perm[i]];
    return OpSignature{in[0]->dtype, std::move(out)};
}

// Concat: the axis grows by the second input's extent (:148-161).
inline auto signature_concat(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    const std::size_t axis = resolve_axis(std::get<ConcatAttrs>(attrs).axis, in[0]->shape.size(), "Concat");
    shape_t out = in[0]->shape;
    out[axis] += in[1]->shape[axis];
    return OpSignature{in[0]->dtype, std::move(out)};
}

// RepeatKV: the axis is multiplied by `repeats` (:163-176).
inline auto signature_repeat_kv(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    const auto& a = std::get<RepeatKVAttrs>(attrs);
    const std::size_t axis = resolve_axis(a.axis, in[0]->shape.size(), "RepeatKV");
    shape_t out = in[0]->shape;
    out[axis] *= static_cast<dim_t>(a.repeats);
    return OpSignature{in[0]->dtype, std::move(out)};
}

// Slice: ceil((end - begin) / stride) per sliced axis after clamping
// (:178-211).
inline auto signature_slice(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    if (in.size() != 1 || !in[0]) throw std::invalid_argument("Slice: expected single input tensor");
    const auto& s = std::get<SliceAttrs>(attrs);
    const auto& shape = in[0]->shape;
    shape_t out;
    for (std::size_t i = 0; i < shape.size(); ++i) {
        if (i >= s.begins.size()) {
            out.push_back(shape[i]);
            continue;
        }
        const dim_t stride = (i < s.strides.size() && s.strides[i] > 0) ? s.strides[i] : 1;
        const auto [b, e] = clamp_slice_bounds(s.begins[i], s.ends[i], shape[i]);
        out.push_back(e > b ? (e - b + stride - 1) / stride : 0);
    }
    return OpSignature{in[0]->dtype, std::move(out)};
}

// FusedAttention: Q's shape with the last dimension of V (:213-262).
inline auto signature_fused_attention(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    if (in.size() != 3 || !in[0] || !in[1] || !in[2])
        throw std::invalid_argument("FusedAttention: expected 3 inputs (Q, K, V)");
    if (!std::get_if<FusedAttentionAttrs>(&attrs)) throw std::invalid_argument("FusedAttention: invalid attributes");
    shape_t out = in[0]->shape;
    out.back() = in[2]->shape.back();
    return OpSignature{in[0]->dtype, std::move(out)};
}

}  // namespace velomind::internal
