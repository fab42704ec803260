// Operator contract checks shared by all devices.
//
// validate_op_metadata: generic input rules (no scalars, no zero
// dimensions, matching dtypes except for mixed-dtype ops) plus the per-op
// shape, attribute and dtype rules (src/internal/op_validation.h:11-184 in
// the reference).
//
// signature_quantized_matmul: A [..., M, K] (F32/F16/BF16), B_q Int8
// [K, N] or INT4-packed [(K+1)/2, N], scales [N] / [1, N] (block_size 0) or
// [ceil(K/block), N] / flat [ceil(K/block) * N] (block_size > 0); output
// A's shape with the last dimension N, A's dtype
// (src/internal/shape_helpers.h:268-339 in the reference).
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <span>
#include <stdexcept>
#include <utility>
#include <vector>
#include <string>
#include <variant>

#include "internal/registry/shape.h"
#include "velomind/ops.h"
#include "velomind/tensor_storage.h"

namespace velomind::internal {

inline bool is_float_dtype(DataType d) {
    return d == DataType::Float32 || d == DataType::Float16 || d == DataType::BFloat16;
}

// Slice bounds of one axis as the reference resolves them
// (src/internal/shape_helpers.h:188-199): negative values count from the
// end, then both clamp to [0, dim].
inline std::pair<dim_t, dim_t> clamp_slice_bounds(int begin, int end, dim_t dim) {
    const auto d = static_cast<std::int64_t>(dim);
    std::int64_t b = begin < 0 ? begin + d : begin;
    std::int64_t e = end < 0 ? end + d : end;
    b = std::clamp<std::int64_t>(b, 0, d);
    e = std::clamp<std::int64_t>(e, 0, d);
    return {static_cast<dim_t>(b), static_cast<dim_t>(e)};
}

inline void validate_op_metadata(Op op, std::span<const pConstTensorStorage> in, const OpAttrs& attrs) {
    const auto fail = [op](const std::string& why) {
        throw std::invalid_argument(std::string(op_name(op)) + ": " + why);
    };
    if (attrs.index() != default_op_attrs(op).index()) fail("invalid attributes");
    for (auto* t : in) {
        if (t->shape.empty()) fail("scalar input is not supported");
        for (dim_t d : t->shape)
            if (d == 0) fail("zero dimension is not supported");
    }
    const bool mixed_ok = op == Op::Embedding || op == Op::MatMul || op == Op::RMSNorm || op == Op::QuantizedMatMul;
    if (!mixed_ok)
        for (auto* t : in)
            if (t->dtype != in[0]->dtype) fail("input dtype mismatch");
    const auto& shape = in[0]->shape;
    switch (op) {
        case Op::Add: case Op::Sub: case Op::Mul: case Op::Div:
            if (in.size() > 1 && in[1]->shape != shape) fail("broadcast is not supported; shapes must match");
            break;
        case Op::MatMul: {
            const auto& a = std::get<MatMulAttrs>(attrs);
            if (a.trans_a || a.trans_b) fail("transpose attributes are not supported");
            if (in[0]->dtype != in[1]->dtype) {
                const bool f32_half = (in[0]->dtype == DataType::Float32 && is_float_dtype(in[1]->dtype)) ||
                                      (in[1]->dtype == DataType::Float32 && is_float_dtype(in[0]->dtype));
                if (!f32_half) fail("unsupported mixed precision dtypes for MatMul");
            }
            break;
        }
        case Op::Reshape: {
            TensorStorage target;
            target.shape = std::get<ReshapeAttrs>(attrs).shape;
            if (storage_numel(target) != storage_numel(*in[0])) fail("element count mismatch");
            break;
        }
        case Op::Transpose: {
            const auto& perm = std::get<TransposeAttrs>(attrs).perm;
            if (perm.empty()) break;
            if (perm.size() != shape.size()) fail("permutation rank mismatch");
            std::vector<bool> seen(shape.size(), false);
            for (int axis : perm) {
                if (axis < 0 || static_cast<std::size_t>(axis) >= shape.size()) fail("permutation axis out of range");
                if (seen[axis]) fail("duplicate permutation axis");
                seen[axis] = true;
            }
            break;
        }
        case Op::Concat: {
            if (shape.size() != in[1]->shape.size()) fail("rank mismatch");
            std::int64_t axis = std::get<ConcatAttrs>(attrs).axis;
            if (axis < 0) axis += static_cast<std::int64_t>(shape.size());
            if (axis < 0 || static_cast<std::size_t>(axis) >= shape.size()) fail("axis out of range");
            for (std::size_t i = 0; i < shape.size(); ++i)
                if (i != static_cast<std::size_t>(axis) && shape[i] != in[1]->shape[i]) fail("non-axis shape mismatch");
            if (shape[axis] > std::numeric_limits<dim_t>::max() - in[1]->shape[axis]) fail("dimension sum overflow");
            break;
        }
        case Op::RMSNorm: {
            const auto& a = std::get<RMSNormAttrs>(attrs);
            std::int64_t axis = a.axis;
            if (axis < 0) axis += static_cast<std::int64_t>(shape.size());
            if (axis != static_cast<std::int64_t>(shape.size()) - 1) fail("only last-axis normalization is supported");
            if (!std::isfinite(a.epsilon) || a.epsilon <= 0) fail("epsilon must be finite and positive");
            if (in[1]->shape != shape_t{shape.back()}) fail("weight shape mismatch");
            if (!is_float_dtype(in[0]->dtype)) fail("expected Float32, Float16, or BFloat16 input for RMSNorm");
            if (in[0]->dtype != in[1]->dtype &&
                !(in[0]->dtype == DataType::Float32 && is_float_dtype(in[1]->dtype)))
                fail("unsupported mixed precision dtypes for RMSNorm");
            break;
        }
        case Op::Embedding:
            if (shape.size() != 2) fail("expected nonempty rank-two table");
            if (in[0]->dtype != DataType::Float32 || in[1]->dtype != DataType::Int32)
                fail("expected Float32 table and Int32 indices");
            break;
        case Op::RotaryEmbedding: {
            if (shape.back() % 2 != 0) fail("head dimension must be positive and even");
            if (in[0]->dtype != DataType::Float32) fail("expected Float32");
            const auto& cache = in[1]->shape;
            if (cache != in[2]->shape || cache.size() > 2 || cache.back() != shape.back() / 2)
                fail("cosine/sine cache shape mismatch");
            if (cache.size() == 2 && cache[0] > 1 && (shape.size() < 2 || shape[shape.size() - 2] != cache[0]))
                fail("position cache length mismatch");
            break;
        }
        case Op::RepeatKV: {
            const auto& a = std::get<RepeatKVAttrs>(attrs);
            if (a.repeats <= 0) fail("repeats must be positive");
            std::int64_t axis = a.axis;
            if (axis < 0) axis += static_cast<std::int64_t>(shape.size());
            if (axis < 0 || static_cast<std::size_t>(axis) >= shape.size()) fail("axis out of range");
            break;
        }
        case Op::Slice: {
            const auto& a = std::get<SliceAttrs>(attrs);
            if (a.begins.size() != a.ends.size()) fail("begins and ends rank mismatch");
            if (!a.strides.empty() && a.strides.size() != a.begins.size()) fail("strides rank mismatch");
            if (a.begins.size() > shape.size()) fail("slice attributes rank exceeds tensor rank");
            for (std::size_t i = 0; i < a.begins.size(); ++i) {
                if (i < a.strides.size() && a.strides[i] <= 0) fail("stride must be positive");
                const auto [b, e] = clamp_slice_bounds(a.begins[i], a.ends[i], shape[i]);
                if (b >= e) fail("slice begin must be strictly less than end");
            }
            break;
        }
        case Op::Softmax:
            if (!is_float_dtype(in[0]->dtype)) fail("expected Float32, Float16, or BFloat16");
            break;
        case Op::FusedAttention: {
            const auto& a = std::get<FusedAttentionAttrs>(attrs);
            if (!is_float_dtype(in[0]->dtype)) fail("expected Float32, Float16, or BFloat16");
            const std::size_t rank = shape.size();
            if (rank < 3 || in[1]->shape.size() != rank || in[2]->shape.size() != rank)
                fail("inputs must have matching rank >= 3");
            for (std::size_t i = 0; i + 3 < rank; ++i)
                if (shape[i] != in[1]->shape[i] || shape[i] != in[2]->shape[i]) fail("batch dimension mismatch");
            const dim_t hk = in[1]->shape[rank - 3];
            if (hk <= 0 || in[2]->shape[rank - 3] != hk || shape[rank - 3] % hk != 0) fail("invalid head counts");
            if (in[1]->shape[rank - 2] != in[2]->shape[rank - 2]) fail("K and V sequence length mismatch");
            if (a.is_causal && in[1]->shape[rank - 2] < shape[rank - 2]) fail("causal attention requires S_k >= S_q");
            if (shape[rank - 1] != in[1]->shape[rank - 1]) fail("Q and K feature dimension mismatch");
            break;
        }
        default:
            break;
    }
    if (op == Op::QuantizedMatMul) {
        const auto& qa = std::get<QuantizedMatMulAttrs>(attrs);
        if (!is_float_dtype(in[0]->dtype)) fail("activation must be Float32, Float16, or BFloat16");
        if (in[1]->dtype != DataType::Int8) fail("quantized weight must be Int8");
        if (!is_float_dtype(in[2]->dtype)) fail("scales must be Float32, Float16, or BFloat16");
        if (in[0]->shape.size() < 2) fail("activation rank must be >= 2");
        if (in[1]->shape.size() != 2) fail("quantized weight must be 2D matrix");
        if (qa.quant_type == QuantType::Int4 && qa.block_size > 0 && qa.block_size % 2 != 0)
            fail("Int4 block_size must be even");
    }
}

inline auto signature_quantized_matmul(std::span<const pConstTensorStorage> in, const OpAttrs& attrs) -> OpSignature {
    const auto fail = [](const char* why) { throw std::invalid_argument(std::string("QuantizedMatMul: ") + why); };
    if (in.size() != 3 || !in[0] || !in[1] || !in[2]) fail("expected 3 inputs (A, B_q, scales)");
    const auto* qa = std::get_if<QuantizedMatMulAttrs>(&attrs);
    if (!qa) fail("invalid attributes");
    const auto& a = in[0]->shape;
    const auto& b = in[1]->shape;
    const auto& s = in[2]->shape;
    if (a.size() < 2) fail("activation rank must be >= 2");
    if (b.size() != 2) fail("quantized weight must be 2D matrix");
    const dim_t k = a.back();
    const dim_t n = b[1];
    if (qa->quant_type == QuantType::Int4) {
        if (b[0] != (k + 1) / 2) fail("(Int4) packed rows mismatch with activation inner dimension");
    } else if (b[0] != k) {
        fail("inner dimension mismatch between activation and weight");
    }
    if (qa->block_size > 0) {
        const dim_t nb = (k + qa->block_size - 1) / qa->block_size;
        if (s.size() == 2) {
            if (s[0] != nb || s[1] != n) fail("block-wise scales shape mismatch");
        } else if (s.size() == 1) {
            if (s[0] != nb * n) fail("flat block-wise scales size mismatch");
        } else {
            fail("invalid scales rank");
        }
    } else {
        if (s.size() == 1) {
            if (s[0] != n) fail("per-channel scales size mismatch with output columns");
        } else if (s.size() == 2) {
            if (s[0] != 1 || s[1] != n) fail("2D per-channel scales shape mismatch");
        } else {
            fail("invalid scales rank");
        }
    }
    shape_t out = a;
    out.back() = n;
    return OpSignature{in[0]->dtype, std::move(out)};
}

}  // namespace velomind::internal
