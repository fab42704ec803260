// Operator contract checks shared by all devices.
//
// validate_op_metadata: generic input rules (no scalars, no zero
// dimensions, matching dtypes except for mixed-dtype ops) plus the
// QuantizedMatMul dtype/rank rules (src/internal/op_validation.h:11-30 and
// :159-184 in the reference).
//
// signature_quantized_matmul: A [..., M, K] (F32/F16/BF16), B_q Int8
// [K, N] or INT4-packed [(K+1)/2, N], scales [N] / [1, N] (block_size 0) or
// [ceil(K/block), N] / flat [ceil(K/block) * N] (block_size > 0); output
// A's shape with the last dimension N, A's dtype
// (src/internal/shape_helpers.h:268-339 in the reference).
#pragma once

#include <span>
#include <stdexcept>
#include <string>
#include <variant>

#include "internal/registry/shape.h"
#include "velomind/ops.h"
#include "velomind/tensor_storage.h"

namespace velomind::internal {

inline bool is_float_dtype(DataType d) {
    return d == DataType::Float32 || d == DataType::Float16 || d == DataType::BFloat16;
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
