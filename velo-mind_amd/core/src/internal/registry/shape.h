// Operator signature registry (output dtype/shape from inputs and attrs)
// and the default-attribute table (the reference's
// src/internal/registry/shape.h:13-50).
#pragma once

#include "internal/registry/macros.h"

#include <array>
#include <span>

#include "velomind/ops.h"
#include "velomind/tensor_storage.h"
#include "velomind/types.h"

namespace velomind::internal {

struct OpSignature {
    DataType dtype;
    shape_t shape;
};

using OpSignatureFn = OpSignature (*)(std::span<const pConstTensorStorage> inputs, const OpAttrs& attrs);

// Checks arity and metadata, then evaluates the registered signature.
auto op_signature(Op op, std::span<const pConstTensorStorage> inputs, const OpAttrs& attrs) -> OpSignature;
auto signatures() -> std::array<OpSignatureFn, MAX_OPS>&;
void register_op_signature(Op op, OpSignatureFn fn);
auto get_op_signature(Op op) -> OpSignatureFn;
auto default_attrs_table() -> std::array<OpAttrs, MAX_OPS>&;
void register_default_op_attrs(Op op, OpAttrs attrs);
using ::velomind::default_op_attrs;

}  // namespace velomind::internal

#define VELOMIND_REGISTER_SIGNATURE(OP_ENUM, FN)                                                  \
    namespace {                                                                                   \
    [[maybe_unused]] const bool VELOMIND_CONCAT_(_velomind_sig_, __LINE__) = [] {                 \
        ::velomind::internal::register_op_signature(OP_ENUM, FN);                                 \
        return true;                                                                              \
    }();                                                                                          \
    }
