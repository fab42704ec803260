// op_signature: arity and metadata checks in front of every registered
// signature (the reference's src/kernel.cpp:16-51), plus the device-
// independent QuantizedMatMul signature registration.
#include <cstring>
#include <span>
#include <type_traits>
#include <stdexcept>
#include <string>

#include "internal/op_contract.h"
#include "internal/registry/kernel.h"
#include "internal/registry/shape.h"
#include "internal/registry/storage.h"
#include "velomind/dtype.h"

namespace velomind::internal {

namespace {
std::size_t expected_arity(Op op) {
    switch (op) {
        case Op::Add: case Op::Sub: case Op::Mul: case Op::Div:
        case Op::MatMul: case Op::Concat: case Op::RMSNorm: case Op::Embedding:
            return 2;
        case Op::RotaryEmbedding: case Op::FusedAttention: case Op::QuantizedMatMul:
            return 3;
        default:
            return 1;
    }
}
}  // namespace

auto op_signature(Op op, std::span<const pConstTensorStorage> inputs, const OpAttrs& attrs) -> OpSignature {
    auto fn = get_op_signature(op);
    if (fn == nullptr) throw std::invalid_argument("Graph::op: unsupported operator signature");
    if (inputs.size() != expected_arity(op))
        throw std::invalid_argument(std::string(op_name(op)) + ": invalid input count");
    for (auto* t : inputs) {
        if (!t) throw std::invalid_argument("Graph::op: null input storage");
        if (t->size_bytes < storage_nbytes(*t)) throw std::invalid_argument("Graph::op: invalid input capacity");
    }
    // The node's own attributes by reference (a copy allocates for every
    // vector-valued attribute, twice per node and decode step); the
    // operator's defaults only when it carries none.
    if (!std::holds_alternative<NoAttrs>(attrs)) {
        validate_op_metadata(op, inputs, attrs);
        return fn(inputs, attrs);
    }
    const OpAttrs effective = default_op_attrs(op);
    validate_op_metadata(op, inputs, effective);
    return fn(inputs, effective);
}

}  // namespace velomind::internal

VELOMIND_REGISTER_SIGNATURE(::velomind::Op::QuantizedMatMul, ::velomind::internal::signature_quantized_matmul)

namespace velomind {

auto is_dtype_supported(DeviceType device, DataType dtype) noexcept -> bool {
    return data_type_size(dtype) != 0 && internal::get_storage_creator(device) != nullptr;
}

auto is_op_dtype_supported(DeviceType device, Op op, std::span<const DataType> input_dtypes,
                           DataType output_dtype) noexcept -> bool {
    try {
        return internal::resolve_op_kernel(op, input_dtypes, output_dtype, device) != nullptr;
    } catch (...) {
        return false;
    }
}

namespace {
template <typename TSrc, typename TDst>
void convert_typed(const void* src, void* dst, std::size_t n) {
    const auto* s = static_cast<const TSrc*>(src);
    auto* d = static_cast<TDst*>(dst);
    for (std::size_t i = 0; i < n; ++i) {
        if constexpr (std::is_same_v<TDst, float16_t> || std::is_same_v<TDst, bfloat16_t>)
            d[i] = TDst(static_cast<float>(s[i]));
        else if constexpr (std::is_same_v<TSrc, float16_t> || std::is_same_v<TSrc, bfloat16_t>)
            d[i] = static_cast<TDst>(static_cast<float>(s[i]));
        else
            d[i] = static_cast<TDst>(s[i]);
    }
}

template <typename TSrc>
void convert_from(const void* src, DataType dst_dtype, void* dst, std::size_t n) {
    switch (dst_dtype) {
        case DataType::Float32: convert_typed<TSrc, float>(src, dst, n); break;
        case DataType::Float16: convert_typed<TSrc, float16_t>(src, dst, n); break;
        case DataType::BFloat16: convert_typed<TSrc, bfloat16_t>(src, dst, n); break;
        case DataType::Int32: convert_typed<TSrc, std::int32_t>(src, dst, n); break;
        case DataType::Int8: convert_typed<TSrc, std::int8_t>(src, dst, n); break;
        case DataType::Bool: convert_typed<TSrc, bool>(src, dst, n); break;
    }
}
}  // namespace

auto convert_dtype(const void* src, DataType src_dtype, void* dst, DataType dst_dtype, std::size_t numel) -> void {
    if (numel == 0) return;
    if (!src || !dst) throw std::invalid_argument("convert_dtype: null buffer pointer");
    if (src_dtype == dst_dtype) {
        std::memcpy(dst, src, numel * data_type_size(src_dtype));
        return;
    }
    switch (src_dtype) {
        case DataType::Float32: convert_from<float>(src, dst_dtype, dst, numel); break;
        case DataType::Float16: convert_from<float16_t>(src, dst_dtype, dst, numel); break;
        case DataType::BFloat16: convert_from<bfloat16_t>(src, dst_dtype, dst, numel); break;
        case DataType::Int32: convert_from<std::int32_t>(src, dst_dtype, dst, numel); break;
        case DataType::Int8: convert_from<std::int8_t>(src, dst_dtype, dst, numel); break;
        case DataType::Bool: convert_from<bool>(src, dst_dtype, dst, numel); break;
    }
}

}  // namespace velomind
