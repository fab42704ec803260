// Operator identifiers, attributes and the kernel function type.  The Op
// enum values and the OpAttrs alternative order are ABI and match the
// reference's include/velomind/ops.h:26-153 (QuantizedMatMul = 26,
// QuantizedMatMulAttrs = alternative 14).
#pragma once

#include <array>
#include <cstdint>
#include <ostream>
#include <string>
#include <variant>
#include <vector>

#include "velomind/quant.h"
#include "velomind/tensor_storage.h"
#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

// inputs[i] / outputs[i] are the storages of the node; attrs points at the
// node's OpDescriptor.  Kernels enqueue work and return; they never
// allocate, free or retain storages.
using KernelFn = void (*)(const pConstTensorStorage* inputs, const pTensorStorage* outputs, const void* attrs);

enum class Op : std::uint16_t {
    NoOp = 0,
    Add,
    Sub,
    Mul,
    Div,
    Neg,
    Abs,
    Relu,
    Sigmoid,
    Tanh,
    Softmax,
    MatMul,
    ReduceSum,
    ReduceMean,
    Conv2D,
    Reshape,
    Transpose,
    Concat,
    Slice,
    Broadcast,
    Rsqrt,
    RMSNorm,
    Embedding,
    RotaryEmbedding,
    RepeatKV,
    FusedAttention,
    QuantizedMatMul,
    Last = QuantizedMatMul,
};

constexpr std::size_t MAX_OPS = static_cast<std::size_t>(Op::Last) + 1;

struct NoAttrs {};
struct BinaryAttrs {};
struct UnaryAttrs {};
struct MatMulAttrs {
    bool trans_a = false;
    bool trans_b = false;
};
struct ReduceAttrs {
    std::vector<int> axes;
    bool keepdim = false;
};
struct Conv2DAttrs {
    std::array<int, 2> padding{0, 0};
    std::array<int, 2> stride{1, 1};
    std::array<int, 2> dilation{1, 1};
    int groups = 1;
};
struct SoftmaxAttrs {
    int axis = -1;
};
struct ReshapeAttrs {
    shape_t shape;
};
struct RMSNormAttrs {
    float epsilon = 1e-5f;
    int axis = -1;
};
struct TransposeAttrs {
    std::vector<int> perm;
};
struct ConcatAttrs {
    int axis = 0;
};
struct SliceAttrs {
    std::vector<int> begins;
    std::vector<int> ends;
    std::vector<int> strides;
};
struct RepeatKVAttrs {
    int repeats = 1;
    int axis = 0;
};
struct FusedAttentionAttrs {
    float scale = 1.0f;
    bool is_causal = true;
};
// block_size == 0: one scale per output column; > 0: one scale per
// (block of K rows, column).  INT4 graphs pass the packer's block (32).
// trans_b is carried for API compatibility and, as in the reference, not read.
struct QuantizedMatMulAttrs {
    QuantType quant_type = QuantType::Int8;
    int block_size = 0;
    bool trans_b = false;
};

using OpAttrs = std::variant<NoAttrs, BinaryAttrs, UnaryAttrs, MatMulAttrs, ReduceAttrs, Conv2DAttrs, SoftmaxAttrs,
                             ReshapeAttrs, TransposeAttrs, ConcatAttrs, SliceAttrs, RMSNormAttrs, RepeatKVAttrs,
                             FusedAttentionAttrs, QuantizedMatMulAttrs>;

struct OpDescriptor {
    Op op = Op::NoOp;
    OpAttrs attrs = NoAttrs{};
};

// Registered default attributes of `op` (used when a node passes NoAttrs).
VELOMIND_CORE_EXPORT auto default_op_attrs(Op op) -> OpAttrs;

constexpr const char* op_name(Op op) {
    switch (op) {
        case Op::NoOp: return "NoOp";
        case Op::Add: return "Add";
        case Op::Sub: return "Sub";
        case Op::Mul: return "Mul";
        case Op::Div: return "Div";
        case Op::Neg: return "Neg";
        case Op::Abs: return "Abs";
        case Op::Relu: return "Relu";
        case Op::Sigmoid: return "Sigmoid";
        case Op::Tanh: return "Tanh";
        case Op::Softmax: return "Softmax";
        case Op::MatMul: return "MatMul";
        case Op::ReduceSum: return "ReduceSum";
        case Op::ReduceMean: return "ReduceMean";
        case Op::Conv2D: return "Conv2D";
        case Op::Reshape: return "Reshape";
        case Op::Transpose: return "Transpose";
        case Op::Concat: return "Concat";
        case Op::Slice: return "Slice";
        case Op::Broadcast: return "Broadcast";
        case Op::Rsqrt: return "Rsqrt";
        case Op::RMSNorm: return "RMSNorm";
        case Op::Embedding: return "Embedding";
        case Op::RotaryEmbedding: return "RotaryEmbedding";
        case Op::RepeatKV: return "RepeatKV";
        case Op::FusedAttention: return "FusedAttention";
        case Op::QuantizedMatMul: return "QuantizedMatMul";
    }
    return "Unknown";
}

inline auto to_string(Op op) -> std::string { return op_name(op); }
inline auto operator<<(std::ostream& os, Op op) -> std::ostream& { return os << op_name(op); }
inline auto to_string(const OpDescriptor& d) -> std::string { return std::string("OpDescriptor(op=") + op_name(d.op) + ")"; }
inline auto operator<<(std::ostream& os, const OpDescriptor& d) -> std::ostream& { return os << to_string(d); }

}  // namespace velomind
