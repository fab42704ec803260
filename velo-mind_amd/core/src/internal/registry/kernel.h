// Per-device operator kernel table keyed by (op, input dtypes, output
// dtype), filled at static-initialisation time by backend registration
// macros and read-only afterwards (the reference's
// src/internal/registry/kernel.h:15-43 and :192-204).
#pragma once

#include "internal/registry/macros.h"

#include <array>
#include <cstddef>
#include <span>
#include <vector>

#include "velomind/dtype.h"
#include "velomind/executable.h"
#include "velomind/ops.h"
#include "velomind/types.h"

namespace velomind::internal {

// Up to four input dtypes; num_inputs says how many take part in matching.
struct KernelDtypeKey {
    std::array<DataType, 4> input_dtypes{};
    std::size_t num_inputs = 0;
    DataType output_dtype = DataType::Float32;
};

auto operator==(const KernelDtypeKey& a, const KernelDtypeKey& b) noexcept -> bool;

struct KernelEntry {
    KernelDtypeKey key;
    Executable::KernelFn fn = nullptr;
};

auto op_kernels(DeviceType device) -> std::array<std::vector<KernelEntry>, MAX_OPS>&;

// Exact-match lookup; nullptr when no kernel is registered.
auto resolve_op_kernel(Op op, std::span<const DataType> input_dtypes, DataType output_dtype, DeviceType device)
    -> Executable::KernelFn;

auto register_op_kernel(DeviceType device, Op op, KernelDtypeKey key, Executable::KernelFn fn) -> void;

// Grouped QuantizedMatMul: sibling fp32 QuantizedMatMul nodes that read the
// same A (q | k | v, gate | up) run as one compiled step when the device
// registers a group kernel.  Its inputs are [A, B_1, scales_1, B_2,
// scales_2, ...], its outputs [C_1, C_2, ...], its attrs a QmmGroupAttrs.
// No counterpart in the reference, which runs every node on its own.
struct QmmGroupAttrs {
    OpDescriptor desc;          // the members' common descriptor
    std::size_t members = 0;    // 2 .. kMaxQmmGroup
};
inline constexpr std::size_t kMaxQmmGroup = 4;

auto register_qmm_group_kernel(DeviceType device, Executable::KernelFn fn) -> void;
// nullptr when the device has none (its QuantizedMatMul nodes run one by one)
auto qmm_group_kernel(DeviceType device) -> Executable::KernelFn;

// Fused steps: a chain of graph nodes that a device runs as one launch,
// the chain's intermediates never materialised.  A device registers one
// kernel per kind; the graph compiler matches the chains
// (graph_compiler.cpp) and hands the kernel the chain's external operands.
// No counterpart in the reference, which runs every node on its own.
enum class FusedKind : int {
    SiluMul = 0,          // Mul(Mul(Sigmoid(g), g), u): inputs [g, u], outputs [y]
    QmmAdd = 1,           // Add(h, QuantizedMatMul(A, B, S)): inputs [A, B, S, h], outputs [C];
                          // attrs the QuantizedMatMul's OpDescriptor
    AttentionDecode = 2,  // one query row per head: RepeatKV(K), RepeatKV(V), Transpose(K),
                          // MatMul, Softmax, MatMul: inputs [q, K, V] (K/V before RepeatKV),
                          // outputs [ctx]
    AttentionGqa = 3,     // FusedAttention on RepeatKV(K), RepeatKV(V): inputs [q, K, V]
                          // (before RepeatKV), outputs [o]; attrs the FusedAttention's OpDescriptor
    RopeAppend = 4,       // one decode position: RoPE(q), Concat(K_past, RoPE(k)), Concat(V_past, v):
                          // inputs [q, k, v, K_past, V_past, cos, sin], outputs [q', K, V]
    NormQmm = 5,          // QuantizedMatMul(s) of RMSNorm(x, w): inputs [x, w, B_1, S_1, ..],
                          // outputs [C_1, ..]; attrs a NormQmmAttrs
    SwigluQmmAdd = 6,     // Add(h, QuantizedMatMul(Mul(Mul(Sigmoid(g), g), u), B, S)): inputs
                          // [g, u, B, S, h], outputs [C]; attrs the QuantizedMatMul's OpDescriptor
};
inline constexpr std::size_t kFusedKinds = 7;

struct NormQmmAttrs {
    OpDescriptor desc;          // the QuantizedMatMuls' common descriptor
    std::size_t members = 0;    // 1 .. kMaxQmmGroup
    float epsilon = 0.0f;       // the RMSNorm's
};

auto register_fused_kernel(DeviceType device, FusedKind kind, Executable::KernelFn fn) -> void;
// nullptr when the device does not run that chain fused
auto fused_kernel(DeviceType device, FusedKind kind) -> Executable::KernelFn;

template <DataType D> struct dtype_to_type;
template <> struct dtype_to_type<DataType::Float32> { using type = float; };
template <> struct dtype_to_type<DataType::Int32> { using type = std::int32_t; };
template <> struct dtype_to_type<DataType::Int8> { using type = std::int8_t; };
template <> struct dtype_to_type<DataType::Bool> { using type = bool; };
template <> struct dtype_to_type<DataType::Float16> { using type = float16_t; };
template <> struct dtype_to_type<DataType::BFloat16> { using type = bfloat16_t; };
template <DataType D> using dtype_t = typename dtype_to_type<D>::type;

}  // namespace velomind::internal


// Registers FN for (DEVICE, OP_ENUM, KEY) during static initialisation.
#define VELOMIND_REGISTER_OP_KERNEL(DEVICE, OP_ENUM, KEY, ...)                                    \
    [[maybe_unused]] static const bool VELOMIND_CONCAT_(_velomind_kr_, __LINE__) = [] {          \
        ::velomind::internal::register_op_kernel((DEVICE), (OP_ENUM), (KEY), (__VA_ARGS__));     \
        return true;                                                                             \
    }();

// QuantizedMatMul: inputs (A: TA, B_q: Int8, scales: TSCALE) -> TC, with
// NAME a template over the three element types.
#define VELOMIND_REGISTER_QUANTIZED_MATMUL(DEVICE, TA_DT, TSCALE_DT, TC_DT, NAME)                 \
    VELOMIND_REGISTER_OP_KERNEL(                                                                 \
        (DEVICE), ::velomind::Op::QuantizedMatMul,                                               \
        (::velomind::internal::KernelDtypeKey{{(TA_DT), ::velomind::DataType::Int8, (TSCALE_DT)}, \
                                              3, (TC_DT)}),                                       \
        (&NAME<::velomind::internal::dtype_t<TA_DT>, ::velomind::internal::dtype_t<TSCALE_DT>,    \
               ::velomind::internal::dtype_t<TC_DT>>))

// Registers FN as DEVICE's kernel for the fused chain KIND.
#define VELOMIND_REGISTER_FUSED(DEVICE, KIND, FN)                                                  \
    [[maybe_unused]] static const bool VELOMIND_CONCAT_(_velomind_fz_, __LINE__) = [] {          \
        ::velomind::internal::register_fused_kernel((DEVICE), (KIND), (FN));                     \
        return true;                                                                             \
    }();

// Registers FN as DEVICE's grouped QuantizedMatMul kernel.
#define VELOMIND_REGISTER_QMM_GROUP(DEVICE, FN)                                                   \
    [[maybe_unused]] static const bool VELOMIND_CONCAT_(_velomind_qg_, __LINE__) = [] {          \
        ::velomind::internal::register_qmm_group_kernel((DEVICE), (FN));                         \
        return true;                                                                             \
    }();
