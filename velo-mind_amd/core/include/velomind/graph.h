// Graph: owns every tensor storage and node of a DAG.  Building a graph
// records shapes (through the operator signature registry) and edges only;
// Graph::build(device) plans memory, allocates it on `device` and resolves
// kernels into an Executable.  Mirrors the reference's
// include/velomind/graph.h:50-137.
#pragma once

#include <array>
#include <cstddef>
#include <memory>
#include <optional>
#include <stdexcept>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "velomind/node.h"
#include "velomind/ops.h"
#include "velomind/ptr.h"
#include "velomind/tensor.h"
#include "velomind/tensor_storage.h"
#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

class Executable;
namespace internal {
class GraphCompiler;
class TensorIndex;
}

template <typename T>
concept TensorHandle = std::is_same_v<std::remove_cvref_t<T>, Tensor>;
template <typename... Ts>
concept AllTensorHandles = (TensorHandle<Ts> && ...);

inline constexpr std::size_t DEFAULT_TENSOR_CAPACITY = 64;
inline constexpr std::size_t DEFAULT_NODE_CAPACITY = 32;
inline constexpr std::size_t MAX_TENSORS_PER_GRAPH = 1U << 16;

// Outcome of the build-time memory plan.
struct MemoryPlanStats {
    std::size_t peak_bytes = 0;                 // arena + dedicated bytes
    std::size_t allocation_count = 0;           // physical allocations made
    std::size_t intermediate_tensor_count = 0;  // tensors placed in the arena
    std::size_t reused_tensor_count = 0;        // tensors sharing bytes with another
    std::size_t bytes_saved = 0;                // versus one allocation per tensor
};

class VELOMIND_CORE_EXPORT Graph {
public:
    explicit Graph(std::size_t initial_tensor_capacity = DEFAULT_TENSOR_CAPACITY,
                   std::size_t initial_node_capacity = DEFAULT_NODE_CAPACITY);
    ~Graph();
    Graph(const Graph&) = delete;
    Graph& operator=(const Graph&) = delete;
    Graph(Graph&&) = delete;
    Graph& operator=(Graph&&) = delete;

    auto reserve(std::size_t tensor_capacity, std::size_t node_capacity = 0) -> void;
    auto tensor_capacity() const noexcept -> std::size_t { return _tensors.capacity(); }
    auto node_capacity() const noexcept -> std::size_t { return _nodes.capacity(); }

    // Declares an input (allocated at build time).
    auto input(shape_t shape, DataType dtype) -> Tensor;
    // Adopts an existing storage (e.g. shared weights) as an input.
    auto input(std::shared_ptr<TensorStorage> storage) -> Tensor;

    auto tensor_storage_at(std::size_t i) const -> pConstTensorStorage;
    auto shared_storage_at(std::size_t i) const -> std::shared_ptr<TensorStorage>;
    auto tensor_storage_at(std::size_t i) -> pTensorStorage;
    auto tensor_count() const noexcept -> std::size_t { return _tensors.size(); }
    auto is_input_tensor(std::size_t i) const noexcept -> bool;
    auto is_output_tensor(std::size_t i) const noexcept -> bool;
    auto lifetime_token() const noexcept -> std::weak_ptr<void> { return _lifetime; }

    // Appends a node; its output's shape and dtype come from the op signature.
    template <typename... Inputs>
        requires AllTensorHandles<Inputs...>
    auto op(Op op, Inputs&&... inputs) -> Tensor;
    template <typename... Inputs>
        requires AllTensorHandles<Inputs...>
    auto op(OpDescriptor desc, Inputs&&... inputs) -> Tensor;

    auto mark_output(Tensor tensor) -> void;
    auto set_outputs(std::vector<Tensor> outputs) -> void;
    auto outputs() const -> std::vector<Tensor>;
    auto has_explicit_outputs() const noexcept -> bool { return _has_explicit_outputs; }

    // Signatures, kernel availability on `device` and acyclicity; allocates nothing.
    auto validate(DeviceType device) const -> void;
    // Dead-code elimination, topological order, liveness-based arena plan,
    // allocation on `device`, kernel resolution.
    auto build(DeviceType device) -> std::unique_ptr<Executable>;

    auto is_built() const noexcept -> bool { return _built; }
    auto bound_device() const noexcept -> std::optional<DeviceType> {
        return _built ? std::make_optional(_bound_device) : std::nullopt;
    }
    auto memory_plan_stats() const noexcept -> const std::optional<MemoryPlanStats>& { return _plan_stats; }
    auto node_count() const noexcept -> std::size_t { return _nodes.size(); }
    auto node_tot() const -> std::size_t { return _nodes.size(); }

private:
    auto _op_impl(OpDescriptor desc, std::span<const pConstTensorStorage> inputs) -> Tensor;
    auto _compute_required_nodes() const -> std::vector<bool>;
    auto _topological_order() const -> std::vector<pConstNode>;
    auto _topological_order(const std::vector<bool>& req) const -> std::vector<pConstNode>;
    // validate()'s checks; returns the topological order of the required
    // nodes (the build's order, computed once).
    auto _validated_order(DeviceType device) const -> std::vector<pConstNode>;
    // The same with the caller's index of _tensors (the build reuses it).
    auto _validated_order(DeviceType device, const internal::TensorIndex& index) const -> std::vector<pConstNode>;

    friend struct GraphTestAccess;
    friend class internal::GraphCompiler;

    std::vector<std::shared_ptr<TensorStorage>> _tensors;
    std::vector<Node> _nodes;
    bool _built = false;
    DeviceType _bound_device = DeviceType::CPU;
    bool _has_explicit_outputs = false;
    std::vector<pConstTensorStorage> _explicit_outputs;
    std::optional<MemoryPlanStats> _plan_stats;
    std::shared_ptr<void> _lifetime;
};

template <typename... Inputs>
    requires AllTensorHandles<Inputs...>
auto Graph::op(Op op_kind, Inputs&&... inputs) -> Tensor {
    return op(OpDescriptor{op_kind, NoAttrs{}}, std::forward<Inputs>(inputs)...);
}

template <typename... Inputs>
    requires AllTensorHandles<Inputs...>
auto Graph::op(OpDescriptor desc, Inputs&&... inputs) -> Tensor {
    if (_built) throw std::logic_error("Graph::op: graph is already built");
    if (((inputs.graph() != this || inputs.storage() == nullptr) || ...))
        throw std::invalid_argument("Graph::op: invalid or foreign tensor handle");
    const std::array<pConstTensorStorage, sizeof...(Inputs)> ptrs{inputs.storage()...};
    return _op_impl(std::move(desc), std::span<const pConstTensorStorage>(ptrs.data(), ptrs.size()));
}

VELOMIND_EXPORT_PTR(Graph);

}  // namespace velomind
