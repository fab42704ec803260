// Compiled execution plan of a Graph: resolved kernels in topological order
// plus the backend's execution context (for HIP: the stream).  The owning
// Graph must outlive it.  Mirrors the reference's
// include/velomind/executable.h:176-242.
#pragma once

#include <cstddef>
#include <array>
#include <memory>
#include <vector>

#include "velomind/graph.h"
#include "velomind/inline_list.h"
#include "velomind/tensor.h"
#include "velomind/tensor_storage.h"
#include "velomind_core_export.h"

namespace velomind {

// An externally owned buffer bound to a graph input without a copy.
struct ExternalBuffer {
    void* data = nullptr;
    std::size_t capacity_bytes = 0;
    DeviceType device = DeviceType::CPU;
    std::shared_ptr<void> owner;
};

class VELOMIND_CORE_EXPORT Executable {
public:
    using KernelFn = ::velomind::KernelFn;

    struct CompiledNode {
        KernelFn kernel = nullptr;
        InlineList<pConstTensorStorage, 8> inputs;
        InlineList<pTensorStorage, 4> outputs;
        std::shared_ptr<const void> attrs;  // the node's OpDescriptor (fused > 1: the group's attrs)
        std::size_t fused = 1;              // graph nodes this step runs (sibling QuantizedMatMuls)
    };

    // A storage the plan reads or writes, with the metadata it had at build
    // time (the fields a run re-checks).  Each storage appears once, however
    // many nodes touch it.
    struct FrozenLayout {
        // The shape: inline up to kInlineRank dimensions (no allocation per
        // watched storage and build), else in `shape`.
        static constexpr std::size_t kInlineRank = 6;
        std::array<dim_t, kInlineRank> dims{};
        std::size_t rank = 0;
        shape_t shape;
        DataType dtype = DataType::Float32;
        DeviceType device = DeviceType::CPU;
        std::size_t size_bytes = 0;
    };
    struct WatchedStorage {
        pConstTensorStorage live = nullptr;
        FrozenLayout frozen;
    };

    // Embedding node whose device-resident indices are read back and range
    // checked before the node launches.
    struct IndexGuard {
        std::size_t node = 0;               // position in topo
        pConstTensorStorage indices = nullptr;
        dim_t vocab_rows = 0;
    };

    struct Impl {
        pConstGraph graph = nullptr;
        std::weak_ptr<void> graph_lifetime;
        DeviceType device = DeviceType::CPU;
        std::vector<CompiledNode> topo;         // the steps, in order
        std::size_t node_count = 0;              // graph nodes the steps run
        std::vector<WatchedStorage> watched;
        std::vector<IndexGuard> index_guards;   // ascending node order
        MemoryPlanStats plan_stats;
        // Backend execution context created by the device's context hook.
        std::shared_ptr<void> device_context;

        // Fills `watched` and `index_guards` from `topo` (called once, at build).
        void derive_run_plan();
    };

    Executable() = default;
    ~Executable();
    Executable(const Executable&) = delete;
    Executable& operator=(const Executable&) = delete;
    Executable(Executable&&) noexcept;
    Executable& operator=(Executable&&) noexcept;

    // Runs every node in order; for GPU devices work is enqueued on the
    // context's stream and the stream is synchronized before returning.
    auto execute() -> void;
    auto bind_input(Tensor tensor, ExternalBuffer external_buffer) -> void;
    auto output(Tensor tensor) -> pTensorStorage;
    auto output(Tensor tensor) const -> pConstTensorStorage;
    auto memory_plan_stats() const noexcept -> const MemoryPlanStats&;
    auto num_nodes() const -> std::size_t;
    // Kernel steps a run enqueues: num_nodes() less the nodes that run
    // grouped with a sibling.
    auto num_steps() const -> std::size_t;
    auto empty() const -> bool { return num_nodes() == 0; }

private:
    friend class Graph;
    friend class internal::GraphCompiler;
    std::unique_ptr<Impl> _impl;
};

}  // namespace velomind
