// Executable: runs compiled nodes in order under the device's execution
// context and synchronizes at the boundary (the reference's
// src/executable.cpp, with the CUDA #ifdefs replaced by the registered
// device-context hooks).
#include "velomind/executable.h"

#include <cstdint>
#include <stdexcept>
#include <vector>

#include "internal/registry/device_context.h"
#include "internal/registry/memory_transfer.h"
#include "velomind/graph.h"

namespace velomind {

Executable::~Executable() {
    if (_impl && _impl->device_context) {
        const auto hooks = internal::get_device_context_hooks(_impl->device);
        if (hooks.synchronize) {
            try {
                hooks.synchronize(_impl->device_context.get());
            } catch (...) {
            }
        }
    }
}

Executable::Executable(Executable&&) noexcept = default;
Executable& Executable::operator=(Executable&&) noexcept = default;

auto Executable::execute() -> void {
    if (!_impl) throw std::logic_error("Executable::execute: not built");
    if (_impl->graph_lifetime.expired()) throw std::logic_error("Executable::execute: owning graph has been destroyed");
    const auto check = [](const TensorStorage& now, const TensorStorage& then) {
        if (now.shape != then.shape || now.dtype != then.dtype || now.device != then.device ||
            now.size_bytes != then.size_bytes)
            throw std::invalid_argument("Executable::execute: tensor metadata changed after build");
        if (storage_nbytes(now) > 0 && !now.data) throw std::invalid_argument("Executable::execute: tensor buffer is null");
    };
    // Check every node first so that a bad late node cannot leave earlier
    // outputs half-written.
    for (const auto& cn : _impl->topo) {
        for (std::size_t i = 0; i < cn.inputs.size(); ++i) check(*cn.inputs[i], cn.input_metadata[i]);
        for (std::size_t i = 0; i < cn.outputs.size(); ++i) check(*cn.outputs[i], cn.output_metadata[i]);
    }
    const auto hooks = internal::get_device_context_hooks(_impl->device);
    internal::ScopedDeviceContext scope(_impl->device, _impl->device_context.get());
    for (auto& cn : _impl->topo) {
        const auto& desc = *static_cast<const OpDescriptor*>(cn.attrs.get());
        if (desc.op == Op::Embedding) {
            // Indices may come from an earlier node: read them back and
            // range-check before the gather (executable.cpp:54-72).
            const auto& idx = *cn.inputs[1];
            const auto count = storage_numel(idx);
            std::vector<std::int32_t> host(count);
            if (count) {
                if (hooks.synchronize && _impl->device_context) hooks.synchronize(_impl->device_context.get());
                const auto t = internal::get_memory_transfer(idx.device);
                if (!t.copy_d2h) throw std::runtime_error("Embedding: no index readback transfer");
                t.copy_d2h(host.data(), idx.data, count * sizeof(std::int32_t));
            }
            for (auto v : host)
                if (v < 0 || v >= cn.inputs[0]->shape[0])
                    throw std::invalid_argument("Embedding: index out of vocabulary range");
        }
        cn.kernel(cn.inputs.data(), cn.outputs.data(), cn.attrs.get());
    }
    if (hooks.synchronize && _impl->device_context) hooks.synchronize(_impl->device_context.get());
}

auto Executable::bind_input(Tensor t, ExternalBuffer buf) -> void {
    if (!_impl) throw std::logic_error("Executable::bind_input: not built");
    if (_impl->graph_lifetime.expired()) throw std::logic_error("Executable::bind_input: owning graph has been destroyed");
    if (t.graph() != _impl->graph || !t.storage()) throw std::invalid_argument("Executable::bind_input: invalid or foreign tensor");
    auto* g = const_cast<Graph*>(_impl->graph);
    if (!g->is_input_tensor(t.index())) throw std::invalid_argument("Executable::bind_input: tensor is not a graph input");
    auto* s = g->tensor_storage_at(t.index());
    if (buf.device != _impl->device || s->device != _impl->device)
        throw std::invalid_argument("Executable::bind_input: device mismatch");
    if (buf.capacity_bytes < s->size_bytes) throw std::invalid_argument("Executable::bind_input: insufficient buffer capacity");
    if (s->size_bytes > 0 && (!buf.data || !buf.owner))
        throw std::invalid_argument("Executable::bind_input: nonempty buffer requires data and owner");
    if (buf.owner && buf.owner.get() != buf.data) throw std::invalid_argument("Executable::bind_input: owner must alias buffer data");
    if (buf.data && reinterpret_cast<std::uintptr_t>(buf.data) % data_type_size(s->dtype) != 0)
        throw std::invalid_argument("Executable::bind_input: unaligned buffer");
    s->external_owner = std::move(buf.owner);
    s->data = buf.data;
}

auto Executable::output(Tensor t) -> pTensorStorage {
    if (!_impl || _impl->graph_lifetime.expired() || t.graph() != _impl->graph) return nullptr;
    return const_cast<Graph*>(_impl->graph)->tensor_storage_at(t.index());
}

auto Executable::output(Tensor t) const -> pConstTensorStorage {
    if (!_impl || _impl->graph_lifetime.expired() || t.graph() != _impl->graph) return nullptr;
    return _impl->graph->tensor_storage_at(t.index());
}

auto Executable::num_nodes() const -> std::size_t { return _impl ? _impl->topo.size() : 0; }

auto Executable::memory_plan_stats() const noexcept -> const MemoryPlanStats& {
    static const MemoryPlanStats empty;
    return _impl ? _impl->plan_stats : empty;
}

}  // namespace velomind
