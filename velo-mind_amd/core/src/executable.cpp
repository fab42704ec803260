// Executable: replays a compiled plan.
//
// The work that does not depend on the run is done once, at build
// (Impl::derive_run_plan): the set of distinct storages the plan touches,
// each with a frozen copy of its metadata, and the positions of the
// Embedding nodes whose indices must be range checked on the host.  A run
// then (1) verifies every watched storage against its frozen copy, before
// anything is launched, so a bad tensor late in the plan cannot leave
// earlier outputs half-written; (2) enqueues the kernels in order under the
// device's execution context, pausing at each index guard to drain the
// context and read the indices back; (3) drains the context before
// returning.  The device context hooks stand in for the reference's CUDA
// blocks; the checks, their order and messages are the reference's contract
// (src/executable.cpp:27-81, :83-109).
#include "velomind/executable.h"

#include <cstdint>
#include <stdexcept>
#include <algorithm>
#include <vector>

#include "internal/registry/device_context.h"
#include "internal/registry/memory_transfer.h"
#include "velomind/graph.h"

namespace velomind {

namespace {

// Waits for the work enqueued on an executable's context, if it has one.
class ContextDrain {
public:
    ContextDrain(DeviceType device, void* ctx) : _sync(internal::get_device_context_hooks(device).synchronize), _ctx(ctx) {}
    void operator()() const {
        if (_sync && _ctx) _sync(_ctx);
    }

private:
    void (*_sync)(void*) = nullptr;
    void* _ctx = nullptr;
};

void require_live(const Executable::Impl* impl, const char* who) {
    if (!impl) throw std::logic_error(std::string(who) + ": not built");
    if (impl->graph_lifetime.expired()) throw std::logic_error(std::string(who) + ": owning graph has been destroyed");
}

Executable::FrozenLayout freeze(const TensorStorage& s) {
    Executable::FrozenLayout f;
    f.rank = s.shape.size();
    if (f.rank <= f.dims.size())
        std::copy(s.shape.begin(), s.shape.end(), f.dims.begin());
    else
        f.shape = s.shape;
    f.dtype = s.dtype;
    f.device = s.device;
    f.size_bytes = s.size_bytes;
    return f;
}

bool same_shape(const shape_t& a, const Executable::FrozenLayout& b) {
    if (a.size() != b.rank) return false;
    if (b.rank > b.dims.size()) return a == b.shape;
    return std::equal(a.begin(), a.end(), b.dims.begin());
}

bool same_layout(const TensorStorage& a, const Executable::FrozenLayout& b) {
    return same_shape(a.shape, b) && a.dtype == b.dtype && a.device == b.device && a.size_bytes == b.size_bytes;
}

void verify_watched(const Executable::WatchedStorage& w) {
    if (!same_layout(*w.live, w.frozen))
        throw std::invalid_argument("Executable::execute: tensor metadata changed after build");
    if (!w.live->data && storage_nbytes(*w.live) > 0)
        throw std::invalid_argument("Executable::execute: tensor buffer is null");
}

// Embedding indices may be produced by an earlier node on the device, so
// the guard drains the context first and checks the values actually there
// (the reference's executable.cpp:54-72).
void check_index_guard(const Executable::IndexGuard& g, const ContextDrain& drain) {
    const std::size_t count = storage_numel(*g.indices);
    if (count == 0) return;
    drain();
    const auto transfer = internal::get_memory_transfer(g.indices->device);
    if (!transfer.copy_d2h) throw std::runtime_error("Embedding: no index readback transfer");
    std::vector<std::int32_t> host(count);
    transfer.copy_d2h(host.data(), g.indices->data, count * sizeof(std::int32_t));
    for (const std::int32_t v : host)
        if (v < 0 || static_cast<dim_t>(v) >= g.vocab_rows)
            throw std::invalid_argument("Embedding: index out of vocabulary range");
}

// First violated rule of Executable::bind_input, or nullptr (the rules and
// their order are the reference's, src/executable.cpp:83-109).
const char* bind_violation(const TensorStorage& slot, const ExternalBuffer& buf, DeviceType plan_device) {
    if (buf.device != plan_device || slot.device != plan_device) return "device mismatch";
    if (buf.capacity_bytes < slot.size_bytes) return "insufficient buffer capacity";
    const bool needs_memory = slot.size_bytes > 0;
    if (needs_memory && (buf.data == nullptr || buf.owner == nullptr)) return "nonempty buffer requires data and owner";
    if (buf.owner && buf.owner.get() != buf.data) return "owner must alias buffer data";
    if (buf.data && reinterpret_cast<std::uintptr_t>(buf.data) % data_type_size(slot.dtype) != 0)
        return "unaligned buffer";
    return nullptr;
}

}  // namespace

void Executable::Impl::derive_run_plan() {
    watched.clear();
    index_guards.clear();
    // Storages already watched: an open-addressing set of pointers in one
    // array (a node-based set allocated once per storage and build).
    std::size_t operands = 16;
    for (const auto& cn : topo) operands += cn.inputs.size() + cn.outputs.size();
    std::size_t cap = 16;
    while (cap < 2 * operands) cap <<= 1;
    std::vector<pConstTensorStorage> seen(cap, nullptr);
    watched.reserve(operands);
    auto watch = [&](pConstTensorStorage s) {
        std::size_t h = (reinterpret_cast<std::uintptr_t>(s) >> 4) * 0x9E3779B97F4A7C15ull;
        for (std::size_t i = h & (cap - 1);; i = (i + 1) & (cap - 1)) {
            if (seen[i] == s) return;
            if (seen[i] == nullptr) {
                seen[i] = s;
                break;
            }
        }
        watched.push_back(WatchedStorage{s, freeze(*s)});
    };
    for (std::size_t i = 0; i < topo.size(); ++i) {
        const CompiledNode& cn = topo[i];
        for (pConstTensorStorage s : cn.inputs) watch(s);
        for (pConstTensorStorage s : cn.outputs) watch(s);
        if (cn.fused > 1) continue;   // grouped QuantizedMatMuls: no index guard
        const auto& desc = *static_cast<const OpDescriptor*>(cn.attrs.get());
        if (desc.op == Op::Embedding && cn.inputs.size() >= 2)
            index_guards.push_back(IndexGuard{i, cn.inputs[1], cn.inputs[0]->shape.empty() ? 0 : cn.inputs[0]->shape[0]});
    }
}

Executable::~Executable() {
    if (!_impl || !_impl->device_context) return;
    try {
        ContextDrain(_impl->device, _impl->device_context.get())();
    } catch (...) {
        // a destructor must not throw; the error was the last run's to report
    }
}

Executable::Executable(Executable&&) noexcept = default;
Executable& Executable::operator=(Executable&&) noexcept = default;

auto Executable::execute() -> void {
    require_live(_impl.get(), "Executable::execute");
    Impl& plan = *_impl;
    for (const WatchedStorage& w : plan.watched) verify_watched(w);

    const ContextDrain drain(plan.device, plan.device_context.get());
    internal::ScopedDeviceContext scope(plan.device, plan.device_context.get());
    auto guard = plan.index_guards.cbegin();
    for (std::size_t i = 0; i < plan.topo.size(); ++i) {
        for (; guard != plan.index_guards.cend() && guard->node == i; ++guard) check_index_guard(*guard, drain);
        const CompiledNode& cn = plan.topo[i];
        cn.kernel(cn.inputs.data(), cn.outputs.data(), cn.attrs.get());
    }
    drain();
}

auto Executable::bind_input(Tensor t, ExternalBuffer buf) -> void {
    require_live(_impl.get(), "Executable::bind_input");
    if (t.graph() != _impl->graph || !t.storage()) throw std::invalid_argument("Executable::bind_input: invalid or foreign tensor");
    auto* owner_graph = const_cast<Graph*>(_impl->graph);
    if (!owner_graph->is_input_tensor(t.index()))
        throw std::invalid_argument("Executable::bind_input: tensor is not a graph input");
    TensorStorage* slot = owner_graph->tensor_storage_at(t.index());
    if (const char* why = bind_violation(*slot, buf, _impl->device))
        throw std::invalid_argument(std::string("Executable::bind_input: ") + why);
    slot->data = buf.data;
    slot->external_owner = std::move(buf.owner);
}

auto Executable::output(Tensor t) -> pTensorStorage {
    const auto* self = this;
    return const_cast<pTensorStorage>(self->output(t));
}

auto Executable::output(Tensor t) const -> pConstTensorStorage {
    if (!_impl || _impl->graph_lifetime.expired() || t.graph() != _impl->graph) return nullptr;
    return _impl->graph->tensor_storage_at(t.index());
}

auto Executable::num_nodes() const -> std::size_t { return _impl ? _impl->node_count : 0; }

auto Executable::num_steps() const -> std::size_t { return _impl ? _impl->topo.size() : 0; }

auto Executable::memory_plan_stats() const noexcept -> const MemoryPlanStats& {
    static const MemoryPlanStats empty;
    return _impl ? _impl->plan_stats : empty;
}

}  // namespace velomind
