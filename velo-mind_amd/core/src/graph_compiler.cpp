// Memory planning and compilation of a Graph into an Executable.
//
// Plan: every tensor the ordered nodes touch is "active".  Graph inputs,
// tensors that already own data and the requested outputs (every active
// tensor when no outputs were marked) get dedicated allocations; the other
// active tensors are intermediates with a lifetime [producer step, last
// consumer step].  Intermediates are packed into ONE arena allocation:
// largest first (ties: longer lifetime, earlier birth, lower index), each at
// the lowest offset that does not overlap a placed intermediate whose
// lifetime intersects its own, slots rounded up to 256 bytes.  On HIP the
// arena is a single device allocation.
//
// Everything is staged on copies of the graph's storage list and only
// committed after the last allocation, so a failed build leaves the graph
// unchanged and buildable again.  VELOMIND_FAIL_GRAPH_BUILD_AFTER_ALLOCATIONS=N
// injects a failure after the N-th allocation (the reference's hook of the
// same name, src/internal/graph_compiler.cpp:563-568).
#include "internal/graph_compiler.h"

#include <algorithm>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "internal/registry/device_context.h"
#include "internal/registry/kernel.h"
#include "internal/registry/storage.h"

namespace velomind::internal {

namespace {

struct Interval {
    std::size_t tensor = 0;  // index into Graph::_tensors
    std::size_t birth = 0;
    std::size_t death = 0;
    std::size_t bytes = 0;
    std::size_t slot = 0;    // bytes rounded up to the arena alignment
    std::size_t offset = 0;
};

std::size_t align_up(std::size_t v, std::size_t a) { return (v + a - 1) / a * a; }

bool lifetimes_overlap(const Interval& a, const Interval& b) {
    return std::max(a.birth, b.birth) <= std::min(a.death, b.death);
}

// Places intervals; returns the arena size.
std::size_t plan_arena(std::vector<Interval>& items) {
    std::sort(items.begin(), items.end(), [](const Interval& a, const Interval& b) {
        if (a.bytes != b.bytes) return a.bytes > b.bytes;
        const std::size_t da = a.death - a.birth, db = b.death - b.birth;
        if (da != db) return da > db;
        if (a.birth != b.birth) return a.birth < b.birth;
        return a.tensor < b.tensor;
    });
    std::size_t total = 0;
    for (std::size_t i = 0; i < items.size(); ++i) {
        Interval& cur = items[i];
        std::vector<const Interval*> live;
        for (std::size_t j = 0; j < i; ++j)
            if (lifetimes_overlap(items[j], cur)) live.push_back(&items[j]);
        std::vector<std::size_t> candidates{0};
        for (const auto* p : live) candidates.push_back(p->offset + p->slot);
        std::sort(candidates.begin(), candidates.end());
        cur.offset = candidates.back();
        for (std::size_t cand : candidates) {
            bool clash = false;
            for (const auto* p : live)
                if (std::max(cand, p->offset) < std::min(cand + cur.slot, p->offset + p->slot)) {
                    clash = true;
                    break;
                }
            if (!clash) {
                cur.offset = cand;
                break;
            }
        }
        total = std::max(total, cur.offset + cur.slot);
    }
    return total;
}

std::size_t injected_failure_point() {
    const char* v = std::getenv("VELOMIND_FAIL_GRAPH_BUILD_AFTER_ALLOCATIONS");
    if (!v || !*v) return 0;
    char* end = nullptr;
    const unsigned long long n = std::strtoull(v, &end, 10);
    return (end && *end == '\0') ? static_cast<std::size_t>(n) : 0;
}

std::shared_ptr<TensorStorage> allocate_checked(std::size_t bytes, DeviceType device) {
    auto s = TensorStorage::allocate(bytes, device);
    if (!s || s->device != device || s->size_bytes < bytes || (bytes > 0 && s->data == nullptr))
        throw std::runtime_error("velomind: backend allocator returned invalid storage for " + std::to_string(bytes) +
                                 " bytes on device [" + device_type_name(device) + "]");
    return s;
}

}  // namespace

auto GraphCompiler::compile(Graph& graph, DeviceType device) -> std::unique_ptr<Executable> {
    if (graph._built) throw std::logic_error("Graph::build: graph is already built");
    graph.validate(device);
    const auto order = graph._topological_order();
    const auto& tensors = graph._tensors;

    std::unordered_map<pConstTensorStorage, std::size_t> index_of;
    for (std::size_t i = 0; i < tensors.size(); ++i) index_of[tensors[i].get()] = i;

    // Activity and lifetimes.
    std::vector<bool> active(tensors.size(), false);
    std::vector<std::size_t> birth(tensors.size(), 0), death(tensors.size(), 0);
    std::vector<bool> born(tensors.size(), false);
    for (std::size_t step = 0; step < order.size(); ++step) {
        for (auto* in : order[step]->inputs()) {
            const auto i = index_of.at(in);
            active[i] = true;
            death[i] = std::max(death[i], step);
        }
        for (auto* out : order[step]->outputs()) {
            const auto i = index_of.at(out);
            active[i] = true;
            if (!born[i]) {
                born[i] = true;
                birth[i] = step;
            }
            death[i] = std::max(death[i], step);
        }
    }
    std::vector<bool> dedicated(tensors.size(), false);
    if (graph._has_explicit_outputs) {
        for (auto* s : graph._explicit_outputs) {
            const auto i = index_of.at(s);
            active[i] = true;
            dedicated[i] = true;
        }
    } else {
        for (std::size_t i = 0; i < tensors.size(); ++i) {
            active[i] = true;
            dedicated[i] = true;
        }
    }
    for (std::size_t i = 0; i < tensors.size(); ++i)
        if (tensors[i]->data != nullptr || graph.is_input_tensor(i)) dedicated[i] = true;

    std::vector<Interval> arena_items;
    for (std::size_t i = 0; i < tensors.size(); ++i) {
        if (!active[i] || dedicated[i] || tensors[i]->size_bytes == 0) continue;
        arena_items.push_back(Interval{i, birth[i], std::max(birth[i], death[i]), tensors[i]->size_bytes,
                                       align_up(tensors[i]->size_bytes, kArenaAlignment), 0});
    }
    const std::size_t arena_bytes = plan_arena(arena_items);

    bool needs_alloc = arena_bytes > 0;
    for (std::size_t i = 0; i < tensors.size(); ++i)
        if (active[i] && dedicated[i] && tensors[i]->data == nullptr) needs_alloc = true;
    if (needs_alloc && get_storage_creator(device) == nullptr)
        throw std::runtime_error(std::string("velomind: no backend allocator registered for device [") +
                                 device_type_name(device) + "]");

    // Stage allocations.
    const std::size_t fail_after = injected_failure_point();
    std::size_t allocations = 0;
    auto count_allocation = [&] {
        if (fail_after != 0 && ++allocations == fail_after)
            throw std::runtime_error("Graph::build: injected allocation-stage failure");
    };
    std::vector<std::shared_ptr<TensorStorage>> staged = tensors;
    MemoryPlanStats stats;
    if (arena_bytes > 0) {
        auto arena = allocate_checked(arena_bytes, device);
        ++stats.allocation_count;
        count_allocation();
        for (const auto& it : arena_items) {
            const auto& src = *tensors[it.tensor];
            auto view = std::make_shared<TensorStorage>();
            view->shape = src.shape;
            view->strides = src.strides.empty() ? default_strides(src.shape) : src.strides;
            view->dtype = src.dtype;
            view->device = device;
            view->size_bytes = src.size_bytes;
            view->offset_bytes = it.offset;
            view->capacity_bytes = arena->capacity_bytes;
            view->data = static_cast<char*>(arena->data) + it.offset;
            view->external_owner = arena;
            staged[it.tensor] = std::move(view);
        }
    }
    std::size_t dedicated_bytes = 0;
    for (std::size_t i = 0; i < tensors.size(); ++i) {
        if (!active[i] || !dedicated[i]) continue;
        const auto& src = *tensors[i];
        dedicated_bytes += src.size_bytes;
        if (src.data != nullptr) continue;
        auto buf = allocate_checked(src.size_bytes, device);
        buf->shape = src.shape;
        buf->strides = src.strides.empty() ? default_strides(src.shape) : src.strides;
        buf->dtype = src.dtype;
        ++stats.allocation_count;
        count_allocation();
        staged[i] = std::move(buf);
    }

    stats.peak_bytes = arena_bytes + dedicated_bytes;
    stats.intermediate_tensor_count = arena_items.size();
    std::size_t unshared = 0;
    for (const auto& it : arena_items) {
        unshared += it.bytes;
        for (const auto& other : arena_items) {
            if (&other == &it || other.death >= it.birth) continue;
            if (std::max(it.offset, other.offset) < std::min(it.offset + it.slot, other.offset + other.slot)) {
                ++stats.reused_tensor_count;
                break;
            }
        }
    }
    stats.bytes_saved = unshared > arena_bytes ? unshared - arena_bytes : 0;

    std::unordered_map<pConstTensorStorage, pTensorStorage> remap;
    for (std::size_t i = 0; i < tensors.size(); ++i) remap[tensors[i].get()] = staged[i].get();

    // Kernels and the executable.
    auto impl = std::make_unique<Executable::Impl>();
    impl->graph = &graph;
    impl->graph_lifetime = graph._lifetime;
    impl->device = device;
    impl->plan_stats = stats;
    if (auto create = get_device_context_hooks(device).create) impl->device_context = create();
    impl->topo.reserve(order.size());
    for (const auto* node : order) {
        Executable::CompiledNode cn;
        std::vector<DataType> dtypes;
        for (auto* in : node->inputs()) {
            auto* s = remap.at(in);
            cn.inputs.push_back(s);
            dtypes.push_back(in->dtype);
        }
        for (auto* out : node->outputs()) {
            auto* s = remap.at(out);
            cn.outputs.push_back(s);
        }
        if (cn.outputs.empty()) throw std::runtime_error("velomind: op node has no outputs");
        cn.kernel = resolve_op_kernel(node->op().op, dtypes, node->outputs().front()->dtype, device);
        if (!cn.kernel) throw std::runtime_error(std::string("velomind: no kernel for op=") + op_name(node->op().op));
        cn.attrs = std::shared_ptr<const void>(new OpDescriptor(node->op()),
                                               [](const void* p) { delete static_cast<const OpDescriptor*>(p); });
        impl->topo.push_back(std::move(cn));
    }
    impl->derive_run_plan();

    // Commit.
    graph._tensors.swap(staged);
    for (auto& node : graph._nodes) {
        for (auto*& in : node._inputs) in = remap.at(in);
        for (auto*& out : node._outputs) out = remap.at(out);
    }
    for (auto*& out : graph._explicit_outputs) out = remap.at(out);
    graph._built = true;
    graph._bound_device = device;
    graph._plan_stats = stats;
    auto exec = std::make_unique<Executable>();
    exec->_impl = std::move(impl);
    return exec;
}

}  // namespace velomind::internal
