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
#include <cstdint>
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

// Places intervals; returns the arena size.  Lifetimes are inclusive
// ranges of step indices, so two intersect exactly when they share a step:
// the placed intervals alive at each step are kept in per-step lists, and
// an interval's conflicts are gathered from the steps it spans instead of
// from every interval placed before it (the scan over all earlier
// intervals made a ~1000-node decode graph's plan quadratic).
std::size_t plan_arena(std::vector<Interval>& items) {
    std::sort(items.begin(), items.end(), [](const Interval& a, const Interval& b) {
        if (a.bytes != b.bytes) return a.bytes > b.bytes;
        const std::size_t da = a.death - a.birth, db = b.death - b.birth;
        if (da != db) return da > db;
        if (a.birth != b.birth) return a.birth < b.birth;
        return a.tensor < b.tensor;
    });
    std::size_t steps = 0;
    for (const auto& it : items) steps = std::max(steps, it.death + 1);
    std::vector<std::vector<std::size_t>> alive(steps);   // placed intervals per step
    std::vector<std::size_t> seen(items.size(), SIZE_MAX);
    std::vector<const Interval*> live;
    std::vector<std::size_t> candidates;
    std::size_t total = 0;
    for (std::size_t i = 0; i < items.size(); ++i) {
        Interval& cur = items[i];
        live.clear();
        for (std::size_t st = cur.birth; st <= cur.death; ++st)
            for (std::size_t j : alive[st])
                if (seen[j] != i) {
                    seen[j] = i;
                    live.push_back(&items[j]);
                }
        candidates.assign(1, 0);
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
        for (std::size_t st = cur.birth; st <= cur.death; ++st) alive[st].push_back(i);
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

// ---- steps -----------------------------------------------------------------
// A compiled step runs one node, or (where the device registers a group
// kernel) up to kMaxQmmGroup sibling QuantizedMatMul nodes that read the
// same fp32 A with the same quantisation and have at most four rows of A:
// decode projections such as q | k | v and gate | up then stream their
// weights in one launch.  A sibling is pulled forward to the first
// member's place only when every tensor it reads is already available
// there; memory lifetimes are planned on the steps, so tensors the group
// writes early never share arena space with anything still live.
// VELOMIND_GROUP_QMM=0 keeps every node on its own.
using Step = std::vector<pConstNode>;

const QuantizedMatMulAttrs* qmm_attrs(pConstNode n) {
    if (n->op().op != Op::QuantizedMatMul) return nullptr;
    return std::get_if<QuantizedMatMulAttrs>(&n->op().attrs);
}

bool qmm_groupable(pConstNode n) {
    const auto* qa = qmm_attrs(n);
    if (!qa || qa->trans_b) return false;
    const auto in = n->inputs();
    const auto out = n->outputs();
    if (in.size() != 3 || out.size() != 1) return false;
    if (in[0]->dtype != DataType::Float32 || in[1]->dtype != DataType::Int8 || in[2]->dtype != DataType::Float32 ||
        out[0]->dtype != DataType::Float32)
        return false;
    if (in[0]->shape.empty() || in[1]->shape.size() != 2) return false;
    dim_t rows = 1;
    for (std::size_t i = 0; i + 1 < in[0]->shape.size(); ++i) rows *= in[0]->shape[i];
    return rows >= 1 && rows <= 4;
}

bool qmm_siblings(pConstNode a, pConstNode b) {
    if (!qmm_groupable(b) || a->inputs()[0] != b->inputs()[0]) return false;
    const auto* qa = qmm_attrs(a);
    const auto* qb = qmm_attrs(b);
    return qa->quant_type == qb->quant_type && qa->block_size == qb->block_size;
}

std::vector<Step> plan_steps(const std::vector<pConstNode>& order, DeviceType device) {
    const char* env = std::getenv("VELOMIND_GROUP_QMM");
    const bool group = qmm_group_kernel(device) != nullptr && !(env && env[0] == '0');
    std::unordered_map<pConstTensorStorage, std::size_t> producer;
    for (std::size_t i = 0; i < order.size(); ++i)
        for (auto* out : order[i]->outputs()) producer.emplace(out, i);
    // groupable nodes by the A they read, in order (siblings share A)
    std::unordered_map<pConstTensorStorage, std::vector<std::size_t>> by_a;
    if (group)
        for (std::size_t i = 0; i < order.size(); ++i)
            if (qmm_groupable(order[i])) by_a[order[i]->inputs()[0]].push_back(i);
    std::vector<bool> done(order.size(), false), taken(order.size(), false);
    std::vector<Step> steps;
    for (std::size_t i = 0; i < order.size(); ++i) {
        if (taken[i]) continue;
        std::vector<std::size_t> members{i};
        taken[i] = true;
        if (group && qmm_groupable(order[i])) {
            for (const std::size_t j : by_a.at(order[i]->inputs()[0])) {
                if (members.size() >= kMaxQmmGroup) break;
                if (j <= i || taken[j] || !qmm_siblings(order[i], order[j])) continue;
                bool ready = true;
                for (auto* in : order[j]->inputs()) {
                    const auto it = producer.find(in);
                    if (it != producer.end() && !done[it->second]) ready = false;
                }
                if (!ready) continue;
                members.push_back(j);
                taken[j] = true;
            }
        }
        Step step;
        for (std::size_t m : members) {
            step.push_back(order[m]);
            done[m] = true;
        }
        steps.push_back(std::move(step));
    }
    return steps;
}

// ---- byte-preserving nodes --------------------------------------------------
// A Reshape, or a Transpose that keeps the order of every axis longer than
// one, writes its input's bytes unchanged.  When input and output are both
// arena intermediates, the output becomes a view of the input's bytes (the
// input's lifetime extended over the output's) and the step launches
// nothing: decode graphs of the reference's LLaMA layer hold ~110 such
// Reshapes and ~140 such Transposes per token.  VELOMIND_GRAPH_ALIAS=0
// keeps the copies.
bool keeps_bytes(pConstNode n) {
    const auto& op = n->op();
    if (n->inputs().size() != 1 || n->outputs().size() != 1) return false;
    const auto* in = n->inputs()[0];
    const auto* out = n->outputs()[0];
    if (in->dtype != out->dtype || in->size_bytes != out->size_bytes || !in->is_contiguous() ||
        !out->is_contiguous())
        return false;
    if (op.op == Op::Reshape) return true;
    if (op.op != Op::Transpose) return false;
    const auto* ta = std::get_if<TransposeAttrs>(&op.attrs);
    if (!ta || ta->perm.size() != in->shape.size()) return false;
    int last = -1;
    for (int axis : ta->perm) {
        if (axis < 0 || static_cast<std::size_t>(axis) >= in->shape.size()) return false;
        if (in->shape[static_cast<std::size_t>(axis)] == 1) continue;
        if (axis < last) return false;
        last = axis;
    }
    return true;
}

void no_launch(const pConstTensorStorage*, const pTensorStorage*, const void*) {}

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
    const auto order = graph._validated_order(device);
    const auto steps = plan_steps(order, device);
    const auto& tensors = graph._tensors;

    std::unordered_map<pConstTensorStorage, std::size_t> index_of;
    for (std::size_t i = 0; i < tensors.size(); ++i) index_of[tensors[i].get()] = i;

    // Activity and lifetimes.
    std::vector<bool> active(tensors.size(), false);
    std::vector<std::size_t> birth(tensors.size(), 0), death(tensors.size(), 0);
    std::vector<bool> born(tensors.size(), false);
    for (std::size_t step = 0; step < steps.size(); ++step) {
        for (const auto* node : steps[step]) {
            for (auto* in : node->inputs()) {
                const auto i = index_of.at(in);
                active[i] = true;
                death[i] = std::max(death[i], step);
            }
            for (auto* out : node->outputs()) {
                const auto i = index_of.at(out);
                active[i] = true;
                if (!born[i]) {
                    born[i] = true;
                    birth[i] = step;
                }
                death[i] = std::max(death[i], step);
            }
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

    // Byte-preserving steps between arena intermediates: the output views
    // its root's bytes, whose lifetime covers the output's.
    std::vector<std::size_t> root(tensors.size());
    for (std::size_t i = 0; i < tensors.size(); ++i) root[i] = i;
    std::vector<bool> alias_step(steps.size(), false);
    {
        const char* env = std::getenv("VELOMIND_GRAPH_ALIAS");
        if (!(env && env[0] == '0')) {
            for (std::size_t step = 0; step < steps.size(); ++step) {
                if (steps[step].size() != 1 || !keeps_bytes(steps[step].front())) continue;
                const auto in = root[index_of.at(steps[step].front()->inputs()[0])];
                const auto out = index_of.at(steps[step].front()->outputs()[0]);
                if (dedicated[in] || dedicated[out] || tensors[in]->size_bytes == 0) continue;
                root[out] = in;
                death[in] = std::max(death[in], death[out]);
                alias_step[step] = true;
            }
        }
    }

    std::vector<Interval> arena_items;
    for (std::size_t i = 0; i < tensors.size(); ++i) {
        if (!active[i] || dedicated[i] || root[i] != i || tensors[i]->size_bytes == 0) continue;
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

    for (std::size_t i = 0; i < tensors.size(); ++i) {
        if (root[i] == i) continue;
        const auto& src = *tensors[i];
        const auto& base = staged[root[i]];
        auto view = std::make_shared<TensorStorage>();
        view->shape = src.shape;
        view->strides = src.strides.empty() ? default_strides(src.shape) : src.strides;
        view->dtype = src.dtype;
        view->device = device;
        view->size_bytes = src.size_bytes;
        view->offset_bytes = base->offset_bytes;
        view->capacity_bytes = base->capacity_bytes;
        view->data = base->data;
        view->external_owner = base->external_owner ? base->external_owner : std::shared_ptr<void>(base);
        staged[i] = std::move(view);
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
    impl->node_count = order.size();
    impl->topo.reserve(steps.size());
    for (const auto& step : steps) {
        if (step.size() > 1) {
            // grouped QuantizedMatMul: [A, B_1, S_1, ..], [C_1, ..]
            Executable::CompiledNode cn;
            cn.inputs.push_back(remap.at(step.front()->inputs()[0]));
            for (const auto* node : step) {
                cn.inputs.push_back(remap.at(node->inputs()[1]));
                cn.inputs.push_back(remap.at(node->inputs()[2]));
                cn.outputs.push_back(remap.at(node->outputs()[0]));
            }
            cn.kernel = qmm_group_kernel(device);
            auto* ga = new QmmGroupAttrs{step.front()->op(), step.size()};
            cn.attrs = std::shared_ptr<const void>(ga, [](const void* p) { delete static_cast<const QmmGroupAttrs*>(p); });
            cn.fused = step.size();
            impl->topo.push_back(std::move(cn));
            continue;
        }
        const auto* node = step.front();
        Executable::CompiledNode cn;
        const bool aliased = alias_step[static_cast<std::size_t>(&step - steps.data())];
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
        cn.kernel = aliased ? &no_launch : resolve_op_kernel(node->op().op, dtypes, node->outputs().front()->dtype, device);
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
