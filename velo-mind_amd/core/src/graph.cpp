// Graph construction, dead-code elimination and topological ordering
// (the reference's src/graph.cpp), written for this build.
#include "velomind/graph.h"

#include <algorithm>
#include <span>
#include <stdexcept>

#include "internal/graph_compiler.h"
#include "internal/registry/kernel.h"
#include "internal/registry/shape.h"
#include "internal/tensor_index.h"
#include "velomind/executable.h"

namespace velomind {

Graph::Graph(std::size_t initial_tensor_capacity, std::size_t initial_node_capacity)
    : _lifetime(std::make_shared<int>(0)) {
    _tensors.reserve(initial_tensor_capacity);
    _nodes.reserve(initial_node_capacity);
}

Graph::~Graph() = default;

auto Graph::reserve(std::size_t tensor_capacity, std::size_t node_capacity) -> void {
    if (_built) throw std::logic_error("Graph::reserve: graph is already built");
    if (tensor_capacity > _tensors.capacity()) _tensors.reserve(tensor_capacity);
    if (node_capacity > _nodes.capacity()) _nodes.reserve(node_capacity);
}

auto Graph::tensor_storage_at(std::size_t i) const -> pConstTensorStorage {
    return i < _tensors.size() ? _tensors[i].get() : nullptr;
}
auto Graph::tensor_storage_at(std::size_t i) -> pTensorStorage { return i < _tensors.size() ? _tensors[i].get() : nullptr; }
auto Graph::shared_storage_at(std::size_t i) const -> std::shared_ptr<TensorStorage> {
    return i < _tensors.size() ? _tensors[i] : nullptr;
}

auto Graph::is_input_tensor(std::size_t i) const noexcept -> bool {
    const auto* s = tensor_storage_at(i);
    if (!s) return false;
    for (const auto& n : _nodes)
        for (auto* o : n.outputs())
            if (o == s) return false;
    return true;
}

auto Graph::is_output_tensor(std::size_t i) const noexcept -> bool {
    const auto* s = tensor_storage_at(i);
    if (!s) return false;
    if (_has_explicit_outputs) return std::find(_explicit_outputs.begin(), _explicit_outputs.end(), s) != _explicit_outputs.end();
    if (is_input_tensor(i)) return false;
    for (const auto& n : _nodes)
        for (auto* in : n.inputs())
            if (in == s) return false;
    return true;
}

auto Graph::input(shape_t shape, DataType dtype) -> Tensor {
    if (_built) throw std::logic_error("Graph::input: graph is already built");
    auto s = std::make_shared<TensorStorage>();
    s->shape = std::move(shape);
    s->strides = default_strides(s->shape);
    s->dtype = dtype;
    s->size_bytes = storage_nbytes(*s);
    s->capacity_bytes = s->size_bytes;
    _tensors.push_back(std::move(s));
    return Tensor{this, _tensors.size() - 1};
}

auto Graph::input(std::shared_ptr<TensorStorage> storage) -> Tensor {
    if (_built) throw std::logic_error("Graph::input: graph is already built");
    if (!storage) throw std::invalid_argument("Graph::input: null storage");
    if (storage->size_bytes < storage_nbytes(*storage))
        throw std::invalid_argument("Graph::input: storage capacity is smaller than tensor");
    if (storage->strides.empty()) storage->strides = default_strides(storage->shape);
    if (storage->capacity_bytes == 0) storage->capacity_bytes = storage->size_bytes;
    _tensors.push_back(std::move(storage));
    return Tensor{this, _tensors.size() - 1};
}

auto Graph::_op_impl(OpDescriptor desc, std::span<const pConstTensorStorage> inputs) -> Tensor {
    if (std::holds_alternative<NoAttrs>(desc.attrs)) desc.attrs = default_op_attrs(desc.op);
    // Shapes and dtypes come only from the signature registry.
    auto sig = internal::op_signature(desc.op, inputs, desc.attrs);
    auto out = std::make_shared<TensorStorage>();
    out->shape = std::move(sig.shape);
    out->strides = default_strides(out->shape);
    out->dtype = sig.dtype;
    out->size_bytes = storage_nbytes(*out);
    out->capacity_bytes = out->size_bytes;
    _tensors.push_back(std::move(out));
    Node node;
    node._op = std::move(desc);
    node._inputs.reserve(inputs.size());
    for (auto* in : inputs) node._inputs.push_back(in);
    node._outputs.push_back(_tensors.back().get());
    _nodes.push_back(std::move(node));
    return Tensor{this, _tensors.size() - 1};
}

auto Graph::mark_output(Tensor t) -> void {
    if (_built) throw std::logic_error("Graph::mark_output: graph is already built");
    if (t.graph() != this || t.storage() == nullptr)
        throw std::invalid_argument("Graph::mark_output: invalid or foreign tensor handle");
    _has_explicit_outputs = true;
    if (std::find(_explicit_outputs.begin(), _explicit_outputs.end(), t.storage()) == _explicit_outputs.end())
        _explicit_outputs.push_back(t.storage());
}

auto Graph::set_outputs(std::vector<Tensor> outputs) -> void {
    if (_built) throw std::logic_error("Graph::set_outputs: graph is already built");
    for (const auto& t : outputs)
        if (t.graph() != this || t.storage() == nullptr)
            throw std::invalid_argument("Graph::set_outputs: invalid or foreign tensor handle");
    _explicit_outputs.clear();
    _has_explicit_outputs = !outputs.empty();
    for (const auto& t : outputs)
        if (std::find(_explicit_outputs.begin(), _explicit_outputs.end(), t.storage()) == _explicit_outputs.end())
            _explicit_outputs.push_back(t.storage());
}

auto Graph::outputs() const -> std::vector<Tensor> {
    std::vector<Tensor> res;
    auto* self = const_cast<Graph*>(this);
    if (_has_explicit_outputs) {
        for (auto* s : _explicit_outputs)
            for (std::size_t i = 0; i < _tensors.size(); ++i)
                if (_tensors[i].get() == s) {
                    res.emplace_back(self, i);
                    break;
                }
    } else {
        for (std::size_t i = 0; i < _tensors.size(); ++i)
            if (is_output_tensor(i)) res.emplace_back(self, i);
    }
    return res;
}

namespace {

// The node writing each tensor (by index into the tensor list; the last
// writer when several do), SIZE_MAX for tensors no node writes.
std::vector<std::size_t> producers_of(const std::vector<Node>& nodes, const internal::TensorIndex& index,
                                      std::size_t tensors) {
    std::vector<std::size_t> p(tensors, SIZE_MAX);
    for (std::size_t i = 0; i < nodes.size(); ++i)
        for (auto* o : nodes[i].outputs()) {
            const std::size_t t = index.find(o);
            if (t != internal::TensorIndex::npos) p[t] = i;
        }
    return p;
}

std::size_t producer_of(pConstTensorStorage s, const internal::TensorIndex& index,
                        const std::vector<std::size_t>& producer) {
    const std::size_t t = index.find(s);
    return t == internal::TensorIndex::npos ? SIZE_MAX : producer[t];
}

// The producing node of every node input (SIZE_MAX: nothing writes it), as
// compressed rows: node v's inputs are node[first[v] .. first[v + 1]).
// Found once, for the passes that walk the graph's edges.
struct InputProducers {
    std::vector<std::size_t> first, node;
};

InputProducers input_producers(const std::vector<Node>& nodes, const internal::TensorIndex& index,
                               const std::vector<std::size_t>& producer) {
    InputProducers ip;
    ip.first.resize(nodes.size() + 1, 0);
    std::size_t edges = 0;
    for (std::size_t v = 0; v < nodes.size(); ++v) edges += nodes[v].inputs().size();
    ip.node.reserve(edges);
    for (std::size_t v = 0; v < nodes.size(); ++v) {
        for (auto* in : nodes[v].inputs()) ip.node.push_back(producer_of(in, index, producer));
        ip.first[v + 1] = ip.node.size();
    }
    return ip;
}

// Nodes reachable backwards from the explicit outputs.
std::vector<bool> required_nodes(const std::vector<Node>& nodes, const std::vector<pConstTensorStorage>& outputs,
                                 const internal::TensorIndex& index, const std::vector<std::size_t>& producer,
                                 const InputProducers& ip) {
    std::vector<bool> req(nodes.size(), false);
    std::vector<std::size_t> stack;
    auto reach = [&](std::size_t p) {
        if (p != SIZE_MAX && !req[p]) {
            req[p] = true;
            stack.push_back(p);
        }
    };
    for (auto* s : outputs) reach(producer_of(s, index, producer));
    while (!stack.empty()) {
        const std::size_t u = stack.back();
        stack.pop_back();
        for (std::size_t e = ip.first[u]; e < ip.first[u + 1]; ++e) reach(ip.node[e]);
    }
    return req;
}

// Kahn's algorithm over the required nodes, in insertion order among ready
// nodes (FIFO); throws on a cycle.
std::vector<pConstNode> topological(const std::vector<Node>& nodes, const std::vector<bool>& req,
                                    const InputProducers& ip) {
    const std::size_t n = nodes.size();
    std::vector<std::size_t> indeg(n, 0), deps, edge_u, edge_v;
    std::size_t active = 0;
    for (std::size_t v = 0; v < n; ++v) {
        if (!req[v]) continue;
        ++active;
        deps.clear();
        for (std::size_t e = ip.first[v]; e < ip.first[v + 1]; ++e) {
            const std::size_t p = ip.node[e];
            if (p != SIZE_MAX && req[p]) deps.push_back(p);
        }
        std::sort(deps.begin(), deps.end());
        deps.erase(std::unique(deps.begin(), deps.end()), deps.end());
        indeg[v] = deps.size();
        for (std::size_t u : deps) {
            edge_u.push_back(u);
            edge_v.push_back(v);
        }
    }
    // users of each node in ascending order, as compressed rows
    std::vector<std::size_t> first(n + 1, 0), users(edge_u.size());
    for (std::size_t u : edge_u) ++first[u + 1];
    for (std::size_t i = 0; i < n; ++i) first[i + 1] += first[i];
    std::vector<std::size_t> fill(first.begin(), first.end() - 1);
    for (std::size_t e = 0; e < edge_u.size(); ++e) users[fill[edge_u[e]]++] = edge_v[e];
    std::vector<std::size_t> ready;
    ready.reserve(active);
    for (std::size_t v = 0; v < n; ++v)
        if (req[v] && indeg[v] == 0) ready.push_back(v);
    std::vector<pConstNode> order;
    order.reserve(active);
    for (std::size_t head = 0; head < ready.size(); ++head) {
        const std::size_t u = ready[head];
        order.push_back(&nodes[u]);
        for (std::size_t e = first[u]; e < first[u + 1]; ++e)
            if (--indeg[users[e]] == 0) ready.push_back(users[e]);
    }
    if (order.size() != active) throw std::invalid_argument("Graph::build: cycle detected in graph");
    return order;
}

}  // namespace

// Nodes reachable backwards from the explicit outputs (all nodes if none).
auto Graph::_compute_required_nodes() const -> std::vector<bool> {
    if (!_has_explicit_outputs) return std::vector<bool>(_nodes.size(), true);
    const internal::TensorIndex index(_tensors);
    const auto producer = producers_of(_nodes, index, _tensors.size());
    return required_nodes(_nodes, _explicit_outputs, index, producer, input_producers(_nodes, index, producer));
}

auto Graph::_topological_order() const -> std::vector<pConstNode> { return _topological_order(_compute_required_nodes()); }

auto Graph::_topological_order(const std::vector<bool>& req) const -> std::vector<pConstNode> {
    const internal::TensorIndex index(_tensors);
    return topological(_nodes, req, input_producers(_nodes, index, producers_of(_nodes, index, _tensors.size())));
}

auto Graph::validate(DeviceType device) const -> void { (void)_validated_order(device); }

auto Graph::_validated_order(DeviceType device) const -> std::vector<pConstNode> {
    if (_built) throw std::logic_error("Graph::validate: graph is already built");
    return _validated_order(device, internal::TensorIndex(_tensors));
}

auto Graph::_validated_order(DeviceType device, const internal::TensorIndex& index) const -> std::vector<pConstNode> {
    if (_built) throw std::logic_error("Graph::validate: graph is already built");
    if (static_cast<std::size_t>(device) >= MAX_DEVICE_TYPES) throw std::invalid_argument("Graph::validate: invalid device");
    for (const auto& s : _tensors) {
        if (s->size_bytes < storage_nbytes(*s)) throw std::invalid_argument("Graph::validate: invalid tensor capacity");
        if (s->data != nullptr && s->device != device)
            throw std::invalid_argument("Graph::validate: populated storage belongs to another device");
    }
    const auto producer = producers_of(_nodes, index, _tensors.size());
    const auto ip = input_producers(_nodes, index, producer);
    const auto req = _has_explicit_outputs ? required_nodes(_nodes, _explicit_outputs, index, producer, ip)
                                           : std::vector<bool>(_nodes.size(), true);
    for (std::size_t i = 0; i < _nodes.size(); ++i) {
        if (!req[i]) continue;
        const auto& n = _nodes[i];
        if (n.outputs().empty()) throw std::invalid_argument("Graph::validate: node has no outputs");
        // Metadata may have changed through shared storages: re-derive.
        const auto sig = internal::op_signature(n.op().op, n.inputs(), n.op().attrs);
        const auto* out = n.outputs().front();
        if (sig.shape != out->shape || sig.dtype != out->dtype)
            throw std::invalid_argument("Graph::validate: output metadata no longer matches signature");
        DataType dtypes[4];
        const auto ins = n.inputs();
        const bool keyed = ins.size() <= 4;
        for (std::size_t j = 0; keyed && j < ins.size(); ++j) dtypes[j] = ins[j]->dtype;
        if (!keyed || !internal::resolve_op_kernel(n.op().op, std::span<const DataType>(dtypes, ins.size()), out->dtype,
                                                   device))
            throw std::invalid_argument(std::string("Graph::validate: unsupported kernel for ") + op_name(n.op().op));
    }
    return topological(_nodes, req, ip);
}

auto Graph::build(DeviceType device) -> std::unique_ptr<Executable> {
    return internal::GraphCompiler::compile(*this, device);
}

}  // namespace velomind
