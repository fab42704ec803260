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
// Allocations are staged on a copy of the graph's storage list (arena
// placements written into the graph's own storages only after the last
// step that can fail, and undone if one does), so a failed build leaves the
// graph unchanged and buildable again.  VELOMIND_FAIL_GRAPH_BUILD_AFTER_ALLOCATIONS=N
// injects a failure after the N-th allocation (the reference's hook of the
// same name, src/internal/graph_compiler.cpp:563-568).
#include "internal/graph_compiler.h"

#include <algorithm>
#include <array>
#include <cstdint>
#include <span>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "internal/registry/device_context.h"
#include "internal/tensor_index.h"
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

// Places intervals; returns the arena size.  Lifetimes are inclusive
// ranges of step indices, so two intersect exactly when they share a step:
// an interval's conflicts are the intervals placed before it that cover
// one of the steps it spans, gathered from per-step lists instead of from
// every interval placed before it (the scan over all earlier intervals
// made a ~1000-node decode graph's plan quadratic).
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
    // The intervals covering each step, in placement order, in one flat
    // array (cover[first[st] .. first[st + 1])): those placed before
    // interval i are the entries below i.  One allocation instead of a
    // growing list per step (~2,400 heap allocations per decode graph).
    std::vector<std::size_t> first(steps + 1, 0);
    for (const auto& it : items)
        for (std::size_t st = it.birth; st <= it.death; ++st) ++first[st + 1];
    for (std::size_t st = 0; st < steps; ++st) first[st + 1] += first[st];
    std::vector<std::size_t> cover(first[steps]);
    {
        std::vector<std::size_t> fill(first.begin(), first.end() - 1);
        for (std::size_t i = 0; i < items.size(); ++i)
            for (std::size_t st = items[i].birth; st <= items[i].death; ++st) cover[fill[st]++] = i;
    }
    std::vector<std::size_t> seen(items.size(), SIZE_MAX);
    std::vector<const Interval*> live;
    std::vector<std::size_t> candidates;
    std::size_t total = 0;
    for (std::size_t i = 0; i < items.size(); ++i) {
        Interval& cur = items[i];
        live.clear();
        for (std::size_t st = cur.birth; st <= cur.death; ++st)
            for (std::size_t e = first[st]; e < first[st + 1] && cover[e] < i; ++e) {
                const std::size_t j = cover[e];
                if (seen[j] != i) {
                    seen[j] = i;
                    live.push_back(&items[j]);
                }
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
// A compiled step runs one node; or (where the device registers a group
// kernel) up to kMaxQmmGroup sibling QuantizedMatMul nodes that read the
// same fp32 A with the same quantisation and have at most four rows of A:
// decode projections such as q | k | v and gate | up then stream their
// weights in one launch; or (where the device registers the kernel) a
// fused chain of nodes (kernel.h FusedKind, matched by fuse_steps below).
// A sibling is pulled forward to the first member's place only when every
// tensor it reads is already available there; memory lifetimes are planned
// on the steps, so tensors the group writes early never share arena space
// with anything still live.  VELOMIND_GROUP_QMM=0 keeps every node on its own.
// The nodes of a step: up to kInline in place, more on the heap (most
// steps run one node; a vector allocated once per step and build).
class StepNodes {
public:
    static constexpr std::size_t kInline = 4;
    StepNodes() = default;
    StepNodes(const StepNodes& o) { *this = o; }
    StepNodes& operator=(const StepNodes& o) {
        if (this == &o) return *this;
        _n = 0;
        _heap.clear();
        for (auto* p : o) push_back(p);
        return *this;
    }
    StepNodes(StepNodes&& o) noexcept : _in(o._in), _heap(std::move(o._heap)), _n(o._n) { o._n = 0; }
    StepNodes& operator=(StepNodes&& o) noexcept {
        _in = o._in;
        _heap = std::move(o._heap);
        _n = o._n;
        o._heap.clear();
        o._n = 0;
        return *this;
    }
    void push_back(pConstNode p) {
        if (_heap.empty() && _n < kInline) {
            _in[_n++] = p;
            return;
        }
        if (_heap.empty()) _heap.assign(_in.begin(), _in.begin() + static_cast<std::ptrdiff_t>(_n));
        _heap.push_back(p);
        _n = _heap.size();
    }
    std::size_t size() const noexcept { return _n; }
    bool empty() const noexcept { return _n == 0; }
    const pConstNode* begin() const noexcept { return _heap.empty() ? _in.data() : _heap.data(); }
    const pConstNode* end() const noexcept { return begin() + _n; }
    pConstNode front() const noexcept { return *begin(); }

private:
    std::array<pConstNode, kInline> _in{};
    std::vector<pConstNode> _heap;   // all nodes once there are more than kInline
    std::size_t _n = 0;
};

struct Step {
    StepNodes nodes;                          // graph nodes the step runs
    int fused = -1;                           // FusedKind, or -1
    std::vector<pConstTensorStorage> ins;     // fused: the chain's external operands
    std::vector<pConstTensorStorage> outs;
    std::shared_ptr<const void> attrs;        // fused: what the kernel takes as attrs, if anything
};

// A node's descriptor as kernel attributes, without a copy: the executable
// runs only while its graph lives (Executable::execute checks the graph's
// lifetime first) and a built graph's nodes never move, so the pointer
// into the node stays valid for every run (an aliasing shared_ptr that owns
// nothing).
std::shared_ptr<const void> node_desc(const OpDescriptor& d) {
    return std::shared_ptr<const void>(std::shared_ptr<const void>{}, &d);
}

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
    for (auto* t : in)
        if (!t->is_contiguous()) return false;
    if (!out[0]->is_contiguous()) return false;
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

std::vector<Step> plan_steps(const std::vector<pConstNode>& order, DeviceType device, const TensorIndex& index,
                             std::size_t tensor_count) {
    const char* env = std::getenv("VELOMIND_GROUP_QMM");
    const bool group = qmm_group_kernel(device) != nullptr && !(env && env[0] == '0');
    std::vector<Step> steps;
    steps.reserve(order.size());
    if (!group) {
        for (auto* n : order) {
            Step st;
            st.nodes.push_back(n);
            steps.push_back(std::move(st));
        }
        return steps;
    }
    std::vector<std::size_t> producer(tensor_count, SIZE_MAX);
    for (std::size_t i = 0; i < order.size(); ++i)
        for (auto* out : order[i]->outputs()) {
            auto& p = producer[index.at(out)];
            if (p == SIZE_MAX) p = i;
        }
    // groupable nodes by the A they read, in order (siblings share A)
    std::vector<std::vector<std::size_t>> by_a(tensor_count);
    for (std::size_t i = 0; i < order.size(); ++i)
        if (qmm_groupable(order[i])) by_a[index.at(order[i]->inputs()[0])].push_back(i);
    std::vector<bool> done(order.size(), false), taken(order.size(), false);
    for (std::size_t i = 0; i < order.size(); ++i) {
        if (taken[i]) continue;
        Step step;
        step.nodes.push_back(order[i]);
        taken[i] = true;
        done[i] = true;
        if (qmm_groupable(order[i])) {
            for (const std::size_t j : by_a[index.at(order[i]->inputs()[0])]) {
                if (step.nodes.size() >= kMaxQmmGroup) break;
                if (j <= i || taken[j] || !qmm_siblings(order[i], order[j])) continue;
                bool ready = true;
                for (auto* in : order[j]->inputs()) {
                    const auto p = producer[index.at(in)];
                    if (p != SIZE_MAX && !done[p]) ready = false;
                }
                if (!ready) continue;
                step.nodes.push_back(order[j]);
                taken[j] = true;
                done[j] = true;
            }
        }
        steps.push_back(std::move(step));
    }
    return steps;
}

// ---- fused chains -------------------------------------------------------------
// Chains of single-node steps that the device runs as one launch
// (kernel.h FusedKind).  A chain's inner tensors must have exactly one
// consumer and must not be kept (requested outputs, graph inputs, tensors
// that own data): they are then never allocated.  The fused step takes the
// place of the chain's last node, where every operand it reads exists.
//   SiluMul          y = Mul(Mul(Sigmoid(g), g), u)      (either operand order)
//   QmmAdd           C = Add(h, QuantizedMatMul(A, ..))  (at most 4 rows of A, fp32, either order)
//   AttentionDecode  ctx = MatMul(Softmax(MatMul(q, Transpose(RepeatKV(K)))), RepeatKV(V))
//                    with q [H, 1, D], K [Hkv, S, D], V [Hkv, S, Dv], the
//                    Transpose swapping the last two axes, the Softmax on the
//                    last one (RepeatKV absent when H == Hkv)
//   AttentionGqa     o = FusedAttention(q, RepeatKV(K), RepeatKV(V))
//   SwigluQmmAdd     C = Add(h, QuantizedMatMul(SiluMul(g, u), ..)): a QmmAdd whose
//                    activations are a fused SiluMul's inner output
//   NormQmm          C_g = QuantizedMatMul(RMSNorm(x, w), ..) for the members of one step
//                    (a single node or a sibling group) that are the norm's only readers
//   RopeAppend       q' = RoPE(q), K = Concat(K_past, RoPE(k)), V = Concat(V_past, v)
//                    at one position (new rows [., 1, .], one cos/sin row), the
//                    four nodes within a few steps of each other and q', K read
//                    by nothing before the fused step's place
// VELOMIND_GRAPH_FUSE=0 keeps every chain as separate launches;
// VELOMIND_GRAPH_FUSE_OFF lists kinds (their numbers) to leave out.
void fuse_steps(std::vector<Step>& steps, DeviceType device, const TensorIndex& index,
                const std::vector<bool>& kept) {
    const char* env = std::getenv("VELOMIND_GRAPH_FUSE");
    if (env && env[0] == '0') return;
    // VELOMIND_GRAPH_FUSE_OFF="k,k,.." leaves the listed kinds out (measurements)
    bool off[kFusedKinds] = {};
    if (const char* list = std::getenv("VELOMIND_GRAPH_FUSE_OFF"))
        for (const char* c = list; *c; ++c)
            if (*c >= '0' && *c <= '9' && static_cast<std::size_t>(*c - '0') < kFusedKinds) off[*c - '0'] = true;
    Executable::KernelFn kernels[kFusedKinds];
    bool any = false;
    for (std::size_t k = 0; k < kFusedKinds; ++k) {
        kernels[k] = off[k] ? nullptr : fused_kernel(device, static_cast<FusedKind>(k));
        any = any || kernels[k];
    }
    if (!any) return;
    const std::size_t nt = kept.size();
    std::vector<std::uint32_t> consumers(nt, 0);
    std::vector<std::size_t> producer(nt, SIZE_MAX);   // single-node step producing the tensor
    std::vector<std::size_t> first_use(nt, SIZE_MAX);  // earliest step reading the tensor
    for (std::size_t s = 0; s < steps.size(); ++s)
        for (auto* n : steps[s].nodes) {
            for (auto* in : n->inputs()) {
                const std::size_t i = index.at(in);
                ++consumers[i];
                first_use[i] = std::min(first_use[i], s);
            }
            if (steps[s].nodes.size() == 1)
                for (auto* out : n->outputs()) producer[index.at(out)] = s;
        }
    std::vector<bool> dead(steps.size(), false);
    // the step producing t when it is a live, unfused single node of op `op` with one output
    auto single = [&](pConstTensorStorage t, Op op) -> std::size_t {
        const std::size_t s = producer[index.at(t)];
        if (s == SIZE_MAX || dead[s] || steps[s].fused >= 0) return SIZE_MAX;
        const auto* n = steps[s].nodes.front();
        return (n->op().op == op && n->outputs().size() == 1) ? s : SIZE_MAX;
    };
    auto inner = [&](pConstTensorStorage t) {
        const std::size_t i = index.at(t);
        return consumers[i] == 1 && !kept[i];
    };
    auto f32 = [](pConstTensorStorage t) { return t->dtype == DataType::Float32; };
    auto node_of = [&](std::size_t s) { return steps[s].nodes.front(); };
    auto is_kv_repeat = [&](std::size_t s) {
        if (s == SIZE_MAX) return false;
        const auto* a = std::get_if<RepeatKVAttrs>(&node_of(s)->op().attrs);
        return a && (a->axis == 0 || a->axis == -3) && node_of(s)->inputs()[0]->shape.size() == 3;
    };
    // K or V as the chain reads it: before its RepeatKV when that is inner
    auto unrepeat = [&](pConstTensorStorage t, std::vector<std::size_t>& absorbed) -> pConstTensorStorage {
        const std::size_t s = single(t, Op::RepeatKV);
        if (!is_kv_repeat(s) || !inner(t)) return t;
        absorbed.push_back(s);
        return node_of(s)->inputs()[0];
    };
    auto make = [&](std::size_t at, FusedKind kind, std::vector<std::size_t> absorbed,
                    std::vector<pConstTensorStorage> ins, std::shared_ptr<const void> attrs,
                    std::vector<pConstTensorStorage> outs = {}) {
        Step f;
        std::sort(absorbed.begin(), absorbed.end());
        for (std::size_t s : absorbed) {
            f.nodes.push_back(node_of(s));
            dead[s] = true;
        }
        f.nodes.push_back(node_of(at));
        f.fused = static_cast<int>(kind);
        f.ins = std::move(ins);
        f.outs = outs.empty() ? std::vector<pConstTensorStorage>{node_of(at)->outputs()[0]} : std::move(outs);
        f.attrs = std::move(attrs);
        steps[at] = std::move(f);
    };

    // RMSNorm read only by the QuantizedMatMul(s) of step j: NormQmm
    auto norm_qmm = [&](std::size_t j) {
        const auto& members = steps[j].nodes;
        if (!kernels[static_cast<int>(FusedKind::NormQmm)] || !qmm_groupable(members.front())) return false;
        const auto* hn = members.front()->inputs()[0];
        const std::size_t sr = single(hn, Op::RMSNorm);
        if (sr == SIZE_MAX) return false;
        const std::size_t i = index.at(hn);
        if (kept[i] || consumers[i] != members.size()) return false;
        const auto* norm = node_of(sr);
        const auto* na = std::get_if<RMSNormAttrs>(&norm->op().attrs);
        const auto* x = norm->inputs()[0];
        const auto* w = norm->inputs()[1];
        const dim_t k = hn->shape.back();
        if (!na || !(na->axis == -1 || na->axis == static_cast<int>(hn->shape.size()) - 1) || x->shape != hn->shape ||
            w->shape != shape_t{k} || !f32(x) || !f32(w))
            return false;
        Step f;
        f.nodes.push_back(norm);
        f.ins = {x, w};
        for (auto* mnode : members) {
            f.nodes.push_back(mnode);
            f.ins.push_back(mnode->inputs()[1]);
            f.ins.push_back(mnode->inputs()[2]);
            f.outs.push_back(mnode->outputs()[0]);
        }
        f.fused = static_cast<int>(FusedKind::NormQmm);
        auto* a = new NormQmmAttrs{members.front()->op(), members.size(), na->epsilon};
        f.attrs = std::shared_ptr<const void>(a, [](const void* p) { delete static_cast<const NormQmmAttrs*>(p); });
        dead[sr] = true;
        steps[j] = std::move(f);
        return true;
    };

    for (std::size_t j = 0; j < steps.size(); ++j) {
        if (dead[j] || steps[j].fused >= 0) continue;
        if (steps[j].nodes.size() > 1) {   // a sibling QuantizedMatMul group
            norm_qmm(j);
            continue;
        }
        const auto* n = node_of(j);
        const auto ins = n->inputs();
        if (n->outputs().size() != 1) continue;
        const auto* out = n->outputs()[0];
        const Op op = n->op().op;

        if (op == Op::Mul && kernels[static_cast<int>(FusedKind::SiluMul)] && ins.size() == 2) {
            bool done = false;
            for (int ti = 0; ti < 2 && !done; ++ti) {
                const auto* t = ins[ti];
                const auto* u = ins[1 - ti];
                const std::size_t st = single(t, Op::Mul);
                if (st == SIZE_MAX || !inner(t)) continue;
                const auto m1 = node_of(st)->inputs();
                for (int si = 0; si < 2 && !done; ++si) {
                    const auto* sg = m1[si];
                    const auto* g = m1[1 - si];
                    const std::size_t ss = single(sg, Op::Sigmoid);
                    if (ss == SIZE_MAX || !inner(sg) || node_of(ss)->inputs()[0] != g) continue;
                    if (!(f32(g) && f32(u) && f32(out) && f32(t) && f32(sg)) || g->shape != u->shape ||
                        g->shape != out->shape || g->shape != t->shape || g->shape != sg->shape)
                        continue;
                    make(j, FusedKind::SiluMul, {ss, st}, {g, u}, nullptr);
                    done = true;
                }
            }
            continue;
        }
        if (op == Op::Add && kernels[static_cast<int>(FusedKind::QmmAdd)] && ins.size() == 2) {
            for (int yi = 1; yi >= 0; --yi) {
                const auto* y = ins[yi];
                const auto* h = ins[1 - yi];
                const std::size_t sq = single(y, Op::QuantizedMatMul);
                if (sq == SIZE_MAX || !inner(y) || !qmm_groupable(node_of(sq))) continue;
                if (!f32(h) || !f32(out) || h->shape != y->shape || out->shape != y->shape) continue;
                const auto q = node_of(sq)->inputs();
                // activations from a fused SiluMul read by this product alone: one launch for all
                const std::size_t sa = producer[index.at(q[0])];
                if (kernels[static_cast<int>(FusedKind::SwigluQmmAdd)] && sa != SIZE_MAX && !dead[sa] &&
                    steps[sa].fused == static_cast<int>(FusedKind::SiluMul) && inner(q[0])) {
                    Step f;
                    f.nodes = steps[sa].nodes;
                    f.nodes.push_back(node_of(sq));
                    f.nodes.push_back(n);
                    f.fused = static_cast<int>(FusedKind::SwigluQmmAdd);
                    f.ins = {steps[sa].ins[0], steps[sa].ins[1], q[1], q[2], h};
                    f.outs = {out};
                    f.attrs = node_desc(node_of(sq)->op());
                    dead[sa] = true;
                    dead[sq] = true;
                    steps[j] = std::move(f);
                    break;
                }
                make(j, FusedKind::QmmAdd, {sq}, {q[0], q[1], q[2], h}, node_desc(node_of(sq)->op()));
                break;
            }
            continue;
        }
        if (op == Op::QuantizedMatMul) {
            norm_qmm(j);
            continue;
        }
        if (op == Op::MatMul && kernels[static_cast<int>(FusedKind::AttentionDecode)] && ins.size() == 2) {
            const std::size_t sp = single(ins[0], Op::Softmax);
            if (sp == SIZE_MAX || !inner(ins[0])) continue;
            const auto* scores = node_of(sp)->inputs()[0];
            const auto* sa = std::get_if<SoftmaxAttrs>(&node_of(sp)->op().attrs);
            if (!sa || !(sa->axis == -1 || sa->axis == 2)) continue;
            const std::size_t sm = single(scores, Op::MatMul);
            if (sm == SIZE_MAX || !inner(scores)) continue;
            const auto* q = node_of(sm)->inputs()[0];
            const auto* kt = node_of(sm)->inputs()[1];
            const std::size_t st = single(kt, Op::Transpose);
            if (st == SIZE_MAX || !inner(kt)) continue;
            const auto* ta = std::get_if<TransposeAttrs>(&node_of(st)->op().attrs);
            if (!ta || ta->perm != std::vector<int>{0, 2, 1}) continue;
            std::vector<std::size_t> absorbed{sp, sm, st};
            const auto* k = unrepeat(node_of(st)->inputs()[0], absorbed);
            const auto* v = unrepeat(ins[1], absorbed);
            if (q->shape.size() != 3 || k->shape.size() != 3 || v->shape.size() != 3 || out->shape.size() != 3) continue;
            const dim_t H = q->shape[0], D = q->shape[2], Hkv = k->shape[0], S = k->shape[1], Dv = v->shape[2];
            // K and V both before their RepeatKV (Hkv heads) or both without one (H heads)
            const bool shapes = q->shape[1] == 1 && k->shape[2] == D && v->shape[0] == Hkv && v->shape[1] == S &&
                                Hkv > 0 && H % Hkv == 0 && S > 0 && S + D <= 16384 &&
                                out->shape == shape_t{H, 1, Dv};
            if (!shapes) continue;
            if (!(f32(q) && f32(k) && f32(v) && f32(out))) continue;
            make(j, FusedKind::AttentionDecode, absorbed, {q, k, v}, nullptr);
            continue;
        }
        if (op == Op::Concat && kernels[static_cast<int>(FusedKind::RopeAppend)] && ins.size() == 2) {
            // the later of the two appends; the other and the two RoPEs come a few steps before it
            auto seq_append = [&](pConstNode c) {
                const auto* a = std::get_if<ConcatAttrs>(&c->op().attrs);
                const auto* p = c->inputs()[0];
                const auto* x = c->inputs()[1];
                return c->outputs().size() == 1 && a && (a->axis == 1 || a->axis == -2) && p->shape.size() == 3 &&
                       x->shape.size() == 3 && x->shape[1] == 1 && x->shape[0] == p->shape[0] &&
                       x->shape[2] == p->shape[2] && f32(p) && f32(x) && f32(c->outputs()[0]);
            };
            auto near_single = [&](std::size_t from, auto&& want) {
                for (std::size_t b = from; b-- > 0 && from - b <= 8;)
                    if (!dead[b] && steps[b].fused < 0 && steps[b].nodes.size() == 1 && want(b)) return b;
                return SIZE_MAX;
            };
            if (!seq_append(n)) continue;
            const auto* past = ins[0];
            const std::size_t so = near_single(j, [&](std::size_t b) {
                const auto* c = node_of(b);
                return c->op().op == Op::Concat && seq_append(c) && c->inputs()[0]->shape[0] == past->shape[0] &&
                       c->inputs()[0]->shape[1] == past->shape[1];
            });
            if (so == SIZE_MAX) continue;
            // the key append is the one whose new row is an inner RoPE output
            auto roped = [&](pConstNode c) {
                const std::size_t r = single(c->inputs()[1], Op::RotaryEmbedding);
                return (r != SIZE_MAX && inner(c->inputs()[1])) ? r : SIZE_MAX;
            };
            const std::size_t r_here = roped(n), r_other = roped(node_of(so));
            if ((r_here == SIZE_MAX) == (r_other == SIZE_MAX)) continue;
            const auto* kcat = r_here != SIZE_MAX ? n : node_of(so);
            const auto* vcat = r_here != SIZE_MAX ? node_of(so) : n;
            const std::size_t sb = r_here != SIZE_MAX ? r_here : r_other;
            if (sb > j) continue;
            const auto* kr = kcat->inputs()[1];
            const auto* k = node_of(sb)->inputs()[0];
            const auto* cs = node_of(sb)->inputs()[1];
            const auto* sn = node_of(sb)->inputs()[2];
            if (cs->shape.size() != 2 || cs->shape[0] != 1 || sn->shape != cs->shape || k->shape != kr->shape) continue;
            const std::size_t sa = near_single(j, [&](std::size_t b) {
                const auto* a = node_of(b);
                return b != sb && a->op().op == Op::RotaryEmbedding && a->outputs().size() == 1 &&
                       a->inputs()[1] == cs && a->inputs()[2] == sn;
            });
            if (sa == SIZE_MAX) continue;
            const auto* q = node_of(sa)->inputs()[0];
            const auto* qr = node_of(sa)->outputs()[0];
            const auto* kc = kcat->outputs()[0];
            const auto* vc = vcat->outputs()[0];
            const dim_t D = k->shape[2];
            if (q->shape.size() != 3 || q->shape[1] != 1 || q->shape[2] != D || qr->shape != q->shape || D % 2 != 0 ||
                cs->shape[1] != D / 2 || !f32(q) || !f32(qr) || !f32(cs) || !f32(sn))
                continue;
            // q' and the other append's cache are computed at step j: nothing may read them before it
            const auto* early = r_here != SIZE_MAX ? vc : kc;
            if (first_use[index.at(qr)] <= j || first_use[index.at(early)] <= j) continue;
            make(j, FusedKind::RopeAppend, {sa, sb, so},
                 {q, k, vcat->inputs()[1], kcat->inputs()[0], vcat->inputs()[0], cs, sn}, nullptr, {qr, kc, vc});
            continue;
        }
        if (op == Op::FusedAttention && kernels[static_cast<int>(FusedKind::AttentionGqa)] && ins.size() == 3) {
            std::vector<std::size_t> absorbed;
            const auto* k = unrepeat(ins[1], absorbed);
            const auto* v = unrepeat(ins[2], absorbed);
            if (absorbed.size() != 2 || k->shape[0] != v->shape[0]) continue;
            make(j, FusedKind::AttentionGqa, absorbed, {ins[0], k, v}, node_desc(n->op()));
            continue;
        }
    }
    std::size_t w = 0;
    for (std::size_t s = 0; s < steps.size(); ++s) {
        if (dead[s]) continue;
        if (w != s) steps[w] = std::move(steps[s]);
        ++w;
    }
    steps.resize(w);
}

// Fused and grouped launches take dense operands only (a single node's
// kernel gathers and scatters strided ones itself): a step that would hand
// such a launch a strided operand runs its nodes one by one instead, at the
// step's place, where every operand of every member exists.  Only a fused
// chain's external operands count; its inner tensors are never allocated.
void split_strided(std::vector<Step>& steps) {
    auto dense = [](const auto& ts) {
        return std::all_of(ts.begin(), ts.end(), [](pConstTensorStorage t) { return t->is_contiguous(); });
    };
    auto launchable = [&](const Step& st) {
        if (st.fused >= 0) return dense(st.ins) && dense(st.outs);
        if (st.nodes.size() < 2) return true;
        return std::all_of(st.nodes.begin(), st.nodes.end(),
                           [&](pConstNode n) { return dense(n->inputs()) && dense(n->outputs()); });
    };
    if (std::all_of(steps.begin(), steps.end(), launchable)) return;
    std::vector<Step> out;
    out.reserve(steps.size());
    for (auto& st : steps) {
        if (launchable(st)) {
            out.push_back(std::move(st));
            continue;
        }
        for (auto* n : st.nodes) {
            Step one;
            one.nodes.push_back(n);
            out.push_back(std::move(one));
        }
    }
    steps = std::move(out);
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
    const auto& tensors = graph._tensors;
    const TensorIndex index(tensors);
    const auto order = graph._validated_order(device, index);

    // Dedicated allocations: requested outputs (every tensor when none were
    // marked), graph inputs and tensors that already own data.
    std::vector<bool> active(tensors.size(), false);
    std::vector<bool> dedicated(tensors.size(), false);
    if (graph._has_explicit_outputs) {
        for (auto* s : graph._explicit_outputs) {
            const auto i = index.at(s);
            active[i] = true;
            dedicated[i] = true;
        }
    } else {
        for (std::size_t i = 0; i < tensors.size(); ++i) {
            active[i] = true;
            dedicated[i] = true;
        }
    }
    // graph inputs: the tensors no node writes (Graph::is_input_tensor, for
    // every tensor at once)
    std::vector<bool> produced(tensors.size(), false);
    for (const auto& node : graph._nodes)
        for (auto* out : node.outputs()) {
            const auto i = index.find(out);
            if (i != TensorIndex::npos) produced[i] = true;
        }
    for (std::size_t i = 0; i < tensors.size(); ++i)
        if (tensors[i]->data != nullptr || !produced[i]) dedicated[i] = true;

    auto steps = plan_steps(order, device, index, tensors.size());
    fuse_steps(steps, device, index, dedicated);
    split_strided(steps);

    // Activity and lifetimes (a fused step touches its chain's external
    // operands only).
    std::vector<std::size_t> birth(tensors.size(), 0), death(tensors.size(), 0);
    std::vector<bool> born(tensors.size(), false);
    auto read = [&](pConstTensorStorage t, std::size_t step) {
        const auto i = index.at(t);
        active[i] = true;
        death[i] = std::max(death[i], step);
    };
    auto write = [&](pConstTensorStorage t, std::size_t step) {
        const auto i = index.at(t);
        active[i] = true;
        if (!born[i]) {
            born[i] = true;
            birth[i] = step;
        }
        death[i] = std::max(death[i], step);
    };
    for (std::size_t step = 0; step < steps.size(); ++step) {
        const Step& st = steps[step];
        if (st.fused >= 0) {
            for (auto* in : st.ins) read(in, step);
            for (auto* out : st.outs) write(out, step);
            continue;
        }
        for (const auto* node : st.nodes) {
            for (auto* in : node->inputs()) read(in, step);
            for (auto* out : node->outputs()) write(out, step);
        }
    }

    // Byte-preserving steps between arena intermediates: the output views
    // its root's bytes, whose lifetime covers the output's.
    std::vector<std::size_t> root(tensors.size());
    for (std::size_t i = 0; i < tensors.size(); ++i) root[i] = i;
    std::vector<bool> alias_step(steps.size(), false);
    {
        const char* env = std::getenv("VELOMIND_GRAPH_ALIAS");
        if (!(env && env[0] == '0')) {
            for (std::size_t step = 0; step < steps.size(); ++step) {
                if (steps[step].fused >= 0 || steps[step].nodes.size() != 1 || !keeps_bytes(steps[step].nodes.front()))
                    continue;
                const auto in = root[index.at(steps[step].nodes.front()->inputs()[0])];
                const auto out = index.at(steps[step].nodes.front()->outputs()[0]);
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
    // Arena intermediates and byte-preserving aliases keep their storage
    // objects: where their bytes live is recorded here and written into
    // them just before the run plan is derived (undone if a later step
    // throws), so the build allocates no second object per tensor.
    struct Placement {
        std::size_t tensor = 0;
        void* data = nullptr;
        std::size_t offset = 0, capacity = 0;
        std::shared_ptr<void> owner;
    };
    std::vector<Placement> placed;
    std::vector<std::size_t> placed_at(tensors.size(), SIZE_MAX);
    placed.reserve(arena_items.size() + tensors.size() / 4);
    MemoryPlanStats stats;
    if (arena_bytes > 0) {
        auto arena = allocate_checked(arena_bytes, device);
        ++stats.allocation_count;
        count_allocation();
        for (const auto& it : arena_items) {
            placed_at[it.tensor] = placed.size();
            placed.push_back(Placement{it.tensor, static_cast<char*>(arena->data) + it.offset, it.offset,
                                       arena->capacity_bytes, arena});
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
        if (placed_at[root[i]] != SIZE_MAX) {
            const Placement b = placed[placed_at[root[i]]];
            placed.push_back(Placement{i, b.data, b.offset, b.capacity, b.owner});
        } else {
            const auto& base = staged[root[i]];
            placed.push_back(Placement{i, base->data, base->offset_bytes, base->capacity_bytes,
                                       base->external_owner ? base->external_owner : std::shared_ptr<void>(base)});
        }
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

    std::vector<pTensorStorage> staged_ptr(tensors.size());
    for (std::size_t i = 0; i < tensors.size(); ++i) staged_ptr[i] = staged[i].get();
    auto remap = [&](pConstTensorStorage t) { return staged_ptr[index.at(t)]; };

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
        if (step.fused >= 0) {
            // fused chain: its external operands, in the order its kind lists them
            Executable::CompiledNode cn;
            cn.inputs.reserve(step.ins.size());
            cn.outputs.reserve(step.outs.size());
            for (auto* in : step.ins) cn.inputs.push_back(remap(in));
            for (auto* out : step.outs) cn.outputs.push_back(remap(out));
            cn.kernel = fused_kernel(device, static_cast<FusedKind>(step.fused));
            cn.attrs = step.attrs;
            cn.fused = step.nodes.size();
            impl->topo.push_back(std::move(cn));
            continue;
        }
        if (step.nodes.size() > 1) {
            // grouped QuantizedMatMul: [A, B_1, S_1, ..], [C_1, ..]
            Executable::CompiledNode cn;
            cn.inputs.reserve(1 + 2 * step.nodes.size());
            cn.outputs.reserve(step.nodes.size());
            cn.inputs.push_back(remap(step.nodes.front()->inputs()[0]));
            for (const auto* node : step.nodes) {
                cn.inputs.push_back(remap(node->inputs()[1]));
                cn.inputs.push_back(remap(node->inputs()[2]));
                cn.outputs.push_back(remap(node->outputs()[0]));
            }
            cn.kernel = qmm_group_kernel(device);
            auto* ga = new QmmGroupAttrs{step.nodes.front()->op(), step.nodes.size()};
            cn.attrs = std::shared_ptr<const void>(ga, [](const void* p) { delete static_cast<const QmmGroupAttrs*>(p); });
            cn.fused = step.nodes.size();
            impl->topo.push_back(std::move(cn));
            continue;
        }
        const auto* node = step.nodes.front();
        Executable::CompiledNode cn;
        const bool aliased = alias_step[static_cast<std::size_t>(&step - steps.data())];
        DataType dtypes[4];
        std::size_t n_in = 0;
        cn.inputs.reserve(node->inputs().size());
        cn.outputs.reserve(node->outputs().size());
        for (auto* in : node->inputs()) {
            cn.inputs.push_back(remap(in));
            if (n_in < 4) dtypes[n_in] = in->dtype;
            ++n_in;
        }
        for (auto* out : node->outputs()) cn.outputs.push_back(remap(out));
        if (cn.outputs.empty()) throw std::runtime_error("velomind: op node has no outputs");
        cn.kernel = aliased ? &no_launch
                            : (n_in > 4 ? nullptr
                                        : resolve_op_kernel(node->op().op, std::span<const DataType>(dtypes, n_in),
                                                            node->outputs().front()->dtype, device));
        if (!cn.kernel) throw std::runtime_error(std::string("velomind: no kernel for op=") + op_name(node->op().op));
        cn.attrs = node_desc(node->op());
        impl->topo.push_back(std::move(cn));
    }
    // Placements into the graph's own storages, then nothing may fail: a
    // throw from here on restores the fields written.
    struct Prior {
        bool no_strides;
        DeviceType device;
        std::size_t offset, capacity;
        void* data;
        std::shared_ptr<void> owner;
    };
    std::vector<Prior> prior;
    prior.reserve(placed.size());
    for (const auto& pl : placed) {
        auto& t = *tensors[pl.tensor];
        prior.push_back(Prior{t.strides.empty(), t.device, t.offset_bytes, t.capacity_bytes, t.data, t.external_owner});
        if (t.strides.empty()) t.strides = default_strides(t.shape);
        t.device = device;
        t.offset_bytes = pl.offset;
        t.capacity_bytes = pl.capacity;
        t.data = pl.data;
        t.external_owner = pl.owner;
    }
    std::unique_ptr<Executable> exec;
    try {
        impl->derive_run_plan();
        exec = std::make_unique<Executable>();
    } catch (...) {
        for (std::size_t j = 0; j < placed.size(); ++j) {
            auto& t = *tensors[placed[j].tensor];
            const auto& pr = prior[j];
            if (pr.no_strides) t.strides.clear();
            t.device = pr.device;
            t.offset_bytes = pr.offset;
            t.capacity_bytes = pr.capacity;
            t.data = pr.data;
            t.external_owner = pr.owner;
        }
        throw;
    }

    // Commit.
    graph._tensors.swap(staged);
    for (auto& node : graph._nodes) {
        for (auto*& in : node._inputs) in = remap(in);
        for (auto*& out : node._outputs) out = remap(out);
    }
    for (auto*& out : graph._explicit_outputs) out = remap(out);
    graph._built = true;
    graph._bound_device = device;
    graph._plan_stats = stats;
    exec->_impl = std::move(impl);
    return exec;
}

}  // namespace velomind::internal
