// The N-D executor's fusion plan (nd_plan.h): a def-use graph of the ONNX nodes and a small
// pattern matcher over it.
#include "nd_plan.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <optional>
#include <set>

namespace ocr {

namespace {

// ---- patterns ---------------------------------------------------------------------------------
// An operand of a pattern node: the value the pattern starts from (X), the output of an earlier
// node of the pattern, a scalar initializer within `tol` of `value`, any scalar initializer, any
// float initializer, or any computed value other than X (a tensor some other step produces).
enum class Arg { X, Out, Near, Scalar, Weight, Value, Any, Ints };
struct Operand {
    Arg kind;
    int ref = -1;
    float value = 0.f, tol = 0.f;
    std::vector<int64_t> ints;  // Ints: an integer initializer holding exactly these values
};
Operand X() { return {Arg::X}; }
Operand Out(int k) { return {Arg::Out, k}; }
Operand Near(float v, float tol) { return {Arg::Near, -1, v, tol}; }
Operand AnyScalar() { return {Arg::Scalar}; }
Operand AnyWeight() { return {Arg::Weight}; }
Operand AnyValue() { return {Arg::Value}; }
Operand AnyInput() { return {Arg::Any}; }
Operand Ints(std::vector<int64_t> v) { return {Arg::Ints, -1, 0.f, 0.f, std::move(v)}; }

struct PNode {
    const char *op;
    std::vector<Operand> in;
    bool (*attrs_ok)(const Node &) = nullptr;
};

// swallows_x: X disappears into the step (an epilogue of the anchor), so nothing outside the
// pattern may read it; otherwise X is the step's input and may have other readers.
struct Pattern {
    const char *name;
    std::vector<PNode> nodes;
    bool swallows_x;
};

bool last_axis_mean(const Node &n) {
    const auto axes = n.ints("axes");
    return axes && axes->size() == 1 && (*axes)[0] == -1 && n.int_("keepdims").value_or(1) == 1;
}

// The chains the exporters write (shapes of the ONNX format, matched node by node).
const Pattern kLayerNorm{"layer_norm",
                         {{"ReduceMean", {X()}, last_axis_mean},
                          {"Sub", {X(), Out(0)}},
                          {"Pow", {Out(1), Near(2.f, 0.f)}},
                          {"ReduceMean", {Out(2)}, last_axis_mean},
                          {"Add", {Out(3), AnyScalar()}},
                          {"Sqrt", {Out(4)}},
                          {"Div", {Out(1), Out(5)}},
                          {"Mul", {Out(6), AnyWeight()}},
                          {"Add", {Out(7), AnyWeight()}}},
                         false};
// x * (erf(x / sqrt 2) + 1) * 0.5
const Pattern kGelu{"gelu",
                    {{"Div", {X(), Near(1.41421356f, 1e-4f)}},
                     {"Erf", {Out(0)}},
                     {"Add", {Out(1), Near(1.f, 1e-6f)}},
                     {"Mul", {X(), Out(2)}},
                     {"Mul", {Out(3), Near(0.5f, 1e-6f)}}},
                    true};
const Pattern kSilu{"silu", {{"Sigmoid", {X()}}, {"Mul", {X(), Out(0)}}}, true};
const Pattern kRelu{"relu", {{"Relu", {X()}}}, true};
const Pattern kSigmoid{"sigmoid", {{"Sigmoid", {X()}}}, true};
const Pattern kBiasAdd{"bias", {{"Add", {X(), AnyWeight()}}}, true};
const Pattern kBatchNorm{
    "batch_norm", {{"BatchNormalization", {X(), AnyWeight(), AnyWeight(), AnyWeight(), AnyWeight()}}}, true};
const Pattern kResidual{"residual", {{"Add", {X(), AnyValue()}}}, true};

bool perm_is(const Node &n, std::vector<int64_t> want) { return n.ints("perm").value_or(std::vector<int64_t>{}) == want; }
bool perm_20314(const Node &n) { return perm_is(n, {2, 0, 3, 1, 4}); }
bool perm_0132(const Node &n) { return perm_is(n, {0, 1, 3, 2}); }
bool perm_0213(const Node &n) { return perm_is(n, {0, 2, 1, 3}); }
bool last_axis_softmax(const Node &n) {
    const int64_t a = n.int_("axis").value_or(-1);
    return a == -1 || a == 3;
}
// Multi-head self-attention as the exporter writes it from a fused QKV projection x [n, T, 3 H d]:
// reshape to [n, T, 3, H, d], transpose to [3, n, H, T, d], slice and squeeze q, k, v, scale q,
// softmax(q k^T) v, back to [n, T, H d]. Captured: the first reshape's shape, the scale, the last
// reshape's shape.
const Pattern kAttention{"attention",
                         {{"Reshape", {X(), AnyInput()}},
                          {"Transpose", {Out(0)}, perm_20314},
                          {"Slice", {Out(1), Ints({0}), Ints({1}), Ints({0})}},
                          {"Squeeze", {Out(2), Ints({0})}},
                          {"Slice", {Out(1), Ints({1}), Ints({2}), Ints({0})}},
                          {"Squeeze", {Out(4), Ints({0})}},
                          {"Slice", {Out(1), Ints({2}), Ints({3}), Ints({0})}},
                          {"Squeeze", {Out(6), Ints({0})}},
                          {"Mul", {Out(3), AnyScalar()}},
                          {"Transpose", {Out(5)}, perm_0132},
                          {"MatMul", {Out(8), Out(9)}},
                          {"Softmax", {Out(10)}, last_axis_softmax},
                          {"MatMul", {Out(11), Out(7)}},
                          {"Transpose", {Out(12)}, perm_0213},
                          {"Reshape", {Out(13), AnyInput()}}},
                         false};

// Epilogue slots of each anchor kind, in order; a slot takes the first of its options that
// matches, or none.
enum class Effect { Bias, BatchNorm, Act, Residual };
struct Option {
    const Pattern *pattern;
    Effect effect;
    int act = ACT_NONE;
};
using Slots = std::vector<std::vector<Option>>;
const Slots kConvSlots{{{&kBiasAdd, Effect::Bias}},
                       {{&kBatchNorm, Effect::BatchNorm}},
                       {{&kRelu, Effect::Act, ACT_RELU}, {&kGelu, Effect::Act, ACT_GELU}},
                       {{&kResidual, Effect::Residual}}};
const Slots kLinearSlots{{{&kBiasAdd, Effect::Bias}}, {{&kSilu, Effect::Act, ACT_SILU}}, {{&kResidual, Effect::Residual}}};
const Slots kConvTSlots{{{&kBiasAdd, Effect::Bias}},
                        {{&kRelu, Effect::Act, ACT_RELU}, {&kSigmoid, Effect::Act, ACT_SIGMOID}}};

struct Match {
    std::vector<int> nodes;              // graph node of each pattern node
    std::vector<std::string> captured;   // AnyScalar / AnyWeight / AnyValue operands, in order met
};

class Planner {
  public:
    Planner(const Onnx &onnx, NdPlan &plan) : onnx_(onnx), plan_(plan) {}
    void run();

  private:
    const Onnx &onnx_;
    NdPlan &plan_;
    std::map<std::string, int> producer_;
    std::map<std::string, std::vector<int>> consumers_;
    std::vector<char> taken_;
    struct Gate {
        int mul;
        std::string x, scale;  // the ungated input and the gate
    };
    std::map<int, Gate> se_;  // dense conv -> the squeeze-excitation Mul in front of it

    const std::vector<Node> &nodes() const { return plan_.nodes; }
    bool is_weight(const std::string &v) const { return onnx_.weights.count(v) > 0; }
    bool is_const(const std::string &v) const { return is_weight(v) || onnx_.ints.count(v) > 0; }
    std::optional<float> scalar(const std::string &v) const {
        auto it = onnx_.weights.find(v);
        if (it == onnx_.weights.end() || it->second.data.size() != 1) return std::nullopt;
        return it->second.data[0];
    }
    bool is_output(const std::string &v) const { return v == plan_.output; }
    const std::vector<int> &users(const std::string &v) const {
        static const std::vector<int> none;
        auto it = consumers_.find(v);
        return it == consumers_.end() ? none : it->second;
    }
    bool read_only_by(const std::string &v, const std::vector<int> &set) const {
        if (is_output(v)) return false;
        for (int u : users(v))
            if (std::find(set.begin(), set.end(), u) == set.end()) return false;
        return true;
    }

    void index();
    void find_se_gates();
    bool operand_ok(const Operand &o, const std::string &name, const std::string &x, const std::vector<int> &bound,
                    std::vector<std::string> &caps) const;
    bool node_ok(const PNode &pn, const Node &n, const std::string &x, const std::vector<int> &bound,
                 std::vector<std::string> &caps) const;
    bool extend(const Pattern &p, const std::string &x, Match &m) const;
    std::optional<Match> match(const Pattern &p, const std::string &x) const;
    void grow(NdStep &s, std::string &v, const Slots &slots, size_t channels);
    size_t weight_dim(const std::string &w, size_t d) const {
        const Weight &t = onnx_.weight(w);
        return d < t.dims.size() ? size_t(t.dims[d]) : 0;
    }
    void take(NdStep &s, const Match &m);
};

void Planner::index() {
    producer_.clear();
    consumers_.clear();
    for (int i = 0; i < int(nodes().size()); i++) {
        for (const auto &o : nodes()[size_t(i)].outputs) producer_[o] = i;
        for (const auto &in : nodes()[size_t(i)].inputs)
            if (!in.empty()) consumers_[in].push_back(i);
    }
}

bool Planner::operand_ok(const Operand &o, const std::string &name, const std::string &x, const std::vector<int> &bound,
                         std::vector<std::string> &caps) const {
    switch (o.kind) {
    case Arg::X:
        return name == x;
    case Arg::Out:
        return o.ref < int(bound.size()) && nodes()[size_t(bound[size_t(o.ref)])].outputs.at(0) == name;
    case Arg::Near: {
        const auto v = scalar(name);
        return v && std::fabs(*v - o.value) <= o.tol;
    }
    case Arg::Scalar:
        if (!scalar(name)) return false;
        caps.push_back(name);
        return true;
    case Arg::Weight:
        if (!is_weight(name)) return false;
        caps.push_back(name);
        return true;
    case Arg::Value:
        if (name == x || name.empty() || is_const(name)) return false;
        caps.push_back(name);
        return true;
    case Arg::Any:
        if (name.empty()) return false;
        caps.push_back(name);
        return true;
    case Arg::Ints: {
        auto it = onnx_.ints.find(name);
        return it != onnx_.ints.end() && it->second == o.ints;
    }
    }
    return false;
}

// Node n matches pattern node pn: same op and attributes, and its inputs match the operands in
// order (Add and Mul of two operands in either order).
bool Planner::node_ok(const PNode &pn, const Node &n, const std::string &x, const std::vector<int> &bound,
                      std::vector<std::string> &caps) const {
    if (n.op != pn.op || n.inputs.size() != pn.in.size() || n.outputs.empty()) return false;
    if (pn.attrs_ok && !pn.attrs_ok(n)) return false;
    const bool commutes = (n.op == "Add" || n.op == "Mul") && n.inputs.size() == 2;
    for (int order = 0; order < (commutes ? 2 : 1); order++) {
        std::vector<std::string> c = caps;
        bool ok = true;
        for (size_t k = 0; k < pn.in.size() && ok; k++)
            ok = operand_ok(pn.in[k], n.inputs[order ? pn.in.size() - 1 - k : k], x, bound, c);
        if (ok) {
            caps = std::move(c);
            return true;
        }
    }
    return false;
}

// Depth-first: pattern node k is looked for among the readers of the first value operand it
// names (X or an earlier node's output); every candidate is tried, so the first complete match
// in node order wins.
bool Planner::extend(const Pattern &p, const std::string &x, Match &m) const {
    const size_t k = m.nodes.size();
    if (k == p.nodes.size()) {
        for (size_t j = 0; j + 1 < k; j++)
            if (!read_only_by(nodes()[size_t(m.nodes[j])].outputs[0], m.nodes)) return false;
        return !p.swallows_x || read_only_by(x, m.nodes);
    }
    const PNode &pn = p.nodes[k];
    std::string from;
    for (const Operand &o : pn.in) {
        if (o.kind == Arg::X) from = x;
        else if (o.kind == Arg::Out) from = nodes()[size_t(m.nodes[size_t(o.ref)])].outputs[0];
        if (!from.empty()) break;
    }
    if (from.empty()) return false;
    for (int c : users(from)) {
        if (taken_[size_t(c)] || std::find(m.nodes.begin(), m.nodes.end(), c) != m.nodes.end()) continue;
        std::vector<std::string> caps = m.captured;
        if (!node_ok(pn, nodes()[size_t(c)], x, m.nodes, caps)) continue;
        Match next{m.nodes, std::move(caps)};
        next.nodes.push_back(c);
        if (extend(p, x, next)) {
            m = std::move(next);
            return true;
        }
    }
    return false;
}

std::optional<Match> Planner::match(const Pattern &p, const std::string &x) const {
    Match m;
    if (extend(p, x, m)) return m;
    return std::nullopt;
}

void Planner::take(NdStep &s, const Match &m) {
    for (int n : m.nodes) {
        taken_[size_t(n)] = 1;
        s.nodes.push_back(n);
        s.last = std::max(s.last, n);
    }
}

// Walks the slots from value v (the anchor's result), taking what matches; v becomes the
// step's output. `channels`: the anchor's output channels (the size a bias must have).
void Planner::grow(NdStep &s, std::string &v, const Slots &slots, size_t channels) {
    for (const auto &slot : slots)
        for (const Option &opt : slot) {
            auto m = match(*opt.pattern, v);
            if (!m) continue;
            if (opt.effect == Effect::Bias) {
                // A bias: one value per output channel, along at most one axis.
                const Weight &w = onnx_.weight(m->captured.at(0));
                const auto non1 = std::count_if(w.dims.begin(), w.dims.end(), [](int64_t d) { return d != 1; });
                if (channels == 0 || w.data.size() != channels || non1 > 1) continue;
                s.bias.push_back(m->captured[0]);
            } else if (opt.effect == Effect::BatchNorm) {
                s.batch_norm = m->nodes[0];
            } else if (opt.effect == Effect::Act) {
                s.act = opt.act;
            } else {
                s.residual = m->captured.at(0);
            }
            take(s, *m);
            v = nodes()[size_t(m->nodes.back())].outputs[0];
            break;
        }
}

// Squeeze-excitation: a dense Conv whose input is Mul(x, g), g a HardSigmoid's output and the
// Mul read by nothing else, reads x and scales it by g per (image, channel) as it loads.
void Planner::find_se_gates() {
    for (int c = 0; c < int(nodes().size()); c++) {
        const Node &conv = nodes()[size_t(c)];
        if (conv.op != "Conv" || conv.int_("group").value_or(1) != 1 || conv.inputs.empty()) continue;
        auto pm = producer_.find(conv.inputs[0]);
        if (pm == producer_.end()) continue;
        const int mi = pm->second;
        const Node &mul = nodes()[size_t(mi)];
        if (mul.op != "Mul" || mul.inputs.size() != 2 || taken_[size_t(mi)]) continue;
        if (!read_only_by(mul.outputs[0], {c})) continue;
        auto hard_sigmoid = [&](const std::string &v) {
            auto p = producer_.find(v);
            return p != producer_.end() && nodes()[size_t(p->second)].op == "HardSigmoid";
        };
        for (int g : {1, 0})
            if (hard_sigmoid(mul.inputs[size_t(g)])) {
                se_[c] = {mi, mul.inputs[size_t(1 - g)], mul.inputs[size_t(g)]};
                taken_[size_t(mi)] = 1;
                break;
            }
    }
}

void Planner::run() {
    index();
    taken_.assign(nodes().size(), 0);
    find_se_gates();
    for (int i = 0; i < int(nodes().size()); i++) {
        if (taken_[size_t(i)]) continue;
        const Node &n = nodes()[size_t(i)];
        NdStep s;
        s.anchor = s.last = i;
        if (n.op == "ReduceMean" && !n.inputs.empty()) {
            auto m = match(kLayerNorm, n.inputs[0]);
            if (m && m->nodes[0] == i) {
                s.kind = NdKind::LayerNorm;
                take(s, *m);
                s.eps = *scalar(m->captured.at(0));
                s.gamma = m->captured.at(1);
                s.beta = m->captured.at(2);
                s.output = nodes()[size_t(s.last)].outputs[0];
                plan_.steps.push_back(std::move(s));
                continue;
            }
        }
        if (n.op == "Reshape" && !n.inputs.empty()) {
            auto m = match(kAttention, n.inputs[0]);
            if (m && m->nodes[0] == i) {
                s.kind = NdKind::Attention;
                take(s, *m);
                s.conv_input = n.inputs[0];
                s.attn_shape = m->captured.at(0);
                s.attn_scale = *scalar(m->captured.at(1));
                s.attn_out_shape = m->captured.at(2);
                s.output = nodes()[size_t(s.last)].outputs[0];
                plan_.steps.push_back(std::move(s));
                continue;
            }
        }
        taken_[size_t(i)] = 1;
        s.nodes.push_back(i);
        std::string v = n.outputs.at(0);
        if (n.op == "Conv" && n.inputs.size() >= 2 && is_weight(n.inputs[1])) {
            s.kind = NdKind::Conv;
            s.conv_input = n.inputs[0];
            auto se = se_.find(i);
            if (se != se_.end()) {
                s.nodes.push_back(se->second.mul);
                s.in_scale = se->second.scale;
                s.conv_input = se->second.x;
            }
            grow(s, v, kConvSlots, weight_dim(n.inputs[1], 0));
        } else if (n.op == "MatMul" && n.inputs.size() == 2 && is_weight(n.inputs[1]) &&
                   onnx_.weight(n.inputs[1]).dims.size() == 2) {
            s.kind = NdKind::Linear;
            grow(s, v, kLinearSlots, weight_dim(n.inputs[1], 1));
        } else if (n.op == "ConvTranspose" && n.inputs.size() >= 2 && is_weight(n.inputs[1])) {
            s.kind = NdKind::ConvT;
            grow(s, v, kConvTSlots, weight_dim(n.inputs[1], 1));
        } else if (n.op == "BatchNormalization") {
            s.kind = NdKind::Affine;
        }
        s.output = v;
        plan_.steps.push_back(std::move(s));
    }
    std::stable_sort(plan_.steps.begin(), plan_.steps.end(), [](const NdStep &a, const NdStep &b) { return a.last < b.last; });
}

const char *kind_name(NdKind k) {
    switch (k) {
    case NdKind::Conv: return "conv";
    case NdKind::ConvT: return "conv_transpose";
    case NdKind::Linear: return "linear";
    case NdKind::LayerNorm: return "layer_norm";
    case NdKind::Affine: return "affine";
    case NdKind::Attention: return "attention";
    default: return "node";
    }
}

const char *act_name(int a) {
    switch (a) {
    case ACT_RELU: return "relu";
    case ACT_SIGMOID: return "sigmoid";
    case ACT_GELU: return "gelu";
    case ACT_SILU: return "silu";
    default: return "none";
    }
}

}  // namespace

NdPlan plan_nd(const Onnx &onnx, bool stop_before_softmax) {
    NdPlan plan;
    // Identity nodes go: a value read through any chain of them resolves to its source.
    std::map<std::string, std::string> source;
    auto resolve = [&](const std::string &v) {
        auto it = source.find(v);
        return it == source.end() ? v : it->second;
    };
    for (const Node &n : onnx.nodes) {
        if (n.op == "Identity") {
            if (n.inputs.empty() || n.outputs.empty()) fail("Identity without input or output");
            source[n.outputs[0]] = resolve(n.inputs[0]);
            continue;
        }
        Node c = n;
        for (auto &in : c.inputs) in = resolve(in);
        plan.nodes.push_back(std::move(c));
    }
    plan.input = onnx.input;
    plan.output = resolve(onnx.output);
    // A final Softmax is cut off on request: the graph then ends at the logits it would read.
    if (stop_before_softmax)
        for (size_t i = plan.nodes.size(); i-- > 0;)
            if (!plan.nodes[i].outputs.empty() && plan.nodes[i].outputs[0] == plan.output) {
                if (plan.nodes[i].op == "Softmax" && !plan.nodes[i].inputs.empty()) {
                    plan.output = plan.nodes[i].inputs[0];
                    plan.nodes.erase(plan.nodes.begin() + long(i));
                }
                break;
            }
    // Nodes nothing needs for the output are dropped (the cut Softmax leaves none, but a graph
    // may hold others).
    std::set<std::string> need{plan.output};
    std::vector<char> live(plan.nodes.size(), 0);
    for (size_t i = plan.nodes.size(); i-- > 0;) {
        const Node &n = plan.nodes[i];
        live[i] = std::any_of(n.outputs.begin(), n.outputs.end(), [&](const std::string &o) { return need.count(o) > 0; });
        if (live[i])
            for (const auto &in : n.inputs) need.insert(in);
    }
    std::vector<Node> kept;
    for (size_t i = 0; i < plan.nodes.size(); i++)
        if (live[i]) kept.push_back(std::move(plan.nodes[i]));
    plan.nodes = std::move(kept);
    Planner(onnx, plan).run();
    return plan;
}

std::string describe(const NdPlan &plan) {
    std::string out;
    for (const NdStep &s : plan.steps) {
        out += std::string(kind_name(s.kind)) + " " + plan.nodes[size_t(s.anchor)].op + "@" + std::to_string(s.anchor) + " [";
        std::vector<int> ns = s.nodes;
        std::sort(ns.begin(), ns.end());
        for (size_t k = 0; k < ns.size(); k++) out += (k ? "," : "") + std::to_string(ns[k]);
        out += "]";
        if (s.act != ACT_NONE) out += std::string(" act=") + act_name(s.act);
        if (!s.bias.empty()) out += " bias=" + std::to_string(s.bias.size());
        if (s.batch_norm >= 0) out += " bn@" + std::to_string(s.batch_norm);
        if (!s.residual.empty()) out += " residual=" + s.residual;
        if (!s.in_scale.empty()) out += " in_scale=" + s.in_scale;
        if (s.kind == NdKind::LayerNorm) out += " gamma=" + s.gamma + " beta=" + s.beta;
        out += " -> " + s.output + "\n";
    }
    return out;
}

}  // namespace ocr
