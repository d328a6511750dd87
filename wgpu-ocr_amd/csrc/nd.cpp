// NdGraph: load-time fusions as the reference's NdGraph::new (src/nd.rs:505-817) decides them,
// plus one of this library's own (a BatchNormalization right after a Conv becomes the conv's
// epilogue affine), and a run loop over the ops of NdGraph::run (nd.rs:834-1195). Buffers come
// from the context's stream-ordered pool and go back after their last reader.
#include "nd.h"

#include <algorithm>
#include <cmath>
#include <functional>
#include <numeric>

namespace ocr {

size_t NdTensor::count() const {
    size_t c = 1;
    for (int64_t d : shape) c *= size_t(d);
    return c;
}

namespace {

int axis_of(int64_t a, size_t rank) {
    const int64_t r = a < 0 ? a + int64_t(rank) : a;
    if (r < 0 || r >= int64_t(std::max<size_t>(rank, 1)))
        fail("axis " + std::to_string(a) + " out of range for rank " + std::to_string(rank));
    return int(r);
}

std::vector<size_t> strides_of(const std::vector<int64_t> &shape) {
    std::vector<size_t> s(shape.size(), 1);
    for (size_t d = shape.size(); d-- > 1;) s[d - 1] = s[d] * size_t(shape[d]);
    return s;
}

std::string shape_str(const std::vector<int64_t> &s) {
    std::string o = "[";
    for (size_t i = 0; i < s.size(); i++) o += (i ? ", " : "") + std::to_string(s[i]);
    return o + "]";
}

bool env_set(const char *n) { return std::getenv(n) != nullptr; }

}  // namespace

// ---------------------------------------------------------------------------------------------
// Build
// ---------------------------------------------------------------------------------------------
NdGraph NdGraph::build(Ctx &ctx, const Onnx &onnx, bool stop_before_softmax) {
    NdGraph g;
    // Identity nodes: readers read their input instead (nd.rs:506-524).
    std::map<std::string, std::string> alias;
    for (const Node &n : onnx.nodes)
        if (n.op == "Identity") {
            auto it = alias.find(n.inputs.at(0));
            alias[n.outputs.at(0)] = it != alias.end() ? it->second : n.inputs.at(0);
        }
    auto resolve = [&](const std::string &s) {
        auto it = alias.find(s);
        return it == alias.end() ? s : it->second;
    };
    std::vector<Node> nodes;
    for (const Node &n : onnx.nodes) {
        if (n.op == "Identity") continue;
        Node c = n;
        for (auto &i : c.inputs) i = resolve(i);
        nodes.push_back(std::move(c));
    }
    std::string output = resolve(onnx.output);
    // Drop a final Softmax (nd.rs:526-532).
    if (stop_before_softmax) {
        for (size_t i = nodes.size(); i-- > 0;)
            if (!nodes[i].outputs.empty() && nodes[i].outputs[0] == output) {
                if (nodes[i].op == "Softmax") {
                    output = nodes[i].inputs.at(0);
                    nodes.resize(i);
                }
                break;
            }
    }
    auto has_weight = [&](const std::string &nm) { return onnx.weights.count(nm) > 0; };
    auto scalar = [&](const std::string &nm) -> std::optional<float> {
        auto it = onnx.weights.find(nm);
        if (it == onnx.weights.end() || it->second.data.size() != 1) return std::nullopt;
        return it->second.data[0];
    };
    std::vector<bool> skip(nodes.size(), false);
    auto count_readers = [&]() {
        std::map<std::string, int> c;
        for (size_t k = 0; k < nodes.size(); k++)
            if (!skip[k])
                for (const auto &i : nodes[k].inputs) c[i]++;
        return c;
    };
    // Squeeze-excitation: Mul(x, HardSigmoid gate) read only by a dense Conv becomes that conv's
    // input scale (nd.rs:552-571).
    std::map<size_t, std::string> in_scale;
    {
        auto first = count_readers();
        auto readers = [&](const std::string &nm) { return first[nm] + (nm == output ? 1 : 0); };
        std::vector<std::tuple<size_t, size_t, std::string, std::string>> se;
        for (size_t mi = 0; mi < nodes.size(); mi++) {
            const Node &m = nodes[mi];
            if (m.op != "Mul" || readers(m.outputs[0]) != 1) continue;
            size_t ci = nodes.size();
            for (size_t c = 0; c < nodes.size(); c++)
                if (nodes[c].op == "Conv" && nodes[c].inputs.at(0) == m.outputs[0] && nodes[c].int_("group").value_or(1) == 1) {
                    ci = c;
                    break;
                }
            if (ci == nodes.size()) continue;
            auto gate = [&](const std::string &nm) {
                return std::any_of(nodes.begin(), nodes.end(),
                                   [&](const Node &x) { return x.op == "HardSigmoid" && x.outputs[0] == nm; });
            };
            if (gate(m.inputs.at(1))) se.emplace_back(mi, ci, m.inputs[0], m.inputs[1]);
            else if (gate(m.inputs.at(0))) se.emplace_back(mi, ci, m.inputs[1], m.inputs[0]);
        }
        if (!env_set("NOSE"))
            for (auto &[mi, ci, x, sc] : se) {
                in_scale[ci] = sc;
                skip[mi] = true;
                nodes[ci].inputs[0] = x;
            }
    }
    auto counts = count_readers();
    auto readers = [&](const std::string &nm) {
        auto it = counts.find(nm);
        return (it == counts.end() ? 0 : it->second) + (nm == output ? 1 : 0);
    };
    // A following Add of a constant `want`-element bias with at most one non-1 dimension.
    auto takes_bias = [&](const Node &next, const std::string &out, size_t want) -> std::optional<std::string> {
        if (next.op != "Add" || readers(out) != 1) return std::nullopt;
        std::string other;
        if (next.inputs.at(0) == out) other = next.inputs.at(1);
        else if (next.inputs.at(1) == out) other = next.inputs.at(0);
        else return std::nullopt;
        auto it = onnx.weights.find(other);
        if (it == onnx.weights.end() || it->second.data.size() != want) return std::nullopt;
        int non1 = 0;
        for (int64_t d : it->second.dims) non1 += d != 1;
        if (non1 > 1) return std::nullopt;
        return other;
    };

    size_t i = 0;
    while (i < nodes.size()) {
        if (skip[i]) {
            i++;
            continue;
        }
        const Node &n = nodes[i];
        NdOp op;
        op.node = int(i);
        op.inputs = n.inputs;
        op.output = n.outputs.at(0);
        size_t j = i + 1;
        std::string out = n.outputs[0];
        // LayerNorm chain (nd.rs:583-611).
        if (n.op == "ReduceMean" && i + 9 <= nodes.size()) {
            const Node &mean = nodes[i], &sub = nodes[i + 1], &pw = nodes[i + 2], &var = nodes[i + 3],
                       &add = nodes[i + 4], &sq = nodes[i + 5], &div = nodes[i + 6], &mul = nodes[i + 7],
                       &beta = nodes[i + 8];
            auto last_axis = [](const Node &x) {
                auto a = x.ints("axes");
                return a && a->size() == 1 && (*a)[0] == -1;
            };
            const bool chain =
                last_axis(mean) && sub.op == "Sub" && sub.inputs[0] == mean.inputs[0] && sub.inputs[1] == mean.outputs[0] &&
                pw.op == "Pow" && pw.inputs[0] == sub.outputs[0] && scalar(pw.inputs[1]) == std::optional<float>(2.f) &&
                var.op == "ReduceMean" && var.inputs[0] == pw.outputs[0] && last_axis(var) && add.op == "Add" &&
                add.inputs[0] == var.outputs[0] && scalar(add.inputs[1]).has_value() && sq.op == "Sqrt" &&
                sq.inputs[0] == add.outputs[0] && div.op == "Div" && div.inputs[0] == sub.outputs[0] &&
                div.inputs[1] == sq.outputs[0] && mul.op == "Mul" && mul.inputs[0] == div.outputs[0] &&
                has_weight(mul.inputs[1]) && beta.op == "Add" && beta.inputs[0] == mul.outputs[0] &&
                has_weight(beta.inputs[1]) && readers(mean.outputs[0]) == 1 && readers(sub.outputs[0]) == 2 &&
                readers(pw.outputs[0]) == 1 && readers(var.outputs[0]) == 1 && readers(add.outputs[0]) == 1 &&
                readers(sq.outputs[0]) == 1 && readers(div.outputs[0]) == 1 && readers(mul.outputs[0]) == 1;
            if (chain) {
                const Weight &gm = onnx.weight(mul.inputs[1]), &bt = onnx.weight(beta.inputs[1]);
                if (gm.data.size() != bt.data.size()) fail("LayerNorm gamma and beta sizes differ");
                std::vector<float> gb = gm.data;
                gb.insert(gb.end(), bt.data.begin(), bt.data.end());
                op.kind = NdKind::LayerNorm;
                op.gb = ctx.upload_weights(gb.data(), gb.size());
                op.len = int(gm.data.size());
                op.eps = *scalar(add.inputs[1]);
                op.inputs = {mean.inputs[0]};
                op.output = beta.outputs[0];
                for (size_t k = i + 1; k < i + 9; k++) skip[k] = true;
                g.ops.push_back(std::move(op));
                i += 9;
                continue;
            }
        }
        if (n.op == "Conv") {
            const Weight &w = onnx.weight(n.inputs.at(1));
            if (w.dims.size() != 4) fail("conv weight not 4D");
            op.kind = NdKind::Conv;
            op.cout = int(w.dims[0]);
            op.cin_g = int(w.dims[1]);
            op.kh = int(w.dims[2]);
            op.kw = int(w.dims[3]);
            op.group = int(n.int_("group").value_or(1));
            op.cin = op.cin_g * op.group;
            std::vector<float> b(size_t(op.cout), 0.f);
            if (n.inputs.size() > 2 && !n.inputs[2].empty()) {
                const Weight &bw = onnx.weight(n.inputs[2]);
                if (bw.data.size() != size_t(op.cout)) fail("Conv bias size");
                b = bw.data;
            }
            if (j < nodes.size())
                if (auto bn = takes_bias(nodes[j], out, size_t(op.cout))) {
                    const Weight &bw = onnx.weight(*bn);
                    for (int c = 0; c < op.cout; c++) b[size_t(c)] += bw.data[size_t(c)];
                    out = nodes[j].outputs[0];
                    j++;
                }
            // This library's fusion: BatchNormalization right after, as the epilogue affine.
            if (j < nodes.size() && nodes[j].op == "BatchNormalization" && nodes[j].inputs.at(0) == out &&
                readers(out) == 1 && !env_set("NOBNFUSE")) {
                const Node &bn = nodes[j];
                const float eps = bn.f32("epsilon").value_or(1e-5f);
                const Weight &sc = onnx.weight(bn.inputs.at(1)), &sf = onnx.weight(bn.inputs.at(2)),
                             &mn = onnx.weight(bn.inputs.at(3)), &vr = onnx.weight(bn.inputs.at(4));
                std::vector<float> st(size_t(2 * op.cout));
                for (int c = 0; c < op.cout; c++) {
                    const float s = sc.data.at(size_t(c)) / std::sqrt(vr.data.at(size_t(c)) + eps);
                    st[size_t(c)] = s;
                    st[size_t(op.cout + c)] = sf.data.at(size_t(c)) - mn.data.at(size_t(c)) * s;
                }
                op.affine = ctx.upload_weights(st.data(), st.size());
                out = bn.outputs[0];
                j++;
            }
            if (j < nodes.size() && nodes[j].op == "Relu" && nodes[j].inputs.at(0) == out && readers(out) == 1) {
                op.act = ACT_RELU;
                out = nodes[j].outputs[0];
                j++;
            }
            // GELU as the exporter writes it: x * (erf(x / sqrt 2) + 1) * 0.5 (nd.rs:650-676).
            if (op.act == ACT_NONE && j + 5 <= nodes.size()) {
                const Node &dv = nodes[j], &ef = nodes[j + 1], &ad = nodes[j + 2], &ml = nodes[j + 3], &hf = nodes[j + 4];
                auto contains = [](const std::vector<std::string> &v, const std::string &x) {
                    return std::find(v.begin(), v.end(), x) != v.end();
                };
                auto any_scalar = [&](const std::vector<std::string> &v, float want, float tol) {
                    return std::any_of(v.begin(), v.end(), [&](const std::string &x) {
                        auto s = scalar(x);
                        return s && std::fabs(*s - want) < tol;
                    });
                };
                auto sq2 = scalar(dv.inputs.size() > 1 ? dv.inputs[1] : "");
                if (dv.op == "Div" && dv.inputs[0] == out && sq2 && std::fabs(*sq2 - 1.41421356f) < 1e-4f &&
                    ef.op == "Erf" && ef.inputs[0] == dv.outputs[0] && ad.op == "Add" && contains(ad.inputs, ef.outputs[0]) &&
                    any_scalar(ad.inputs, 1.f, 1e-6f) && ml.op == "Mul" && contains(ml.inputs, out) &&
                    contains(ml.inputs, ad.outputs[0]) && hf.op == "Mul" && contains(hf.inputs, ml.outputs[0]) &&
                    any_scalar(hf.inputs, 0.5f, 1e-6f) && readers(out) == 2 && readers(dv.outputs[0]) == 1 &&
                    readers(ef.outputs[0]) == 1 && readers(ad.outputs[0]) == 1 && readers(ml.outputs[0]) == 1) {
                    op.act = ACT_GELU;
                    out = hf.outputs[0];
                    j += 5;
                }
            }
            // A residual Add of another computed tensor (nd.rs:678-690).
            if (j < nodes.size() && nodes[j].op == "Add" && readers(out) == 1) {
                const Node &ad = nodes[j];
                const std::string *other = nullptr;
                if (ad.inputs.at(0) == out) other = &ad.inputs.at(1);
                else if (ad.inputs.at(1) == out) other = &ad.inputs.at(0);
                if (other && !onnx.weights.count(*other) && !onnx.ints.count(*other)) {
                    op.residual = *other;
                    out = ad.outputs[0];
                    j++;
                }
            }
            if (auto d = n.ints("dilations"))
                for (int64_t v : *d)
                    if (v != 1) fail("dilated conv");
            auto st = n.ints("strides").value_or(std::vector<int64_t>{1, 1});
            op.sh = int(st.at(0));
            op.sw = int(st.at(1));
            const auto ap = n.str("auto_pad").value_or("NOTSET");
            op.same_upper = ap == "SAME_UPPER";
            if (ap != "NOTSET" && ap != "SAME_UPPER") fail("Conv auto_pad " + ap);
            if (auto p = n.ints("pads")) {
                if (p->size() != 4) fail("Conv pads");
                for (int k = 0; k < 4; k++) op.pads[k] = int((*p)[size_t(k)]);
            }
            auto isc = in_scale.find(i);
            if (isc != in_scale.end()) op.in_scale = isc->second;
            if ((op.group != 1) && (!op.residual.empty() || !op.in_scale.empty()))
                fail("residual or input scale after a grouped conv");
            op.b = ctx.upload_weights(b.data(), b.size());
            op.mfma = op.group == 1 && conv_mfma_supported(op.kh, op.kw, op.sh, op.sw);
            if (op.mfma) {
                op.pk = plan_conv_pack(op.cin, op.cout, op.kh, op.kw);
                std::vector<uint16_t> hi(op.pk.halves()), lo(op.pk.halves());
                bool exact = true;
                pack_conv_weights(op.pk, w.data.data(), hi.data(), lo.data(), &exact);
                op.pk.exact = exact;
                op.whi = ctx.upload_weights(hi.data(), hi.size());
                if (!exact) op.wlo = ctx.upload_weights(lo.data(), lo.size());
            } else {
                op.w = ctx.upload_weights(w.data.data(), w.data.size());
            }
            op.inputs = {nodes[i].inputs[0]};
        } else if (n.op == "MatMul" && onnx.weights.count(n.inputs.at(1)) &&
                   onnx.weight(n.inputs[1]).dims.size() == 2) {
            const Weight &w = onnx.weight(n.inputs[1]);
            op.kind = NdKind::Linear;
            op.k = int(w.dims[0]);
            op.n = int(w.dims[1]);
            std::vector<float> b(size_t(op.n), 0.f);
            if (j < nodes.size())
                if (auto bn = takes_bias(nodes[j], out, size_t(op.n))) {
                    b = onnx.weight(*bn).data;
                    out = nodes[j].outputs[0];
                    j++;
                }
            // SiLU: x * sigmoid(x) (nd.rs:738-752).
            if (j + 2 <= nodes.size()) {
                const Node &sg = nodes[j], &ml = nodes[j + 1];
                if (sg.op == "Sigmoid" && sg.inputs.at(0) == out && ml.op == "Mul" &&
                    std::find(ml.inputs.begin(), ml.inputs.end(), out) != ml.inputs.end() &&
                    std::find(ml.inputs.begin(), ml.inputs.end(), sg.outputs[0]) != ml.inputs.end() &&
                    readers(out) == 2 && readers(sg.outputs[0]) == 1) {
                    op.act = ACT_SILU;
                    out = ml.outputs[0];
                    j += 2;
                }
            }
            // [k][n] -> rows [n][k] for the GEMM's packed layout.
            std::vector<float> t(size_t(op.n) * op.k);
            for (int kk = 0; kk < op.k; kk++)
                for (int c = 0; c < op.n; c++) t[size_t(c) * op.k + kk] = w.data[size_t(kk) * op.n + c];
            op.pk = plan_conv_pack(op.k, op.n, 1, 1);
            std::vector<uint16_t> hi(op.pk.halves()), lo(op.pk.halves());
            bool exact = true;
            pack_conv_weights(op.pk, t.data(), hi.data(), lo.data(), &exact);
            op.pk.exact = exact;
            op.whi = ctx.upload_weights(hi.data(), hi.size());
            if (!exact) op.wlo = ctx.upload_weights(lo.data(), lo.size());
            op.b = ctx.upload_weights(b.data(), b.size());
            op.inputs = {n.inputs[0]};
        } else if (n.op == "ConvTranspose") {
            const Weight &w = onnx.weight(n.inputs.at(1));
            if (w.dims.size() != 4) fail("ConvTranspose weight not 4D");
            auto st = n.ints("strides").value_or(std::vector<int64_t>{1, 1});
            bool bad = n.int_("group").value_or(1) != 1 || st.size() != 2 || st[0] != st[1];
            for (const char *a : {"pads", "output_padding"})
                if (auto p = n.ints(a))
                    for (int64_t v : *p) bad |= v != 0;
            if (bad) fail("unsupported ConvTranspose attributes");
            op.kind = NdKind::ConvT;
            op.cin = int(w.dims[0]);
            op.cout = int(w.dims[1]);
            op.kh = int(w.dims[2]);
            op.kw = int(w.dims[3]);
            op.sh = op.sw = int(st[0]);
            std::vector<float> b(size_t(op.cout), 0.f);
            if (n.inputs.size() > 2 && !n.inputs[2].empty()) b = onnx.weight(n.inputs[2]).data;
            if (j < nodes.size())
                if (auto bn = takes_bias(nodes[j], out, size_t(op.cout))) {
                    const Weight &bw = onnx.weight(*bn);
                    for (int c = 0; c < op.cout; c++) b[size_t(c)] += bw.data[size_t(c)];
                    out = nodes[j].outputs[0];
                    j++;
                }
            if (j < nodes.size() && (nodes[j].op == "Relu" || nodes[j].op == "Sigmoid") &&
                nodes[j].inputs.at(0) == out && readers(out) == 1) {
                op.act = nodes[j].op == "Relu" ? ACT_RELU : ACT_SIGMOID;
                out = nodes[j].outputs[0];
                j++;
            }
            op.w = ctx.upload_weights(w.data.data(), w.data.size());
            op.b = ctx.upload_weights(b.data(), b.size());
            op.inputs = {n.inputs[0]};
        } else if (n.op == "BatchNormalization") {
            const float eps = n.f32("epsilon").value_or(1e-5f);
            const Weight &sc = onnx.weight(n.inputs.at(1)), &sf = onnx.weight(n.inputs.at(2)),
                         &mn = onnx.weight(n.inputs.at(3)), &vr = onnx.weight(n.inputs.at(4));
            const size_t c = sc.data.size();
            std::vector<float> st(2 * c);
            for (size_t ch = 0; ch < c; ch++) {
                const float s = sc.data[ch] / std::sqrt(vr.data.at(ch) + eps);
                st[ch] = s;
                st[c + ch] = sf.data.at(ch) - mn.data.at(ch) * s;
            }
            op.kind = NdKind::Affine;
            op.st = ctx.upload_weights(st.data(), st.size());
            op.cout = int(c);
            op.inputs = {n.inputs[0]};
        }
        for (size_t k = i + 1; k < j; k++) skip[k] = true;
        op.output = out;
        g.ops.push_back(std::move(op));
        i = j;
    }
    // Weights every generic op may read, and small constants kept on the host too.
    for (const auto &kv : onnx.weights) {
        DevW w;
        w.shape = kv.second.dims;
        w.p = ctx.upload_weights(kv.second.data.data(), std::max<size_t>(kv.second.data.size(), 1));
        if (kv.second.data.size() <= 16) w.host = kv.second.data;
        g.weights_[kv.first] = std::move(w);
    }
    g.ints_ = onnx.ints;
    g.nodes_ = std::move(nodes);
    g.input = onnx.input;
    g.output = output;
    for (size_t k = 0; k < g.ops.size(); k++) {
        for (const auto &nm : g.ops[k].inputs) g.last_use_[nm] = k;
        if (!g.ops[k].residual.empty()) g.last_use_[g.ops[k].residual] = k;
        if (!g.ops[k].in_scale.empty()) g.last_use_[g.ops[k].in_scale] = k;
    }
    return g;
}

// ---------------------------------------------------------------------------------------------
// Run
// ---------------------------------------------------------------------------------------------
NdValue NdGraph::get(const std::map<std::string, NdValue> &vals, const std::string &name) const {
    auto it = vals.find(name);
    if (it != vals.end()) return it->second;
    auto wt = weights_.find(name);
    if (wt != weights_.end()) {
        NdValue v;
        v.t.p = const_cast<float *>(wt->second.p);
        v.t.shape = wt->second.shape;
        return v;
    }
    auto in = ints_.find(name);
    if (in != ints_.end()) {
        NdValue v;
        v.is_int = true;
        v.iv = in->second;
        v.ishape = {int64_t(in->second.size())};
        return v;
    }
    fail("missing value " + name);
}

NdTensor NdGraph::run_ops(Ctx *ctx, const NdTensor &x, size_t nops, std::map<std::string, NdValue> *vals_out) const {
    // Without a context only shapes are worked out (no memory, no launches).
    const bool shapes_only = ctx == nullptr;
    const hipStream_t st = shapes_only ? nullptr : ctx->stream();
    std::map<std::string, NdValue> vals;
    NdValue xin;
    xin.t = x;
    vals[input] = xin;
    auto alloc = [&](const std::vector<int64_t> &shape) {
        NdTensor t;
        t.shape = shape;
        if (!shapes_only) {
            t.buf = std::make_shared<DBuf>(ctx, std::max<size_t>(t.count(), 1) * sizeof(float));
            t.p = t.buf->as<float>();
        }
        return t;
    };
    for (size_t oi = 0; oi < nops; oi++) {
        const NdOp &op = ops[oi];
        const Node &n = nodes_[size_t(op.node)];
        auto arg = [&](size_t k) { return get(vals, op.inputs.at(k)); };
        auto flt = [&](size_t k) {
            NdValue v = arg(k);
            if (v.is_int) fail(n.op + ": input " + std::to_string(k) + " is not float");
            return v.t;
        };
        auto ints = [&](size_t k) {
            NdValue v = arg(k);
            if (!v.is_int) fail(n.op + ": input " + std::to_string(k) + " is not an integer constant");
            return v.iv;
        };
        NdValue out;
        switch (op.kind) {
        case NdKind::Conv: {
            const NdTensor a = flt(0);
            if (a.shape.size() != 4) fail("Conv input " + shape_str(a.shape));
            const int nb = int(a.shape[0]), cin = int(a.shape[1]), h = int(a.shape[2]), w = int(a.shape[3]);
            if (cin != op.cin) fail("Conv expects " + std::to_string(op.cin) + " channels, has " + std::to_string(cin));
            int pt = op.pads[0], pl = op.pads[1], pb = op.pads[2], pr = op.pads[3];
            if (op.same_upper) {
                const int oh = (h + op.sh - 1) / op.sh, ow = (w + op.sw - 1) / op.sw;
                const int th = std::max(0, (oh - 1) * op.sh + op.kh - h), tw = std::max(0, (ow - 1) * op.sw + op.kw - w);
                pt = th / 2, pl = tw / 2, pb = th - th / 2, pr = tw - tw / 2;
            }
            if (h + pt + pb < op.kh || w + pl + pr < op.kw) fail("Conv input smaller than its kernel");
            const int oh = (h + pt + pb - op.kh) / op.sh + 1, ow = (w + pl + pr - op.kw) / op.sw + 1;
            out.t = alloc({nb, op.cout, oh, ow});
            NdTensor res, sc;
            if (!op.residual.empty()) {
                res = get(vals, op.residual).t;
                if (res.shape != out.t.shape)
                    fail("residual " + shape_str(res.shape) + " for a conv giving " + shape_str(out.t.shape));
            }
            if (!op.in_scale.empty()) {
                sc = get(vals, op.in_scale).t;
                if (sc.count() != size_t(nb) * cin) fail("input scale " + shape_str(sc.shape) + " for " + shape_str(a.shape));
            }
            if (shapes_only) break;
            if (op.mfma) {
                ConvArgs ca;
                ca.x = Act{a.p, nb, h, w, cin, cin};
                ca.y = Act{out.t.p, nb, oh, ow, op.cout, op.cout};
                ca.nchw = true;
                ca.wt_hi = op.whi;
                ca.wt_lo = op.wlo;
                ca.bias = op.b;
                ca.affine = op.affine;
                ca.res = res.p;
                ca.in_scale = sc.p;
                ca.pt = pt;
                ca.pl = pl;
                ca.act = op.act;
                ca.pk = op.pk;
                conv_mfma(ca, st);
            } else {
                NdConvArgs ca;
                ca.x = a.p;
                ca.n = nb;
                ca.cin = cin;
                ca.h = h;
                ca.w = w;
                ca.wt = op.w;
                ca.b = op.b;
                ca.affine = op.affine;
                ca.res = res.p;
                ca.in_scale = sc.p;
                ca.y = out.t.p;
                ca.cout = op.cout;
                ca.oh = oh;
                ca.ow = ow;
                ca.kh = op.kh;
                ca.kw = op.kw;
                ca.sh = op.sh;
                ca.sw = op.sw;
                ca.pt = pt;
                ca.pl = pl;
                ca.group = op.group;
                ca.act = op.act;
                nd_conv_generic(ca, st);
            }
            break;
        }
        case NdKind::ConvT: {
            const NdTensor a = flt(0);
            if (a.shape.size() != 4) fail("ConvTranspose input " + shape_str(a.shape));
            if (a.shape[1] != op.cin) fail("ConvTranspose expects " + std::to_string(op.cin) + " channels");
            const int nb = int(a.shape[0]), h = int(a.shape[2]), w = int(a.shape[3]);
            out.t = alloc({nb, op.cout, (h - 1) * op.sh + op.kh, (w - 1) * op.sw + op.kw});
            if (!shapes_only)
                nd_conv_transpose(a.p, nb, op.cin, h, w, op.w, op.b, out.t.p, op.cout, op.kh, op.kw, op.sh, op.act, st);
            break;
        }
        case NdKind::Linear: {
            const NdTensor a = flt(0);
            if (a.shape.empty() || a.shape.back() != op.k)
                fail("MatMul: " + shape_str(a.shape) + " by [" + std::to_string(op.k) + ", " + std::to_string(op.n) + "]");
            const size_t m = a.count() / size_t(op.k);
            auto shape = a.shape;
            shape.back() = op.n;
            out.t = alloc(shape);
            if (shapes_only || m == 0) break;
            if (m > 0x7fffffff) fail("MatMul: too many rows");
            ConvArgs ca;
            ca.x = Act{a.p, 1, 1, int(m), op.k, op.k};
            ca.y = Act{out.t.p, 1, 1, int(m), op.n, op.n};
            ca.wt_hi = op.whi;
            ca.wt_lo = op.wlo;
            ca.bias = op.b;
            ca.act = op.act;
            ca.pk = op.pk;
            conv_mfma(ca, st);
            break;
        }
        case NdKind::LayerNorm: {
            const NdTensor a = flt(0);
            if (a.shape.empty() || a.shape.back() != op.len)
                fail("LayerNorm over " + shape_str(a.shape) + ", expects " + std::to_string(op.len));
            out.t = alloc(a.shape);
            if (!shapes_only) nd_layer_norm(a.p, op.gb, out.t.p, a.count() / size_t(op.len), op.len, op.eps, st);
            break;
        }
        case NdKind::Affine: {
            const NdTensor a = flt(0);
            const int c = a.shape.size() > 1 ? int(a.shape[1]) : 1;
            if (c != op.cout) fail("BatchNormalization over " + std::to_string(c) + " channels, has " + std::to_string(op.cout));
            size_t inner = 1;
            for (size_t d = 2; d < a.shape.size(); d++) inner *= size_t(a.shape[d]);
            out.t = alloc(a.shape);
            if (!shapes_only) nd_affine(a.p, op.st, out.t.p, a.count(), c, std::max<size_t>(inner, 1), st);
            break;
        }
        case NdKind::Generic: {
            const std::string &o = n.op;
            if (o == "Add" || o == "Sub" || o == "Mul" || o == "Div" || o == "Pow") {
                NdValue va = arg(0), vb = arg(1);
                if (va.is_int && vb.is_int) {
                    out.is_int = true;
                    out.ishape = va.ishape;
                    for (size_t k = 0; k < va.iv.size(); k++) {
                        const int64_t xa = va.iv[k], xb = vb.iv.size() == 1 ? vb.iv[0] : vb.iv.at(k);
                        int64_t r = xa;
                        if (o == "Add") r = xa + xb;
                        else if (o == "Sub") r = xa - xb;
                        else if (o == "Mul") r = xa * xb;
                        else if (o == "Div") r = xb == 0 ? 0 : xa / xb;
                        out.iv.push_back(r);
                    }
                    break;
                }
                if (va.is_int || vb.is_int) fail(o + ": mixed integer and float inputs");
                const auto &sa0 = va.t.shape, &sb0 = vb.t.shape;
                const size_t r = std::max(sa0.size(), sb0.size());
                if (r > size_t(ND_RANK)) fail("rank above 6");
                auto pad = [&](const std::vector<int64_t> &s) {
                    std::vector<int64_t> p(r - s.size(), 1);
                    p.insert(p.end(), s.begin(), s.end());
                    return p;
                };
                const auto sa = pad(sa0), sb = pad(sb0);
                std::vector<int64_t> shape(r);
                for (size_t d = 0; d < r; d++) {
                    if (sa[d] != sb[d] && sa[d] != 1 && sb[d] != 1)
                        fail(o + ": shapes " + shape_str(sa0) + " and " + shape_str(sb0) + " do not broadcast");
                    shape[d] = std::max(sa[d], sb[d]);
                }
                out.t = alloc(shape);
                if (shapes_only) break;
                NdIndex ix;
                ix.total = out.t.count();
                ix.rank = int(r);
                const auto ta = strides_of(sa), tb = strides_of(sb);
                for (size_t d = 0; d < r; d++) {
                    ix.dims[d] = size_t(shape[d]);
                    ix.s0[d] = sa[d] == 1 ? 0 : ta[d];
                    ix.s1[d] = sb[d] == 1 ? 0 : tb[d];
                }
                const int bop = o == "Add" ? BIN_ADD : o == "Sub" ? BIN_SUB : o == "Mul" ? BIN_MUL : o == "Div" ? BIN_DIV : BIN_POW;
                nd_binary(va.t.p, vb.t.p, out.t.p, ix, bop, st);
            } else if (o == "Relu" || o == "Sigmoid" || o == "HardSigmoid" || o == "Erf" || o == "Sqrt") {
                const NdTensor a = flt(0);
                out.t = alloc(a.shape);
                const int u = o == "Relu" ? UN_RELU : o == "Sigmoid" ? UN_SIGMOID : o == "HardSigmoid" ? UN_HARDSIGMOID
                            : o == "Erf" ? UN_ERF : UN_SQRT;
                if (!shapes_only)
                    nd_unary(a.p, out.t.p, a.count(), u, n.f32("alpha").value_or(0.2f), n.f32("beta").value_or(0.5f), st);
            } else if (o == "ReduceMean" || o == "GlobalAveragePool") {
                const NdTensor a = flt(0);
                const size_t r = a.shape.size();
                std::vector<int> axes;
                if (o == "GlobalAveragePool") {
                    if (r < 3) fail("GlobalAveragePool on " + shape_str(a.shape));
                    for (size_t d = 2; d < r; d++) axes.push_back(int(d));
                } else if (auto ax = n.ints("axes")) {
                    for (int64_t v : *ax) axes.push_back(axis_of(v, r));
                } else {
                    for (size_t d = 0; d < r; d++) axes.push_back(int(d));
                }
                std::sort(axes.begin(), axes.end());
                for (size_t k = 0; k < axes.size(); k++)
                    if (axes[k] != int(r - axes.size() + k)) fail("ReduceMean over non-trailing axes");
                size_t inner = 1;
                for (int d : axes) inner *= size_t(a.shape[size_t(d)]);
                const bool keep = o == "GlobalAveragePool" || n.int_("keepdims").value_or(1) == 1;
                std::vector<int64_t> shape;
                for (size_t d = 0; d < r; d++) {
                    const bool red = std::find(axes.begin(), axes.end(), int(d)) != axes.end();
                    if (!red) shape.push_back(a.shape[d]);
                    else if (keep) shape.push_back(1);
                }
                out.t = alloc(shape);
                if (!shapes_only) nd_reduce_mean(a.p, out.t.p, a.count() / std::max<size_t>(inner, 1), int(inner), st);
            } else if (o == "Softmax") {
                const NdTensor a = flt(0);
                const int ax = axis_of(n.int_("axis").value_or(-1), a.shape.size());
                size_t len = 1;
                for (size_t d = size_t(ax); d < a.shape.size(); d++) len *= size_t(a.shape[d]);
                out.t = alloc(a.shape);
                if (!shapes_only) nd_softmax(a.p, out.t.p, a.count() / std::max<size_t>(len, 1), int(len), st);
            } else if (o == "MatMul") {
                const NdTensor a = flt(0), b = flt(1);
                const size_t r = a.shape.size();
                if (r < 2 || b.shape.size() != r || !std::equal(a.shape.begin(), a.shape.end() - 2, b.shape.begin()) ||
                    a.shape[r - 1] != b.shape[r - 2])
                    fail("MatMul shapes " + shape_str(a.shape) + " x " + shape_str(b.shape));
                const int64_t m = a.shape[r - 2], k = a.shape[r - 1], nn = b.shape[r - 1];
                size_t batch = 1;
                for (size_t d = 0; d + 2 < r; d++) batch *= size_t(a.shape[d]);
                auto shape = a.shape;
                shape[r - 1] = nn;
                out.t = alloc(shape);
                if (shapes_only) break;
                BgemmArgs gm;
                gm.a = a.p;
                gm.b = b.p;
                gm.c = out.t.p;
                gm.batch = int(batch);
                gm.m = int(m);
                gm.n = int(nn);
                gm.k = int(k);
                gm.sab = size_t(m * k), gm.sam = size_t(k), gm.sak = 1;
                gm.sbb = size_t(k * nn), gm.sbk = size_t(nn), gm.sbn = 1;
                gm.scb = size_t(m * nn), gm.scm = size_t(nn), gm.scn = 1;
                nd_bgemm(gm, st);
            } else if (o == "Transpose") {
                const NdTensor a = flt(0);
                const size_t r = a.shape.size();
                if (r > size_t(ND_RANK)) fail("rank above 6");
                std::vector<int64_t> perm;
                if (auto p = n.ints("perm")) perm = *p;
                else for (size_t d = r; d-- > 0;) perm.push_back(int64_t(d));
                if (perm.size() != r) fail("Transpose perm");
                std::vector<int64_t> shape(r);
                for (size_t d = 0; d < r; d++) shape[d] = a.shape.at(size_t(perm[d]));
                out.t = alloc(shape);
                if (shapes_only) break;
                const auto is = strides_of(a.shape), os = strides_of(shape);
                NdIndex ix;
                ix.total = out.t.count();
                ix.rank = int(r);
                for (size_t d = 0; d < r; d++) {
                    ix.dims[d] = size_t(shape[d]);
                    ix.s0[d] = is[size_t(perm[d])];
                    ix.s1[d] = os[d];
                }
                nd_copy(a.p, out.t.p, ix, 0, 0, st);
            } else if (o == "Slice") {
                const auto starts = ints(1), ends = ints(2);
                NdValue data = arg(0);
                const auto shape = data.is_int ? data.ishape : data.t.shape;
                const size_t r = shape.size();
                std::vector<int64_t> axes;
                if (op.inputs.size() > 3 && !op.inputs[3].empty()) axes = ints(3);
                else for (size_t k = 0; k < starts.size(); k++) axes.push_back(int64_t(k));
                if (op.inputs.size() > 4 && !op.inputs[4].empty())
                    for (int64_t v : ints(4))
                        if (v != 1) fail("Slice with steps");
                std::vector<int64_t> lo(r, 0), oshape = shape;
                for (size_t k = 0; k < starts.size() && k < ends.size() && k < axes.size(); k++) {
                    const int ax = axis_of(axes[k], r);
                    const int64_t dim = shape[size_t(ax)];
                    auto cl = [&](int64_t v) { return std::clamp<int64_t>(v < 0 ? v + dim : v, 0, dim); };
                    const int64_t s0 = cl(starts[k]), e0 = cl(ends[k]);
                    lo[size_t(ax)] = s0;
                    oshape[size_t(ax)] = std::max<int64_t>(0, e0 - s0);
                }
                if (data.is_int) {
                    out.is_int = true;
                    out.ishape = oshape;
                    for (int64_t k = lo[0]; k < lo[0] + oshape[0] && k < int64_t(data.iv.size()); k++)
                        out.iv.push_back(data.iv[size_t(k)]);
                    break;
                }
                out.t = alloc(oshape);
                if (shapes_only) break;
                const auto is = strides_of(shape), os = strides_of(oshape);
                NdIndex ix;
                ix.total = out.t.count();
                ix.rank = int(r);
                size_t base = 0;
                for (size_t d = 0; d < r; d++) {
                    ix.dims[d] = size_t(oshape[d]);
                    ix.s0[d] = is[d];
                    ix.s1[d] = os[d];
                    base += size_t(lo[d]) * is[d];
                }
                nd_copy(data.t.p, out.t.p, ix, base, 0, st);
            } else if (o == "Concat") {
                std::vector<NdValue> parts;
                for (size_t k = 0; k < op.inputs.size(); k++) parts.push_back(arg(k));
                if (std::all_of(parts.begin(), parts.end(), [](const NdValue &v) { return v.is_int; })) {
                    out.is_int = true;
                    for (const auto &p : parts) out.iv.insert(out.iv.end(), p.iv.begin(), p.iv.end());
                    out.ishape = {int64_t(out.iv.size())};
                    break;
                }
                for (const auto &p : parts)
                    if (p.is_int) fail("Concat of mixed values");
                const size_t r = parts[0].t.shape.size();
                const int ax = axis_of(n.int_("axis").value_or(0), r);
                auto shape = parts[0].t.shape;
                shape[size_t(ax)] = 0;
                for (const auto &p : parts) {
                    if (p.t.shape.size() != r) fail("Concat ranks differ");
                    for (size_t d = 0; d < r; d++)
                        if (int(d) != ax && p.t.shape[d] != parts[0].t.shape[d]) fail("Concat shapes differ");
                    shape[size_t(ax)] += p.t.shape[size_t(ax)];
                }
                out.t = alloc(shape);
                if (shapes_only) break;
                const auto os = strides_of(shape);
                size_t off = 0;
                for (const auto &p : parts) {
                    const auto is = strides_of(p.t.shape);
                    NdIndex ix;
                    ix.total = p.t.count();
                    ix.rank = int(r);
                    for (size_t d = 0; d < r; d++) {
                        ix.dims[d] = size_t(p.t.shape[d]);
                        ix.s0[d] = is[d];
                        ix.s1[d] = os[d];
                    }
                    nd_copy(p.t.p, out.t.p, ix, 0, off * os[size_t(ax)], st);
                    off += size_t(p.t.shape[size_t(ax)]);
                }
            } else if (o == "MaxPool" || o == "AveragePool") {
                const NdTensor a = flt(0);
                if (a.shape.size() != 4) fail("pool input " + shape_str(a.shape));
                auto k = n.ints("kernel_shape");
                if (!k || k->size() != 2) fail("pool without kernel_shape");
                auto s = n.ints("strides").value_or(std::vector<int64_t>{1, 1});
                if (n.int_("ceil_mode").value_or(0) != 0) fail("pool with ceil_mode");
                if (o == "AveragePool" && n.int_("count_include_pad").value_or(0) != 0) fail("AveragePool counting padding");
                const int h = int(a.shape[2]), w = int(a.shape[3]), kh = int((*k)[0]), kw = int((*k)[1]);
                const int sh = int(s.at(0)), sw = int(s.at(1));
                int pt = 0, pl = 0, pb = 0, pr = 0;
                if (n.str("auto_pad").value_or("NOTSET") == "SAME_UPPER") {
                    const int oh = (h + sh - 1) / sh, ow = (w + sw - 1) / sw;
                    const int th = std::max(0, (oh - 1) * sh + kh - h), tw = std::max(0, (ow - 1) * sw + kw - w);
                    pt = th / 2, pl = tw / 2, pb = th - th / 2, pr = tw - tw / 2;
                } else if (auto p = n.ints("pads")) {
                    pt = int(p->at(0)), pl = int(p->at(1)), pb = int(p->at(2)), pr = int(p->at(3));
                }
                if (h + pt + pb < kh || w + pl + pr < kw) fail("pool input smaller than its kernel");
                const int oh = (h + pt + pb - kh) / sh + 1, ow = (w + pl + pr - kw) / sw + 1;
                out.t = alloc({a.shape[0], a.shape[1], oh, ow});
                if (!shapes_only)
                    nd_pool(a.p, out.t.p, size_t(a.shape[0] * a.shape[1]), h, w, oh, ow, kh, kw, sh, sw, pt, pl,
                            o == "AveragePool", st);
            } else if (o == "Resize") {
                const NdTensor a = flt(0);
                if (n.str("mode").value_or("") != "nearest" ||
                    n.str("coordinate_transformation_mode").value_or("") != "asymmetric")
                    fail("Resize other than nearest / asymmetric");
                auto wt = weights_.find(op.inputs.size() > 2 ? op.inputs[2] : "");
                if (wt == weights_.end() || wt->second.host.size() != 4) fail("Resize scales");
                const auto &sc = wt->second.host;
                if (a.shape.size() != 4 || sc[0] != 1.f || sc[1] != 1.f) fail("Resize scales on batch or channels");
                const int h = int(a.shape[2]), w = int(a.shape[3]);
                const int oh = int(std::floor(float(h) * sc[2])), ow = int(std::floor(float(w) * sc[3]));
                out.t = alloc({a.shape[0], a.shape[1], oh, ow});
                if (!shapes_only)
                    nd_resize_nearest(a.p, out.t.p, size_t(a.shape[0] * a.shape[1]), h, w, oh, ow, sc[2], sc[3], st);
            } else if (o == "Reshape") {
                const NdTensor a = flt(0);
                const auto want = ints(1);
                const size_t total = a.count();
                std::vector<int64_t> shape;
                for (size_t d = 0; d < want.size(); d++)
                    shape.push_back(want[d] == 0 ? (d < a.shape.size() ? a.shape[d] : 1) : std::max<int64_t>(want[d], 1));
                auto neg = std::find(want.begin(), want.end(), -1);
                if (neg != want.end()) {
                    const size_t p = size_t(neg - want.begin());
                    size_t known = 1;
                    for (size_t d = 0; d < shape.size(); d++)
                        if (d != p) known *= size_t(shape[d]);
                    shape[p] = int64_t(total / std::max<size_t>(known, 1));
                }
                size_t got = 1;
                for (int64_t d : shape) got *= size_t(d);
                if (got != total) fail("Reshape " + shape_str(a.shape) + " to " + shape_str(want));
                out.t = a;
                out.t.shape = shape;
            } else if (o == "Squeeze" || o == "Unsqueeze") {
                std::vector<int64_t> axes;
                if (auto ax = n.ints("axes")) axes = *ax;
                else axes = ints(1);
                NdValue a = arg(0);
                if (a.is_int) {
                    out = a;
                    if (o == "Squeeze") {
                        std::vector<int64_t> s;
                        for (int64_t d : a.ishape)
                            if (d != 1) s.push_back(d);
                        out.ishape = s;
                    } else {
                        out.ishape = {int64_t(a.iv.size())};
                    }
                    break;
                }
                std::vector<int64_t> shape;
                if (o == "Squeeze") {
                    std::vector<int> ax;
                    for (int64_t v : axes) ax.push_back(axis_of(v, a.t.shape.size()));
                    for (size_t d = 0; d < a.t.shape.size(); d++)
                        if (std::find(ax.begin(), ax.end(), int(d)) == ax.end()) shape.push_back(a.t.shape[d]);
                } else {
                    const size_t r = a.t.shape.size() + axes.size();
                    std::vector<int> ax;
                    for (int64_t v : axes) ax.push_back(axis_of(v, r));
                    size_t k = 0;
                    for (size_t d = 0; d < r; d++)
                        shape.push_back(std::find(ax.begin(), ax.end(), int(d)) != ax.end() ? 1 : a.t.shape.at(k++));
                }
                out.t = a.t;
                out.t.shape = shape;
            } else if (o == "Shape") {
                NdValue a = arg(0);
                out.is_int = true;
                out.iv = a.is_int ? a.ishape : a.t.shape;
                out.ishape = {int64_t(out.iv.size())};
            } else if (o == "Gather") {
                const auto data = ints(0), idx = ints(1);
                if (n.int_("axis").value_or(0) != 0) fail("Gather on an axis other than 0");
                out.is_int = true;
                for (int64_t k : idx) {
                    const int64_t kk = k < 0 ? k + int64_t(data.size()) : k;
                    out.iv.push_back(kk >= 0 && kk < int64_t(data.size()) ? data[size_t(kk)] : 0);
                }
                out.ishape = {int64_t(out.iv.size())};
            } else if (o == "Cast") {
                out = arg(0);
            } else {
                fail("unsupported op " + o);
            }
            break;
        }
        }
        vals[op.output] = std::move(out);
        // Values whose last reader was this op go back to the pool (stream order keeps reuse safe).
        for (const auto &nm : op.inputs) {
            auto lu = last_use_.find(nm);
            if (lu != last_use_.end() && lu->second == oi && nm != output && nm != input) vals.erase(nm);
        }
        for (const std::string *nm : {&op.residual, &op.in_scale}) {
            if (nm->empty()) continue;
            auto lu = last_use_.find(*nm);
            if (lu != last_use_.end() && lu->second == oi && *nm != output) vals.erase(*nm);
        }
    }
    if (vals_out) {
        *vals_out = std::move(vals);
        return NdTensor{};
    }
    auto it = vals.find(output);
    if (it == vals.end() || it->second.is_int) fail("output " + output + " not computed");
    return it->second.t;
}

NdTensor NdGraph::run(Ctx &ctx, const NdTensor &x) const { return run_ops(&ctx, x, ops.size(), nullptr); }

std::vector<int64_t> NdGraph::output_shape(const std::vector<int64_t> &in) const {
    NdTensor x;
    x.shape = in;
    return run_ops(nullptr, x, ops.size(), nullptr).shape;
}

void NdGraph::run_argmax(Ctx &ctx, const NdTensor &x, uint32_t *d_best, std::vector<int64_t> *out_shape) const {
    const hipStream_t st = ctx.stream();
    if (!ops.empty() && ops.back().kind == NdKind::Linear && ops.back().act == ACT_NONE && ops.back().output == output) {
        // The head's logits are never written: per-block (max, index) pairs, then one reduction.
        std::map<std::string, NdValue> vals;
        run_ops(&ctx, x, ops.size() - 1, &vals);
        const NdOp &op = ops.back();
        auto it = vals.find(op.inputs.at(0));
        if (it == vals.end() || it->second.is_int) fail("head input not computed");
        const NdTensor &a = it->second.t;
        if (a.shape.empty() || a.shape.back() != op.k) fail("head input " + shape_str(a.shape));
        const size_t m = a.count() / size_t(op.k);
        if (out_shape) {
            *out_shape = a.shape;
            out_shape->back() = op.n;
        }
        if (m == 0) return;
        if (m > 0x7fffffff) fail("head: too many rows");
        DBuf part(&ctx, m * size_t(op.pk.nblocks) * 2 * sizeof(float));
        ConvArgs ca;
        ca.x = Act{a.p, 1, 1, int(m), op.k, op.k};
        ca.y = Act{nullptr, 1, 1, int(m), op.n, op.n};
        ca.wt_hi = op.whi;
        ca.wt_lo = op.wlo;
        ca.bias = op.b;
        ca.pk = op.pk;
        ca.amax_part = part.as<float>();
        conv_mfma(ca, st);
        nd_argmax_partials(part.as<float>(), op.pk.nblocks, m, d_best, st);
        return;
    }
    NdTensor y = run(ctx, x);
    if (out_shape) *out_shape = y.shape;
    if (y.shape.empty()) fail("arg-max of a scalar");
    const size_t len = size_t(y.shape.back());
    nd_argmax(y.p, d_best, y.count() / std::max<size_t>(len, 1), int(len), st);
}

}  // namespace ocr
