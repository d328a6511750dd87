// Graph::build follows the reference's operator contract (src/gpu.rs:1101-1240): Conv (dense,
// depthwise, one-input-channel direct with a fused MaxPool), ConvTranspose, MaxPool (kernel =
// stride, no pad, no ceil), Slice (constant, step 1), Concat (channels), all-zero Pad, Relu and
// Sigmoid (fused into the Conv / ConvTranspose before them when they are its only reader).
// Graph::run differs in how it runs, not in what it computes: shapes are inferred first, every
// Concat's inputs are written by their producers straight into the Concat's channel range (no
// copy), and each buffer goes back to the stream-ordered pool after its last reader.
#include "graph.h"

#include <algorithm>
#include <cstdlib>
#include <map>
#include <memory>
#include <set>

namespace ocr {

namespace {

int act_of(const std::string &op) {
    if (op == "Relu") return ACT_RELU;
    if (op == "Sigmoid") return ACT_SIGMOID;
    return -1;
}

// One value for a symmetric 2-D attribute ([a, a] or [a, a, a, a]); `def` when absent (gpu.rs:1091-1099).
int symmetric(const Node &n, const char *name, int def) {
    auto v = n.ints(name);
    if (!v || v->empty()) return def;
    for (int64_t x : *v)
        if (x != (*v)[0]) fail(n.op + ": asymmetric " + name);
    if ((*v)[0] < 0) fail(n.op + ": negative " + name);
    return int((*v)[0]);
}

bool env_set(const char *name) { return std::getenv(name) != nullptr; }

}  // namespace

Graph Graph::build(Ctx &ctx, const Onnx &onnx, const char *stop, Node *stop_node, bool *found_stop) {
    Graph g;
    g.input = onnx.input;
    if (found_stop) *found_stop = false;
    const auto &nodes = onnx.nodes;
    const Node *stopn = nullptr;
    for (size_t i = 0; i < nodes.size(); i++) {
        const Node &n = nodes[i];
        if (stop && n.op == stop) {
            stopn = &n;
            break;
        }
        Step s;
        s.output = n.outputs.at(0);
        // An activation right after, reading only this output, is fused into it (gpu.rs:1116-1127).
        int fused = ACT_NONE;
        if ((n.op == "Conv" || n.op == "ConvTranspose") && i + 1 < nodes.size() && act_of(nodes[i + 1].op) >= 0 &&
            nodes[i + 1].inputs.at(0) == s.output && onnx.readers(s.output) == 1) {
            fused = act_of(nodes[i + 1].op);
            s.output = nodes[i + 1].outputs.at(0);
            i++;
        }
        auto bias = [&](size_t idx, int count) -> const float * {
            if (idx < n.inputs.size() && !n.inputs[idx].empty()) {
                const Weight &b = onnx.weight(n.inputs[idx]);
                if (int(b.data.size()) != count) fail(n.op + ": bias size");
                return ctx.upload_weights(b.data.data(), b.data.size());
            }
            std::vector<float> z(size_t(count), 0.f);
            return ctx.upload_weights(z.data(), z.size());
        };
        if (n.op == "Conv") {
            const Weight &w = onnx.weight(n.inputs.at(1));
            if (w.dims.size() != 4) fail("conv weight not 4D");
            const int cout = int(w.dims[0]), cin_g = int(w.dims[1]), kh = int(w.dims[2]), kw = int(w.dims[3]);
            const int group = int(n.int_("group").value_or(1));
            if (symmetric(n, "dilations", 1) != 1) fail("dilated conv");
            auto ap = n.str("auto_pad");
            if (ap && *ap != "NOTSET") fail("Conv auto_pad " + *ap + " unsupported");
            std::vector<int64_t> pads = n.ints("pads").value_or(std::vector<int64_t>{});
            if (pads.empty()) pads = {0, 0, 0, 0};
            if (pads.size() != 4) fail("Conv pads");
            auto st = n.ints("strides").value_or(std::vector<int64_t>{1, 1});
            if (st.size() != 2) fail("Conv strides");
            s.cout = cout;
            s.kh = kh;
            s.kw = kw;
            s.pt = int(pads[0]);
            s.pl = int(pads[1]);
            s.pb = int(pads[2]);
            s.pr = int(pads[3]);
            s.sh = int(st[0]);
            s.sw = int(st[1]);
            s.group = group;
            s.act = fused;
            s.b = bias(2, cout);
            const bool square = s.pt == s.pb && s.pl == s.pr && s.pt == s.pl;
            if (group == 1 && cin_g == 1 && s.sh == 1 && s.sw == 1 && square && !env_set("NODIRECT")) {
                // A MaxPool right after, reading only this output, is fused in (gpu.rs:1144-1160).
                s.kind = OpKind::Direct;
                s.cin = 1;
                if (i + 1 < nodes.size()) {
                    const Node &nx = nodes[i + 1];
                    auto k = nx.ints("kernel_shape");
                    auto ks = nx.ints("strides");
                    const int rd = onnx.readers(s.output);
                    if (nx.op == "MaxPool" && nx.inputs.at(0) == s.output && (rd == 1 || rd == 2) && k &&
                        k->size() == 2 && (!ks || *ks == *k) && symmetric(nx, "pads", 0) == 0 &&
                        nx.int_("ceil_mode").value_or(0) == 0 && (rd == 1 || ((*k)[0] == 2 && (*k)[1] == 2)) &&
                        s.output != onnx.output) {
                        s.ph = int((*k)[0]);
                        s.pw = int((*k)[1]);
                        // The only reader: the pooled value replaces the output. Two readers (a 2 x 2
                        // pool): both are written, the pooled one as pool_output.
                        if (rd == 1) s.output = nx.outputs.at(0);
                        else s.pool_output = nx.outputs.at(0);
                        i++;
                    }
                }
                s.w = ctx.upload_weights(w.data.data(), w.data.size());
                bool exact = kh == 3 && kw == 3 && cout % 16 == 0 && cout <= 64;
                for (size_t k = 0; exact && k < w.data.size(); k++)
                    exact = float(_Float16(w.data[k])) == w.data[k];
                if (exact) {
                    std::vector<uint16_t> frag(size_t(cout) / 16 * 64 * 8);
                    pack_conv1_frags(w.data.data(), cout, frag.data());
                    s.w1frag = ctx.upload_weights(frag.data(), frag.size());
                }
            } else if (group == 1) {
                s.kind = OpKind::Conv;
                s.cin = cin_g;
                s.mfma = conv_mfma_supported(kh, kw, s.sh, s.sw);
                // A MaxPool right after (kernel = stride, no padding) runs in the conv's epilogue:
                // alone when it is the conv's only reader, next to the full output otherwise.
                if (s.mfma && kh == 3 && kw == 3 && i + 1 < nodes.size() && !env_set("NOPOOLFUSE")) {
                    const Node &nx = nodes[i + 1];
                    auto k = nx.ints("kernel_shape");
                    auto ks = nx.ints("strides");
                    const int rd = onnx.readers(s.output);
                    if (nx.op == "MaxPool" && nx.inputs.at(0) == s.output && k && k->size() == 2 && (!ks || *ks == *k) &&
                        symmetric(nx, "pads", 0) == 0 && nx.int_("ceil_mode").value_or(0) == 0 && (*k)[0] >= 1 &&
                        (*k)[0] <= 8 && (*k)[1] >= 1 && (*k)[1] <= 16 && s.output != onnx.output && (rd == 1 || rd == 2)) {
                        s.ph = int((*k)[0]);
                        s.pw = int((*k)[1]);
                        if (rd == 1) {
                            s.pool_only = true;
                            s.output = nx.outputs.at(0);
                        } else {
                            s.pool_output = nx.outputs.at(0);
                        }
                        i++;
                    }
                }
                if (s.mfma) {
                    s.pk = plan_conv_pack(cin_g, cout, kh, kw);
                    std::vector<uint16_t> hi(s.pk.halves()), lo(s.pk.halves());
                    bool exact = true;
                    pack_conv_weights(s.pk, w.data.data(), hi.data(), lo.data(), &exact);
                    s.pk.exact = exact;
                    s.whi = ctx.upload_weights(hi.data(), hi.size());
                    if (!exact) s.wlo = ctx.upload_weights(lo.data(), lo.size());
                    std::vector<uint16_t> frag(s.pk.frag_halves());
                    pack_conv_frags(s.pk, hi.data(), lo.data(), frag.data());
                    s.wfrag = ctx.upload_weights(frag.data(), frag.size());
                    // A 1 x 1 conv to a few channels (a head) also keeps float32 weights for the
                    // bandwidth-bound kernel.
                    if (kh == 1 && kw == 1 && cout <= 4 && cin_g % 4 == 0 && s.pt == 0 && s.pl == 0 && s.pb == 0 &&
                        s.pr == 0 && s.sh == 1 && s.sw == 1)
                        s.w = ctx.upload_weights(w.data.data(), w.data.size());
                } else {
                    s.w = ctx.upload_weights(w.data.data(), w.data.size());
                }
            } else if (cin_g == 1 && group == cout) {
                s.kind = OpKind::Conv;  // depthwise: the generic kernel with groups
                s.cin = cout;
                s.w = ctx.upload_weights(w.data.data(), w.data.size());
            } else {
                fail("grouped conv with group " + std::to_string(group));
            }
        } else if (n.op == "ConvTranspose") {
            const Weight &w = onnx.weight(n.inputs.at(1));
            if (w.dims.size() != 4) fail("convT weight not 4D");
            if (n.int_("group").value_or(1) != 1 || symmetric(n, "pads", 0) != 0 ||
                symmetric(n, "output_padding", 0) != 0)
                fail("unsupported ConvTranspose attributes");
            s.kind = OpKind::ConvT;
            s.cin = int(w.dims[0]);
            s.cout = int(w.dims[1]);
            s.kh = int(w.dims[2]);
            s.kw = int(w.dims[3]);
            s.sh = s.sw = symmetric(n, "strides", 1);
            s.act = fused;
            s.b = bias(2, s.cout);
            // [cin][cout][kh][kw] -> [ky][kx][cin][cout]
            std::vector<float> t(w.data.size());
            for (int ci = 0; ci < s.cin; ci++)
                for (int co = 0; co < s.cout; co++)
                    for (int ky = 0; ky < s.kh; ky++)
                        for (int kx = 0; kx < s.kw; kx++)
                            t[((size_t(ky) * s.kw + kx) * s.cin + ci) * s.cout + co] =
                                w.data[((size_t(ci) * s.cout + co) * s.kh + ky) * s.kw + kx];
            s.w = ctx.upload_weights(t.data(), t.size());
            // Sub-pixel phases for the matrix cores: y[s*i + py][s*j + px] sums the taps
            // ky = py + s*m, kx = px + s*q of x[i - m][j - q]; as a conv with leading pads
            // (ty - 1, tx - 1), tap (a, b) reads x[i - ty + 1 + a][j - tx + 1 + b], i.e. m = ty-1-a.
            const int st2 = s.sh;
            bool ok = st2 >= 1 && s.kh >= st2 && s.kw >= st2 && !env_set("NOCONVTMFMA");
            for (int py = 0; ok && py < st2; py++)
                for (int px = 0; ok && px < st2; px++) {
                    Step::TPhase ph;
                    ph.py = py, ph.px = px;
                    ph.ty = (s.kh - py + st2 - 1) / st2, ph.tx = (s.kw - px + st2 - 1) / st2;
                    if (ph.ty < 1 || ph.tx < 1 || ph.ty > 3 || ph.tx > 3) {
                        ok = false;
                        break;
                    }
                    std::vector<float> cw(size_t(s.cout) * s.cin * ph.ty * ph.tx);
                    for (int co = 0; co < s.cout; co++)
                        for (int ci = 0; ci < s.cin; ci++)
                            for (int a2 = 0; a2 < ph.ty; a2++)
                                for (int b2 = 0; b2 < ph.tx; b2++) {
                                    const int ky = py + st2 * (ph.ty - 1 - a2), kx = px + st2 * (ph.tx - 1 - b2);
                                    cw[((size_t(co) * s.cin + ci) * ph.ty + a2) * ph.tx + b2] =
                                        w.data[((size_t(ci) * s.cout + co) * s.kh + ky) * s.kw + kx];
                                }
                    ph.pk = plan_conv_pack(s.cin, s.cout, ph.ty, ph.tx);
                    std::vector<uint16_t> hi(ph.pk.halves()), lo(ph.pk.halves());
                    bool exact = true;
                    pack_conv_weights(ph.pk, cw.data(), hi.data(), lo.data(), &exact);
                    ph.pk.exact = exact;
                    ph.whi = ctx.upload_weights(hi.data(), hi.size());
                    if (!exact) ph.wlo = ctx.upload_weights(lo.data(), lo.size());
                    std::vector<uint16_t> frag(ph.pk.frag_halves());
                    pack_conv_frags(ph.pk, hi.data(), lo.data(), frag.data());
                    ph.wfrag = ctx.upload_weights(frag.data(), frag.size());
                    s.phases.push_back(std::move(ph));
                }
            if (!ok) s.phases.clear();
            const int aty = (s.kh + st2 - 1) / st2, atx = (s.kw + st2 - 1) / st2;
            if (ok && s.cout % 16 == 0 && aty <= 3 && atx <= 3) {
                // All phases as one conv over the input: output channel k * cout + co is phase
                // k = py * s + px; tap (a, b) of the aty x atx kernel (leading pads aty - 1,
                // atx - 1) reads x[i - (aty - 1 - a)][j - (atx - 1 - b)], i.e. the weight of
                // ky = py + s (aty - 1 - a), kx = px + s (atx - 1 - b) (zero past the kernel).
                const int nph = st2 * st2;
                std::vector<float> cw(size_t(nph) * s.cout * s.cin * aty * atx, 0.f);
                for (int k = 0; k < nph; k++)
                    for (int co = 0; co < s.cout; co++)
                        for (int ci = 0; ci < s.cin; ci++)
                            for (int a2 = 0; a2 < aty; a2++)
                                for (int b2 = 0; b2 < atx; b2++) {
                                    const int ky = k / st2 + st2 * (aty - 1 - a2), kx = k % st2 + st2 * (atx - 1 - b2);
                                    if (ky < s.kh && kx < s.kw)
                                        cw[(((size_t(k) * s.cout + co) * s.cin + ci) * aty + a2) * atx + b2] =
                                            w.data[((size_t(ci) * s.cout + co) * s.kh + ky) * s.kw + kx];
                                }
                Step::TPhase &ap = s.allph;
                ap.ty = aty, ap.tx = atx;
                ap.pk = plan_conv_pack(s.cin, nph * s.cout, aty, atx);
                std::vector<uint16_t> hi(ap.pk.halves()), lo(ap.pk.halves());
                bool exact = true;
                pack_conv_weights(ap.pk, cw.data(), hi.data(), lo.data(), &exact);
                ap.pk.exact = exact;
                ap.whi = ctx.upload_weights(hi.data(), hi.size());
                if (!exact) ap.wlo = ctx.upload_weights(lo.data(), lo.size());
                std::vector<uint16_t> frag(ap.pk.frag_halves());
                pack_conv_frags(ap.pk, hi.data(), lo.data(), frag.data());
                ap.wfrag = ctx.upload_weights(frag.data(), frag.size());
            }
        } else if (n.op == "MaxPool") {
            auto k = n.ints("kernel_shape");
            if (!k || k->size() != 2) fail("MaxPool without kernel_shape");
            auto st = n.ints("strides").value_or(*k);
            if (st != *k || symmetric(n, "pads", 0) != 0 || n.int_("ceil_mode").value_or(0) != 0)
                fail("unsupported MaxPool attributes");
            s.kind = OpKind::MaxPool;
            s.ph = int((*k)[0]);
            s.pw = int((*k)[1]);
        } else if (n.op == "Slice") {
            auto get = [&](size_t idx) -> const std::vector<int64_t> * {
                if (idx >= n.inputs.size() || n.inputs[idx].empty()) return nullptr;
                auto it = onnx.ints.find(n.inputs[idx]);
                return it == onnx.ints.end() ? nullptr : &it->second;
            };
            if (auto steps = get(4))
                for (int64_t v : *steps)
                    if (v != 1) fail("Slice with steps");
            if (!get(1)) fail("Slice starts not constant");
            if (!get(2)) fail("Slice ends not constant");
            s.kind = OpKind::Slice;
            s.starts = *get(1);
            s.ends = *get(2);
            if (get(3)) s.axes = *get(3);
            else for (size_t a = 0; a < s.starts.size(); a++) s.axes.push_back(int64_t(a));
        } else if (n.op == "Concat") {
            if (n.int_("axis") != std::optional<int64_t>(1)) fail("Concat not on channels");
            s.kind = OpKind::Concat;
        } else if (n.op == "Pad") {
            std::vector<int64_t> pads;
            if (n.inputs.size() > 1) {
                auto it = onnx.ints.find(n.inputs[1]);
                if (it != onnx.ints.end()) pads = it->second;
                else if (onnx.weights.count(n.inputs[1]))
                    for (float v : onnx.weights.at(n.inputs[1]).data) pads.push_back(int64_t(v));
            }
            for (int64_t v : pads)
                if (v != 0) fail("non-zero Pad");
            s.kind = OpKind::Identity;
        } else if (act_of(n.op) >= 0) {
            s.kind = OpKind::Act;
            s.act = act_of(n.op);
        } else {
            fail("unsupported op " + n.op);
        }
        if (s.kind == OpKind::Concat) s.inputs = n.inputs;
        else s.inputs = {n.inputs.at(0)};
        g.steps.push_back(std::move(s));
    }
    if (stopn) {
        if (stop_node) *stop_node = *stopn;
        if (found_stop) *found_stop = true;
        g.output = stopn->inputs.at(0);
    } else {
        g.output = onnx.output;
    }
    return g;
}

std::vector<Shape> Graph::shapes(const Shape &in) const {
    std::map<std::string, Shape> sh;
    sh[input] = in;
    std::vector<Shape> out;
    out.reserve(steps.size());
    for (const Step &s : steps) {
        auto it = sh.find(s.inputs[0]);
        if (it == sh.end()) fail("missing value " + s.inputs[0]);
        const auto [n, h, w, c] = it->second;
        Shape o = it->second;
        switch (s.kind) {
        case OpKind::Conv:
            if (c != s.cin)
                fail("Conv input has " + std::to_string(c) + " channels, weights take " + std::to_string(s.cin));
            o = {n, (h + s.pt + s.pb - s.kh) / s.sh + 1, (w + s.pl + s.pr - s.kw) / s.sw + 1, s.cout};
            if (h + s.pt + s.pb < s.kh || w + s.pl + s.pr < s.kw) fail("Conv input smaller than its kernel");
            if (s.pool_only || !s.pool_output.empty()) {
                const Shape pooled{o[0], o[1] / s.ph, o[2] / s.pw, o[3]};
                if (pooled[1] < 1 || pooled[2] < 1) fail("empty output shape");
                if (s.pool_only) o = pooled;
                else sh[s.pool_output] = pooled;
            }
            break;
        case OpKind::Direct: {
            if (c != 1) fail("direct conv takes one channel");
            const int ch = h + 2 * s.pt - s.kh + 1, cw = w + 2 * s.pt - s.kw + 1;
            if (ch < 1 || cw < 1) fail("Conv input smaller than its kernel");
            if (s.pool_output.empty()) {
                o = {n, ch / s.ph, cw / s.pw, s.cout};
            } else {
                o = {n, ch, cw, s.cout};
                if (ch / s.ph < 1 || cw / s.pw < 1) fail("empty output shape");
                sh[s.pool_output] = Shape{n, ch / s.ph, cw / s.pw, s.cout};
            }
            break;
        }
        case OpKind::ConvT:
            if (c != s.cin) fail("ConvTranspose input channels");
            o = {n, (h - 1) * s.sh + s.kh, (w - 1) * s.sw + s.kw, s.cout};
            break;
        case OpKind::MaxPool: o = {n, h / s.ph, w / s.pw, c}; break;
        case OpKind::Slice: {
            // Starts / ends clamped ONNX-style on NCHW axes (gpu.rs:1299-1309).
            int nchw[4] = {n, c, h, w}, lo[4] = {0, 0, 0, 0};
            int dims[4] = {n, c, h, w};
            for (size_t k = 0; k < s.starts.size() && k < s.ends.size() && k < s.axes.size(); k++) {
                int64_t ax = s.axes[k] < 0 ? s.axes[k] + 4 : s.axes[k];
                if (ax < 0 || ax > 3) fail("Slice axis");
                int64_t dim = nchw[ax];
                auto clampv = [&](int64_t v) { return std::clamp<int64_t>(v < 0 ? v + dim : v, 0, dim); };
                int64_t s0 = clampv(s.starts[k]), e0 = clampv(s.ends[k]);
                lo[ax] = int(s0);
                dims[ax] = int(std::max<int64_t>(0, e0 - s0));
            }
            if (lo[0] != 0 || lo[1] != 0 || dims[0] != n || dims[1] != c) fail("Slice on batch or channels");
            o = {n, dims[2], dims[3], c};
            break;
        }
        case OpKind::Concat: {
            int ctot = 0;
            for (const std::string &nm : s.inputs) {
                auto jt = sh.find(nm);
                if (jt == sh.end()) fail("missing value " + nm);
                if (jt->second[0] != n || jt->second[1] != h || jt->second[2] != w) fail("Concat shapes differ");
                ctot += jt->second[3];
            }
            o = {n, h, w, ctot};
            break;
        }
        case OpKind::Act:
        case OpKind::Identity: break;
        }
        if (o[1] < 1 || o[2] < 1) fail("empty output shape");
        sh[s.output] = o;
        out.push_back(o);
    }
    return out;
}

Shape Graph::infer(const Shape &in) const {
    auto sh = shapes(in);
    for (size_t i = steps.size(); i-- > 0;)
        if (steps[i].output == output) return sh[i];
    if (output == input) return in;
    fail("graph output " + output + " not computed");
}

// One input's walk through the steps: shapes, liveness, views and buffers.
struct Graph::Exec {
    const Graph &g;
    Ctx &ctx;
    hipStream_t st;
    Act x;
    std::vector<Shape> shp;
    std::map<std::string, size_t> last;                  // last reader of every value
    std::map<std::string, std::pair<size_t, int>> into;  // value -> (concat step, channel offset)
    std::map<std::string, Act> view;
    std::map<std::string, DBuf> owned;  // buffers by the value that owns them

    Exec(const Graph &graph, Ctx &c, const Act &in) : g(graph), ctx(c), st(c.stream()), x(in) {
        shp = g.shapes({x.n, x.h, x.w, x.c});
        std::set<std::string> produced;
        for (size_t i = 0; i < g.steps.size(); i++) {
            for (const std::string &nm : g.steps[i].inputs) last[nm] = i;
            if (g.steps[i].kind != OpKind::Identity) produced.insert(g.steps[i].output);
            if (!g.steps[i].pool_output.empty()) produced.insert(g.steps[i].pool_output);
        }
        for (size_t i = 0; i < g.steps.size(); i++) {
            const Step &s = g.steps[i];
            if (s.kind != OpKind::Concat) continue;
            int off = 0;
            for (const std::string &nm : s.inputs) {
                const int c2 = [&] {
                    for (size_t j = 0; j < i; j++)
                        if (g.steps[j].output == nm || g.steps[j].pool_output == nm) return shp[j][3];
                    return x.c;
                }();
                if (produced.count(nm) && !into.count(nm) && nm != g.output && nm != g.input) into[nm] = {i, off};
                off += c2;
            }
        }
        // A value written into a Concat's buffer keeps that buffer alive until its own last reader.
        for (const auto &kv : into) {
            auto lv = last.find(kv.first);
            if (lv == last.end()) continue;
            size_t &lc = last[g.steps[kv.second.first].output];
            lc = std::max(lc, lv->second);
        }
        view[g.input] = x;
    }
    Act alloc(const std::string &name, const Shape &sh) {
        Act a{nullptr, sh[0], sh[1], sh[2], sh[3], sh[3]};
        DBuf b(&ctx, a.count() * sizeof(float));
        a.p = b.as<float>();
        owned[name] = std::move(b);
        return a;
    }
    // Where a value of shape sh is written: its own buffer, or its channel range of a Concat's.
    Act view_for(const std::string &name, const Shape &sh) {
        auto it = into.find(name);
        if (it == into.end()) return alloc(name, sh);
        const size_t ci = it->second.first;
        const std::string &cname = g.steps[ci].output;
        if (!view.count(cname)) view[cname] = alloc(cname, shp[ci]);
        Act whole = view[cname];
        Act a{whole.p + it->second.second, sh[0], sh[1], sh[2], sh[3], whole.cs};
        return a;
    }
    Act out_view(size_t i) { return view_for(g.steps[i].output, shp[i]); }
    // Buffers whose last reader was step i go back to the pool (stream order keeps the reuse
    // safe). A value inside a Concat's buffer is freed with that buffer, whose last use was
    // extended above to cover it.
    void release(size_t i) {
        for (const auto &kv : last) {
            if (kv.second != i || kv.first == g.output || into.count(kv.first)) continue;
            owned.erase(kv.first);
        }
    }
    void done(size_t i, const Act &y) {
        view[g.steps[i].output] = y;
        release(i);
    }
    // Step i is a dense conv on the matrix cores (not the narrow 1 x 1 one).
    bool mfma_conv(size_t i) const {
        const Step &s = g.steps[i];
        if (s.kind != OpKind::Conv || !s.mfma) return false;
        const Act &a = view.at(s.inputs[0]);
        return !(s.w && !s.pool_only && s.pool_output.empty() && a.cs % 4 == 0 &&
                 (reinterpret_cast<uintptr_t>(a.p) & 15) == 0);
    }
    // The arguments of such a step (its outputs get their views); y: the step's value.
    ConvArgs conv_args(size_t i, Act &y) {
        const Step &s = g.steps[i];
        const Act a = view.at(s.inputs[0]);
        y = out_view(i);
        ConvArgs ca;
        ca.x = a;
        ca.y = y;
        if (s.pool_only) {
            // y is the pooled value; the full-size output is never written.
            ca.ypool = y;
            ca.y = Act{nullptr, y.n, (a.h + s.pt + s.pb - s.kh) + 1, (a.w + s.pl + s.pr - s.kw) + 1, y.c, y.c};
            ca.keep_full = false;
        } else if (!s.pool_output.empty()) {
            ca.ypool = view_for(s.pool_output, {y.n, y.h / s.ph, y.w / s.pw, y.c});
            view[s.pool_output] = ca.ypool;
        }
        ca.ph = s.ph;
        ca.pw = s.pw;
        ca.wt_hi = s.whi;
        ca.wt_lo = s.wlo;
        ca.wt_frag = s.wfrag;
        ca.bias = s.b;
        ca.pt = s.pt;
        ca.pl = s.pl;
        ca.act = s.act;
        ca.pk = s.pk;
        return ca;
    }
    // Step i is a one-channel conv the matrix-core kernel takes (3 x 3, pad 1, packed weights).
    bool direct_mfma(size_t i) const {
        const Step &s = g.steps[i];
        return s.kind == OpKind::Direct && s.w1frag && s.kh == 3 && s.kw == 3 && s.pt == 1;
    }
    // The output views of a one-channel conv: y, and with a fused pool its pooled output yp.
    void direct_views(size_t i, Act &y, Act &yp) {
        const Step &s = g.steps[i];
        y = out_view(i);
        yp = Act{};
        if (!s.pool_output.empty()) {
            yp = view_for(s.pool_output, {y.n, y.h / s.ph, y.w / s.pw, y.c});
            view[s.pool_output] = yp;
        }
    }
    // The same step without the matrix-core kernel: the conv and then the pool.
    void direct_fallback(size_t i, const Act &a, const Act &y, const Act &yp) {
        const Step &s = g.steps[i];
        if (s.pool_output.empty()) {
            conv_direct(a, y, s.w, s.b, s.kh, s.kw, s.pt, s.act, s.ph, s.pw, st, s.w1frag);
        } else {
            conv_direct(a, y, s.w, s.b, s.kh, s.kw, s.pt, s.act, 1, 1, st, s.w1frag);
            maxpool(y, yp, s.ph, s.pw, st);
        }
    }
    void step(size_t i);
    Out result();
};

void Graph::Exec::step(size_t i) {
    const Step &s = g.steps[i];
    const Act a = view.at(s.inputs[0]);
    Act y;
    switch (s.kind) {
    case OpKind::Conv: {
        if (mfma_conv(i)) {
            conv_mfma(conv_args(i, y), st);
        } else if (s.mfma) {
            y = out_view(i);
            conv1x1_narrow(a, y, s.w, s.b, s.act, st);
        } else {
            y = out_view(i);
            conv_generic(a, y, s.w, s.b, s.kh, s.kw, s.sh, s.sw, s.pt, s.pl, s.group, s.act, st);
        }
        break;
    }
    case OpKind::Direct: {
        Act yp;
        direct_views(i, y, yp);
        if (s.pool_output.empty()) {
            conv_direct(a, y, s.w, s.b, s.kh, s.kw, s.pt, s.act, s.ph, s.pw, st, s.w1frag);
        } else if (!(direct_mfma(i) && conv1_mfma(a, y, s.w1frag, s.b, s.act, s.ph, s.pw, st, &yp))) {
            direct_fallback(i, a, y, yp);
        }
        break;
    }
    case OpKind::ConvT:
        y = out_view(i);
        if (s.phases.empty()) {
            conv_transpose(a, y, s.w, s.b, s.kh, s.kw, s.sh, s.act, st);
            break;
        }
        // All phases as one GEMM over the output's s x s blocks whose epilogue writes the phases
        // (operands read straight into the matrix cores, no staging set-up to pay back); a
        // kernel past the stride adds taps (the detector's 2 x 3 upsampler: a 1 x 2 window).
        if (s.allph.whi && s.sh == s.sw && !env_set("NOCONVTROWS") &&
            convt_rows(a, y, s.allph.whi, s.allph.wlo, s.allph.pk, s.b, s.sh, s.act, st))
            break;
        // Kernel = stride = 2 with few channels: a float32 pass with the weights in LDS.
        if (convt_k2s2(a, y, s.w, s.b, s.kh, s.kw, s.sh, s.act, st)) break;
        if (s.allph.whi) {
            // All phases as one GEMM over the input pixels.
            ConvArgs ca;
            ca.x = a;
            ca.y = y;
            ca.wt_hi = s.allph.whi;
            ca.wt_lo = s.allph.wlo;
            ca.wt_frag = s.allph.wfrag;
            ca.bias = s.b;
            ca.act = s.act;
            ca.pk = s.allph.pk;
            ca.pt = s.allph.ty - 1;
            ca.pl = s.allph.tx - 1;
            ca.ph_cout = s.cout;
            ca.ph_s = s.sh;
            if (conv_igemm(ca, st)) break;
        }
        for (const Step::TPhase &ph : s.phases) {
            const int st2 = s.sh;
            const int ohp = (y.h - ph.py + st2 - 1) / st2, owp = (y.w - ph.px + st2 - 1) / st2;
            if (ohp < 1 || owp < 1) continue;
            ConvArgs ca;
            ca.x = a;
            ca.y = Act{y.p + (size_t(ph.py) * y.w + ph.px) * y.cs, y.n, ohp, owp, y.c, y.cs};
            ca.y_px = st2;
            ca.y_row = long(st2) * y.w;
            ca.y_img = long(y.h) * y.w;
            ca.wt_hi = ph.whi;
            ca.wt_lo = ph.wlo;
            ca.wt_frag = ph.wfrag;
            ca.bias = s.b;
            ca.pt = ph.ty - 1;
            ca.pl = ph.tx - 1;
            ca.act = s.act;
            ca.pk = ph.pk;
            conv_mfma(ca, st);
        }
        break;
    case OpKind::MaxPool:
        y = out_view(i);
        maxpool(a, y, s.ph, s.pw, st);
        break;
    case OpKind::Slice: {
        y = out_view(i);
        int y0 = 0, x0 = 0;
        for (size_t k = 0; k < s.starts.size() && k < s.axes.size(); k++) {
            int64_t ax = s.axes[k] < 0 ? s.axes[k] + 4 : s.axes[k];
            int64_t dim = ax == 2 ? a.h : a.w;
            int64_t v = s.starts[k] < 0 ? s.starts[k] + dim : s.starts[k];
            v = std::clamp<int64_t>(v, 0, dim);
            if (ax == 2) y0 = int(v);
            if (ax == 3) x0 = int(v);
        }
        copy_act(a, y, y0, x0, st);
        break;
    }
    case OpKind::Concat: {
        if (!view.count(s.output)) view[s.output] = alloc(s.output, shp[i]);
        y = view[s.output];
        int off = 0;
        for (const std::string &nm : s.inputs) {
            const Act part = view.at(nm);
            auto it = into.find(nm);
            if (it == into.end() || it->second.first != i) {
                Act dst{y.p + off, part.n, part.h, part.w, part.c, y.cs};
                copy_act(part, dst, 0, 0, st);
            }
            off += part.c;
        }
        break;
    }
    case OpKind::Act:
        y = out_view(i);
        activate(a, y, s.act, st);
        break;
    case OpKind::Identity: y = a; break;
    }
    done(i, y);
}

Graph::Out Graph::Exec::result() {
    Out out;
    auto vit = view.find(g.output);
    if (vit == view.end()) fail("graph output " + g.output + " not computed");
    out.act = vit->second;
    auto oit = owned.find(g.output);
    if (oit != owned.end() && out.act.cs == out.act.c) {
        out.buf = std::move(oit->second);
    } else {
        // The output is a view (a Concat slice or the input): give the caller its own copy.
        Act dst{nullptr, out.act.n, out.act.h, out.act.w, out.act.c, out.act.c};
        out.buf = DBuf(&ctx, dst.count() * sizeof(float));
        dst.p = out.buf.as<float>();
        copy_act(out.act, dst, 0, 0, st);
        out.act = dst;
    }
    return out;
}

Graph::Out Graph::run(Ctx &ctx, const Act &x) const {
    Exec e(*this, ctx, x);
    for (size_t i = 0; i < steps.size(); i++) e.step(i);
    return e.result();
}

std::vector<Graph::Out> Graph::run_multi(Ctx &ctx, const std::vector<Act> &xs) const {
    std::vector<Out> outs;
    run_multi_tm(ctx, xs, 0, nullptr, 0, outs, {});
    return outs;
}

bool Graph::run_multi_time_major(Ctx &ctx, const std::vector<Act> &xs, int kh, float *X, int ntot,
                                 std::vector<Out> &outs, const std::function<void(int)> &after_step) const {
    if (!X || kh != 2) fail("run_multi_time_major: X and an average pool over 2 rows");
    return run_multi_tm(ctx, xs, kh, X, ntot, outs, after_step);
}

bool Graph::run_multi_tm(Ctx &ctx, const std::vector<Act> &xs, int kh, float *X, int ntot,
                         std::vector<Out> &outs, const std::function<void(int)> &after_step) const {
    std::vector<std::unique_ptr<Exec>> es;
    for (const Act &x : xs) es.emplace_back(new Exec(*this, ctx, x));
    std::vector<ConvArgs> cas;
    std::vector<Act> as, ys, yps;
    outs.clear();
    for (size_t i = 0; i < steps.size(); i++) {
        if (X && i + 1 == steps.size() && !es.empty()) {
            // The last layer: conv + ReLU + MaxPool (2, 1) of four rows, then the average pool
            // to one row, time-major, in the conv's epilogue.
            const Step &s = steps[i];
            bool all = s.pool_only && s.ph == 2 && s.pw == 1 && s.output == output;
            for (auto &e : es) all = all && e->mfma_conv(i) && e->shp[i][1] * 2 == 4;
            if (all) {
                cas.clear();
                int noff = 0;
                for (auto &e : es) {
                    const Act a = e->view.at(s.inputs[0]);
                    ConvArgs ca;
                    ca.x = a;
                    ca.y = Act{nullptr, a.n, a.h + s.pt + s.pb - s.kh + 1, a.w + s.pl + s.pr - s.kw + 1, s.cout, s.cout};
                    ca.ph = 2;
                    ca.pw = 1;
                    ca.keep_full = false;
                    ca.wt_hi = s.whi;
                    ca.wt_lo = s.wlo;
                    ca.wt_frag = s.wfrag;
                    ca.bias = s.b;
                    ca.pt = s.pt;
                    ca.pl = s.pl;
                    ca.act = s.act;
                    ca.pk = s.pk;
                    ca.tm = X;
                    ca.tm_ntot = ntot;
                    ca.tm_noff = noff;
                    noff += a.n;
                    cas.push_back(ca);
                }
                if (noff <= ntot && conv3x3_dma_multi(cas.data(), int(cas.size()), ctx.stream())) {
                    outs.resize(es.size());
                    return true;
                }
            }
        }
        bool all = !es.empty(), all1 = !es.empty();
        for (auto &e : es) all = all && e->mfma_conv(i), all1 = all1 && e->direct_mfma(i);
        if (all1 && es.size() > 1) {
            // The one-channel first layer of every input in one launch.
            const Step &s = steps[i];
            as.clear();
            ys.assign(es.size(), Act{});
            yps.assign(es.size(), Act{});
            for (size_t k = 0; k < es.size(); k++) {
                as.push_back(es[k]->view.at(s.inputs[0]));
                es[k]->direct_views(i, ys[k], yps[k]);
            }
            const bool pooled = !s.pool_output.empty();
            if (!conv1_mfma_multi(as.data(), ys.data(), pooled ? yps.data() : nullptr, int(es.size()), s.w1frag, s.b,
                                  s.act, s.ph, s.pw, ctx.stream()))
                for (size_t k = 0; k < es.size(); k++) es[k]->direct_fallback(i, as[k], ys[k], yps[k]);
            for (size_t k = 0; k < es.size(); k++) es[k]->done(i, ys[k]);
        } else if (all && es.size() > 1) {
            // One launch for every input's conv when the kernel takes them together.
            cas.clear();
            ys.assign(es.size(), Act{});
            for (size_t k = 0; k < es.size(); k++) cas.push_back(es[k]->conv_args(i, ys[k]));
            if (!conv3x3_dma_multi(cas.data(), int(cas.size()), ctx.stream()))
                for (const ConvArgs &ca : cas) conv_mfma(ca, ctx.stream());
            for (size_t k = 0; k < es.size(); k++) es[k]->done(i, ys[k]);
        } else {
            for (auto &e : es) e->step(i);
        }
        if (after_step) after_step(int(i));
    }
    for (auto &e : es) outs.push_back(e->result());
    return false;
}

}  // namespace ocr
