// NdGraph: the fusion plan of nd_plan.cpp (the operator contract of the reference's
// NdGraph::new, src/nd.rs:505-817) with each step's weights laid out for its kernel, and a run
// loop over the steps (NdGraph::run, nd.rs:834-1195). Buffers come from the context's
// stream-ordered pool and go back after their last reader.
#include "nd.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
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

// OCR_NO_NDCONV=1 keeps the N-D convs and MatMuls on the general kernels (for side-by-side
// timing of the two paths on one GPU).
bool no_ndconv() {
    static const bool off = [] {
        const char *e = std::getenv("OCR_NO_NDCONV");
        return e && *e && *e != '0';
    }();
    return off;
}

std::string shape_str(const std::vector<int64_t> &s) {
    std::string o = "[";
    for (size_t i = 0; i < s.size(); i++) o += (i ? ", " : "") + std::to_string(s[i]);
    return o + "]";
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// Build
// ---------------------------------------------------------------------------------------------
namespace {

// Scale and shift of an inference BatchNormalization node: y = s x + t per channel, with
// s = gamma / sqrt(var + eps) and t = beta - mean s. Returned as [s..., t...].
std::vector<float> batch_norm_affine(const Onnx &onnx, const Node &bn, size_t channels) {
    const float eps = bn.f32("epsilon").value_or(1e-5f);
    const Weight &gamma = onnx.weight(bn.inputs.at(1)), &beta = onnx.weight(bn.inputs.at(2)),
                 &mean = onnx.weight(bn.inputs.at(3)), &var = onnx.weight(bn.inputs.at(4));
    for (const Weight *w : {&gamma, &beta, &mean, &var})
        if (w->data.size() != channels)
            fail("BatchNormalization parameters of " + std::to_string(w->data.size()) + " values for " +
                 std::to_string(channels) + " channels");
    std::vector<float> st(2 * channels);
    for (size_t c = 0; c < channels; c++) {
        st[c] = gamma.data[c] / std::sqrt(var.data[c] + eps);
        st[channels + c] = beta.data[c] - mean.data[c] * st[c];
    }
    return st;
}

// Packs [rows][k] float weights into the matrix-core layout as float16 hi (+ lo when some value
// is not a float16 value) and uploads them.
void pack_upload(Ctx &ctx, NdOp &op, const float *w, int cin, int cout, int kh, int kw) {
    op.pk = plan_conv_pack(cin, cout, kh, kw);
    std::vector<uint16_t> hi(op.pk.halves()), lo(op.pk.halves());
    bool exact = true;
    pack_conv_weights(op.pk, w, hi.data(), lo.data(), &exact);
    op.pk.exact = exact;
    op.whi = ctx.upload_weights(hi.data(), hi.size());
    if (!exact) op.wlo = ctx.upload_weights(lo.data(), lo.size());
}

// The epilogue bias of a step: the anchor's own bias input (if any) plus every bias Add taken.
std::vector<float> step_bias(const Onnx &onnx, const NdStep &s, const Node &anchor, size_t channels) {
    std::vector<float> b(channels, 0.f);
    auto add = [&](const std::string &name, const char *what) {
        const Weight &w = onnx.weight(name);
        if (w.data.size() != channels)
            fail(std::string(what) + " of " + std::to_string(w.data.size()) + " values for " + std::to_string(channels) +
                 " output channels");
        for (size_t c = 0; c < channels; c++) b[c] += w.data[c];
    };
    if (anchor.inputs.size() > 2 && !anchor.inputs[2].empty()) add(anchor.inputs[2], (anchor.op + " bias").c_str());
    for (const auto &name : s.bias) add(name, "added bias");
    return b;
}

}  // namespace

// The plan (nd_plan.cpp) decides which nodes run together; here each step's weights are laid out
// for its kernel and uploaded once.
NdGraph NdGraph::build(Ctx &ctx, const Onnx &onnx, bool stop_before_softmax) {
    NdPlan plan = plan_nd(onnx, stop_before_softmax);
    NdGraph g;
    for (const NdStep &s : plan.steps) {
        const Node &n = plan.nodes[size_t(s.anchor)];
        NdOp op;
        op.kind = s.kind;
        op.node = s.anchor;
        op.inputs = n.inputs;
        op.output = s.output;
        op.act = s.act;
        switch (s.kind) {
        case NdKind::Generic:
            break;
        case NdKind::LayerNorm: {
            const Weight &gm = onnx.weight(s.gamma), &bt = onnx.weight(s.beta);
            if (gm.data.size() != bt.data.size()) fail("LayerNorm: " + std::to_string(gm.data.size()) + " scales and " +
                                                       std::to_string(bt.data.size()) + " shifts");
            std::vector<float> gb = gm.data;
            gb.insert(gb.end(), bt.data.begin(), bt.data.end());
            op.gb = ctx.upload_weights(gb.data(), gb.size());
            op.len = int(gm.data.size());
            op.eps = s.eps;
            op.inputs = {n.inputs.at(0)};
            break;
        }
        case NdKind::Affine: {
            const size_t c = onnx.weight(n.inputs.at(1)).data.size();
            const std::vector<float> st = batch_norm_affine(onnx, n, c);
            op.st = ctx.upload_weights(st.data(), st.size());
            op.cout = int(c);
            op.inputs = {n.inputs.at(0)};
            break;
        }
        case NdKind::Conv: {
            const Weight &w = onnx.weight(n.inputs.at(1));
            if (w.dims.size() != 4) fail("Conv weight of rank " + std::to_string(w.dims.size()) + ", not 4");
            if (auto d = n.ints("dilations"))
                for (int64_t v : *d)
                    if (v != 1) fail("Conv dilation " + std::to_string(v) + " (only 1 is supported)");
            op.cout = int(w.dims[0]);
            op.cin_g = int(w.dims[1]);
            op.kh = int(w.dims[2]);
            op.kw = int(w.dims[3]);
            op.group = int(n.int_("group").value_or(1));
            op.cin = op.cin_g * op.group;
            const auto strides = n.ints("strides").value_or(std::vector<int64_t>{1, 1});
            if (strides.size() != 2) fail("Conv strides of rank " + std::to_string(strides.size()));
            op.sh = int(strides[0]);
            op.sw = int(strides[1]);
            const std::string pad_mode = n.str("auto_pad").value_or("NOTSET");
            if (pad_mode != "NOTSET" && pad_mode != "SAME_UPPER") fail("Conv auto_pad " + pad_mode + " is not supported");
            op.same_upper = pad_mode == "SAME_UPPER";
            if (auto p = n.ints("pads")) {
                if (p->size() != 4) fail("Conv pads of length " + std::to_string(p->size()));
                for (int k = 0; k < 4; k++) op.pads[k] = int((*p)[size_t(k)]);
            }
            std::vector<float> b = step_bias(onnx, s, n, size_t(op.cout));
            if (s.batch_norm >= 0) {
                const std::vector<float> st = batch_norm_affine(onnx, plan.nodes[size_t(s.batch_norm)], size_t(op.cout));
                op.affine = ctx.upload_weights(st.data(), st.size());
            }
            op.residual = s.residual;
            op.in_scale = s.in_scale;
            if (op.group != 1 && (!op.residual.empty() || !op.in_scale.empty()))
                fail("a grouped Conv cannot take a residual or an input scale");
            op.b = ctx.upload_weights(b.data(), b.size());
            op.mfma = op.group == 1 && conv_mfma_supported(op.kh, op.kw, op.sh, op.sw);
            if (op.mfma) pack_upload(ctx, op, w.data.data(), op.cin, op.cout, op.kh, op.kw);
            else op.w = ctx.upload_weights(w.data.data(), w.data.size());
            op.inputs = {s.conv_input};
            break;
        }
        case NdKind::Attention:
            op.inputs = {s.conv_input, s.attn_shape, s.attn_out_shape};
            op.scale = s.attn_scale;
            break;
        case NdKind::Linear: {
            const Weight &w = onnx.weight(n.inputs.at(1));
            op.k = int(w.dims.at(0));
            op.n = int(w.dims.at(1));
            const std::vector<float> b = step_bias(onnx, s, n, size_t(op.n));
            // The weight [k][n] is packed as n rows of k (a 1 x 1 conv from k to n channels).
            std::vector<float> rows(size_t(op.n) * op.k);
            for (int kk = 0; kk < op.k; kk++)
                for (int c = 0; c < op.n; c++) rows[size_t(c) * op.k + kk] = w.data[size_t(kk) * op.n + c];
            pack_upload(ctx, op, rows.data(), op.k, op.n, 1, 1);
            op.b = ctx.upload_weights(b.data(), b.size());
            op.inputs = {n.inputs.at(0)};
            op.residual = s.residual;
            break;
        }
        case NdKind::ConvT: {
            const Weight &w = onnx.weight(n.inputs.at(1));
            if (w.dims.size() != 4) fail("ConvTranspose weight of rank " + std::to_string(w.dims.size()) + ", not 4");
            const auto strides = n.ints("strides").value_or(std::vector<int64_t>{1, 1});
            bool ok = n.int_("group").value_or(1) == 1 && strides.size() == 2 && strides[0] == strides[1];
            for (const char *a : {"pads", "output_padding", "dilations"})
                if (auto p = n.ints(a))
                    for (int64_t v : *p) ok &= v == (std::string(a) == "dilations" ? 1 : 0);
            if (!ok) fail("ConvTranspose: only group 1, equal strides, no padding and no dilation are supported");
            op.cin = int(w.dims[0]);
            op.cout = int(w.dims[1]);
            op.kh = int(w.dims[2]);
            op.kw = int(w.dims[3]);
            op.sh = op.sw = int(strides[0]);
            const std::vector<float> b = step_bias(onnx, s, n, size_t(op.cout));
            op.w = ctx.upload_weights(w.data.data(), w.data.size());
            op.b = ctx.upload_weights(b.data(), b.size());
            op.inputs = {n.inputs.at(0)};
            break;
        }
        }
        g.ops.push_back(std::move(op));
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
    g.nodes_ = std::move(plan.nodes);
    g.input = plan.input;
    g.output = plan.output;
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
                NdMfmaConvArgs ma;
                ma.x = a.p;
                ma.n = nb;
                ma.cin = cin;
                ma.h = h;
                ma.w = w;
                ma.y = out.t.p;
                ma.cout = op.cout;
                ma.oh = oh;
                ma.ow = ow;
                ma.wt_hi = op.whi;
                ma.wt_lo = op.wlo;
                ma.pk = op.pk;
                ma.bias = op.b;
                ma.affine = op.affine;
                ma.res = res.p;
                ma.in_scale = sc.p;
                ma.pt = pt;
                ma.pl = pl;
                ma.act = op.act;
                if (!no_ndconv() && nd_conv_nchw_mfma(ma, st)) break;
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
                if (!no_ndconv() && (nd_conv_dw(ca, st) || nd_conv_small(ca, st))) break;
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
            NdTensor res;
            if (!op.residual.empty()) {
                res = get(vals, op.residual).t;
                if (res.shape != out.t.shape)
                    fail("residual " + shape_str(res.shape) + " for a MatMul giving " + shape_str(out.t.shape));
            }
            NdRowsArgs ra;
            ra.res = res.p;
            ra.x = a.p;
            ra.m = int(m);
            ra.k = op.k;
            ra.n = op.n;
            ra.wt_hi = op.whi;
            ra.wt_lo = op.wlo;
            ra.pk = op.pk;
            ra.bias = op.b;
            ra.y = out.t.p;
            ra.act = op.act;
            if (!no_ndconv() && nd_gemm_rows(ra, st)) break;
            ConvArgs ca;
            ca.x = Act{a.p, 1, 1, int(m), op.k, op.k};
            ca.y = Act{out.t.p, 1, 1, int(m), op.n, op.n};
            ca.wt_hi = op.whi;
            ca.wt_lo = op.wlo;
            ca.bias = op.b;
            ca.act = op.act;
            ca.pk = op.pk;
            ca.res = res.p;
            ca.res_cs = op.n;
            conv_mfma(ca, st);
            break;
        }
        case NdKind::Attention: {
            const NdTensor qkv = flt(0);
            if (qkv.shape.size() != 3) fail("attention input " + shape_str(qkv.shape) + ", expects [n, T, 3 H d]");
            const int64_t nb = qkv.shape[0], tt = qkv.shape[1], c3 = qkv.shape[2];
            // The first Reshape's shape [n, T, 3, H, d] (0 copies a dimension, one -1 is inferred).
            std::vector<int64_t> s5 = ints(1);
            if (s5.size() != 5) fail("attention: a reshape to " + std::to_string(s5.size()) + " dimensions");
            const int64_t in_dims[3] = {nb, tt, c3};
            int64_t known = 1;
            int infer = -1;
            for (int d = 0; d < 5; d++) {
                if (s5[size_t(d)] == 0 && d < 3) s5[size_t(d)] = in_dims[d];
                if (s5[size_t(d)] == -1) {
                    if (infer >= 0) fail("attention: two inferred dimensions");
                    infer = d;
                } else {
                    known *= s5[size_t(d)];
                }
            }
            if (infer >= 0 && known > 0) s5[size_t(infer)] = nb * tt * c3 / known;
            const int64_t heads = s5[3], hd = s5[4];
            if (s5[0] != nb || s5[1] != tt || s5[2] != 3 || heads <= 0 || hd <= 0 || 3 * heads * hd != c3)
                fail("attention: reshape of " + shape_str(qkv.shape) + " to " + shape_str(s5));
            // The last Reshape must give [n, T, H d].
            std::vector<int64_t> s3 = ints(2);
            const int64_t od[3] = {nb, tt, heads * hd};
            for (size_t d = 0; d < s3.size() && d < 3; d++)
                if (s3[d] == 0) s3[d] = od[d];
            if (s3.size() == 3)
                for (size_t d = 0; d < 3; d++)
                    if (s3[d] == -1) s3[d] = od[d];
            if (s3 != std::vector<int64_t>(od, od + 3)) fail("attention: output reshape to " + shape_str(s3));
            out.t = alloc({nb, tt, heads * hd});
            if (shapes_only || nb * tt == 0) break;
            if (hd > 64 || nb > 65535 || heads > 65535) fail("attention: heads of " + std::to_string(hd) + " values");
            nd_attention(qkv.p, int(nb), int(tt), int(heads), int(hd), op.scale, out.t.p, st);
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
        if (!no_ndconv() && op.pk.bn == 64 && op.pk.chunks <= 8) {
            const int parts = nd_head_parts(int(m), op.pk);
            DBuf hp(&ctx, m * size_t(parts) * 2 * sizeof(float));
            NdRowsArgs ra;
            ra.x = a.p;
            ra.m = int(m);
            ra.k = op.k;
            ra.n = op.n;
            ra.wt_hi = op.whi;
            ra.wt_lo = op.wlo;
            ra.pk = op.pk;
            ra.bias = op.b;
            if (nd_head_argmax(ra, hp.as<float>(), parts, st)) {
                nd_argmax_partials(hp.as<float>(), parts, m, d_best, st);
                return;
            }
        }
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
