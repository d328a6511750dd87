#include "models.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace ocr {

// ---------------------------------------------------------------------------------------------
// Detector
// ---------------------------------------------------------------------------------------------
Detector::Detector(Ctx &ctx, const Onnx &onnx) : ctx_(ctx) {
    graph_ = Graph::build(ctx, onnx, nullptr, nullptr, nullptr);
}

void Detector::detect_pages_device(const uint8_t *const *rgb, const int *w, const int *h, int count, float thr,
                                   uint32_t *const *bits) {
    if (count <= 0) return;
    const hipStream_t st = ctx_.stream();
    Act in{nullptr, count, DET_MH, DET_MW, 1, 1};
    DBuf inbuf(&ctx_, in.count() * sizeof(float));
    in.p = inbuf.as<float>();
    std::vector<GreyPage> gp;
    for (int k = 0; k < count; k++) {
        if (w[k] <= 0 || h[k] <= 0) fail("empty page");
        const int ph = std::max(h[k], DET_MH), pw = std::max(w[k], DET_MW);
        gp.push_back({rgb[k], w[k], h[k], pw, ph, in.p + size_t(k) * DET_MH * DET_MW, float(pw) / float(DET_MW),
                      float(ph) / float(DET_MH)});
    }
    grey_resize(gp.data(), count, DET_MW, DET_MH, st);
    Graph::Out out = graph_.run(ctx_, in);
    if (out.act.h != DET_MH || out.act.w != DET_MW || out.act.c != 1)
        fail("detection model output is not [n, 1, 800, 600]");
    std::vector<MaskPage> mp;
    for (int k = 0; k < count; k++) {
        const int ph = std::max(h[k], DET_MH), pw = std::max(w[k], DET_MW);
        // The part of the mask that covers the page, not the padding (gpu.rs:1413-1414).
        const int vh = DET_MH - (ph - h[k]) * DET_MH / ph, vw = DET_MW - (pw - w[k]) * DET_MW / pw;
        mp.push_back({out.act.p + size_t(k) * DET_MH * DET_MW, vw, vh, bits[k], w[k], h[k], float(vw) / float(w[k]),
                      float(vh) / float(h[k])});
    }
    mask_up(mp.data(), count, DET_MW, thr, st);
}

std::vector<float> Detector::detect(const float *input, int h, int w) {
    Act in{nullptr, 1, h, w, 1, 1};
    DBuf inbuf(&ctx_, in.count() * sizeof(float));
    in.p = inbuf.as<float>();
    ctx_.h2d(in.p, input, in.count() * sizeof(float));
    Graph::Out out = graph_.run(ctx_, in);
    std::vector<float> prob(out.act.count());
    // The output is NHWC; for one channel that is NCHW too.
    if (out.act.c != 1) {
        std::vector<float> nhwc(out.act.count());
        ctx_.d2h(nhwc.data(), out.act.p, nhwc.size() * sizeof(float));
        const size_t hw = size_t(out.act.h) * out.act.w;
        for (size_t p = 0; p < hw; p++)
            for (int c = 0; c < out.act.c; c++) prob[c * hw + p] = nhwc[p * out.act.c + c];
        return prob;
    }
    ctx_.d2h(prob.data(), out.act.p, prob.size() * sizeof(float));
    return prob;
}

// ---------------------------------------------------------------------------------------------
// Recognizer
// ---------------------------------------------------------------------------------------------
namespace {

void pack_linear(Ctx &ctx, const std::vector<float> &w_rows, int rows, int cols, ConvPack &pk, const uint16_t *&hi,
                 const uint16_t *&lo, const uint16_t *&frag) {
    // w_rows is [rows = outputs][cols = inputs]: a 1 x 1 convolution's [cout][cin][1][1].
    pk = plan_conv_pack(cols, rows, 1, 1);
    std::vector<uint16_t> h(pk.halves()), l(pk.halves());
    bool exact = true;
    pack_conv_weights(pk, w_rows.data(), h.data(), l.data(), &exact);
    pk.exact = exact;
    hi = ctx.upload_weights(h.data(), h.size());
    lo = exact ? nullptr : ctx.upload_weights(l.data(), l.size());
    std::vector<uint16_t> f(pk.frag_halves());
    pack_conv_frags(pk, h.data(), l.data(), f.data());
    frag = ctx.upload_weights(f.data(), f.size());
}

}  // namespace

Recognizer::Recognizer(Ctx &ctx, const Onnx &onnx, uint32_t lines) : ctx_(ctx), lines_(lines) {
    Node pool;
    bool found = false;
    trunk_ = Graph::build(ctx, onnx, "AveragePool", &pool, &found);
    if (!found) fail("no AveragePool in the recognition model");
    auto k = pool.ints("kernel_shape");
    if (!k) fail("AveragePool without kernel_shape");
    auto s = pool.ints("strides");
    if (k->size() != 2 || (*k)[1] != 1 || !s || *s != *k) fail("unsupported AveragePool");
    pool_kh_ = int((*k)[0]);
    int nl = 0;
    for (const Node &n : onnx.nodes) {
        if (n.op != "GRU") continue;
        if (nl >= 2) fail("more than 2 GRU layers");
        if (n.int_("hidden_size") != std::optional<int64_t>(256) ||
            n.int_("linear_before_reset") != std::optional<int64_t>(1) ||
            n.str("direction") != std::optional<std::string>("bidirectional"))
            fail("unsupported GRU attributes");
        const Weight &w = onnx.weight(n.inputs.at(1)), &r = onnx.weight(n.inputs.at(2)),
                     &b = onnx.weight(n.inputs.at(3));
        if (w.dims.size() != 3 || w.dims[0] != 2 || w.dims[1] != 768) fail("GRU W shape");
        if (r.dims != std::vector<int64_t>{2, 768, 256}) fail("GRU R shape");
        if (b.data.size() != 2 * 1536) fail("GRU B shape");
        Layer &L = layers_[nl++];
        L.input = int(w.dims[2]);
        // W [2][768][in] is already the projection's [1536 outputs][in] (gpu.rs:1466-1472).
        pack_linear(ctx, w.data, 1536, L.input, L.pk, L.w_hi, L.w_lo, L.w_frag);
        std::vector<float> wb, rb;
        for (int d = 0; d < 2; d++) {
            wb.insert(wb.end(), b.data.begin() + d * 1536, b.data.begin() + d * 1536 + 768);
            rb.insert(rb.end(), b.data.begin() + d * 1536 + 768, b.data.begin() + d * 1536 + 1536);
        }
        L.wb = ctx.upload_weights(wb.data(), wb.size());
        L.rb = ctx.upload_weights(rb.data(), rb.size());
        // R in float16 (gpu.rs:1478-1484): exact for float16-valued weights; otherwise rounded,
        // as the reference does with F16 on (its default). With F16=0 the reference keeps R in
        // float32, and so does this library for R that is not float16-valued: the recurrence
        // then streams R^T in float32 (gru_recurrence_f32).
        std::vector<uint16_t> rh(r.data.size());
        bool exact = true;
        for (size_t i = 0; i < r.data.size(); i++) {
            _Float16 v = (_Float16)r.data[i];
            if ((float)v != r.data[i]) exact = false;
            std::memcpy(&rh[i], &v, 2);
        }
        r_exact_ = r_exact_ && exact;
        const char *f16 = std::getenv("F16");
        if (!exact && f16 && std::string(f16) == "0") {
            std::vector<float> rt(r.data.size());
            for (int d = 0; d < 2; d++)
                for (int row = 0; row < 768; row++)
                    for (int k = 0; k < 256; k++)
                        rt[(size_t(d) * 256 + k) * 768 + row] = r.data[(size_t(d) * 768 + row) * 256 + k];
            L.r32 = ctx.upload_weights(rt.data(), rt.size());
        }
        L.r = ctx.upload_weights(rh.data(), rh.size());
    }
    if (nl != 2) fail(std::to_string(nl) + " GRU layers");
    const Node *mm = nullptr;
    for (const Node &n : onnx.nodes)
        if (n.op == "MatMul") { mm = &n; break; }
    if (!mm) fail("no MatMul");
    const Weight &lin = onnx.weight(mm->inputs.at(1));  // [512][classes]: [in][out]
    if (lin.dims.size() != 2 || lin.dims[0] != 512) fail("output MatMul weight shape");
    classes_ = int(lin.dims[1]);
    const Node *add = nullptr;
    for (const Node &n : onnx.nodes)
        if (n.op == "Add" && std::find(n.inputs.begin(), n.inputs.end(), mm->outputs.at(0)) != n.inputs.end()) {
            add = &n;
            break;
        }
    if (!add) fail("no bias Add");
    const Weight *bias = nullptr;
    for (const std::string &i : add->inputs)
        if (onnx.weights.count(i)) bias = &onnx.weights.at(i);
    if (!bias || int(bias->data.size()) != classes_) fail("no bias weight");
    std::vector<float> t(size_t(classes_) * 512);
    for (int i = 0; i < 512; i++)
        for (int c = 0; c < classes_; c++) t[size_t(c) * 512 + i] = lin.data[size_t(i) * classes_ + c];
    pack_linear(ctx, t, classes_, 512, lin_pk_, lin_hi_, lin_lo_, lin_frag_);
    lin_b_ = ctx.upload_weights(bias->data.data(), bias->data.size());
}

Recognizer::~Recognizer() = default;

Recognizer::Dims Recognizer::dims(const Batch *batches, int count) const {
    Dims d{0, 0, classes_};
    for (int b = 0; b < count; b++) {
        if (batches[b].n <= 0 || batches[b].w <= 0) fail("empty recognition batch");
        const Shape s = trunk_.infer({batches[b].n, 64, batches[b].w, 1});
        d.tmax = std::max(d.tmax, s[2]);
        d.ntot += batches[b].n;
    }
    return d;
}

void Recognizer::recognize_device(const Batch *batches, int count, float *logits, uint32_t *best, uint32_t *lens,
                                  const std::function<void()> &between, hipStream_t gru_stream) {
    const hipStream_t st = ctx_.stream();
    const Dims d = dims(batches, count);
    if (d.ntot == 0) return;
    const int M = d.tmax * d.ntot;
    if (double(d.tmax) * d.ntot >= 2147483647.0) fail("recognition pass too large");
    // X [t][ntot][256] time-major (gpu.rs:1538-1555); rows t >= a line's length are never read.
    DBuf X(&ctx_, size_t(M) * 256 * sizeof(float));
    // The trunks first (gpu.rs:1516-1526). The width batches share the 64-row height, so each
    // trunk layer runs once over all of them: one launch a dense conv layer fills the GPU where
    // a launch per width batch would not.
    // The average pool (gpu.rs:595-614) runs in the last trunk layer's epilogue when that layer
    // takes it, else as its own kernel over all width batches.
    std::vector<Act> xs;
    int noff = 0;
    for (int b = 0; b < count; b++) {
        xs.push_back(Act{const_cast<float *>(batches[b].data), batches[b].n, 64, batches[b].w, 1, 1});
        const Shape t = trunk_.infer({batches[b].n, 64, batches[b].w, 1});
        if (t[3] != layers_[0].input)
            fail("trunk gives " + std::to_string(t[3]) + " features, GRU takes " + std::to_string(layers_[0].input));
        if ((t[1] - pool_kh_) / pool_kh_ + 1 != 1)
            fail("trunk height " + std::to_string(t[1]) + " does not pool to one row");
        for (int i = 0; i < t[0]; i++) lens[noff + i] = uint32_t(t[2]);
        noff += t[0];
    }
    const int tmax = d.tmax, ntot = d.ntot;
    // The rows that carry a step of some line, t-major: (t, line) with t < lens[line]. The
    // projections and the output layer run on these rows only (the reference computes all
    // tmax x ntot rows and ignores the padding ones); G, Y and the logits keep the [t][ntot]
    // layout, so the recurrence and the caller see the reference's layout.
    // Lines come in batches of one length each: per step, the runs of lines still going.
    std::vector<int32_t> rows;
    {
        std::vector<std::pair<int, int>> runs;  // (first line, length) of each batch
        size_t total = 0;
        for (int i = 0; i < ntot;) {
            int j = i + 1;
            while (j < ntot && lens[j] == lens[i]) j++;
            runs.push_back({i, j});
            total += size_t(j - i) * lens[i];
            i = j;
        }
        rows.resize(total);
        size_t k = 0;
        for (int t = 0; t < tmax; t++)
            for (const auto &rn : runs)
                if (uint32_t(t) < lens[rn.first])
                    for (int i = rn.first; i < rn.second; i++) rows[k++] = t * ntot + i;
    }
    const int P = int(rows.size());
    const long long steps = P;
    // Lengths and rows in one upload, ahead of the trunk's kernels.
    const size_t rows_at = (size_t(ntot) * 4 + 15) & ~size_t(15);
    std::vector<char> tab(rows_at + rows.size() * 4, 0);
    std::memcpy(tab.data(), lens, size_t(ntot) * 4);
    std::memcpy(tab.data() + rows_at, rows.data(), rows.size() * 4);
    DBuf tabd(&ctx_, tab.size());
    ctx_.h2d(tabd.get(), tab.data(), tab.size());
    const uint32_t *lensd = reinterpret_cast<const uint32_t *>(tabd.as<char>());
    const int32_t *rowsd = reinterpret_cast<const int32_t *>(tabd.as<char>() + rows_at);
    std::vector<Graph::Out> trunks;
    // A stage boundary also in the middle of the trunk (its five layers carry similar work), so a
    // caller's work queued from between() waits for half the trunk rather than all of it.
    const int mid = (int(trunk_.steps.size()) + 1) / 2;
    auto after = [&](int i) {
        if (between && i + 1 == mid) between();
    };
    const bool fused = pool_kh_ == 2 && trunk_.run_multi_time_major(ctx_, xs, pool_kh_, X.as<float>(), d.ntot, trunks,
                                                                    after);
    if (!fused) {
        if (pool_kh_ != 2) trunks = trunk_.run_multi(ctx_, xs);
        std::vector<Act> feats;
        for (const Graph::Out &t : trunks) feats.push_back(t.act);
        avgpool_t(feats.data(), count, pool_kh_, X.as<float>(), d.ntot, st);
    }
    trunks.clear();
    if (between) between();
    DBuf G(&ctx_, size_t(M) * 1536 * sizeof(float));
    DBuf Y[2] = {DBuf(&ctx_, size_t(M) * 512 * sizeof(float)), DBuf(&ctx_, size_t(M) * 512 * sizeof(float))};
    const float *in = X.as<float>();
    int in_c = 256;
    // With a stream for the recurrences: each waits for its projection; the context's stream
    // waits for the first (join) before the second projection reads its output, and the second
    // recurrence, the output layer and the arg-max stay on the recurrence stream (the caller
    // orders its reads of logits and best after that stream). The buffers the recurrence stream
    // touches are marked as used on it, so the pool hands them out again only after its work.
    const hipStream_t gs = gru_stream ? gru_stream : st;
    if (gs != st) {
        G.used_on(gs);
        Y[0].used_on(gs);
        Y[1].used_on(gs);
        tabd.used_on(gs);
    }
    hipEvent_t join = nullptr;
    auto fork = [&]() {
        if (gs == st) return;
        hipEvent_t e = nullptr;
        OCR_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        OCR_HIP(hipEventRecord(e, st));
        OCR_HIP(hipStreamWaitEvent(gs, e, 0));
        OCR_HIP(hipEventDestroy(e));  // the wait holds what it needs
    };
    auto join_back = [&]() {
        if (!join) return;
        OCR_HIP(hipStreamWaitEvent(st, join, 0));
        OCR_HIP(hipEventDestroy(join));
        join = nullptr;
    };
    // If anything throws, the context's stream still waits for the recurrence stream before the
    // buffers (declared above, so released after this) go back.
    struct Unwind {
        hipStream_t st, gs;
        hipEvent_t &join;
        bool settled = false;
        ~Unwind() {
            if (join) (void)hipEventDestroy(join);
            if (settled || gs == st) return;
            hipEvent_t e = nullptr;
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return;
            if (hipEventRecord(e, gs) == hipSuccess) (void)hipStreamWaitEvent(st, e, 0);
            (void)hipEventDestroy(e);
        }
    } unwind{st, gs, join};
    for (int l = 0; l < 2; l++) {
        join_back();
        const Layer &L = layers_[l];
        if (in_c != L.input) fail("GRU layer input size");
        ConvArgs ca;
        ca.x = Act{const_cast<float *>(in), 1, 1, P, in_c, in_c};
        ca.y = Act{G.as<float>(), 1, 1, P, 1536, 1536};
        ca.rows = rowsd;
        ca.wt_hi = L.w_hi;
        ca.wt_lo = L.w_lo;
        ca.wt_frag = L.w_frag;
        ca.bias = L.wb;
        ca.pk = L.pk;
        conv_mfma(ca, st);
        fork();
        if (L.r32) gru_recurrence_f32(G.as<float>(), L.r32, L.rb, Y[l].as<float>(), lensd, ntot, steps, gs);
        else gru_recurrence(G.as<float>(), L.r, L.rb, Y[l].as<float>(), lensd, ntot, tmax, steps, gs);
        if (gs != st && l == 0) {
            OCR_HIP(hipEventCreateWithFlags(&join, hipEventDisableTiming));
            OCR_HIP(hipEventRecord(join, gs));
        }
        in = Y[l].as<float>();
        in_c = 512;
        if (between) between();
    }
    ConvArgs ca;
    ca.x = Act{const_cast<float *>(in), 1, 1, P, 512, 512};
    ca.y = Act{logits, 1, 1, P, classes_, classes_};
    ca.rows = rowsd;
    ca.wt_hi = lin_hi_;
    ca.wt_lo = lin_lo_;
    ca.wt_frag = lin_frag_;
    ca.bias = lin_b_;
    ca.pk = lin_pk_;
    conv_mfma(ca, gs);
    if (best) argmax_rows(logits, P, classes_, best, gs, rowsd);
    unwind.settled = true;
}

}  // namespace ocr
