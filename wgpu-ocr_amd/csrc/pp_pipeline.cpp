#include "pp_pipeline.h"

#include <algorithm>
#include <cmath>
#include <memory>
#include <mutex>

#include "crop.h"
#include "host_util.h"
#include "pipeline_core.h"
#include "upload.h"

namespace ocr {

namespace {

// nd.rs:1356-1358 (the same rule as the C ABI's detection-input size).
void det_size(int w, int h, int max_side, int *ow, int *oh) {
    const float ratio = std::max(w, h) > max_side ? float(max_side) / float(std::max(w, h)) : 1.f;
    auto round32 = [](float v) { return std::max(int(std::lround(v / 32.f)) * 32, 32); };
    *ow = round32(float(w) * ratio);
    *oh = round32(float(h) * ratio);
}

struct PageBoxes {
    std::vector<PpLine> lines;
    BatchPlan plan;
};

}  // namespace

struct PpPipeline::Impl {
    Ctx &ctx;
    NdGraph &det, &rec;
    PpPipelineOpts opts;
    Workers workers;
    std::vector<Pinned> prob_host, bits_host, best_host;
    std::unique_ptr<PageUploader> upl;  // made by the first run from host memory
    Impl(Ctx &c, NdGraph &d, NdGraph &r, const PpPipelineOpts &o)
        : ctx(c), det(d), rec(r), opts(o), workers(worker_count(o.threads)) {}
};

PpPipeline::PpPipeline(Ctx &ctx, NdGraph &det, NdGraph &rec, const PpPipelineOpts &opts)
    : impl_(new Impl(ctx, det, rec, opts)) {
    if (opts.merge < 1 || opts.det_batch < 1 || opts.per_batch < 1 || opts.max_side < 32)
        fail("pp pipeline: merge, det_batch and per_batch must be at least 1, max_side at least 32");
}

PpPipeline::~PpPipeline() { delete impl_; }

void PpPipeline::run(const uint8_t *const *d_rgb, const int *w, const int *h, int npages) {
    run_pages(d_rgb, false, w, h, npages);
}

void PpPipeline::run_host(const uint8_t *const *rgb, const int *w, const int *h, int npages) {
    run_pages(rgb, true, w, h, npages);
}

namespace {

// One run of the PP-OCR pipeline as the page pipeline's schedule (pipeline_core.h) drives it:
// groups of pages upload (host pages), are detected (detection input, DB graph, threshold, the
// map and mask to pinned memory) and boxed on the host a page at a time; recognition passes
// (line images, SVTR graph with the fused arg-max) go out as soon as their pages are boxed, and
// their CTC runs on the host. Hooks run on the schedule's threads: stage on the stager,
// detect and recognize on the calling thread, detect_wait on the watcher, layout and decode on
// the workers.
struct PpRun final : PipelineHooks {
    PpPipeline::Impl &I;
    Ctx &ctx;
    hipStream_t st, up = nullptr;
    const PipelinePlan &P;
    const uint8_t *const *src;
    bool on_host;
    const int *w, *h;
    std::vector<int> ow, oh;
    std::vector<PageText> &pages;
    PipelineStats &stats;
    std::vector<DBuf> dpages;              // host pages' device copies
    std::vector<const uint8_t *> d_rgb;    // every page's device RGB
    std::vector<char> pinned;
    std::vector<hipEvent_t> up_ev, det_ev, rec_ev;
    std::vector<std::vector<DBuf>> keep;   // a group's detection buffers, until the run ends
    std::vector<std::shared_ptr<DBuf>> keep_in;
    std::vector<PageBoxes> boxes;
    struct Row {
        int page, line, steps;
        size_t off;
    };
    std::vector<std::vector<Row>> rows;
    std::vector<DBuf> best;

    PpRun(PpPipeline::Impl &impl, Ctx &c, const PipelinePlan &plan, const uint8_t *const *s_, bool host, const int *w_,
          const int *h_, const std::vector<int> &ow_, const std::vector<int> &oh_, std::vector<PageText> &pg,
          PipelineStats &stt)
        : I(impl), ctx(c), st(c.stream()), P(plan), src(s_), on_host(host), w(w_), h(h_), ow(ow_), oh(oh_), pages(pg),
          stats(stt) {
        const int np = P.npages;
        up_ev.assign(size_t(P.groups()), nullptr);
        det_ev.assign(size_t(P.groups()), nullptr);
        rec_ev.assign(size_t(P.passes()), nullptr);
        keep.resize(size_t(P.groups()));
        keep_in.resize(size_t(P.groups()));
        boxes.resize(size_t(np));
        rows.resize(size_t(P.passes()));
        best.resize(size_t(P.passes()));
        // Pinned landing places, made here (one thread) before any hook runs.
        if (I.prob_host.size() < size_t(np)) I.prob_host.resize(size_t(np)), I.bits_host.resize(size_t(np));
        if (I.best_host.size() < size_t(P.passes())) I.best_host.resize(size_t(P.passes()));
        for (int p = 0; p < np; p++) {
            I.prob_host[size_t(p)].ensure(size_t(ow[size_t(p)]) * oh[size_t(p)] * 4);
            I.bits_host[size_t(p)].ensure(size_t((ow[size_t(p)] + 31) / 32) * oh[size_t(p)] * 4);
        }
        if (on_host) {
            if (!I.upl) I.upl.reset(new PageUploader(ctx));
            up = I.upl->stream();
            pinned.resize(size_t(np));
            for (int p = 0; p < np; p++) {
                dpages.emplace_back(&ctx, size_t(w[p]) * h[p] * 3);
                dpages.back().used_on(up);
                d_rgb.push_back(dpages.back().as<uint8_t>());
                pinned[size_t(p)] = host_pinned(src[p]);
            }
            // The page buffers come from the pool in the compute stream's order.
            hipEvent_t ready = nullptr;
            OCR_HIP(hipEventCreateWithFlags(&ready, hipEventDisableTiming));
            OCR_HIP(hipEventRecord(ready, st));
            OCR_HIP(hipStreamWaitEvent(up, ready, 0));
            OCR_HIP(hipEventDestroy(ready));
        } else {
            d_rgb.assign(src, src + np);
        }
    }
    ~PpRun() override {
        if (up) drain_stream(up, "the uploads of a pp run");
        for (auto *v : {&up_ev, &det_ev, &rec_ev})
            for (hipEvent_t e : *v)
                if (e) (void)hipEventDestroy(e);
    }
    hipEvent_t record(hipStream_t s) {
        hipEvent_t e = nullptr;
        OCR_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        OCR_HIP(hipEventRecord(e, s));
        return e;
    }

    void stage(int g) override {
        if (!on_host) return;
        ctx.bind();
        for (int p = P.group_p0[size_t(g)]; p < P.group_p0[size_t(g) + 1]; p++)
            I.upl->upload(dpages[size_t(p)].as<uint8_t>(), src[p], size_t(w[p]) * h[p] * 3, pinned[size_t(p)] != 0);
        up_ev[size_t(g)] = record(up);
    }
    bool landed(int g) override {
        const hipEvent_t e = up_ev[size_t(g)];
        return !e || event_query(e, true);
    }
    void detect(int g) override {
        const int p = P.group_p0[size_t(g)], q = P.group_p0[size_t(g) + 1], n = q - p;
        if (up_ev[size_t(g)]) OCR_HIP(hipStreamWaitEvent(st, up_ev[size_t(g)], 0));
        const int W = ow[size_t(p)], H = oh[size_t(p)];
        const size_t plane = size_t(W) * H, words = size_t((W + 31) / 32) * H;
        NdTensor in;
        in.shape = {n, 3, H, W};
        in.buf = std::make_shared<DBuf>(&ctx, size_t(n) * 3 * plane * sizeof(float));
        in.p = in.buf->as<float>();
        keep_in[size_t(g)] = in.buf;
        for (int k = 0; k < n; k++) nd_det_prep(d_rgb[size_t(p + k)], w[p + k], h[p + k], in.p + size_t(k) * 3 * plane, W, H, st);
        NdTensor prob = I.det.run(ctx, in);
        if (prob.count() != size_t(n) * plane) fail("pp pipeline: detector output is not [n, 1, h, w]");
        DBuf bits(&ctx, size_t(n) * words * 4);
        for (int k = 0; k < n; k++) {
            nd_threshold_bits(prob.p + size_t(k) * plane, W, H, I.opts.thr, bits.as<uint32_t>() + size_t(k) * words, st);
            OCR_HIP(hipMemcpyAsync(I.prob_host[size_t(p + k)].p, prob.p + size_t(k) * plane, plane * 4,
                                   hipMemcpyDeviceToHost, st));
            OCR_HIP(hipMemcpyAsync(I.bits_host[size_t(p + k)].p, bits.as<uint32_t>() + size_t(k) * words, words * 4,
                                   hipMemcpyDeviceToHost, st));
        }
        det_ev[size_t(g)] = record(st);
        keep[size_t(g)].push_back(std::move(bits));
        if (prob.buf) keep_in.push_back(prob.buf);
    }
    void detect_wait(int g) override {
        wait_event(det_ev[size_t(g)], "the probability maps and masks of detection group " + std::to_string(g));
    }
    void layout(int k) override {
        (void)hipSetDevice(ctx.device());
        const float *pr = static_cast<const float *>(I.prob_host[size_t(k)].p);
        const uint32_t *bt = static_cast<const uint32_t *>(I.bits_host[size_t(k)].p);
        const int mw = ow[size_t(k)], mh = oh[size_t(k)];
        PageBoxes B;
        for (const RRect &r : db_boxes(bt, pr, mw, mh, float(w[k]) / float(mw), float(h[k]) / float(mh), I.opts.db))
            B.lines.push_back(pp_line_box(r, I.opts.relv, w[k], h[k]));
        std::vector<int> ow_l;
        for (const PpLine &l : B.lines) ow_l.push_back(l.out_w);
        B.plan = plan_pp_batches(ow_l, I.opts.per_batch);
        boxes[size_t(k)] = std::move(B);
    }
    void recognize(int r, const std::vector<char> &ok) override {
        const int p0 = P.pass_p0[size_t(r)], p1 = P.pass_p0[size_t(r) + 1];
        struct Batch {
            NdTensor in;
            size_t best_off;
            int steps;
        };
        std::vector<Batch> batches;
        std::vector<PpCropLine> crops;
        size_t best_total = 0;
        int max_wb = 0;
        for (int k = p0; k < p1; k++) {
            if (!ok[size_t(k - p0)]) continue;
            const PageBoxes &B = boxes[size_t(k)];
            pages[size_t(k)].words = int(B.lines.size());
            pages[size_t(k)].lines.assign(B.lines.size(), std::string());
            for (size_t b = 0; b < B.plan.lines.size(); b++) {
                const int wb = B.plan.width[b], n = int(B.plan.lines[b].size());
                Batch bt;
                bt.in.shape = {n, 3, PP_LINE_H, wb};
                bt.in.buf = std::make_shared<DBuf>(&ctx, size_t(n) * 3 * PP_LINE_H * wb * sizeof(float));
                bt.in.p = bt.in.buf->as<float>();
                const auto os = I.rec.output_shape(bt.in.shape);
                if (os.size() != 3 || os[0] != n) fail("pp pipeline: recogniser output is not [n, steps, classes]");
                bt.steps = int(os[1]);
                bt.best_off = best_total;
                best_total += size_t(n) * bt.steps;
                max_wb = std::max(max_wb, wb);
                for (int j = 0; j < n; j++) {
                    const int li = B.plan.lines[b][size_t(j)];
                    const PpLine &L = B.lines[size_t(li)];
                    crops.push_back({d_rgb[size_t(k)], w[k], h[k], L.left, L.top, L.cw, L.ch, L.out_w,
                                     bt.in.p + size_t(j) * 3 * PP_LINE_H * wb, wb});
                    rows[size_t(r)].push_back({k, li, bt.steps, bt.best_off + size_t(j) * bt.steps});
                }
                batches.push_back(std::move(bt));
            }
        }
        stats.batches += int(batches.size());
        if (batches.empty()) return;
        DBuf dcrops(&ctx, crops.size() * sizeof(PpCropLine));
        ctx.h2d(dcrops.get(), crops.data(), crops.size() * sizeof(PpCropLine));
        pp_line_crop(dcrops.as<PpCropLine>(), int(crops.size()), max_wb, st);
        best[size_t(r)] = DBuf(&ctx, best_total * 4);
        for (const Batch &bt : batches) I.rec.run_argmax(ctx, bt.in, best[size_t(r)].as<uint32_t>() + bt.best_off, nullptr);
        I.best_host[size_t(r)].ensure(best_total * 4);
        OCR_HIP(hipMemcpyAsync(I.best_host[size_t(r)].p, best[size_t(r)].get(), best_total * 4, hipMemcpyDeviceToHost, st));
        rec_ev[size_t(r)] = record(st);
        stats.rec_passes++;
    }
    void decode(int r, bool) override {
        if (!rec_ev[size_t(r)]) return;  // no lines in the pass
        wait_event(rec_ev[size_t(r)], "the arg-max of recognition pass " + std::to_string(r));
        const uint32_t *bh = static_cast<const uint32_t *>(I.best_host[size_t(r)].p);
        for (const Row &row : rows[size_t(r)])
            pages[size_t(row.page)].lines[size_t(row.line)] = pp_ctc_decode(bh + row.off, row.steps);
    }
};

}  // namespace

void PpPipeline::run_pages(const uint8_t *const *src, bool on_host, const int *w, const int *h, int npages) {
    Impl &I = *impl_;
    Ctx &ctx = I.ctx;
    const auto t0 = Clock::now();
    pages_.assign(size_t(std::max(npages, 0)), PageText{});
    stats_ = PipelineStats{};
    stats_.pages = npages;
    if (npages <= 0) return;
    for (int p = 0; p < npages; p++) {
        if (!src[p]) fail("pp pipeline: page " + std::to_string(p) + " has no pixels");
        if (w[p] <= 0 || h[p] <= 0) fail("pp pipeline: empty page " + std::to_string(p));
    }
    ctx.bind();
    std::vector<int> ow(static_cast<size_t>(npages)), oh(static_cast<size_t>(npages));
    for (int p = 0; p < npages; p++) det_size(w[p], h[p], I.opts.max_side, &ow[size_t(p)], &oh[size_t(p)]);
    // The page pipeline's plan, with a detection group also cut where the detection input's
    // size changes (a group is one batched detector run).
    PipelinePlan plan = plan_pipeline(npages, I.opts.merge, I.opts.det_batch, on_host);
    std::vector<int> cuts;
    for (int g = 0; g < plan.groups(); g++) {
        cuts.push_back(plan.group_p0[size_t(g)]);
        for (int p = plan.group_p0[size_t(g)] + 1; p < plan.group_p0[size_t(g) + 1]; p++)
            if (ow[size_t(p)] != ow[size_t(p - 1)] || oh[size_t(p)] != oh[size_t(p - 1)]) cuts.push_back(p);
    }
    cuts.push_back(npages);
    plan.group_p0 = cuts;
    for (int g = 0; g < plan.groups(); g++)
        for (int p = plan.group_p0[size_t(g)]; p < plan.group_p0[size_t(g) + 1]; p++) plan.group_of[size_t(p)] = g;
    std::vector<std::string> errs;
    double busy = 0;
    {
        PpRun R(I, ctx, plan, src, on_host, w, h, ow, oh, pages_, stats_);
        errs = run_schedule(plan, R, [&](std::function<void()> f) { I.workers.submit(std::move(f)); }, &busy,
                            !on_host);
        for (const auto &rr : R.rows)
            for (const auto &row : rr) stats_.rec_steps += row.steps;
        ctx.sync();
    }
    for (int p = 0; p < npages; p++)
        if (!errs[size_t(p)].empty()) fail("pp pipeline: " + errs[size_t(p)]);
    stats_.ms = ms_since(t0);
    stats_.cpu_busy_ms = busy;
    for (const PageText &pt : pages_) {
        stats_.lines += int(pt.lines.size());
        stats_.words += pt.words;
    }
}

}  // namespace ocr
