#include "pp_pipeline.h"

#include <algorithm>
#include <cmath>
#include <memory>
#include <mutex>

#include "crop.h"
#include "host_util.h"
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
    run_pages(d_rgb, w, h, npages, [](int, int) {});
}

void PpPipeline::run_host(const uint8_t *const *rgb, const int *w, const int *h, int npages) {
    Impl &I = *impl_;
    Ctx &ctx = I.ctx;
    ctx.bind();
    if (!I.upl) I.upl.reset(new PageUploader(ctx));
    const hipStream_t up = I.upl->stream(), st = ctx.stream();
    std::vector<DBuf> dpages;
    std::vector<const uint8_t *> ptrs;
    std::vector<char> pinned(size_t(std::max(npages, 0)));
    for (int p = 0; p < npages; p++) {
        if (!rgb[p]) fail("pp pipeline: page " + std::to_string(p) + " has no pixels");
        if (w[p] <= 0 || h[p] <= 0) fail("pp pipeline: empty page " + std::to_string(p));
        dpages.emplace_back(&ctx, size_t(w[p]) * h[p] * 3);
        dpages.back().used_on(up);
        ptrs.push_back(dpages.back().as<uint8_t>());
        pinned[size_t(p)] = host_pinned(rgb[p]);
    }
    // The page buffers come from the pool in the compute stream's order: the uploads wait for it.
    hipEvent_t ready, done;
    OCR_HIP(hipEventCreateWithFlags(&ready, hipEventDisableTiming));
    OCR_HIP(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    struct Events {
        hipEvent_t a, b;
        ~Events() {
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
        }
    } guard{ready, done};
    OCR_HIP(hipEventRecord(ready, st));
    OCR_HIP(hipStreamWaitEvent(up, ready, 0));
    try {
        run_pages(ptrs.data(), w, h, npages, [&](int p, int q) {
            for (int k = p; k < q; k++)
                I.upl->upload(dpages[size_t(k)].as<uint8_t>(), rgb[k], size_t(w[k]) * h[k] * 3, pinned[size_t(k)] != 0);
            OCR_HIP(hipEventRecord(done, up));
            OCR_HIP(hipStreamWaitEvent(st, done, 0));
        });
    } catch (...) {
        drain_stream(up, "the uploads of a failed run");
        throw;
    }
}

void PpPipeline::run_pages(const uint8_t *const *d_rgb, const int *w, const int *h, int npages,
                           const std::function<void(int, int)> &before_pass) {
    Impl &I = *impl_;
    Ctx &ctx = I.ctx;
    const hipStream_t st = ctx.stream();
    const auto t0 = Clock::now();
    pages_.assign(size_t(std::max(npages, 0)), PageText{});
    stats_ = PipelineStats{};
    stats_.pages = npages;
    if (npages <= 0) return;
    for (int p = 0; p < npages; p++)
        if (w[p] <= 0 || h[p] <= 0) fail("pp pipeline: empty page " + std::to_string(p));
    std::vector<int> ow(static_cast<size_t>(npages)), oh(static_cast<size_t>(npages));
    for (int p = 0; p < npages; p++) det_size(w[p], h[p], I.opts.max_side, &ow[size_t(p)], &oh[size_t(p)]);

    std::mutex mu;
    std::condition_variable cv;
    std::vector<int> ready(static_cast<size_t>(npages), 0);
    std::vector<PageBoxes> boxes(static_cast<size_t>(npages));
    std::string error;
    double cpu_busy = 0;
    int pending = 0;
    auto task_done = [&](double busy, const std::string &err) {
        std::lock_guard<std::mutex> lk(mu);
        cpu_busy += busy;
        if (!err.empty() && error.empty()) error = err;
        pending--;
        cv.notify_all();
    };
    std::vector<hipEvent_t> events;
    const int dev = ctx.device();
    // Per recognition pass, where each line's arg-max lands (read by the decoding tasks, so it
    // lives until they have all finished).
    struct Row {
        int page, line, steps;
        size_t off;
    };
    const int nrec = (npages + I.opts.merge - 1) / I.opts.merge;
    std::vector<std::vector<Row>> rows(static_cast<size_t>(nrec));
    try {
        // 1. Detection: consecutive pages of one input size, det_batch a pass; the map and its
        // threshold bits come back to pinned memory asynchronously.
        if (I.prob_host.size() < size_t(npages)) {
            I.prob_host.resize(size_t(npages));
            I.bits_host.resize(size_t(npages));
        }
        int p = 0;
        while (p < npages) {
            int q = p + 1;
            while (q < npages && q - p < I.opts.det_batch && ow[size_t(q)] == ow[size_t(p)] && oh[size_t(q)] == oh[size_t(p)])
                q++;
            const int n = q - p, W = ow[size_t(p)], H = oh[size_t(p)];
            const size_t plane = size_t(W) * H, words = size_t((W + 31) / 32) * H;
            before_pass(p, q);
            NdTensor in;
            in.shape = {n, 3, H, W};
            in.buf = std::make_shared<DBuf>(&ctx, size_t(n) * 3 * plane * sizeof(float));
            in.p = in.buf->as<float>();
            for (int k = 0; k < n; k++) nd_det_prep(d_rgb[p + k], w[p + k], h[p + k], in.p + size_t(k) * 3 * plane, W, H, st);
            NdTensor prob = I.det.run(ctx, in);
            if (prob.count() != size_t(n) * plane) fail("pp pipeline: detector output is not [n, 1, h, w]");
            DBuf bits(&ctx, size_t(n) * words * 4);
            for (int k = 0; k < n; k++) {
                nd_threshold_bits(prob.p + size_t(k) * plane, W, H, I.opts.thr, bits.as<uint32_t>() + size_t(k) * words, st);
                I.prob_host[size_t(p + k)].ensure(plane * 4);
                I.bits_host[size_t(p + k)].ensure(words * 4);
                OCR_HIP(hipMemcpyAsync(I.prob_host[size_t(p + k)].p, prob.p + size_t(k) * plane, plane * 4,
                                       hipMemcpyDeviceToHost, st));
                OCR_HIP(hipMemcpyAsync(I.bits_host[size_t(p + k)].p, bits.as<uint32_t>() + size_t(k) * words, words * 4,
                                       hipMemcpyDeviceToHost, st));
            }
            hipEvent_t ev;
            OCR_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
            events.push_back(ev);
            OCR_HIP(hipEventRecord(ev, st));
            // 2. Host DB boxes of each page of the pass as soon as its map is on the host.
            for (int k = p; k < q; k++) {
                {
                    std::lock_guard<std::mutex> lk(mu);
                    pending++;
                }
                const float *pr = static_cast<const float *>(I.prob_host[size_t(k)].p);
                const uint32_t *bt = static_cast<const uint32_t *>(I.bits_host[size_t(k)].p);
                const int pw = w[k], ph = h[k], mw = W, mh = H;
                I.workers.submit([&, k, ev, pr, bt, pw, ph, mw, mh, dev] {
                    std::string err;
                    double busy = 0;
                    try {
                        (void)hipSetDevice(dev);
                        wait_event(ev, "the probability map and mask of page " + std::to_string(k));
                        const auto tc = Clock::now();
                        PageBoxes B;
                        for (const RRect &r : db_boxes(bt, pr, mw, mh, float(pw) / float(mw), float(ph) / float(mh), I.opts.db))
                            B.lines.push_back(pp_line_box(r, I.opts.relv, pw, ph));
                        std::vector<int> ow_l;
                        for (const PpLine &l : B.lines) ow_l.push_back(l.out_w);
                        B.plan = plan_pp_batches(ow_l, I.opts.per_batch);
                        busy = ms_since(tc);
                        std::lock_guard<std::mutex> lk(mu);
                        boxes[size_t(k)] = std::move(B);
                        ready[size_t(k)] = 1;
                    } catch (const std::exception &e) {
                        err = e.what();
                        std::lock_guard<std::mutex> lk(mu);
                        ready[size_t(k)] = -1;
                    }
                    task_done(busy, err);
                });
            }
            p = q;
        }
        // 3. Recognition, `merge` pages a pass: every page's own batches (ocr-bench.rs:240-284).
        if (I.best_host.size() < size_t(nrec)) I.best_host.resize(size_t(nrec));
        for (int r = 0; r < nrec; r++) {
            const int p0 = r * I.opts.merge, p1 = std::min(npages, p0 + I.opts.merge);
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] {
                    for (int k = p0; k < p1; k++)
                        if (!ready[size_t(k)]) return false;
                    return true;
                });
                if (!error.empty()) break;
            }
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
                const PageBoxes &B = boxes[size_t(k)];
                pages_[size_t(k)].words = int(B.lines.size());
                pages_[size_t(k)].lines.assign(B.lines.size(), std::string());
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
                        crops.push_back({d_rgb[k], w[k], h[k], L.left, L.top, L.cw, L.ch, L.out_w,
                                         bt.in.p + size_t(j) * 3 * PP_LINE_H * wb, wb});
                        rows[size_t(r)].push_back({k, li, bt.steps, bt.best_off + size_t(j) * bt.steps});
                    }
                    batches.push_back(std::move(bt));
                }
            }
            stats_.batches += int(batches.size());
            if (batches.empty()) continue;
            DBuf dcrops(&ctx, crops.size() * sizeof(PpCropLine));
            ctx.h2d(dcrops.get(), crops.data(), crops.size() * sizeof(PpCropLine));
            pp_line_crop(dcrops.as<PpCropLine>(), int(crops.size()), max_wb, st);
            DBuf best(&ctx, best_total * 4);
            for (const Batch &bt : batches) I.rec.run_argmax(ctx, bt.in, best.as<uint32_t>() + bt.best_off, nullptr);
            I.best_host[size_t(r)].ensure(best_total * 4);
            OCR_HIP(hipMemcpyAsync(I.best_host[size_t(r)].p, best.get(), best_total * 4, hipMemcpyDeviceToHost, st));
            hipEvent_t ev;
            OCR_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
            events.push_back(ev);
            OCR_HIP(hipEventRecord(ev, st));
            stats_.rec_passes++;
            // 4. Greedy CTC on the host once the arg-max is back.
            {
                std::lock_guard<std::mutex> lk(mu);
                pending++;
            }
            const uint32_t *bh = static_cast<const uint32_t *>(I.best_host[size_t(r)].p);
            I.workers.submit([&, ev, bh, r, dev] {
                std::string err;
                double busy = 0;
                try {
                    (void)hipSetDevice(dev);
                    wait_event(ev, "the arg-max of recognition pass " + std::to_string(r));
                    const auto tc = Clock::now();
                    for (const Row &row : rows[size_t(r)])
                        pages_[size_t(row.page)].lines[size_t(row.line)] = pp_ctc_decode(bh + row.off, row.steps);
                    busy = ms_since(tc);
                } catch (const std::exception &e) {
                    err = e.what();
                }
                task_done(busy, err);
            });
        }
        for (const auto &rr : rows)
            for (const Row &row : rr) stats_.rec_steps += row.steps;
    } catch (const std::exception &e) {
        std::lock_guard<std::mutex> lk(mu);
        if (error.empty()) error = e.what();
    }
    {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return pending == 0; });
    }
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
    if (!error.empty()) fail("pp pipeline: " + error);
    ctx.sync();
    stats_.ms = ms_since(t0);
    stats_.cpu_busy_ms = cpu_busy;
    for (const PageText &pt : pages_) {
        stats_.lines += int(pt.lines.size());
        stats_.words += pt.words;
    }
}

}  // namespace ocr
