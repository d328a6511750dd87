#include "pipeline.h"

#include <algorithm>
#include <map>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <functional>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <thread>

#include "crop.h"
#include "host_util.h"

namespace ocr {

// Waits for a GPU event by polling every 20 microseconds: the worker threads waiting for
// detection or recognition results sleep instead of spinning, so the host cores go to the
// layouts; spin: yield between polls instead (the last pass, when no layout is left to run and
// a sleep's wake-up latency would add to the run).
static void wait_event(hipEvent_t ev, bool spin = false) {
    for (;;) {
        const hipError_t e = hipEventQuery(ev);
        if (e == hipSuccess) return;
        if (e != hipErrorNotReady) OCR_HIP(e);
        if (spin) std::this_thread::yield();
        else std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

PageLayout layout_page(const uint32_t *bits, int w, int h, float relv, float relend, int threads, int page_prio,
                       const MaskRows *rows) {
    set_loop_priority(page_prio);
    PageLayout L;
    std::vector<RRect> words =
        rows ? word_rects_from_rows(rows->comps, rows->ncomps, rows->xmin, rows->xmax, rows->nslots, 3.f, 100.f,
                                    threads)
             : word_rects(bits, w, h, 3.f, 100.f, threads);
    L.words = int(words.size());
    auto lines = find_text_lines(words);
    pad_lines(lines, relv, relend);
    lines.erase(std::remove_if(lines.begin(), lines.end(), [](const std::vector<RRect> &l) { return l.empty(); }),
                lines.end());
    L.lines.resize(lines.size());
    const int n = int(lines.size());
    if (threads <= 1) {
        for (int i = 0; i < n; i++) L.lines[size_t(i)] = line_geometry(lines[size_t(i)]);
    } else {
        LoopPool::get().run(n, [&](int i) { L.lines[size_t(i)] = line_geometry(lines[size_t(i)]); }, page_prio);
    }
    std::vector<int> out_w;
    for (const LineGeom &g : L.lines) out_w.push_back(g.out_w);
    L.plan = plan_batches(out_w);
    for (const LineGeom &g : L.lines) {
        L.line_row0.push_back(int32_t(L.row_off.size()));
        const int32_t sbase = int32_t(L.spans.size());
        for (int32_t o : g.row_off) L.row_off.push_back(o + sbase);
        L.spans.insert(L.spans.end(), g.spans.begin(), g.spans.end());
    }
    return L;
}


struct Pipeline::Impl {
    Ctx &ctx;
    Detector &det;
    Recognizer &rec;
    PipelineOpts opts;
    Workers workers;
    std::vector<Pinned> bits_host, best_host, runs_host;
    // The masks and labelled runs go to the host on a stream of their own, so the next
    // detection pass does not wait for the copies.
    hipStream_t copy = nullptr;
    // Host threads the layouts of one recognition pass share (a page's word boxes in row bands,
    // its lines side by side).
    int host_threads;
    explicit Impl(Ctx &c, Detector &d, Recognizer &r, const PipelineOpts &o, int nthreads)
        : ctx(c), det(d), rec(r), opts(o), workers(nthreads),
          host_threads(std::max(1, int(std::thread::hardware_concurrency()))) {
        ctx.bind();
        OCR_HIP(hipStreamCreateWithFlags(&copy, hipStreamNonBlocking));
    }
    ~Impl() {
        if (copy) {
            (void)hipStreamSynchronize(copy);
            (void)hipStreamDestroy(copy);
        }
    }
};

Pipeline::Pipeline(Ctx &ctx, Detector &det, Recognizer &rec, const PipelineOpts &opts)
    : impl_(new Impl(ctx, det, rec, opts, worker_count(opts.threads))) {
    if (opts.merge < 1 || opts.det_batch < 1) fail("pipeline: merge and det_batch must be at least 1");
}

Pipeline::~Pipeline() { delete impl_; }

void Pipeline::run(const uint8_t *const *d_rgb, const int *w, const int *h, int npages) {
    Impl &I = *impl_;
    Ctx &ctx = I.ctx;
    const hipStream_t st = ctx.stream();
    const auto t0 = Clock::now();
    pages_.assign(size_t(std::max(npages, 0)), PageText{});
    stats_ = PipelineStats{};
    stats_.pages = npages;
    if (npages <= 0) return;
    for (int p = 0; p < npages; p++)
        if (w[p] <= 0 || h[p] <= 0) fail("pipeline: empty page " + std::to_string(p));

    std::mutex mu;
    std::condition_variable cv;
    // OCR_PIPE_TRACE=1: host timestamps of the pipeline's steps, printed to stderr at the end.
    static const bool tracing = std::getenv("OCR_PIPE_TRACE") != nullptr;
    std::vector<std::pair<double, std::string>> trace;
    auto mark = [&](const std::string &what) {
        if (!tracing) return;
        std::lock_guard<std::mutex> lk(mu);
        trace.push_back({ms_since(t0), what});
    };
    std::vector<int> layout_ready(size_t(npages), 0);
    std::vector<PageLayout> layouts(static_cast<size_t>(npages));
    std::string error;
    double cpu_busy = 0;
    int pending_tasks = 0;
    auto task_done = [&](double busy, const std::string &err) {
        std::lock_guard<std::mutex> lk(mu);
        cpu_busy += busy;
        if (!err.empty() && error.empty()) error = err;
        pending_tasks--;
        cv.notify_all();
    };

    // Recognition passes of `merge` pages, in page order.
    std::vector<int> pass_p0;
    for (int p = 0; p < npages; p += I.opts.merge) pass_p0.push_back(p);
    pass_p0.push_back(npages);
    const int nrec = int(pass_p0.size()) - 1;
    // 1. Detection of every page in groups of at most det_batch pages (near-equal sizes) that
    // never straddle a recognition pass: the first pass's layouts then start while the later
    // pages are still being detected. The first group is a third of det_batch (at least one
    // page), so the host starts on layouts early. The bit masks come back asynchronously.
    std::vector<int> group_of(static_cast<size_t>(npages)), group_p0;
    for (int r = 0; r < nrec; r++) {
        int q0 = pass_p0[size_t(r)];
        const int r1 = pass_p0[size_t(r) + 1];
        if (r == 0 && r1 - q0 > 1) {
            const int first = std::min(r1 - q0, std::max(1, I.opts.det_batch / 3));
            group_p0.push_back(q0);
            for (int p = q0; p < q0 + first; p++) group_of[size_t(p)] = int(group_p0.size()) - 1;
            q0 += first;
        }
        const int ng = (r1 - q0 + I.opts.det_batch - 1) / I.opts.det_batch;
        for (int k = 0; k < ng; k++) {
            const int g0 = q0 + int(long(r1 - q0) * k / ng), g1 = q0 + int(long(r1 - q0) * (k + 1) / ng);
            group_p0.push_back(g0);
            for (int p = g0; p < g1; p++) group_of[size_t(p)] = int(group_p0.size()) - 1;
        }
    }
    const int ngroups = int(group_p0.size());
    std::vector<hipEvent_t> det_ev(size_t(ngroups), nullptr), ccl_ev(size_t(ngroups), nullptr);
    // Each detection pass's masks and runs on the device, kept until the run ends: the copy
    // stream reads them while the next passes run.
    std::vector<std::vector<DBuf>> keep_bits(static_cast<size_t>(ngroups)), keep_runs(static_cast<size_t>(ngroups));
    std::vector<hipEvent_t> rec_ev(size_t(nrec), nullptr), am_ev(size_t(nrec), nullptr);
    struct RecPass {
        std::vector<std::pair<int, int>> rows;  // (page, line in page) of every recogniser line
        std::vector<uint32_t> lens;
        std::vector<int> widths;
        int tmax = 0, ntot = 0;
        std::vector<CropLine> crops;
        std::vector<int32_t> row_off, spans;
        DBuf best;  // the arg-max classes, read by the copy to the host after the pass's kernels
    };
    std::vector<RecPass> passes(static_cast<size_t>(nrec));
    // Detection groups completed so far (set by the watcher thread below).
    int det_done = 0;
    struct Joiner {
        std::thread t;
        ~Joiner() {
            if (t.joinable()) t.join();
        }
    } watcher;
    // Worker tasks refer to the locals above: whatever happens, wait for them before returning.
    try {
    if (I.bits_host.size() < size_t(npages)) I.bits_host.resize(size_t(npages));
    if (I.runs_host.size() < size_t(npages)) I.runs_host.resize(size_t(npages));
    // Each page's labelled components (ccl_runs) in one device block, whose head goes to the
    // host: the totals (runs, components, row slots), the component records (RCOMPS of 16
    // bytes), each row slot's leftmost then rightmost pixel (RSLOTS of 4 bytes each). The runs
    // themselves (row offsets, roots, first and last pixels, rows, root bottoms; runs_cap each)
    // follow on the device only.
    constexpr int RCOMPS = 16384, RSLOTS = 65536;
    constexpr size_t HEAD = 16 + size_t(RCOMPS) * 16 + size_t(RSLOTS) * 8;
    std::vector<size_t> words_of(static_cast<size_t>(npages));
    std::vector<int> runs_cap(static_cast<size_t>(npages));
    auto roff_bytes = [&](int p) { return (size_t(h[p] + 1) * 4 + 15) & ~size_t(15); };
    auto block_bytes = [&](int p) { return HEAD + roff_bytes(p) + size_t(runs_cap[size_t(p)]) * 14; };
    for (int p = 0; p < npages; p++) {
        words_of[size_t(p)] = size_t((w[p] + 31) / 32) * h[p];
        I.bits_host[size_t(p)].ensure(words_of[size_t(p)] * 4);
        runs_cap[size_t(p)] = int(std::min<size_t>(words_of[size_t(p)] * 16, size_t(1) << 17));
        I.runs_host[size_t(p)].ensure(HEAD);
    }
    for (int g = 0; g < ngroups; g++) {
        const int p0 = group_p0[size_t(g)], p1 = g + 1 < ngroups ? group_p0[size_t(g) + 1] : npages;
        std::vector<DBuf> &bits = keep_bits[size_t(g)];
        std::vector<uint32_t *> bp;
        for (int p = p0; p < p1; p++) {
            bits.emplace_back(&ctx, words_of[size_t(p)] * 4);
            bp.push_back(bits.back().as<uint32_t>());
        }
        I.det.detect_pages_device(d_rgb + p0, w + p0, h + p0, p1 - p0, I.opts.thr, bp.data());
        std::vector<DBuf> &rbuf = keep_runs[size_t(g)];
        std::vector<CclPage> cp;
        for (int p = p0; p < p1; p++) {
            rbuf.emplace_back(&ctx, block_bytes(p));
            char *b = rbuf.back().as<char>();
            const size_t cap = size_t(runs_cap[size_t(p)]);
            char *comps = b + 16, *xmin = comps + size_t(RCOMPS) * 16, *xmax = xmin + size_t(RSLOTS) * 4;
            char *roff = b + HEAD, *root = roff + roff_bytes(p), *cbot = root + cap * 4;
            char *x0 = cbot + cap * 4, *x1 = x0 + cap * 2, *ry = x1 + cap * 2;
            CclPage pg{};
            pg.bits = bp[size_t(p - p0)], pg.w = w[p], pg.h = h[p];
            pg.x0 = reinterpret_cast<uint16_t *>(x0), pg.x1 = reinterpret_cast<uint16_t *>(x1);
            pg.root = reinterpret_cast<int32_t *>(root), pg.row_off = reinterpret_cast<int32_t *>(roff);
            pg.cap = int(cap), pg.total = reinterpret_cast<int32_t *>(b);
            pg.ry = reinterpret_cast<uint16_t *>(ry), pg.cbot = reinterpret_cast<int32_t *>(cbot);
            pg.comps = reinterpret_cast<int32_t *>(comps);
            pg.xmin = reinterpret_cast<uint32_t *>(xmin), pg.xmax = reinterpret_cast<uint32_t *>(xmax);
            pg.ccap = RCOMPS, pg.scap = RSLOTS;
            cp.push_back(pg);
        }
        ccl_runs(cp.data(), int(cp.size()), st);
        OCR_HIP(hipEventCreateWithFlags(&ccl_ev[size_t(g)], hipEventDisableTiming));
        OCR_HIP(hipEventRecord(ccl_ev[size_t(g)], st));
        OCR_HIP(hipStreamWaitEvent(I.copy, ccl_ev[size_t(g)], 0));
        for (int p = p0; p < p1; p++) {
            OCR_HIP(hipMemcpyAsync(I.bits_host[size_t(p)].p, bp[size_t(p - p0)], words_of[size_t(p)] * 4,
                                   hipMemcpyDeviceToHost, I.copy));
            OCR_HIP(hipMemcpyAsync(I.runs_host[size_t(p)].p, rbuf[size_t(p - p0)].get(), HEAD,
                                   hipMemcpyDeviceToHost, I.copy));
        }
        OCR_HIP(hipEventCreateWithFlags(&det_ev[size_t(g)], hipEventDisableTiming | hipEventBlockingSync));
        OCR_HIP(hipEventRecord(det_ev[size_t(g)], I.copy));
        mark("det group " + std::to_string(g) + " enqueued");
    }
    // One thread waits for the detection groups in order and wakes the layouts; the layout
    // tasks sleep meanwhile, so the host cores go to the layouts that can run.
    const int dev = ctx.device();
    watcher.t = std::thread([&, dev] {
        std::string err;
        try {
            (void)hipSetDevice(dev);
            for (int g = 0; g < ngroups; g++) {
                OCR_HIP(hipEventSynchronize(det_ev[size_t(g)]));
                std::lock_guard<std::mutex> lk(mu);
                det_done = g + 1;
                cv.notify_all();
            }
        } catch (const std::exception &e) {
            err = e.what();
        }
        std::lock_guard<std::mutex> lk(mu);
        if (!err.empty() && error.empty()) error = err;
        det_done = ngroups;
        cv.notify_all();
    });
    // 2. Host layout of each page once its mask is on the host and every page of the earlier
    // recognition passes is laid out; its loops run on the shared host loop pool, earlier pages
    // first.
    for (int p = 0; p < npages; p++) {
        {
            std::lock_guard<std::mutex> lk(mu);
            pending_tasks++;
        }
        const int grp = group_of[size_t(p)];
        const uint32_t *bits = static_cast<const uint32_t *>(I.bits_host[size_t(p)].p);
        const char *rblk = static_cast<const char *>(I.runs_host[size_t(p)].p);
        const int rcap = runs_cap[size_t(p)];
        const int pw = w[p], ph = h[p];
        int pr = 0;
        while (pass_p0[size_t(pr) + 1] <= p) pr++;
        const int before = pass_p0[size_t(pr)], threads = I.host_threads;
        I.workers.submit([&, p, grp, bits, rblk, rcap, pw, ph, dev, before, threads] {
            std::string err;
            double busy = 0;
            try {
                (void)hipSetDevice(dev);
                {
                    std::unique_lock<std::mutex> lk(mu);
                    cv.wait(lk, [&] {
                        if (!error.empty()) return true;
                        if (det_done <= grp) return false;
                        for (int q = 0; q < before; q++)
                            if (!layout_ready[size_t(q)]) return false;
                        return true;
                    });
                    if (!error.empty()) fail("an earlier step failed");
                }
                mark("layout " + std::to_string(p) + " start");
                const auto tc = Clock::now();
                // The GPU's labelled components unless the page had more runs, components or
                // row slots than the buffers hold.
                const int32_t *tot = reinterpret_cast<const int32_t *>(rblk);
                const char *comps = rblk + 16, *xmin = comps + size_t(RCOMPS) * 16;
                const MaskRows mr{reinterpret_cast<const int32_t *>(comps), tot[1],
                                  reinterpret_cast<const uint32_t *>(xmin),
                                  reinterpret_cast<const uint32_t *>(xmin + size_t(RSLOTS) * 4), tot[2]};
                const bool fits = tot[0] <= rcap && tot[1] <= RCOMPS && tot[2] <= RSLOTS;
                PageLayout L = layout_page(bits, pw, ph, I.opts.relv, I.opts.relend, threads, p, fits ? &mr : nullptr);
                busy = ms_since(tc);
                mark("layout " + std::to_string(p) + " done");
                std::lock_guard<std::mutex> lk(mu);
                layouts[size_t(p)] = std::move(L);
                layout_ready[size_t(p)] = 1;
            } catch (const std::exception &e) {
                err = e.what();
                std::lock_guard<std::mutex> lk(mu);
                layout_ready[size_t(p)] = -1;
            }
            task_done(busy, err);
        });
    }
    // 3. Recognition, pass by pass in page order.
    if (I.best_host.size() < size_t(nrec)) I.best_host.resize(size_t(nrec));
    for (int r = 0; r < nrec; r++) {
        const int p0 = pass_p0[size_t(r)], p1 = pass_p0[size_t(r) + 1];
        {
            std::unique_lock<std::mutex> lk(mu);
            cv.wait(lk, [&] {
                for (int p = p0; p < p1; p++)
                    if (!layout_ready[size_t(p)]) return false;
                return true;
            });
            if (!error.empty()) break;
        }
        mark("rec " + std::to_string(r) + " layouts ready");
        RecPass &R = passes[size_t(r)];
        // A line's recognition depends on its batch's width (the padding), not on which lines
        // share the batch, so every page's batches of one width run as one trunk batch: the
        // same results with fewer, fuller launches. Widths ascending, pages and batches in order.
        std::map<int, std::vector<std::pair<int, int>>> by_width;  // width -> (page, line)
        // The pages' row offsets and spans, appended page by page (offsets rebased).
        std::vector<int> page_row0(size_t(p1 - p0));
        for (int p = p0; p < p1; p++) {
            const PageLayout &L = layouts[size_t(p)];
            page_row0[size_t(p - p0)] = int(R.row_off.size());
            const int32_t sbase = int32_t(R.spans.size());
            const size_t r0 = R.row_off.size();
            R.row_off.resize(r0 + L.row_off.size());
            for (size_t k = 0; k < L.row_off.size(); k++) R.row_off[r0 + k] = L.row_off[k] + sbase;
            R.spans.insert(R.spans.end(), L.spans.begin(), L.spans.end());
        }
        for (int p = p0; p < p1; p++) {
            const PageLayout &L = layouts[size_t(p)];
            pages_[size_t(p)].words = L.words;
            pages_[size_t(p)].lines.assign(L.lines.size(), std::string());
            for (size_t b = 0; b < L.plan.lines.size(); b++) {
                stats_.batches++;
                for (int li : L.plan.lines[b]) by_width[L.plan.width[b]].push_back({p, li});
            }
        }
        std::vector<Recognizer::Batch> batches;
        std::vector<DBuf> batch_bufs;
        for (const auto &kv : by_width) {
            const int wb = kv.first, n = int(kv.second.size());
            batch_bufs.emplace_back(&ctx, size_t(n) * LINE_H * wb * sizeof(float));
            float *base = batch_bufs.back().as<float>();
            batches.push_back({base, n, wb});
            for (int k = 0; k < n; k++) {
                const int p = kv.second[size_t(k)].first, li = kv.second[size_t(k)].second;
                const PageLayout &L = layouts[size_t(p)];
                const LineGeom &g = L.lines[size_t(li)];
                CropLine c{d_rgb[p], w[p], h[p], g.left, g.top, g.bw, g.bh, g.out_w,
                           page_row0[size_t(p - p0)] + L.line_row0[size_t(li)], base + size_t(k) * LINE_H * wb, wb};
                R.crops.push_back(c);
                R.rows.push_back({p, li});
                R.widths.push_back(g.out_w);
            }
        }
        if (batches.empty()) continue;
        mark("rec " + std::to_string(r) + " crops built");
        line_crop(ctx, R.crops, R.row_off, R.spans, st);
        const Recognizer::Dims d = I.rec.dims(batches.data(), int(batches.size()));
        R.tmax = d.tmax;
        R.ntot = d.ntot;
        R.lens.assign(size_t(d.ntot), 0);
        DBuf logits(&ctx, size_t(d.tmax) * d.ntot * d.classes * sizeof(float));
        R.best = DBuf(&ctx, size_t(d.tmax) * d.ntot * sizeof(uint32_t));
        I.rec.recognize_device(batches.data(), int(batches.size()), logits.as<float>(), R.best.as<uint32_t>(),
                               R.lens.data());
        mark("rec " + std::to_string(r) + " enqueued");
        // The arg-max goes to the host on the copy stream, so the next pass's kernels do not
        // wait for the copy.
        I.best_host[size_t(r)].ensure(size_t(d.tmax) * d.ntot * sizeof(uint32_t));
        OCR_HIP(hipEventCreateWithFlags(&am_ev[size_t(r)], hipEventDisableTiming));
        OCR_HIP(hipEventRecord(am_ev[size_t(r)], st));
        OCR_HIP(hipStreamWaitEvent(I.copy, am_ev[size_t(r)], 0));
        OCR_HIP(hipMemcpyAsync(I.best_host[size_t(r)].p, R.best.get(), size_t(d.tmax) * d.ntot * sizeof(uint32_t),
                               hipMemcpyDeviceToHost, I.copy));
        OCR_HIP(hipEventCreateWithFlags(&rec_ev[size_t(r)], hipEventDisableTiming));
        OCR_HIP(hipEventRecord(rec_ev[size_t(r)], I.copy));
        stats_.rec_passes++;
        // 4. Greedy CTC on the host once the arg-max is back.
        {
            std::lock_guard<std::mutex> lk(mu);
            pending_tasks++;
        }
        hipEvent_t ev = rec_ev[size_t(r)];
        const uint32_t *bh = static_cast<const uint32_t *>(I.best_host[size_t(r)].p);
        const bool last = r == nrec - 1;
        I.workers.submit([&, ev, bh, r, dev, last] {
            std::string err;
            double busy = 0;
            try {
                (void)hipSetDevice(dev);
                wait_event(ev, last);
                mark("ctc " + std::to_string(r) + " start");
                const auto tc = Clock::now();
                const RecPass &R2 = passes[size_t(r)];
                // Lines in chunks on the loop pool (each line's text has a slot of its own).
                const int nl = int(R2.rows.size()), chunks = std::min(nl, 32);
                LoopPool::get().run(chunks, [&](int c) {
                    for (int j = int(long(nl) * c / chunks); j < int(long(nl) * (c + 1) / chunks); j++) {
                        std::string s = ctc_decode(bh + j, int(R2.lens[size_t(j)]), R2.ntot, R2.widths[size_t(j)]);
                        pages_[size_t(R2.rows[size_t(j)].first)].lines[size_t(R2.rows[size_t(j)].second)] = std::move(s);
                    }
                }, -1);
                busy = ms_since(tc);
                mark("ctc " + std::to_string(r) + " done");
            } catch (const std::exception &e) {
                err = e.what();
            }
            task_done(busy, err);
        });
    }
    } catch (const std::exception &e) {
        std::lock_guard<std::mutex> lk(mu);
        if (error.empty()) error = e.what();
    }
    {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return pending_tasks == 0; });
    }
    mark("tasks done");
    (void)hipStreamSynchronize(I.copy);
    for (hipEvent_t e : det_ev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : ccl_ev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : rec_ev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : am_ev)
        if (e) (void)hipEventDestroy(e);
    if (!error.empty()) fail("pipeline: " + error);
    ctx.sync();
    stats_.ms = ms_since(t0);
    if (tracing) {
        mark("end");
        std::sort(trace.begin(), trace.end());
        for (const auto &e : trace) std::fprintf(stderr, "[pipe] %8.3f ms  %s\n", e.first, e.second.c_str());
    }
    stats_.cpu_busy_ms = cpu_busy;
    for (const PageText &pt : pages_) {
        stats_.lines += int(pt.lines.size());
        stats_.words += pt.words;
    }
    for (const RecPass &R : passes)
        for (uint32_t l : R.lens) stats_.rec_steps += l;
}

}  // namespace ocr
