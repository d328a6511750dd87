#include "pipeline.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <map>
#include <condition_variable>
#include <deque>
#include <functional>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>

#include "crop.h"
#include "host_util.h"
#include "pipeline_core.h"
#include "upload.h"

namespace ocr {

// Worker threads wait for detection and recognition results with wait_event (runtime.h): after a
// short yielding phase they sleep between polls, so the host cores go to the layouts; the last
// pass's wait keeps yielding (a sleep's wake-up would add to the run). Every wait is bounded.

PageLayout layout_page(const uint32_t *bits, int w, int h, float relv, float relend, int threads, int page_prio,
                       const MaskRows *rows) {
    set_loop_priority(page_prio);
    PageLayout L;
    const auto t0 = Clock::now();
    std::vector<RRect> words =
        rows ? word_rects_from_rows(bits, w, h, rows->comps, rows->ncomps, rows->xmin, rows->xmax, rows->nslots, 3.f,
                                    100.f, threads)
             : word_rects(bits, w, h, 3.f, 100.f, threads);
    L.words = int(words.size());
    L.ms_words = ms_since(t0);
    const auto t1 = Clock::now();
    auto lines = find_text_lines(words);
    pad_lines(lines, relv, relend);
    L.ms_lines = ms_since(t1);
    const auto t2 = Clock::now();
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
    L.ms_geom = ms_since(t2);
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
    // detection group does not wait for the copies; pages handed over in host memory go to the
    // device on the uploader's. Detection and recognition share the context's stream: their
    // kernels take every CU (persistent workgroups), so running them side by side only slows
    // both.
    hipStream_t copy = nullptr;
    // The recurrences of a recognition pass run on a stream of their own when pages come from host
    // memory: a recurrence occupies one CU per 8 lines and direction (a third to a half of the GPU
    // at the bench's passes), and the detection groups queued between the pass's stages run on
    // the rest of the CUs meanwhile.
    hipStream_t gru = nullptr;
    PageUploader upl;
    hipStream_t up;
    // Host threads the layouts of one recognition pass share (a page's word boxes in row bands,
    // its lines side by side).
    int host_threads;
    explicit Impl(Ctx &c, Detector &d, Recognizer &r, const PipelineOpts &o, int nthreads)
        : ctx(c), det(d), rec(r), opts(o), workers(nthreads), upl(c), up(upl.stream()),
          host_threads(std::max(1, int(std::thread::hardware_concurrency()))) {
        ctx.bind();
        OCR_HIP(hipStreamCreateWithFlags(&copy, hipStreamNonBlocking));
        OCR_HIP(hipStreamCreateWithFlags(&gru, hipStreamNonBlocking));
    }
    ~Impl() {
        if (gru) {
            drain_stream(gru, "the pipeline's recurrence stream");
            (void)hipStreamDestroy(gru);
        }
        if (copy) {
            drain_stream(copy, "the pipeline's copy stream");
            ctx.pool().retire_stream(copy);
            (void)hipStreamDestroy(copy);
        }
    }
    void upload(uint8_t *dst, const uint8_t *src, size_t bytes, bool pinned) { upl.upload(dst, src, bytes, pinned); }
};

Pipeline::Pipeline(Ctx &ctx, Detector &det, Recognizer &rec, const PipelineOpts &opts)
    : impl_(new Impl(ctx, det, rec, opts, worker_count(opts.threads))) {
    if (opts.merge < 1 || opts.det_batch < 1) fail("pipeline: merge and det_batch must be at least 1");
}

Pipeline::~Pipeline() { delete impl_; }

namespace {

// Each page's labelled components (ccl_runs) in one device block, whose head goes to the host:
// the totals (runs, components, row slots), the component records (16 bytes each), each row
// slot's leftmost then rightmost pixel (4 bytes each). The runs themselves (row offsets, roots,
// first and last pixels, rows, root bottoms) follow on the device only.
struct LabelCaps {
    int runs, comps, slots;
    size_t head() const { return 16 + size_t(comps) * 16 + size_t(slots) * 8; }
};

}  // namespace

// One run of the pipeline: the hooks of the schedule (pipeline_core.h) on this GPU.
struct PipelineRun final : PipelineHooks {
    Pipeline::Impl &I;
    Ctx &ctx;
    hipStream_t st;
    const PipelinePlan &P;
    const uint8_t *const *src;  // the pages: device pointers, or host pointers when on_host
    bool on_host;
    const int *w, *h;
    std::vector<PageText> &pages;
    LabelCaps caps;
    const Clock::time_point t0;
    // OCR_PIPE_TRACE=1: host timestamps of the steps, printed to stderr at the end.
    bool tracing;
    bool interleave = false;  // recognition passes queued in stages, detections between them
    // OCR_PIPE_FAIL_LAYOUT=p: page p's layout fails (tests of the per-page error path).
    int fail_layout = -1;
    // With tracing: GPU timestamps (events on the streams) of each upload group, detection group
    // and recognition pass, against one taken at the start on the compute stream.
    hipEvent_t gpu_t0 = nullptr;
    std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> gpu_marks;
    hipEvent_t gpu_event(hipStream_t s) {
        hipEvent_t e = nullptr;
        if (!tracing) return e;
        OCR_HIP(hipEventCreate(&e));
        OCR_HIP(hipEventRecord(e, s));
        return e;
    }
    void gpu_span(const std::string &what, hipEvent_t a, hipEvent_t b) {
        if (!tracing) return;
        std::lock_guard<std::mutex> lk(trace_mu);
        gpu_marks.push_back({what, {a, b}});
    }
    std::mutex trace_mu;
    std::vector<std::pair<double, std::string>> trace;

    // Device pages (host mode: uploaded here), each group's upload event.
    std::vector<DBuf> dpages;
    std::vector<const uint8_t *> d_rgb;
    std::vector<char> pinned;
    std::vector<hipEvent_t> up_ev, det_ev;
    // Each detection group's masks and runs on the device, kept until the run ends: the copy
    // stream reads them while the next groups run.
    std::vector<std::vector<DBuf>> keep_bits, keep_runs;
    std::vector<size_t> words_of;
    std::vector<int> runs_cap;
    // Pages whose mask the GPU labels (the labelling stores columns and rows as 16 bits): the
    // others are labelled on the host from their bits.
    std::vector<char> gpu_label;
    std::atomic<int> host_labelled{0};
    std::vector<PageLayout> layouts;
    struct RecPass {
        std::vector<std::pair<int, int>> rows;  // (page, line in page) of every recogniser line
        std::vector<uint32_t> lens;
        std::vector<int> widths;
        int tmax = 0, ntot = 0;
        std::vector<CropLine> crops;
        std::vector<int32_t> row_off, spans;
        DBuf best;  // the arg-max classes, read by the copy to the host after the pass's kernels
        std::vector<DBuf> batch_bufs;
        hipEvent_t done = nullptr;
    };
    std::vector<RecPass> passes;
    int batches = 0, rec_passes = 0;

    PipelineRun(Pipeline::Impl &impl, const PipelinePlan &plan, const uint8_t *const *pages_src, bool host,
                const int *pw, const int *ph, std::vector<PageText> &out)
        : I(impl), ctx(impl.ctx), st(impl.ctx.stream()), P(plan), src(pages_src), on_host(host), w(pw), h(ph),
          pages(out), t0(Clock::now()) {
        tracing = std::getenv("OCR_PIPE_TRACE") != nullptr;
        if (const char *f = std::getenv("OCR_PIPE_FAIL_LAYOUT")) fail_layout = std::atoi(f);
        if (tracing) {
            OCR_HIP(hipEventCreate(&gpu_t0));
            OCR_HIP(hipEventRecord(gpu_t0, st));
            OCR_HIP(hipStreamWaitEvent(I.up, gpu_t0, 0));
        }
        const int np = P.npages, ng = P.groups();
        caps.runs = I.opts.label_runs > 0 ? I.opts.label_runs : 1 << 17;
        caps.comps = I.opts.label_comps > 0 ? I.opts.label_comps : 16384;
        caps.slots = I.opts.label_slots > 0 ? I.opts.label_slots : 65536;
        up_ev.assign(size_t(ng), nullptr);
        det_ev.assign(size_t(ng), nullptr);
        keep_bits.resize(size_t(ng));
        keep_runs.resize(size_t(ng));
        layouts.resize(size_t(np));
        passes.resize(size_t(P.passes()));
        if (I.bits_host.size() < size_t(np)) I.bits_host.resize(size_t(np));
        if (I.runs_host.size() < size_t(np)) I.runs_host.resize(size_t(np));
        if (I.best_host.size() < size_t(P.passes())) I.best_host.resize(size_t(P.passes()));
        words_of.resize(size_t(np));
        runs_cap.resize(size_t(np));
        gpu_label.resize(size_t(np));
        for (int p = 0; p < np; p++) {
            gpu_label[size_t(p)] = w[p] <= 65536 && h[p] <= 65536;
            words_of[size_t(p)] = size_t((w[p] + 31) / 32) * h[p];
            I.bits_host[size_t(p)].ensure(words_of[size_t(p)] * 4);
            runs_cap[size_t(p)] = int(std::min<size_t>(words_of[size_t(p)] * 16, size_t(caps.runs)));
            I.runs_host[size_t(p)].ensure(caps.head());
        }
        // Host pages: every page's device buffer now, before this run queues any work, so the
        // uploads never wait for this run's kernels.
        d_rgb.resize(size_t(np));
        if (on_host) {
            pinned.resize(size_t(np));
            for (int p = 0; p < np; p++) {
                dpages.emplace_back(&ctx, size_t(w[p]) * h[p] * 3, I.up);
                dpages.back().used_on(st);
                d_rgb[size_t(p)] = dpages.back().as<uint8_t>();
                pinned[size_t(p)] = host_pinned(src[p]);
            }
        } else {
            for (int p = 0; p < np; p++) d_rgb[size_t(p)] = src[p];
        }
    }
    ~PipelineRun() override {
        // Nothing may still use the run's buffers once they go back to the pool.
        drain_stream(I.up, "a finished run's uploads");
        drain_stream(I.copy, "a finished run's copies to the host");
        drain_stream(st, "a finished run's kernels");
        for (hipEvent_t e : up_ev)
            if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : det_ev)
            if (e) (void)hipEventDestroy(e);
        for (RecPass &R : passes)
            if (R.done) (void)hipEventDestroy(R.done);
        if (gpu_t0) (void)hipEventDestroy(gpu_t0);
    }
    void mark(const std::string &what) {
        if (!tracing) return;
        std::lock_guard<std::mutex> lk(trace_mu);
        trace.push_back({ms_since(t0), what});
    }
    void print_trace() {
        if (!tracing) return;
        (void)hipDeviceSynchronize();
        for (auto &m : gpu_marks) {
            float a = 0, b = 0;
            (void)hipEventElapsedTime(&a, gpu_t0, m.second.first);
            (void)hipEventElapsedTime(&b, gpu_t0, m.second.second);
            char buf[160];
            std::snprintf(buf, sizeof buf, "GPU %s: %.3f .. %.3f ms", m.first.c_str(), a, b);
            trace.push_back({double(a), buf});
            (void)hipEventDestroy(m.second.first);
            (void)hipEventDestroy(m.second.second);
        }
        gpu_marks.clear();
        mark("end");
        std::sort(trace.begin(), trace.end());
        for (const auto &e : trace) std::fprintf(stderr, "[pipe] %8.3f ms  %s\n", e.first, e.second.c_str());
    }
    size_t roff_bytes(int p) const { return (size_t(h[p] + 1) * 4 + 15) & ~size_t(15); }
    size_t block_bytes(int p) const { return caps.head() + roff_bytes(p) + size_t(runs_cap[size_t(p)]) * 14; }

    void stage(int g) override {
        const int p0 = P.group_p0[size_t(g)], p1 = P.group_p0[size_t(g) + 1];
        if (!on_host) return;
        ctx.bind();
        mark("stage " + std::to_string(g) + " start");
        hipEvent_t ga = gpu_event(I.up);
        for (int p = p0; p < p1; p++)
            I.upload(dpages[size_t(p)].as<uint8_t>(), src[p], size_t(w[p]) * h[p] * 3, pinned[size_t(p)] != 0);
        gpu_span("upload " + std::to_string(g), ga, gpu_event(I.up));
        OCR_HIP(hipEventCreateWithFlags(&up_ev[size_t(g)], hipEventDisableTiming));
        OCR_HIP(hipEventRecord(up_ev[size_t(g)], I.up));
        mark("stage " + std::to_string(g) + " queued");
    }

    bool landed(int g) override {
        const hipEvent_t e = up_ev[size_t(g)];
        return !e || event_query(e, true);
    }

    // Detection of a group's pages, the labelling of their masks, and the copies of masks and
    // labels to the host (on the copy stream).
    void detect(int g) override {
        const int p0 = P.group_p0[size_t(g)], p1 = P.group_p0[size_t(g) + 1];
        const hipStream_t ds = st;
        if (up_ev[size_t(g)]) OCR_HIP(hipStreamWaitEvent(ds, up_ev[size_t(g)], 0));
        hipEvent_t ga = gpu_event(ds);
        std::vector<DBuf> &bits = keep_bits[size_t(g)];
        std::vector<uint32_t *> bp;
        for (int p = p0; p < p1; p++) {
            bits.emplace_back(&ctx, words_of[size_t(p)] * 4);
            bits.back().used_on(I.copy);
            bp.push_back(bits.back().as<uint32_t>());
        }
        mark("det group " + std::to_string(g) + " model");
        I.det.detect_pages_device(d_rgb.data() + p0, w + p0, h + p0, p1 - p0, I.opts.thr, bp.data());
        mark("det group " + std::to_string(g) + " labels");
        std::vector<DBuf> &rbuf = keep_runs[size_t(g)];
        std::vector<CclPage> cp;
        for (int p = p0; p < p1; p++) {
            if (!gpu_label[size_t(p)]) {
                rbuf.emplace_back();
                continue;
            }
            rbuf.emplace_back(&ctx, block_bytes(p));
            rbuf.back().used_on(I.copy);
            char *b = rbuf.back().as<char>();
            const size_t cap = size_t(runs_cap[size_t(p)]);
            char *comps = b + 16, *xmin = comps + size_t(caps.comps) * 16, *xmax = xmin + size_t(caps.slots) * 4;
            char *roff = b + caps.head(), *root = roff + roff_bytes(p), *cbot = root + cap * 4;
            char *x0 = cbot + cap * 4, *x1 = x0 + cap * 2, *ry = x1 + cap * 2;
            CclPage pg{};
            pg.bits = bp[size_t(p - p0)], pg.w = w[p], pg.h = h[p];
            pg.x0 = reinterpret_cast<uint16_t *>(x0), pg.x1 = reinterpret_cast<uint16_t *>(x1);
            pg.root = reinterpret_cast<int32_t *>(root), pg.row_off = reinterpret_cast<int32_t *>(roff);
            pg.cap = int(cap), pg.total = reinterpret_cast<int32_t *>(b);
            pg.ry = reinterpret_cast<uint16_t *>(ry), pg.cbot = reinterpret_cast<int32_t *>(cbot);
            pg.comps = reinterpret_cast<int32_t *>(comps);
            pg.xmin = reinterpret_cast<uint32_t *>(xmin), pg.xmax = reinterpret_cast<uint32_t *>(xmax);
            pg.ccap = caps.comps, pg.scap = caps.slots;
            cp.push_back(pg);
        }
        ccl_runs(cp.data(), int(cp.size()), ds);
        gpu_span("detect " + std::to_string(g), ga, gpu_event(ds));
        hipEvent_t ready = nullptr;
        OCR_HIP(hipEventCreateWithFlags(&ready, hipEventDisableTiming));
        OCR_HIP(hipEventRecord(ready, ds));
        OCR_HIP(hipStreamWaitEvent(I.copy, ready, 0));
        OCR_HIP(hipEventDestroy(ready));  // the wait above holds what it needs
        for (int p = p0; p < p1; p++) {
            OCR_HIP(hipMemcpyAsync(I.bits_host[size_t(p)].p, bp[size_t(p - p0)], words_of[size_t(p)] * 4,
                                   hipMemcpyDeviceToHost, I.copy));
            if (gpu_label[size_t(p)])
                OCR_HIP(hipMemcpyAsync(I.runs_host[size_t(p)].p, rbuf[size_t(p - p0)].get(), caps.head(),
                                       hipMemcpyDeviceToHost, I.copy));
        }
        OCR_HIP(hipEventCreateWithFlags(&det_ev[size_t(g)], hipEventDisableTiming | hipEventBlockingSync));
        OCR_HIP(hipEventRecord(det_ev[size_t(g)], I.copy));
        mark("det group " + std::to_string(g) + " queued");
    }

    void detect_wait(int g) override {
        ctx.bind();
        // The last group's result is on the run's critical path and the layouts before it are
        // done by then: poll it (yielding) rather than sleep in the blocking wait.
        wait_event(det_ev[size_t(g)], "detection group " + std::to_string(g) + " of " + std::to_string(P.groups()),
                   g + 1 == P.groups());
        mark("det group " + std::to_string(g) + " done");
    }

    // Words, lines and line geometry of page p on the host, from its mask's labelled components
    // (the GPU's, unless the page had more runs, components or row slots than the buffers hold:
    // then from the bits).
    void layout(int p) override {
        ctx.bind();
        mark("layout " + std::to_string(p) + " start");
        const uint32_t *bits = static_cast<const uint32_t *>(I.bits_host[size_t(p)].p);
        const char *rblk = static_cast<const char *>(I.runs_host[size_t(p)].p);
        const int32_t *tot = reinterpret_cast<const int32_t *>(rblk);
        const char *comps = rblk + 16, *xmin = comps + size_t(caps.comps) * 16;
        const MaskRows mr{reinterpret_cast<const int32_t *>(comps), tot[1], reinterpret_cast<const uint32_t *>(xmin),
                          reinterpret_cast<const uint32_t *>(xmin + size_t(caps.slots) * 4), tot[2]};
        const bool fits = gpu_label[size_t(p)] && tot[0] <= runs_cap[size_t(p)] && tot[1] <= caps.comps &&
                          tot[2] <= caps.slots;
        if (!fits) host_labelled++;
        layouts[size_t(p)] = layout_page(bits, w[p], h[p], I.opts.relv, I.opts.relend, I.host_threads, p,
                                         fits ? &mr : nullptr);
        if (p == fail_layout) fail("layout of page " + std::to_string(p) + " failed (injected)");
        if (tracing) {
            const PageLayout &L = layouts[size_t(p)];
            char buf[128];
            std::snprintf(buf, sizeof buf, "layout %d done (words %.3f, lines %.3f, geometry %.3f ms)", p, L.ms_words,
                          L.ms_lines, L.ms_geom);
            mark(buf);
        }
    }

    // Line images and recognition of pass r's laid-out pages, and the arg-max copy to the host.
    void recognize(int r, const std::vector<char> &ok) override {
        const int p0 = P.pass_p0[size_t(r)], p1 = P.pass_p0[size_t(r) + 1];
        RecPass &R = passes[size_t(r)];
        mark("rec " + std::to_string(r) + " layouts ready");
        // The line crops read the pages: after their uploads (long done: their masks were on the
        // host before the layouts ran, but the streams say so too).
        for (int g = P.group_of[size_t(p0)]; g <= P.group_of[size_t(p1 - 1)]; g++)
            if (up_ev[size_t(g)]) OCR_HIP(hipStreamWaitEvent(st, up_ev[size_t(g)], 0));
        // A line's recognition depends on its batch's width (the padding), not on which lines
        // share the batch, so every page's batches of one width run as one trunk batch: the
        // same results with fewer, fuller launches. Widths ascending, pages and batches in order.
        std::map<int, std::vector<std::pair<int, int>>> by_width;  // width -> (page, line)
        // The pages' row offsets and spans, appended page by page (offsets rebased).
        std::vector<int> page_row0(size_t(p1 - p0));
        for (int p = p0; p < p1; p++) {
            if (!ok[size_t(p - p0)]) continue;
            const PageLayout &L = layouts[size_t(p)];
            page_row0[size_t(p - p0)] = int(R.row_off.size());
            const int32_t sbase = int32_t(R.spans.size());
            const size_t r0 = R.row_off.size();
            R.row_off.resize(r0 + L.row_off.size());
            for (size_t k = 0; k < L.row_off.size(); k++) R.row_off[r0 + k] = L.row_off[k] + sbase;
            R.spans.insert(R.spans.end(), L.spans.begin(), L.spans.end());
        }
        for (int p = p0; p < p1; p++) {
            if (!ok[size_t(p - p0)]) continue;
            const PageLayout &L = layouts[size_t(p)];
            pages[size_t(p)].words = L.words;
            pages[size_t(p)].lines.assign(L.lines.size(), std::string());
            for (size_t b = 0; b < L.plan.lines.size(); b++) {
                batches++;
                for (int li : L.plan.lines[b]) by_width[L.plan.width[b]].push_back({p, li});
            }
        }
        std::vector<Recognizer::Batch> rb;
        for (const auto &kv : by_width) {
            const int wb = kv.first, n = int(kv.second.size());
            R.batch_bufs.emplace_back(&ctx, size_t(n) * LINE_H * wb * sizeof(float));
            float *base = R.batch_bufs.back().as<float>();
            rb.push_back({base, n, wb});
            for (int k = 0; k < n; k++) {
                const int p = kv.second[size_t(k)].first, li = kv.second[size_t(k)].second;
                const PageLayout &L = layouts[size_t(p)];
                const LineGeom &g = L.lines[size_t(li)];
                CropLine c{d_rgb[size_t(p)], w[p], h[p], g.left, g.top, g.bw, g.bh, g.out_w,
                           page_row0[size_t(p - p0)] + L.line_row0[size_t(li)], base + size_t(k) * LINE_H * wb, wb};
                R.crops.push_back(c);
                R.rows.push_back({p, li});
                R.widths.push_back(g.out_w);
            }
        }
        if (rb.empty()) return;
        mark("rec " + std::to_string(r) + " crops built");
        hipEvent_t ga = gpu_event(st);
        line_crop(ctx, R.crops, R.row_off, R.spans, st);
        const Recognizer::Dims d = I.rec.dims(rb.data(), int(rb.size()));
        R.tmax = d.tmax;
        R.ntot = d.ntot;
        R.lens.assign(size_t(d.ntot), 0);
        DBuf logits(&ctx, size_t(d.tmax) * d.ntot * d.classes * sizeof(float));
        R.best = DBuf(&ctx, size_t(d.tmax) * d.ntot * sizeof(uint32_t));
        R.best.used_on(I.copy);
        // Between the recogniser's stages (trunk, each GRU layer): the groups staged meanwhile
        // are queued right behind the stage just queued, and the next stage waits until the one
        // before it has finished, so at most one stage is ahead of a group that lands late.
        std::vector<hipEvent_t> stage_ev;
        auto between = [&]() {
            if (!interleave) return;
            hipEvent_t e = nullptr;
            OCR_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
            OCR_HIP(hipEventRecord(e, st));
            stage_ev.push_back(e);
            if (poll_detections) poll_detections();
            // With a detection group still to come, wait for the stage just queued (a group
            // staged meanwhile then runs right after it); otherwise for the one before it, so the
            // stage just queued keeps the GPU busy while the next one is queued.
            const bool pending = detections_pending && detections_pending();
            if (!pending && stage_ev.size() < 2) return;
            const size_t k = pending ? stage_ev.size() - 1 : stage_ev.size() - 2;
            const hipEvent_t prev = stage_ev[k];
            wait_until(
                [&] {
                    const hipError_t q = hipEventQuery(prev);
                    if (q == hipSuccess) return true;
                    if (q != hipErrorNotReady) OCR_HIP(q);
                    if (poll_detections) poll_detections();
                    return false;
                },
                [&] {
                    return "stage " + std::to_string(k) + " of recognition pass " + std::to_string(r) +
                           " on the compute stream";
                });
        };
        // With host pages the pass ends on the recurrence stream (its second recurrence, output
        // layer and arg-max), and the next pass's trunk may start beside it.
        const hipStream_t tail = interleave ? I.gru : st;
        if (tail != st) {
            logits.used_on(tail);
            R.best.used_on(tail);
        }
        I.rec.recognize_device(rb.data(), int(rb.size()), logits.as<float>(), R.best.as<uint32_t>(), R.lens.data(),
                               between, interleave ? I.gru : nullptr);
        for (hipEvent_t e : stage_ev) OCR_HIP(hipEventDestroy(e));
        gpu_span("recognize " + std::to_string(r), ga, gpu_event(tail));
        mark("rec " + std::to_string(r) + " queued");
        // The arg-max goes to the host on the copy stream, so the next pass's kernels do not
        // wait for the copy.
        I.best_host[size_t(r)].ensure(size_t(d.tmax) * d.ntot * sizeof(uint32_t));
        hipEvent_t am = nullptr;
        OCR_HIP(hipEventCreateWithFlags(&am, hipEventDisableTiming));
        OCR_HIP(hipEventRecord(am, tail));
        OCR_HIP(hipStreamWaitEvent(I.copy, am, 0));
        OCR_HIP(hipEventDestroy(am));
        OCR_HIP(hipMemcpyAsync(I.best_host[size_t(r)].p, R.best.get(), size_t(d.tmax) * d.ntot * sizeof(uint32_t),
                               hipMemcpyDeviceToHost, I.copy));
        OCR_HIP(hipEventCreateWithFlags(&R.done, hipEventDisableTiming));
        OCR_HIP(hipEventRecord(R.done, I.copy));
        rec_passes++;
    }

    // Greedy CTC of pass r on the host once its arg-max is there.
    void decode(int r, bool last) override {
        ctx.bind();
        const RecPass &R = passes[size_t(r)];
        if (!R.done) return;
        wait_event(R.done, "recognition pass " + std::to_string(r) + " and its arg-max copy", last);
        mark("ctc " + std::to_string(r) + " start");
        const uint32_t *bh = static_cast<const uint32_t *>(I.best_host[size_t(r)].p);
        // Lines in chunks on the loop pool (each line's text has a slot of its own).
        const int nl = int(R.rows.size()), chunks = std::min(nl, 32);
        LoopPool::get().run(chunks, [&](int c) {
            for (int j = int(long(nl) * c / chunks); j < int(long(nl) * (c + 1) / chunks); j++) {
                std::string s = ctc_decode(bh + j, int(R.lens[size_t(j)]), R.ntot, R.widths[size_t(j)]);
                pages[size_t(R.rows[size_t(j)].first)].lines[size_t(R.rows[size_t(j)].second)] = std::move(s);
            }
        }, -1);
        mark("ctc " + std::to_string(r) + " done");
    }
};

void Pipeline::run_pages(const uint8_t *const *src, bool on_host, const int *w, const int *h, int npages) {
    Impl &I = *impl_;
    const auto t0 = Clock::now();
    pages_.assign(size_t(std::max(npages, 0)), PageText{});
    stats_ = PipelineStats{};
    stats_.pages = npages;
    if (npages <= 0) return;
    for (int p = 0; p < npages; p++) {
        if (!src[p]) fail("pipeline: page " + std::to_string(p) + " is null");
        if (w[p] <= 0 || h[p] <= 0) fail("pipeline: empty page " + std::to_string(p));
    }
    I.ctx.bind();
    const PipelinePlan plan = plan_pipeline(npages, I.opts.merge, I.opts.det_batch, on_host);
    std::vector<std::string> errs;
    double busy = 0;
    int failed = 0;
    {
        PipelineRun R(I, plan, src, on_host, w, h, pages_);
        // Pages from host memory reach the device one group at a time; a recognition pass then
        // goes out as soon as its pages are laid out, in stages with the groups that have landed
        // meanwhile queued between them (OCR_PIPE_INTERLEAVE=0: the whole pass at once, after
        // the next pass's detections). Device-resident pages keep the lookahead order.
        const char *il = std::getenv("OCR_PIPE_INTERLEAVE");
        R.interleave = on_host && !(il && std::atoi(il) == 0);
        const char *la = std::getenv("OCR_PIPE_LOOKAHEAD");
        const bool lookahead = la ? std::atoi(la) != 0 : (R.interleave ? false : I.opts.lookahead);
        errs = run_schedule(plan, R, [&](std::function<void()> f) { I.workers.submit(std::move(f)); }, &busy,
                            lookahead);
        for (int p = 0; p < npages; p++) {
            pages_[size_t(p)].error = errs[size_t(p)];
            if (!errs[size_t(p)].empty()) {
                pages_[size_t(p)].lines.clear();
                failed++;
            }
        }
        stats_.batches = R.batches;
        stats_.rec_passes = R.rec_passes;
        stats_.host_labelled = R.host_labelled.load();
        for (const auto &Rp : R.passes)
            for (uint32_t l : Rp.lens) stats_.rec_steps += l;
        R.print_trace();
    }  // R's destructor waits for the streams before its buffers go back to the pool
    stats_.ms = ms_since(t0);
    stats_.cpu_busy_ms = busy;
    for (const PageText &pt : pages_) {
        stats_.lines += int(pt.lines.size());
        stats_.words += pt.words;
    }
    if (failed) {
        int first = 0;
        while (errs[size_t(first)].empty()) first++;
        fail("pipeline: " + std::to_string(failed) + " of " + std::to_string(npages) + " pages failed; page " +
             std::to_string(first) + ": " + errs[size_t(first)]);
    }
}

void Pipeline::run(const uint8_t *const *d_rgb, const int *w, const int *h, int npages) {
    run_pages(d_rgb, false, w, h, npages);
}

void Pipeline::run_host(const uint8_t *const *rgb, const int *w, const int *h, int npages) {
    run_pages(rgb, true, w, h, npages);
}

}  // namespace ocr
