// The C ABI (include/ocrhip.h): status codes and a thread-local message, nothing thrown across.
#include "../../include/ocrhip.h"

#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "models.h"
#include "noalloc.h"
#include "nd.h"
#include "pipeline.h"
#include "png.h"
#include "crop.h"
#include "pp_pipeline.h"

using namespace ocr;

struct ocr_ctx {
    std::unique_ptr<Ctx> ctx;
};
struct ocr_detector {
    ocr_ctx *owner;
    std::unique_ptr<Detector> det;
};
struct ocr_graph {
    ocr_ctx *owner;
    Graph graph;
};
struct ocr_recognizer {
    ocr_ctx *owner;
    std::unique_ptr<Recognizer> rec;
};
struct ocr_layout {
    PageLayout layout;
};
struct ocr_pipeline {
    ocr_ctx *owner;
    std::unique_ptr<Pipeline> pipe;
};
struct ocr_nd {
    ocr_ctx *owner;
    NdGraph graph;
};
struct ocr_pp_pipeline {
    ocr_ctx *owner;
    std::unique_ptr<PpPipeline> pipe;
};

namespace {

thread_local std::string g_error;

template <class F> int guard(F &&f) {
    try {
        f();
        g_error.clear();
        return OCR_OK;
    } catch (const std::exception &e) {
        g_error = e.what();
    } catch (...) {
        g_error = "unknown error";
    }
    return OCR_ERR;
}

template <class T, class F> T *guard_ptr(F &&f) {
    T *out = nullptr;
    guard([&] { out = f(); });
    return out;
}

void need(const void *p, const char *what) {
    if (!p) fail(std::string(what) + " is NULL");
}

std::vector<Recognizer::Batch> to_batches(const ocr_batch *b, uint32_t count) {
    if (count) need(b, "batches");
    std::vector<Recognizer::Batch> out(count);
    for (uint32_t i = 0; i < count; i++) {
        need(b[i].data, "batch data");
        out[i] = {b[i].data, int(b[i].n), int(b[i].w)};
    }
    return out;
}

}  // namespace

namespace {

// The host-parsed graph of the C ABI as this library's Onnx (the reference's onnx.rs struct),
// every string and array copied.
Onnx onnx_of(const ocr_onnx *g) {
    need(g, "graph");
    auto str = [](const char *p, const char *what) -> std::string {
        if (!p) fail(std::string("graph: missing ") + what);
        return std::string(p);
    };
    Onnx m;
    if (g->nnodes) need(g->nodes, "graph nodes");
    if (g->ntensors) need(g->tensors, "graph tensors");
    m.input = str(g->input, "input name");
    m.output = str(g->output, "output name");
    for (uint32_t k = 0; k < g->ntensors; k++) {
        const ocr_onnx_tensor &t = g->tensors[k];
        const std::string name = str(t.name, "tensor name");
        if (t.rank && !t.dims) fail("graph: tensor " + name + " has a rank but no dims");
        uint64_t n = 1;
        std::vector<int64_t> dims(t.dims, t.dims + t.rank);
        for (int64_t d : dims) {
            if (d < 0) fail("graph: tensor " + name + " has a negative dimension");
            // Refuse dims whose product overflows (it could wrap round to the value count).
            if (__builtin_mul_overflow(n, uint64_t(d), &n) || n > (uint64_t(1) << 40))
                fail("graph: tensor " + name + " has more elements than a model tensor can hold");
        }
        if ((t.data != nullptr) == (t.ints != nullptr)) fail("graph: tensor " + name + " needs exactly one of data, ints");
        if (t.data) {
            if (n != t.count) fail("graph: tensor " + name + ": " + std::to_string(t.count) + " values for its dims");
            m.weights[name] = Weight{dims, std::vector<float>(t.data, t.data + t.count)};
        } else {
            m.ints[name] = std::vector<int64_t>(t.ints, t.ints + t.count);
        }
    }
    for (uint32_t k = 0; k < g->nnodes; k++) {
        const ocr_onnx_node &cn = g->nodes[k];
        Node n;
        n.op = str(cn.op, "node op");
        if (cn.ninputs) need(cn.inputs, "node inputs");
        if (cn.noutputs) need(cn.outputs, "node outputs");
        if (cn.nattrs) need(cn.attrs, "node attributes");
        for (uint32_t i = 0; i < cn.ninputs; i++) n.inputs.push_back(cn.inputs[i] ? cn.inputs[i] : "");
        for (uint32_t i = 0; i < cn.noutputs; i++) n.outputs.push_back(str(cn.outputs[i], "node output"));
        for (uint32_t i = 0; i < cn.nattrs; i++) {
            const ocr_onnx_attr &ca = cn.attrs[i];
            Attr a;
            a.name = str(ca.name, "attribute name");
            a.type = ca.type;
            switch (ca.type) {
            case 1: a.f = ca.f, a.has_f = true; break;
            case 2: a.i = ca.i, a.has_i = true; break;
            case 3: a.s = str(ca.s, "string attribute"), a.has_s = true; break;
            case 6:
                if (ca.count) need(ca.floats, "float list attribute");
                a.floats.assign(ca.floats, ca.floats + ca.count);
                break;
            case 7:
                if (ca.count) need(ca.ints, "int list attribute");
                a.ints.assign(ca.ints, ca.ints + ca.count);
                break;
            default: fail("graph: attribute " + a.name + " of unsupported type " + std::to_string(ca.type));
            }
            n.attrs.push_back(std::move(a));
        }
        m.nodes.push_back(std::move(n));
    }
    return m;
}

}  // namespace

extern "C" {

const char *ocr_last_error(void) { return g_error.c_str(); }
const char *ocr_version(void) { return "ocrhip 0.1 (gfx950)"; }

ocr_ctx *ocr_create(const ocr_opts *opts) {
    return guard_ptr<ocr_ctx>([&] {
        ocr_opts o{8, 8192, 0};
        if (opts) o = *opts;
        if (o.lines == 0) o.lines = 8;
        if (o.pool_mb == 0) o.pool_mb = 8192;
        auto c = std::make_unique<ocr_ctx>();
        c->ctx = std::make_unique<Ctx>(o.device, o.lines, size_t(o.pool_mb));
        // The fixed device array of ocr_word_rects_gpu_noalloc: its address on this device.
        noalloc_init(o.device);
        return c.release();
    });
}

void ocr_destroy(ocr_ctx *ctx) { delete ctx; }

int ocr_synchronize(ocr_ctx *ctx) {
    return guard([&] {
        need(ctx, "ctx");
        ctx->ctx->bind();
        ctx->ctx->sync();
    });
}

void *ocr_device_alloc(ocr_ctx *ctx, size_t bytes) {
    return guard_ptr<void>([&]() -> void * {
        need(ctx, "ctx");
        ctx->ctx->bind();
        void *p = nullptr;
        device_malloc(&p, bytes ? bytes : 16);
        return p;
    });
}

int ocr_device_free(ocr_ctx *ctx, void *p) {
    return guard([&] {
        need(ctx, "ctx");
        ctx->ctx->bind();
        ctx->ctx->sync();
        OCR_HIP(hipFree(p));
    });
}

int ocr_memory_stats(ocr_ctx *ctx, uint64_t *device_allocs, uint64_t *host_allocs, uint64_t *pool_live,
                     uint64_t *pool_held) {
    return guard([&] {
        need(ctx, "ctx");
        if (device_allocs) *device_allocs = device_allocations();
        if (host_allocs) *host_allocs = host_allocations();
        if (pool_live) *pool_live = ctx->ctx->pool().live();
        if (pool_held) *pool_held = ctx->ctx->pool().held();
    });
}

void *ocr_host_alloc(ocr_ctx *ctx, size_t bytes) {
    return guard_ptr<void>([&]() -> void * {
        need(ctx, "ctx");
        ctx->ctx->bind();
        void *p = nullptr;
        host_malloc(&p, bytes ? bytes : 16);
        return p;
    });
}

int ocr_host_free(ocr_ctx *ctx, void *p) {
    return guard([&] {
        need(ctx, "ctx");
        ctx->ctx->bind();
        ctx->ctx->sync();
        OCR_HIP(hipHostFree(p));
    });
}

int ocr_png_dims(const uint8_t *png, size_t n, uint32_t *w, uint32_t *h) {
    return guard([&] {
        need(w, "w");
        need(h, "h");
        const PngHeader hd = png_header(png, n);
        *w = hd.w;
        *h = hd.h;
    });
}

int ocr_png_decode(const uint8_t *png, size_t n, uint8_t *rgb, size_t cap, uint32_t *w, uint32_t *h) {
    return guard([&] {
        const PngHeader hd = png_decode_rgb(png, n, rgb, cap);
        if (w) *w = hd.w;
        if (h) *h = hd.h;
    });
}

int ocr_memcpy_h2d(ocr_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return guard([&] {
        need(ctx, "ctx");
        ctx->ctx->bind();
        ctx->ctx->h2d(dst, src, bytes);
    });
}

int ocr_memcpy_d2h(ocr_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return guard([&] {
        need(ctx, "ctx");
        ctx->ctx->bind();
        ctx->ctx->d2h(dst, src, bytes);
    });
}

ocr_detector *ocr_detector_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph) {
    return guard_ptr<ocr_detector>([&] {
        need(ctx, "ctx");
        Onnx m = onnx_of(graph);
        ctx->ctx->bind();
        auto d = std::make_unique<ocr_detector>();
        d->owner = ctx;
        d->det = std::make_unique<Detector>(*ctx->ctx, m);
        return d.release();
    });
}

ocr_graph *ocr_graph_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph, const char *stop_op) {
    return guard_ptr<ocr_graph>([&] {
        need(ctx, "ctx");
        Onnx m = onnx_of(graph);
        ctx->ctx->bind();
        auto g = std::make_unique<ocr_graph>();
        g->owner = ctx;
        g->graph = Graph::build(*ctx->ctx, m, stop_op, nullptr, nullptr);
        return g.release();
    });
}

ocr_recognizer *ocr_recognizer_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph, uint32_t lines) {
    return guard_ptr<ocr_recognizer>([&] {
        need(ctx, "ctx");
        Onnx m = onnx_of(graph);
        ctx->ctx->bind();
        auto r = std::make_unique<ocr_recognizer>();
        r->owner = ctx;
        r->rec = std::make_unique<Recognizer>(*ctx->ctx, m, lines ? lines : 8);
        return r.release();
    });
}

ocr_nd *ocr_nd_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph, int stop_before_softmax) {
    return guard_ptr<ocr_nd>([&] {
        need(ctx, "ctx");
        Onnx m = onnx_of(graph);
        ctx->ctx->bind();
        auto g = std::make_unique<ocr_nd>();
        g->owner = ctx;
        g->graph = NdGraph::build(*ctx->ctx, m, stop_before_softmax != 0);
        return g.release();
    });
}

ocr_detector *ocr_detector_new(ocr_ctx *ctx, const char *onnx_path) {
    return guard_ptr<ocr_detector>([&] {
        need(ctx, "ctx");
        need(onnx_path, "onnx_path");
        ctx->ctx->bind();
        Onnx m = Onnx::load(onnx_path);
        auto d = std::make_unique<ocr_detector>();
        d->owner = ctx;
        d->det = std::make_unique<Detector>(*ctx->ctx, m);
        return d.release();
    });
}

void ocr_detector_free(ocr_detector *det) { delete det; }

int ocr_detect_page(ocr_detector *det, const uint8_t *rgb, uint32_t w, uint32_t h, float thr, uint32_t *bits) {
    return guard([&] {
        need(det, "det");
        need(rgb, "rgb");
        need(bits, "bits");
        Ctx &c = *det->owner->ctx;
        c.bind();
        const size_t bytes = size_t(w) * h * 3, words = size_t((w + 31) / 32) * h;
        DBuf drgb(&c, bytes), dbits(&c, words * 4);
        c.h2d(drgb.get(), rgb, bytes);
        const uint8_t *pr = drgb.as<uint8_t>();
        uint32_t *pb = dbits.as<uint32_t>();
        const int wi = int(w), hi = int(h);
        det->det->detect_pages_device(&pr, &wi, &hi, 1, thr, &pb);
        c.d2h(bits, pb, words * 4);
    });
}

int ocr_detect_pages_device(ocr_detector *det, const uint8_t *const *d_rgb, const uint32_t *w, const uint32_t *h,
                            uint32_t count, float thr, uint32_t *const *d_bits) {
    return guard([&] {
        need(det, "det");
        if (count == 0) return;
        need(d_rgb, "d_rgb");
        need(w, "w");
        need(h, "h");
        need(d_bits, "d_bits");
        det->owner->ctx->bind();
        std::vector<int> wi(count), hi(count);
        for (uint32_t k = 0; k < count; k++) {
            wi[k] = int(w[k]);
            hi[k] = int(h[k]);
        }
        det->det->detect_pages_device(d_rgb, wi.data(), hi.data(), int(count), thr, d_bits);
    });
}

int ocr_detect(ocr_detector *det, const float *input, uint32_t h, uint32_t w, float *prob) {
    return guard([&] {
        need(det, "det");
        need(input, "input");
        need(prob, "prob");
        det->owner->ctx->bind();
        std::vector<float> out = det->det->detect(input, int(h), int(w));
        std::copy(out.begin(), out.end(), prob);
    });
}

ocr_graph *ocr_graph_new(ocr_ctx *ctx, const char *onnx_path, const char *stop_op) {
    return guard_ptr<ocr_graph>([&] {
        need(ctx, "ctx");
        need(onnx_path, "onnx_path");
        ctx->ctx->bind();
        Onnx m = Onnx::load(onnx_path);
        auto g = std::make_unique<ocr_graph>();
        g->owner = ctx;
        g->graph = Graph::build(*ctx->ctx, m, stop_op, nullptr, nullptr);
        return g.release();
    });
}

void ocr_graph_free(ocr_graph *g) { delete g; }

int ocr_graph_dims(ocr_graph *g, uint32_t n, uint32_t c, uint32_t h, uint32_t w, uint32_t *out_nchw) {
    return guard([&] {
        need(g, "graph");
        need(out_nchw, "out");
        Shape s = g->graph.infer({int(n), int(h), int(w), int(c)});
        out_nchw[0] = uint32_t(s[0]);
        out_nchw[1] = uint32_t(s[3]);
        out_nchw[2] = uint32_t(s[1]);
        out_nchw[3] = uint32_t(s[2]);
    });
}

int ocr_graph_run(ocr_graph *g, const float *in, uint32_t n, uint32_t c, uint32_t h, uint32_t w, float *out) {
    return guard([&] {
        need(g, "graph");
        need(in, "in");
        need(out, "out");
        Ctx &cx = *g->owner->ctx;
        cx.bind();
        const size_t hw = size_t(h) * w;
        std::vector<float> nhwc(size_t(n) * c * hw);
        for (size_t b = 0; b < n; b++)
            for (size_t ch = 0; ch < c; ch++)
                for (size_t p = 0; p < hw; p++) nhwc[(b * hw + p) * c + ch] = in[(b * c + ch) * hw + p];
        Act x{nullptr, int(n), int(h), int(w), int(c), int(c)};
        DBuf xb(&cx, nhwc.size() * sizeof(float));
        x.p = xb.as<float>();
        cx.h2d(x.p, nhwc.data(), nhwc.size() * sizeof(float));
        Graph::Out o = g->graph.run(cx, x);
        std::vector<float> res(o.act.count());
        cx.d2h(res.data(), o.act.p, res.size() * sizeof(float));
        const size_t ohw = size_t(o.act.h) * o.act.w;
        for (size_t b = 0; b < size_t(o.act.n); b++)
            for (size_t ch = 0; ch < size_t(o.act.c); ch++)
                for (size_t p = 0; p < ohw; p++)
                    out[(b * o.act.c + ch) * ohw + p] = res[(b * ohw + p) * o.act.c + ch];
    });
}

ocr_recognizer *ocr_recognizer_new(ocr_ctx *ctx, const char *onnx_path, uint32_t lines) {
    return guard_ptr<ocr_recognizer>([&] {
        need(ctx, "ctx");
        need(onnx_path, "onnx_path");
        ctx->ctx->bind();
        Onnx m = Onnx::load(onnx_path);
        auto r = std::make_unique<ocr_recognizer>();
        r->owner = ctx;
        r->rec = std::make_unique<Recognizer>(*ctx->ctx, m, lines ? lines : 8);
        return r.release();
    });
}

void ocr_recognizer_free(ocr_recognizer *rec) { delete rec; }

int ocr_recognize_dims(ocr_recognizer *rec, const ocr_batch *batches, uint32_t count, uint32_t *tmax, uint32_t *ntot,
                       uint32_t *classes) {
    return guard([&] {
        need(rec, "rec");
        auto bs = to_batches(batches, count);
        Recognizer::Dims d = rec->rec->dims(bs.data(), int(bs.size()));
        if (tmax) *tmax = uint32_t(d.tmax);
        if (ntot) *ntot = uint32_t(d.ntot);
        if (classes) *classes = uint32_t(d.classes);
    });
}

int ocr_recognize(ocr_recognizer *rec, const ocr_batch *batches, uint32_t count, float *logits, uint32_t *lens,
                  uint32_t *best) {
    return guard([&] {
        need(rec, "rec");
        need(lens, "lens");
        Ctx &c = *rec->owner->ctx;
        c.bind();
        auto bs = to_batches(batches, count);
        Recognizer::Dims d = rec->rec->dims(bs.data(), int(bs.size()));
        std::vector<DBuf> data;
        std::vector<Recognizer::Batch> dev(bs.size());
        for (size_t i = 0; i < bs.size(); i++) {
            const size_t bytes = size_t(bs[i].n) * 64 * bs[i].w * sizeof(float);
            data.emplace_back(&c, bytes);
            c.h2d(data.back().get(), bs[i].data, bytes);
            dev[i] = {data.back().as<float>(), bs[i].n, bs[i].w};
        }
        const size_t rows = size_t(d.tmax) * d.ntot;
        DBuf dl(&c, rows * d.classes * sizeof(float)), db(&c, rows * sizeof(uint32_t));
        rec->rec->recognize_device(dev.data(), int(dev.size()), dl.as<float>(), best ? db.as<uint32_t>() : nullptr,
                                   lens);
        if (logits) c.d2h(logits, dl.get(), rows * d.classes * sizeof(float));
        if (best) c.d2h(best, db.get(), rows * sizeof(uint32_t));
        c.sync();
    });
}

int ocr_recognize_device(ocr_recognizer *rec, const ocr_batch *d_batches, uint32_t count, float *d_logits,
                         uint32_t *d_best, uint32_t *lens) {
    return guard([&] {
        need(rec, "rec");
        need(lens, "lens");
        Ctx &c = *rec->owner->ctx;
        c.bind();
        auto bs = to_batches(d_batches, count);
        Recognizer::Dims d = rec->rec->dims(bs.data(), int(bs.size()));
        DBuf tmp;
        float *logits = d_logits;
        if (!logits) {
            tmp = DBuf(&c, size_t(d.tmax) * d.ntot * d.classes * sizeof(float));
            logits = tmp.as<float>();
        }
        rec->rec->recognize_device(bs.data(), int(bs.size()), logits, d_best, lens);
    });
}

int ocr_probe_start(const char *family) {
    return guard([&] {
        need(family, "family");
        Probe::get().start(family);
    });
}

int ocr_probe_stop(const char *family, uint32_t *calls, double *ms, double *flops, double *bytes) {
    return guard([&] {
        need(family, "family");
        if (!Probe::get().stop(family, calls, ms, flops, bytes)) fail(std::string("not probing ") + family);
    });
}

int ocr_word_rects(const uint32_t *bits, uint32_t w, uint32_t h, ocr_rrect *out, uint32_t cap, uint32_t *count) {
    return guard([&] {
        need(bits, "bits");
        need(count, "count");
        std::vector<RRect> r = word_rects(bits, int(w), int(h));
        *count = uint32_t(r.size());
        for (size_t i = 0; i < r.size() && i < cap; i++) out[i] = {r[i].cx, r[i].cy, r[i].ux, r[i].uy, r[i].w, r[i].h};
    });
}

int ocr_word_rects_mt(const uint32_t *bits, uint32_t w, uint32_t h, uint32_t threads, ocr_rrect *out, uint32_t cap,
                      uint32_t *count) {
    return guard([&] {
        need(bits, "bits");
        need(count, "count");
        if (threads < 1 || threads > 256) fail("threads must be 1..256");
        std::vector<RRect> r = word_rects(bits, int(w), int(h), 3.f, 100.f, int(threads));
        *count = uint32_t(r.size());
        for (size_t i = 0; i < r.size() && i < cap; i++) out[i] = {r[i].cx, r[i].cy, r[i].ux, r[i].uy, r[i].w, r[i].h};
    });
}

int ocr_word_rects_gpu(ocr_ctx *ctx, const uint32_t *bits, uint32_t w, uint32_t h, ocr_rrect *out, uint32_t cap,
                       uint32_t *count) {
    return guard([&] {
        need(ctx, "ctx");
        need(bits, "bits");
        need(count, "count");
        if (w == 0 || h == 0 || w > 65536 || h > 65536) fail("mask size");
        Ctx &c = *ctx->ctx;
        c.bind();
        const size_t words = size_t(w + 31) / 32 * h;
        const int runs_cap = int(std::min<size_t>(words * 16, size_t(1) << 26));
        // Components and row slots are at most one a run.
        const size_t rc = size_t(runs_cap);
        DBuf db(&c, words * 4), dx0(&c, rc * 2), dx1(&c, rc * 2), droot(&c, rc * 4), droff(&c, size_t(h + 1) * 4),
            dtot(&c, 16), dry(&c, rc * 2), dcbot(&c, rc * 4), dcomps(&c, rc * 16), dxmin(&c, rc * 4), dxmax(&c, rc * 4);
        c.h2d(db.get(), bits, words * 4);
        CclPage pg{};
        pg.bits = db.as<uint32_t>(), pg.w = int(w), pg.h = int(h);
        pg.x0 = dx0.as<uint16_t>(), pg.x1 = dx1.as<uint16_t>(), pg.root = droot.as<int32_t>();
        pg.row_off = droff.as<int32_t>(), pg.cap = runs_cap, pg.total = dtot.as<int32_t>();
        pg.ry = dry.as<uint16_t>(), pg.cbot = dcbot.as<int32_t>(), pg.comps = dcomps.as<int32_t>();
        pg.xmin = dxmin.as<uint32_t>(), pg.xmax = dxmax.as<uint32_t>(), pg.ccap = runs_cap, pg.scap = runs_cap;
        ccl_runs(&pg, 1, c.stream());
        int32_t tot[4] = {0, 0, 0, 0};
        c.d2h(tot, dtot.get(), 16);
        if (tot[0] > runs_cap) fail("too many runs");
        const size_t nc = size_t(tot[1]), ns = size_t(tot[2]);
        std::vector<int32_t> comps(nc * 4);
        std::vector<uint32_t> xmin(ns), xmax(ns);
        if (nc) {
            c.d2h(comps.data(), dcomps.get(), nc * 16);
            c.d2h(xmin.data(), dxmin.get(), ns * 4);
            c.d2h(xmax.data(), dxmax.get(), ns * 4);
        }
        std::vector<RRect> r = word_rects_from_rows(bits, int(w), int(h), comps.data(), int(nc), xmin.data(), xmax.data(), int(ns));
        *count = uint32_t(r.size());
        for (size_t i = 0; i < r.size() && i < cap; i++) out[i] = {r[i].cx, r[i].cy, r[i].ux, r[i].uy, r[i].w, r[i].h};
    });
}

int ocr_word_rects_gpu_noalloc(ocr_ctx *ctx, const uint32_t *bits, uint32_t w, uint32_t h, ocr_rrect *out,
                               uint32_t cap, uint32_t *count) {
    return guard([&] {
        need(ctx, "ctx");
        need(bits, "bits");
        need(count, "count");
        std::vector<RRect> r = word_rects_gpu_noalloc(*ctx->ctx, bits, int(w), int(h));
        *count = uint32_t(r.size());
        for (size_t i = 0; i < r.size() && i < cap; i++) out[i] = {r[i].cx, r[i].cy, r[i].ux, r[i].uy, r[i].w, r[i].h};
    });
}

ocr_layout *ocr_layout_page(const uint32_t *bits, uint32_t w, uint32_t h, float relv, float relend) {
    return guard_ptr<ocr_layout>([&] {
        need(bits, "bits");
        auto l = std::make_unique<ocr_layout>();
        l->layout = layout_page(bits, int(w), int(h), relv, relend);
        return l.release();
    });
}

void ocr_layout_free(ocr_layout *lay) { delete lay; }

int ocr_layout_counts(ocr_layout *lay, uint32_t *words, uint32_t *lines, uint32_t *batches) {
    return guard([&] {
        need(lay, "layout");
        if (words) *words = uint32_t(lay->layout.words);
        if (lines) *lines = uint32_t(lay->layout.lines.size());
        if (batches) *batches = uint32_t(lay->layout.plan.lines.size());
    });
}

int ocr_layout_line(ocr_layout *lay, uint32_t i, int32_t *box, int32_t *row_off, int32_t *spans, uint32_t *nspans) {
    return guard([&] {
        need(lay, "layout");
        if (i >= lay->layout.lines.size()) fail("line index out of range");
        const LineGeom &g = lay->layout.lines[i];
        if (box) {
            box[0] = g.left, box[1] = g.top, box[2] = g.bw, box[3] = g.bh, box[4] = g.out_w;
        }
        if (nspans) *nspans = uint32_t(g.spans.size() / 2);
        if (row_off) std::copy(g.row_off.begin(), g.row_off.end(), row_off);
        if (spans) std::copy(g.spans.begin(), g.spans.end(), spans);
    });
}

int ocr_layout_batch(ocr_layout *lay, uint32_t i, uint32_t *width, uint32_t *lines, uint32_t *count) {
    return guard([&] {
        need(lay, "layout");
        if (i >= lay->layout.plan.lines.size()) fail("batch index out of range");
        const auto &m = lay->layout.plan.lines[i];
        if (width) *width = uint32_t(lay->layout.plan.width[i]);
        if (count) *count = uint32_t(m.size());
        if (lines)
            for (size_t k = 0; k < m.size(); k++) lines[k] = uint32_t(m[k]);
    });
}

ocr_pipeline *ocr_pipeline_new(ocr_detector *det, ocr_recognizer *rec, const ocr_pipeline_opts *opts) {
    return guard_ptr<ocr_pipeline>([&] {
        need(det, "det");
        need(rec, "rec");
        if (det->owner != rec->owner) fail("detector and recogniser belong to different contexts");
        PipelineOpts o;
        if (opts) {
            if (opts->merge) o.merge = int(opts->merge);
            if (opts->relv != 0.f) o.relv = opts->relv;
            if (opts->relend != 0.f) o.relend = opts->relend;
            if (opts->thr != 0.f) o.thr = opts->thr;
            o.threads = int(opts->threads);
            if (opts->det_batch) o.det_batch = int(opts->det_batch);
            if (opts->label_runs > (1u << 30) || opts->label_comps > (1u << 30) || opts->label_slots > (1u << 30))
                fail("label capacities above 2^30");
            o.label_runs = int(opts->label_runs);
            o.label_comps = int(opts->label_comps);
            o.label_slots = int(opts->label_slots);
        }
        det->owner->ctx->bind();
        auto p = std::make_unique<ocr_pipeline>();
        p->owner = det->owner;
        p->pipe = std::make_unique<Pipeline>(*det->owner->ctx, *det->det, *rec->rec, o);
        return p.release();
    });
}

void ocr_pipeline_free(ocr_pipeline *pipe) { delete pipe; }

int ocr_pipeline_run_device(ocr_pipeline *pipe, const uint8_t *const *d_rgb, const uint32_t *w, const uint32_t *h,
                            uint32_t npages) {
    return guard([&] {
        need(pipe, "pipeline");
        if (npages) {
            need(d_rgb, "d_rgb");
            need(w, "w");
            need(h, "h");
        }
        pipe->owner->ctx->bind();
        std::vector<int> wi(npages), hi(npages);
        for (uint32_t k = 0; k < npages; k++) wi[k] = int(w[k]), hi[k] = int(h[k]);
        pipe->pipe->run(d_rgb, wi.data(), hi.data(), int(npages));
    });
}

int ocr_pipeline_run(ocr_pipeline *pipe, const uint8_t *const *rgb, const uint32_t *w, const uint32_t *h,
                     uint32_t npages) {
    return guard([&] {
        need(pipe, "pipeline");
        if (npages) {
            need(rgb, "rgb");
            need(w, "w");
            need(h, "h");
        }
        pipe->owner->ctx->bind();
        std::vector<int> wi(npages), hi(npages);
        for (uint32_t k = 0; k < npages; k++) wi[k] = int(w[k]), hi[k] = int(h[k]);
        pipe->pipe->run_host(rgb, wi.data(), hi.data(), int(npages));
    });
}

int ocr_pipeline_page_error(ocr_pipeline *pipe, uint32_t page, char *buf, uint32_t cap, uint32_t *len) {
    return guard([&] {
        need(pipe, "pipeline");
        const auto &pages = pipe->pipe->pages();
        if (page >= pages.size()) fail("page index out of range");
        const std::string &s = pages[page].error;
        if (len) *len = uint32_t(s.size());
        if (buf && cap) {
            const size_t n = std::min<size_t>(s.size(), cap - 1);
            std::copy(s.begin(), s.begin() + long(n), buf);
            buf[n] = 0;
        }
    });
}

int ocr_pipeline_stats_get(ocr_pipeline *pipe, ocr_pipeline_stats *out) {
    return guard([&] {
        need(pipe, "pipeline");
        need(out, "out");
        const PipelineStats &s = pipe->pipe->stats();
        *out = {s.ms, s.cpu_busy_ms, uint32_t(s.pages), uint32_t(s.lines), uint32_t(s.words), uint32_t(s.batches),
                uint32_t(s.rec_passes), uint64_t(s.rec_steps), uint32_t(s.host_labelled)};
    });
}

int ocr_pipeline_page(ocr_pipeline *pipe, uint32_t page, uint32_t *lines, uint32_t *words) {
    return guard([&] {
        need(pipe, "pipeline");
        const auto &pages = pipe->pipe->pages();
        if (page >= pages.size()) fail("page index out of range");
        if (lines) *lines = uint32_t(pages[page].lines.size());
        if (words) *words = uint32_t(pages[page].words);
    });
}

int ocr_pipeline_line_text(ocr_pipeline *pipe, uint32_t page, uint32_t line, char *buf, uint32_t cap, uint32_t *len) {
    return guard([&] {
        need(pipe, "pipeline");
        const auto &pages = pipe->pipe->pages();
        if (page >= pages.size() || line >= pages[page].lines.size()) fail("line index out of range");
        const std::string &s = pages[page].lines[line];
        if (len) *len = uint32_t(s.size());
        if (buf && cap) {
            const size_t n = std::min<size_t>(s.size(), cap - 1);
            std::copy(s.begin(), s.begin() + long(n), buf);
            buf[n] = 0;
        }
    });
}


}  // extern "C"

// ---- N-D executor (PP-OCRv6) -------------------------------------------------------------------

namespace {

std::vector<int64_t> shape_in(const int64_t *shape, uint32_t rank) {
    if (rank == 0 || rank > uint32_t(ND_RANK)) fail("rank must be 1 to 6");
    need(shape, "shape");
    std::vector<int64_t> s(shape, shape + rank);
    for (int64_t d : s)
        if (d <= 0) fail("shape with a zero or negative dimension");
    return s;
}

size_t count_of(const std::vector<int64_t> &s) {
    size_t c = 1;
    for (int64_t d : s) c *= size_t(d);
    return c;
}

// PP-OCR detection input size (src/nd.rs:1356-1358): long side at most max_side, each side
// rounded to the nearest multiple of 32 (at least 32).
void det_input_size(uint32_t w, uint32_t h, uint32_t max_side, int *ow, int *oh) {
    if (w == 0 || h == 0 || max_side == 0) fail("det input: empty page or max_side 0");
    const float ratio = std::max(w, h) > max_side ? float(max_side) / float(std::max(w, h)) : 1.f;
    auto round32 = [](float v) { return std::max(int(std::lround(v / 32.f)) * 32, 32); };
    *ow = round32(float(w) * ratio);
    *oh = round32(float(h) * ratio);
}

}  // namespace

extern "C" {

int ocr_nd_plan(const char *onnx_path, int stop_before_softmax, char *buf, uint32_t cap, uint32_t *len) {
    return guard([&] {
        need(onnx_path, "onnx_path");
        const std::string text = describe(plan_nd(Onnx::load(onnx_path), stop_before_softmax != 0));
        if (len) *len = uint32_t(text.size());
        if (buf && cap) {
            const size_t n = std::min<size_t>(text.size(), cap - 1);
            std::memcpy(buf, text.data(), n);
            buf[n] = 0;
        }
    });
}

ocr_nd *ocr_nd_new(ocr_ctx *ctx, const char *onnx_path, int stop_before_softmax) {
    return guard_ptr<ocr_nd>([&] {
        need(ctx, "ctx");
        need(onnx_path, "onnx_path");
        ctx->ctx->bind();
        Onnx m = Onnx::load(onnx_path);
        auto g = std::make_unique<ocr_nd>();
        g->owner = ctx;
        g->graph = NdGraph::build(*ctx->ctx, m, stop_before_softmax != 0);
        return g.release();
    });
}

void ocr_nd_free(ocr_nd *g) { delete g; }

int ocr_nd_dims(ocr_nd *g, const int64_t *in_shape, uint32_t rank, int64_t *out_shape, uint32_t *out_rank) {
    return guard([&] {
        need(g, "graph");
        need(out_shape, "out_shape");
        need(out_rank, "out_rank");
        auto s = g->graph.output_shape(shape_in(in_shape, rank));
        if (s.size() > size_t(ND_RANK)) fail("output rank above 6");
        std::copy(s.begin(), s.end(), out_shape);
        *out_rank = uint32_t(s.size());
    });
}

int ocr_nd_run_device(ocr_nd *g, const float *d_in, const int64_t *in_shape, uint32_t rank, float *d_out) {
    return guard([&] {
        need(g, "graph");
        need(d_in, "input");
        need(d_out, "output");
        Ctx &c = *g->owner->ctx;
        c.bind();
        NdTensor x;
        x.p = const_cast<float *>(d_in);
        x.shape = shape_in(in_shape, rank);
        NdTensor y = g->graph.run(c, x);
        OCR_HIP(hipMemcpyAsync(d_out, y.p, y.count() * sizeof(float), hipMemcpyDeviceToDevice, c.stream()));
    });
}

int ocr_nd_run(ocr_nd *g, const float *in, const int64_t *in_shape, uint32_t rank, float *out) {
    return guard([&] {
        need(g, "graph");
        need(in, "input");
        need(out, "output");
        Ctx &c = *g->owner->ctx;
        c.bind();
        NdTensor x;
        x.shape = shape_in(in_shape, rank);
        DBuf din(&c, count_of(x.shape) * sizeof(float));
        x.p = din.as<float>();
        c.h2d(x.p, in, count_of(x.shape) * sizeof(float));
        NdTensor y = g->graph.run(c, x);
        c.d2h(out, y.p, y.count() * sizeof(float));
    });
}

int ocr_nd_argmax_device(ocr_nd *g, const float *d_in, const int64_t *in_shape, uint32_t rank, uint32_t *d_best) {
    return guard([&] {
        need(g, "graph");
        need(d_in, "input");
        need(d_best, "best");
        Ctx &c = *g->owner->ctx;
        c.bind();
        NdTensor x;
        x.p = const_cast<float *>(d_in);
        x.shape = shape_in(in_shape, rank);
        g->graph.run_argmax(c, x, d_best, nullptr);
    });
}

int ocr_nd_argmax(ocr_nd *g, const float *in, const int64_t *in_shape, uint32_t rank, uint32_t *best) {
    return guard([&] {
        need(g, "graph");
        need(in, "input");
        need(best, "best");
        Ctx &c = *g->owner->ctx;
        c.bind();
        NdTensor x;
        x.shape = shape_in(in_shape, rank);
        auto os = g->graph.output_shape(x.shape);
        if (os.empty()) fail("arg-max of a scalar output");
        const size_t rows = count_of(os) / size_t(os.back());
        DBuf din(&c, count_of(x.shape) * sizeof(float)), dbest(&c, std::max<size_t>(rows, 1) * 4);
        x.p = din.as<float>();
        c.h2d(x.p, in, count_of(x.shape) * sizeof(float));
        g->graph.run_argmax(c, x, dbest.as<uint32_t>(), nullptr);
        c.d2h(best, dbest.get(), rows * 4);
    });
}

int ocr_nd_det_input_dims(uint32_t w, uint32_t h, uint32_t max_side, uint32_t *ow, uint32_t *oh, float *to_page) {
    return guard([&] {
        need(ow, "ow");
        need(oh, "oh");
        int a = 0, b = 0;
        det_input_size(w, h, max_side, &a, &b);
        *ow = uint32_t(a);
        *oh = uint32_t(b);
        if (to_page) {
            to_page[0] = float(w) / float(a);
            to_page[1] = float(h) / float(b);
        }
    });
}

int ocr_nd_det_input_device(ocr_ctx *ctx, const uint8_t *d_rgb, uint32_t w, uint32_t h, uint32_t max_side,
                            float *d_out) {
    return guard([&] {
        need(ctx, "ctx");
        need(d_rgb, "rgb");
        need(d_out, "output");
        ctx->ctx->bind();
        int ow = 0, oh = 0;
        det_input_size(w, h, max_side, &ow, &oh);
        nd_det_prep(d_rgb, int(w), int(h), d_out, ow, oh, ctx->ctx->stream());
    });
}

int ocr_nd_det_input(ocr_ctx *ctx, const uint8_t *rgb, uint32_t w, uint32_t h, uint32_t max_side, float *out) {
    return guard([&] {
        need(ctx, "ctx");
        need(rgb, "rgb");
        need(out, "output");
        Ctx &c = *ctx->ctx;
        c.bind();
        int ow = 0, oh = 0;
        det_input_size(w, h, max_side, &ow, &oh);
        DBuf drgb(&c, size_t(w) * h * 3), dout(&c, size_t(3) * ow * oh * sizeof(float));
        c.h2d(drgb.get(), rgb, size_t(w) * h * 3);
        nd_det_prep(drgb.as<uint8_t>(), int(w), int(h), dout.as<float>(), ow, oh, c.stream());
        c.d2h(out, dout.get(), size_t(3) * ow * oh * sizeof(float));
    });
}

int ocr_db_threshold_device(ocr_ctx *ctx, const float *d_prob, uint32_t w, uint32_t h, float thr, uint32_t *d_bits) {
    return guard([&] {
        need(ctx, "ctx");
        need(d_prob, "prob");
        need(d_bits, "bits");
        if (w == 0 || h == 0) fail("empty probability map");
        ctx->ctx->bind();
        nd_threshold_bits(d_prob, int(w), int(h), thr, d_bits, ctx->ctx->stream());
    });
}

int ocr_db_threshold(ocr_ctx *ctx, const float *prob, uint32_t w, uint32_t h, float thr, uint32_t *bits) {
    return guard([&] {
        need(ctx, "ctx");
        need(prob, "prob");
        need(bits, "bits");
        if (w == 0 || h == 0) fail("empty probability map");
        Ctx &c = *ctx->ctx;
        c.bind();
        const size_t words = size_t((w + 31) / 32) * h;
        DBuf dp(&c, size_t(w) * h * sizeof(float)), db(&c, words * 4);
        c.h2d(dp.get(), prob, size_t(w) * h * sizeof(float));
        nd_threshold_bits(dp.as<float>(), int(w), int(h), thr, db.as<uint32_t>(), c.stream());
        c.d2h(bits, db.get(), words * 4);
    });
}


ocr_pp_pipeline *ocr_pp_pipeline_new(ocr_nd *det, ocr_nd *rec, const ocr_pp_opts *opts) {
    return guard_ptr<ocr_pp_pipeline>([&] {
        need(det, "det");
        need(rec, "rec");
        if (det->owner != rec->owner) fail("detector and recogniser belong to different contexts");
        PpPipelineOpts o;
        if (opts) {
            if (opts->merge) o.merge = int(opts->merge);
            if (opts->thr > 0) o.thr = opts->thr;
            if (opts->relv > 0) o.relv = opts->relv;
            if (opts->max_side) o.max_side = int(opts->max_side);
            if (opts->per_batch) o.per_batch = int(opts->per_batch);
            if (opts->threads) o.threads = int(opts->threads);
            if (opts->det_batch) o.det_batch = int(opts->det_batch);
            if (opts->box_thresh > 0) o.db.box_thresh = opts->box_thresh;
            if (opts->unclip_ratio > 0) o.db.unclip_ratio = opts->unclip_ratio;
            if (opts->min_size > 0) o.db.min_size = opts->min_size;
        }
        det->owner->ctx->bind();
        auto p = std::make_unique<ocr_pp_pipeline>();
        p->owner = det->owner;
        p->pipe = std::make_unique<PpPipeline>(*det->owner->ctx, det->graph, rec->graph, o);
        return p.release();
    });
}

void ocr_pp_pipeline_free(ocr_pp_pipeline *pipe) { delete pipe; }

int ocr_pp_pipeline_run_device(ocr_pp_pipeline *pipe, const uint8_t *const *d_rgb, const uint32_t *w, const uint32_t *h,
                               uint32_t npages) {
    return guard([&] {
        need(pipe, "pipeline");
        if (npages) {
            need(d_rgb, "d_rgb");
            need(w, "w");
            need(h, "h");
        }
        pipe->owner->ctx->bind();
        std::vector<int> wi(npages), hi(npages);
        for (uint32_t k = 0; k < npages; k++) wi[k] = int(w[k]), hi[k] = int(h[k]);
        pipe->pipe->run(d_rgb, wi.data(), hi.data(), int(npages));
    });
}

int ocr_pp_pipeline_run(ocr_pp_pipeline *pipe, const uint8_t *const *rgb, const uint32_t *w, const uint32_t *h,
                        uint32_t npages) {
    return guard([&] {
        need(pipe, "pipeline");
        if (npages) {
            need(rgb, "rgb");
            need(w, "w");
            need(h, "h");
        }
        std::vector<int> wi(npages), hi(npages);
        for (uint32_t k = 0; k < npages; k++) {
            need(rgb[k], "page");
            if (w[k] > 0x7fffffffu || h[k] > 0x7fffffffu) fail("pp pipeline: page size");
            wi[k] = int(w[k]), hi[k] = int(h[k]);
        }
        pipe->pipe->run_host(rgb, wi.data(), hi.data(), int(npages));
    });
}

int ocr_pp_pipeline_stats_get(ocr_pp_pipeline *pipe, ocr_pipeline_stats *out) {
    return guard([&] {
        need(pipe, "pipeline");
        need(out, "out");
        const PipelineStats &s = pipe->pipe->stats();
        *out = ocr_pipeline_stats{s.ms, s.cpu_busy_ms, uint32_t(s.pages), uint32_t(s.lines), uint32_t(s.words),
                                  uint32_t(s.batches), uint32_t(s.rec_passes), uint64_t(s.rec_steps), 0u};
    });
}

int ocr_pp_pipeline_line_text(ocr_pp_pipeline *pipe, uint32_t page, uint32_t line, char *buf, uint32_t cap,
                              uint32_t *len) {
    return guard([&] {
        need(pipe, "pipeline");
        const auto &pages = pipe->pipe->pages();
        if (page >= pages.size() || line >= pages[page].lines.size()) fail("line index out of range");
        const std::string &s = pages[page].lines[line];
        if (len) *len = uint32_t(s.size());
        if (buf && cap) {
            const size_t n = std::min<size_t>(s.size(), cap - 1);
            std::copy(s.begin(), s.begin() + long(n), buf);
            buf[n] = 0;
        }
    });
}

int ocr_pp_pipeline_page(ocr_pp_pipeline *pipe, uint32_t page, uint32_t *lines) {
    return guard([&] {
        need(pipe, "pipeline");
        const auto &pages = pipe->pipe->pages();
        if (page >= pages.size()) fail("page index out of range");
        if (lines) *lines = uint32_t(pages[page].lines.size());
    });
}

int ocr_db_boxes(const uint32_t *bits, const float *prob, uint32_t w, uint32_t h, float to_page_x, float to_page_y,
                 float box_thresh, float unclip_ratio, float min_size, ocr_rrect *out, uint32_t cap, uint32_t *count) {
    return guard([&] {
        need(bits, "bits");
        need(prob, "prob");
        need(count, "count");
        DbParams db;
        if (box_thresh > 0) db.box_thresh = box_thresh;
        if (unclip_ratio > 0) db.unclip_ratio = unclip_ratio;
        if (min_size > 0) db.min_size = min_size;
        auto boxes = db_boxes(bits, prob, int(w), int(h), to_page_x, to_page_y, db);
        *count = uint32_t(boxes.size());
        for (size_t i = 0; i < boxes.size() && i < cap; i++) {
            need(out, "out");
            const RRect &r = boxes[i];
            out[i] = ocr_rrect{r.cx, r.cy, r.ux, r.uy, r.w, r.h};
        }
    });
}

int ocr_pp_line_box(const ocr_rrect *box, float relv, uint32_t page_w, uint32_t page_h, int32_t *out) {
    return guard([&] {
        need(box, "box");
        need(out, "out");
        RRect r;
        r.cx = box->cx, r.cy = box->cy, r.ux = box->ux, r.uy = box->uy, r.w = box->w, r.h = box->h;
        const PpLine l = pp_line_box(r, relv, int(page_w), int(page_h));
        out[0] = l.left, out[1] = l.top, out[2] = l.cw, out[3] = l.ch, out[4] = l.out_w;
    });
}


int ocr_line_images(ocr_ctx *ctx, const uint8_t *rgb, uint32_t page_w, uint32_t page_h, const int32_t *lines,
                    uint32_t count, const int32_t *row_off, uint32_t n_row_off, const int32_t *spans, uint32_t n_spans,
                    uint32_t wb, float *out) {
    return guard([&] {
        need(ctx, "ctx");
        need(rgb, "rgb");
        need(lines, "lines");
        need(row_off, "row_off");
        need(out, "out");
        if (count == 0) return;
        if (wb == 0 || page_w == 0 || page_h == 0) fail("empty page or batch width");
        if (n_spans && !spans) fail("spans is null");
        for (uint32_t i = 0; i < n_row_off; i++)
            if (row_off[i] < 0 || uint32_t(row_off[i]) > n_spans || (i && row_off[i] < row_off[i - 1]))
                fail("row offsets out of range");
        Ctx &c = *ctx->ctx;
        c.bind();
        const size_t slot = size_t(LINE_H) * wb;
        DBuf drgb(&c, size_t(page_w) * page_h * 3), dout(&c, size_t(count) * slot * sizeof(float));
        c.h2d(drgb.get(), rgb, size_t(page_w) * page_h * 3);
        const std::vector<int32_t> roff(row_off, row_off + n_row_off),
            sp(spans ? spans : row_off, spans ? spans + n_spans : row_off);
        std::vector<CropLine> crops;
        for (uint32_t i = 0; i < count; i++) {
            const int32_t *l = lines + size_t(i) * 6;
            if (l[2] < 1 || l[3] < 1 || l[4] < 1 || uint32_t(l[4]) > wb) fail("line box or width out of range");
            if (l[5] < 0 || size_t(l[5]) + size_t(l[3]) + 1 > n_row_off) fail("line row offsets out of range");
            crops.push_back({drgb.as<uint8_t>(), int(page_w), int(page_h), l[0], l[1], l[2], l[3], l[4], l[5],
                             dout.as<float>() + size_t(i) * slot, int(wb)});
        }
        line_crop(c, crops, roff, sp, c.stream());
        c.d2h(out, dout.get(), size_t(count) * slot * sizeof(float));
    });
}

int ocr_pp_line_images(ocr_ctx *ctx, const uint8_t *rgb, uint32_t page_w, uint32_t page_h, const int32_t *lines,
                       uint32_t count, uint32_t wb, float *out) {
    return guard([&] {
        need(ctx, "ctx");
        need(rgb, "rgb");
        need(lines, "lines");
        need(out, "out");
        if (count == 0) return;
        if (wb == 0 || page_w == 0 || page_h == 0) fail("empty page or batch width");
        Ctx &c = *ctx->ctx;
        c.bind();
        const size_t slot = size_t(3) * PP_LINE_H * wb;
        DBuf drgb(&c, size_t(page_w) * page_h * 3), dout(&c, size_t(count) * slot * sizeof(float));
        c.h2d(drgb.get(), rgb, size_t(page_w) * page_h * 3);
        std::vector<PpCropLine> crops;
        for (uint32_t i = 0; i < count; i++) {
            const int32_t *l = lines + size_t(i) * 5;
            if (l[2] < 1 || l[3] < 1 || l[4] < 1 || uint32_t(l[4]) > wb) fail("line box or width out of range");
            crops.push_back({drgb.as<uint8_t>(), int(page_w), int(page_h), l[0], l[1], l[2], l[3], l[4],
                             dout.as<float>() + size_t(i) * slot, int(wb)});
        }
        DBuf dc(&c, crops.size() * sizeof(PpCropLine));
        c.h2d(dc.get(), crops.data(), crops.size() * sizeof(PpCropLine));
        pp_line_crop(dc.as<PpCropLine>(), int(count), int(wb), c.stream());
        c.d2h(out, dout.get(), size_t(count) * slot * sizeof(float));
    });
}

}  // extern "C"
