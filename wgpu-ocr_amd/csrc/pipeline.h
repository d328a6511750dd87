// The whole-page pipeline (the reference's ocr-bench gpu_thread and run, src/bin/ocr-bench.rs:
// 133-310 and 458-585): GPU detection, host words and lines, GPU line images and recognition,
// host CTC, with the GPU and the host cores working on different pages at once.
#pragma once

#include <string>
#include <vector>

#include "geometry.h"
#include "models.h"

namespace ocr {

struct PipelineOpts {
    int merge = 2;        // pages per recognition pass (MERGE, ocr-bench.rs:164; README tuned value 2)
    float relv = 0.15f;   // line padding across, fraction of the median word height (RELV)
    float relend = 0.1f;  // line padding at the ends (RELEND)
    float thr = 0.5f;     // detection threshold
    int threads = 0;      // host worker threads (0: hardware concurrency, at most 16)
    int det_batch = 3;    // pages per detection pass
    bool lookahead = true;  // a recognition pass waits for the next pass's detections to be queued
    // Capacities of the GPU labelling of a page's mask (0: 2^17 runs, 16384 components, 65536
    // row slots); a page that needs more, or is wider or taller than 65536 pixels, is labelled
    // on the host from its bits.
    int label_runs = 0, label_comps = 0, label_slots = 0;
};

struct PageText {
    std::vector<std::string> lines;  // reading order
    int words = 0;
    std::string error;  // why the page failed ("" when it finished)
};

struct PipelineStats {
    double ms = 0, cpu_busy_ms = 0;
    int pages = 0, lines = 0, words = 0, batches = 0, rec_passes = 0;
    long long rec_steps = 0;  // sum over lines of their GRU steps
    int host_labelled = 0;    // pages whose mask was labelled on the host (over the GPU capacities)
};

// Words -> lines -> padding -> line images -> batches for one page (all host work before the
// recogniser), as ocr-bench.rs:503-559 does it per page.
struct PageLayout {
    int words = 0;
    double ms_words = 0, ms_lines = 0, ms_geom = 0;  // wall time of the three steps
    std::vector<LineGeom> lines;
    BatchPlan plan;
    // Every line's row offsets and spans one after another: line i's offsets start at
    // row_off[line_row0[i]] and index this page's spans.
    std::vector<int32_t> row_off, spans, line_row0;
};
// The page mask's components as labelled on the GPU (ccl_runs): its word boxes come from their
// row extremes (word_rects_from_rows) instead of the bits.
struct MaskRows {
    const int32_t *comps;
    int ncomps;
    const uint32_t *xmin, *xmax;
    int nslots;
};
// threads > 1: its loops run on the shared host loop pool at priority page_prio (lower first).
PageLayout layout_page(const uint32_t *bits, int w, int h, float relv, float relend, int threads = 1,
                       int page_prio = 0, const MaskRows *rows = nullptr);

class Pipeline {
  public:
    Pipeline(Ctx &ctx, Detector &det, Recognizer &rec, const PipelineOpts &opts);
    ~Pipeline();
    // All pages' RGB bytes already in device memory.
    void run(const uint8_t *const *d_rgb, const int *w, const int *h, int npages);
    // The pages in host memory: each detection group's pages go to the device on a stream of
    // their own (through pinned staging unless already page-locked) while earlier groups are
    // detected and recognised. A page that fails leaves its error in pages()[p].error and the
    // others finish; the call then throws, naming how many failed and the first error.
    void run_host(const uint8_t *const *rgb, const int *w, const int *h, int npages);
    const std::vector<PageText> &pages() const { return pages_; }
    const PipelineStats &stats() const { return stats_; }
    struct Impl;

  private:
    void run_pages(const uint8_t *const *src, bool on_host, const int *w, const int *h, int npages);
    Impl *impl_;
    std::vector<PageText> pages_;
    PipelineStats stats_;
};

}  // namespace ocr
