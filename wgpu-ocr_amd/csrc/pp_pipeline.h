// The PP-OCR whole-page pipeline (the reference's ocr-bench with DET=ppocr REC=ppocr,
// src/bin/ocr-bench.rs:186-225, 240-284, 500-560): GPU detection input, DB detector and
// threshold; host DB boxes; GPU line images; SVTR recognition with the fused arg-max head;
// host CTC. Pages overlap: the host works on one page's boxes while the GPU detects the next.
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "geometry.h"
#include "nd.h"
#include "pipeline.h"

namespace ocr {

struct PpPipelineOpts {
    int merge = 2;          // pages per recognition pass (MERGE)
    float thr = 0.3f;       // DB threshold
    float relv = 0.1f;      // box padding across, fraction of its height (RELV with DET=ppocr)
    int max_side = 960;     // detection input's long side (DETMAX)
    int per_batch = 16;     // lines per recognition batch (PPBATCH)
    int threads = 0;        // host worker threads (0: hardware concurrency, at most 16)
    int det_batch = 4;      // same-size pages per detection pass
    DbParams db;
};

class PpPipeline {
  public:
    PpPipeline(Ctx &ctx, NdGraph &det, NdGraph &rec, const PpPipelineOpts &opts);
    ~PpPipeline();
    // All pages' RGB bytes already in device memory.
    void run(const uint8_t *const *d_rgb, const int *w, const int *h, int npages);
    // Pages in host memory (page-locked or pageable): a detection group's pages go up on the
    // uploader's stream as the schedule stages them, so later pages upload while earlier ones are
    // detected and recognised (the reference uploads each page in its detection path,
    // src/nd.rs:1353-1369).
    void run_host(const uint8_t *const *rgb, const int *w, const int *h, int npages);
    const std::vector<PageText> &pages() const { return pages_; }
    const PipelineStats &stats() const { return stats_; }

    struct Impl;

  private:
    Impl *impl_;
    // Both entry points: the page pipeline's schedule (pipeline_core.h) over this run's hooks.
    void run_pages(const uint8_t *const *src, bool on_host, const int *w, const int *h, int npages);
    std::vector<PageText> pages_;
    PipelineStats stats_;
};

}  // namespace ocr
