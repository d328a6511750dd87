/*
 * ocrhip: the GPU path of wgpu-ocr (huppiflupp/wgpu-ocr) rebuilt for AMD Instinct MI355X
 * (gfx950) as HIP kernels behind a C ABI.
 *
 * Each entry point names the reference interface it replaces (file:line in the reference tree).
 * Conventions: functions returning int give OCR_OK (0) or OCR_ERR (1); the message of the last
 * failure on the calling thread is ocr_last_error(). Functions returning a pointer give NULL on
 * failure. No exception or abort crosses this boundary. A context, and everything made from it,
 * is used by one host thread at a time (the reference's Gpu is !Sync, src/gpu.rs:835). Output
 * buffers belong to the caller and are sized with the *_dims queries.
 */
#ifndef OCRHIP_H
#define OCRHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OCR_OK 0
#define OCR_ERR 1

typedef struct ocr_ctx ocr_ctx;
typedef struct ocr_detector ocr_detector;
typedef struct ocr_recognizer ocr_recognizer;
typedef struct ocr_pipeline ocr_pipeline;

/* Options of a context. lines: lines per GRU workgroup (LINES, src/bin/ocr-bench.rs:135; this
 * build's recurrence always groups 8, the lines whose hi and lo parts fill one MFMA operand's 16
 * columns; any value is taken). pool_mb: the scratch pool's cap (POOLMB, src/gpu.rs:919).
 * device: the HIP device index. */
typedef struct ocr_opts {
    uint32_t lines;
    uint32_t pool_mb;
    int32_t device;
} ocr_opts;

/* Message of the last failure on this thread ("" if none). */
const char *ocr_last_error(void);
const char *ocr_version(void);

/* Gpu::new (src/gpu.rs:850-920): the device, its stream and the scratch pool. opts may be NULL. */
ocr_ctx *ocr_create(const ocr_opts *opts);
void ocr_destroy(ocr_ctx *ctx);
/* Wait for all work queued on the context (the reference's submit_wait, src/gpu.rs:1005-1008). */
int ocr_synchronize(ocr_ctx *ctx);

/* Device memory of the context's GPU, for callers that keep inputs resident in HBM
 * (the reference's upload / read, src/gpu.rs:922-936, 1039-1055). Copies are ordered on the
 * context's stream; ocr_memcpy_d2h returns when the data is on the host. */
void *ocr_device_alloc(ocr_ctx *ctx, size_t bytes);
int ocr_device_free(ocr_ctx *ctx, void *p);
int ocr_memcpy_h2d(ocr_ctx *ctx, void *dst, const void *src, size_t bytes);
int ocr_memcpy_d2h(ocr_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Page-locked host memory (hipHostMalloc) for pages a caller renders straight into: the page
 * pipeline's upload copies from it with no staging copy. The reference has no counterpart (its
 * uploads go through wgpu's staging, src/gpu.rs:922-936). ocr_host_free waits for the context's
 * stream first. */
void *ocr_host_alloc(ocr_ctx *ctx, size_t bytes);
int ocr_host_free(ocr_ctx *ctx, void *p);
/* Memory accounting, no counterpart in the reference: device_allocs and host_allocs count every
 * device (hipMalloc) and page-locked host (hipHostMalloc) allocation the library has made in
 * this process; pool_live and pool_held are the bytes of ctx's scratch pool handed out and kept
 * for reuse (src/gpu.rs:938-966 keeps the same pool without reporting it). Any pointer may be
 * NULL. */
int ocr_memory_stats(ocr_ctx *ctx, uint64_t *device_allocs, uint64_t *host_allocs, uint64_t *pool_live,
                     uint64_t *pool_held);

/* ---- Page images ------------------------------------------------------------------------------
 * The reference's page decode, image::open(p)?.into_rgb8() (src/bin/ocr-bench.rs:424, also
 * src/bin/stages.rs:94 and src/bin/ppocr-bench.rs:69; image 0.25.10 over png 0.18.1), for PNG
 * files given as their bytes. ocr_png_dims reads the signature and the IHDR chunk. ocr_png_decode
 * writes w x h RGB triples, row by row, into rgb (cap bytes, at least w * h * 3; memory from
 * ocr_host_alloc is uploaded by the page pipeline with no staging copy). Every colour type, bit
 * depth and Adam7 interlacing: grey replicated, alpha dropped, 16-bit samples rounded to 8 bits.
 * Chunk CRCs are checked. Host only and thread-safe, so pages decode side by side on the caller's
 * threads; no context is needed. */
int ocr_png_dims(const uint8_t *png, size_t n, uint32_t *w, uint32_t *h);
int ocr_png_decode(const uint8_t *png, size_t n, uint8_t *rgb, size_t cap, uint32_t *w, uint32_t *h);

/* ---- A graph parsed on the host ---------------------------------------------------------------
 * The reference parses the .onnx file on its own side (Onnx::load, src/onnx.rs:88-123) and hands
 * the parsed Onnx to the constructors (Detector::new(&Gpu, &Onnx), src/gpu.rs:1385). These
 * structs carry the same content (src/onnx.rs:8-56): nodes with their attributes (Constant nodes
 * already turned into weights or integer lists), float weights, int64 constants, the input and
 * output names. Everything is copied during the constructor call; the caller's memory may be
 * released afterwards. */
typedef struct ocr_onnx_attr {
    const char *name;
    int32_t type;     /* ONNX AttributeProto type: 1 FLOAT, 2 INT, 3 STRING, 6 FLOATS, 7 INTS */
    float f;          /* FLOAT */
    int64_t i;        /* INT */
    const char *s;    /* STRING (NUL-terminated) */
    const float *floats;  /* FLOATS */
    const int64_t *ints;  /* INTS */
    uint32_t count;       /* entries of floats or ints */
} ocr_onnx_attr;

typedef struct ocr_onnx_node {
    const char *op;
    const char *const *inputs;  /* "" for an omitted optional input */
    uint32_t ninputs;
    const char *const *outputs;
    uint32_t noutputs;
    const ocr_onnx_attr *attrs;
    uint32_t nattrs;
} ocr_onnx_node;

/* One named tensor: float32 data (Onnx::weights) or int64 values (Onnx::ints), count entries. */
typedef struct ocr_onnx_tensor {
    const char *name;
    const int64_t *dims;
    uint32_t rank;
    const float *data;   /* float32 weights, or NULL */
    const int64_t *ints; /* int64 constants, or NULL */
    uint64_t count;
} ocr_onnx_tensor;

typedef struct ocr_onnx {
    const ocr_onnx_node *nodes;
    uint32_t nnodes;
    const ocr_onnx_tensor *tensors;
    uint32_t ntensors;
    const char *input;
    const char *output;
} ocr_onnx;

/* Detector::new (src/gpu.rs:1385-1387) from an ONNX file (Onnx::load, src/onnx.rs:88-123). */
ocr_detector *ocr_detector_new(ocr_ctx *ctx, const char *onnx_path);
/* Detector::new(&Gpu, &Onnx) (src/gpu.rs:1385) from a graph the host has parsed. */
ocr_detector *ocr_detector_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph);
void ocr_detector_free(ocr_detector *det);

/* Detector::detect_page (src/gpu.rs:1393-1422): rgb is h x w x 3 bytes (host); bits receives
 * h rows of ceil(w / 32) words, bit x % 32 of word x / 32 set where the page-size mask is above
 * thr. Returns when bits is filled. */
int ocr_detect_page(ocr_detector *det, const uint8_t *rgb, uint32_t w, uint32_t h, float thr, uint32_t *bits);

/* The same for `count` pages whose RGB bytes are already in device memory; bits are device
 * buffers too. The pages go through the model as one batch. Queued on the context's stream. */
int ocr_detect_pages_device(ocr_detector *det, const uint8_t *const *d_rgb, const uint32_t *w, const uint32_t *h,
                            uint32_t count, float thr, uint32_t *const *d_bits);

/* Detector::detect (src/gpu.rs:1425-1430): the model's probability map for a [1, 1, h, w]
 * float input (host); prob receives h * w floats. */
int ocr_detect(ocr_detector *det, const float *input, uint32_t h, uint32_t w, float *prob);

/* Graph::build (src/gpu.rs:1104-1240): a convolutional ONNX graph up to (not including) the
 * first node of type stop_op (NULL: the whole graph). The same operator contract as Detector. */
typedef struct ocr_graph ocr_graph;
ocr_graph *ocr_graph_new(ocr_ctx *ctx, const char *onnx_path, const char *stop_op);
/* The same from a graph the host has parsed (Graph::build takes &Onnx, src/gpu.rs:1104). */
ocr_graph *ocr_graph_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph, const char *stop_op);
void ocr_graph_free(ocr_graph *g);
/* Output shape [n, c, h, w] of the graph for an input of shape [n, c, h, w]. */
int ocr_graph_dims(ocr_graph *g, uint32_t n, uint32_t c, uint32_t h, uint32_t w, uint32_t *out_nchw);
/* Graph::run (src/gpu.rs:1243-1377) on a host NCHW float input; out receives the NCHW output
 * (size from ocr_graph_dims). */
int ocr_graph_run(ocr_graph *g, const float *in, uint32_t n, uint32_t c, uint32_t h, uint32_t w, float *out);

/* Recognizer::new (src/gpu.rs:1452-1506). lines as in ocr_opts. */
ocr_recognizer *ocr_recognizer_new(ocr_ctx *ctx, const char *onnx_path, uint32_t lines);
/* Recognizer::new(&Gpu, &Onnx, lines) (src/gpu.rs:1452) from a graph the host has parsed. */
ocr_recognizer *ocr_recognizer_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph, uint32_t lines);
void ocr_recognizer_free(ocr_recognizer *rec);

/* One batch of n line images [n][64][w] (float, the ocrs input convention). */
typedef struct ocr_batch {
    const float *data;
    uint32_t n;
    uint32_t w;
} ocr_batch;

/* Output sizes of ocr_recognize for these batches: tmax steps, ntot lines, classes. */
int ocr_recognize_dims(ocr_recognizer *rec, const ocr_batch *batches, uint32_t count, uint32_t *tmax,
                       uint32_t *ntot, uint32_t *classes);

/* Recognizer::recognize (src/gpu.rs:1510-1602): batches' data on the host. logits receives the
 * raw logits [tmax][ntot][classes] (rows t >= lens[line] are undefined, as in the reference),
 * lens [ntot] every line's step count (its batch's trunk width, src/gpu.rs:1552). best, if not
 * NULL, receives [tmax][ntot] arg-max class per step (the last index on ties, as
 * src/bin/ocr-bench.rs:67 decodes). logits may be NULL when only best is wanted. */
int ocr_recognize(ocr_recognizer *rec, const ocr_batch *batches, uint32_t count, float *logits, uint32_t *lens,
                  uint32_t *best);

/* The same with the batches' data, logits and best in device memory (either may be NULL);
 * lens on the host. Queued on the context's stream. */
int ocr_recognize_device(ocr_recognizer *rec, const ocr_batch *d_batches, uint32_t count, float *d_logits,
                         uint32_t *d_best, uint32_t *lens);

/* Kernel timing for measurement (the role of the reference's OPPROFILE, src/gpu.rs:1247-1368,
 * without its waits): between start and stop, every launch of the kernel family (process-wide:
 * "conv_mfma", "gru", "conv_transpose", "conv_direct", "conv_generic", "maxpool", "mask_up",
 * "grey_resize", "line_crop", "avgpool_t", "argmax", "copy") is bracketed by HIP events on its
 * own stream. stop waits for them and returns the launches, their summed duration in ms and
 * their summed algorithmic FLOPs and bytes. */
int ocr_probe_start(const char *family);
int ocr_probe_stop(const char *family, uint32_t *calls, double *ms, double *flops, double *bytes);

/* ---- Host geometry of the page pipeline (no GPU involved) ------------------------------ */

/* A rotated rectangle: centre, unit up axis (y down), width across it, height along it. */
typedef struct ocr_rrect {
    float cx, cy, ux, uy, w, h;
} ocr_rrect;

/* word_rects (src/bin/ocr-bench.rs:40-60): the words of a page mask (h rows of ceil(w / 32)
 * words): 8-connected components, minimum-area rectangles grown by 3 px, area >= 100. Writes
 * at most cap rectangles; *count receives the number found. */
int ocr_word_rects(const uint32_t *bits, uint32_t w, uint32_t h, ocr_rrect *out, uint32_t cap, uint32_t *count);
/* The same on `threads` host threads (the page cut into row bands labelled side by side, joined
 * across the cuts): the same rectangles in the same order. The page pipeline's layout runs so. */
int ocr_word_rects_mt(const uint32_t *bits, uint32_t w, uint32_t h, uint32_t threads, ocr_rrect *out, uint32_t cap,
                      uint32_t *count);
/* The same with the mask's components labelled on the GPU of ctx, down to each component's
 * leftmost and rightmost pixel per row (the page pipeline's path: the host only turns those rows
 * into a hull and a rectangle). The same rectangles in the same order; no counterpart in the
 * reference, which finds the components on the host. */
int ocr_word_rects_gpu(ocr_ctx *ctx, const uint32_t *bits, uint32_t w, uint32_t h, ocr_rrect *out, uint32_t cap,
                       uint32_t *count);

/* The same rectangles as ocr_word_rects_gpu without any device allocation: no counterpart in the
 * reference; for callers that cannot allocate device memory (serving loops, harnesses that forbid
 * hipMalloc). The labelling runs in one fixed device array of 4.56 MiB per GPU, set up by
 * ocr_create and held until the process ends. Limits: at most 16384 rows and 2^19 mask words
 * (ceil(w / 32) * h; a 4096 x 4096 page); larger masks fail with an error. A mask with more than
 * 131072 runs, 16384 components or 65536 component rows is labelled on the host instead (the
 * same rectangles). Calls on one GPU share the array and run one at a time. Host-side geometry
 * uses ordinary heap memory. */
int ocr_word_rects_gpu_noalloc(ocr_ctx *ctx, const uint32_t *bits, uint32_t w, uint32_t h, ocr_rrect *out,
                               uint32_t cap, uint32_t *count);

/* The page layout before recognition (src/bin/ocr-bench.rs:503-559): words, text lines in
 * reading order, line padding (relv, relend), every line's crop box, polygon spans and resized
 * width, and the batches (ocr-bench.rs:385-407). */
typedef struct ocr_layout ocr_layout;
ocr_layout *ocr_layout_page(const uint32_t *bits, uint32_t w, uint32_t h, float relv, float relend);
void ocr_layout_free(ocr_layout *lay);
/* Counts: words, lines, batches. */
int ocr_layout_counts(ocr_layout *lay, uint32_t *words, uint32_t *lines, uint32_t *batches);
/* Line i: box = {left, top, width, height, resized width}; row_off (height + 1 entries) and
 * spans (pairs of crop columns [x0, x1)) may be NULL to query nspans first. */
int ocr_layout_line(ocr_layout *lay, uint32_t i, int32_t *box, int32_t *row_off, int32_t *spans, uint32_t *nspans);
/* Batch i: its width and members (line indices, at most 20). */
int ocr_layout_batch(ocr_layout *lay, uint32_t i, uint32_t *width, uint32_t *lines, uint32_t *count);

/* ---- The page pipeline (src/bin/ocr-bench.rs:133-310, 458-585) ------------------------- */

/* merge: pages per recognition pass (MERGE); relv / relend: line padding (RELV, RELEND);
 * thr: detection threshold; threads: host worker threads (0 = up to 16); det_batch: pages per
 * detection pass. Zeros take the defaults 2, 0.15, 0.1, 0.5, 0, 3.
 * label_runs / label_comps / label_slots: capacities of the GPU labelling of a page's mask
 * (0 = 131072 runs, 16384 components, 65536 component rows). A page that needs more, or is
 * wider or taller than 65536 pixels, is labelled on the host from its mask bits instead, with
 * the same words. */
typedef struct ocr_pipeline_opts {
    uint32_t merge;
    float relv;
    float relend;
    float thr;
    uint32_t threads;
    uint32_t det_batch;
    uint32_t label_runs;
    uint32_t label_comps;
    uint32_t label_slots;
} ocr_pipeline_opts;

typedef struct ocr_pipeline_stats {
    double ms;           /* wall time of the last run */
    double cpu_busy_ms;  /* host worker time spent on layout and decoding */
    uint32_t pages, lines, words, batches, rec_passes;
    uint64_t rec_steps;      /* GRU steps summed over lines */
    uint32_t host_labelled;  /* pages whose mask was labelled on the host (over the capacities) */
} ocr_pipeline_stats;

ocr_pipeline *ocr_pipeline_new(ocr_detector *det, ocr_recognizer *rec, const ocr_pipeline_opts *opts);
void ocr_pipeline_free(ocr_pipeline *pipe);
/* Runs every page: RGB bytes (h x w x 3) already in device memory. Returns when all text is
 * decoded. */
int ocr_pipeline_run_device(ocr_pipeline *pipe, const uint8_t *const *d_rgb, const uint32_t *w, const uint32_t *h,
                            uint32_t npages);
/* The same with the pages in host memory, as the reference's run receives them
 * (src/bin/ocr-bench.rs:458-587; each page uploaded inside detect_page, src/gpu.rs:1402-1406).
 * Each detection group's pages go to the device on a copy stream of their own while the earlier
 * groups are detected and recognised: through a pinned staging ring (host copies on the host
 * worker threads), or straight from the caller's memory when it is page-locked
 * (ocr_host_alloc). Per-page errors (ocr-bench.rs:277-281, 303-307): a page that fails keeps its
 * error (ocr_pipeline_page_error) and the other pages finish; the call then returns OCR_ERR with
 * the number of failed pages and the first error. */
int ocr_pipeline_run(ocr_pipeline *pipe, const uint8_t *const *rgb, const uint32_t *w, const uint32_t *h,
                     uint32_t npages);
/* Why a page of the last run failed ("" when it finished); *len receives the message length. */
int ocr_pipeline_page_error(ocr_pipeline *pipe, uint32_t page, char *buf, uint32_t cap, uint32_t *len);
int ocr_pipeline_stats_get(ocr_pipeline *pipe, ocr_pipeline_stats *out);
/* Lines and words found on a page of the last run. */
int ocr_pipeline_page(ocr_pipeline *pipe, uint32_t page, uint32_t *lines, uint32_t *words);
/* Text of one line (UTF-8, NUL-terminated, truncated to cap bytes); *len receives its length. */
int ocr_pipeline_line_text(ocr_pipeline *pipe, uint32_t page, uint32_t line, char *buf, uint32_t cap, uint32_t *len);

/* ---- The N-D executor for the PP-OCRv6 models (src/nd.rs) ----------------------------------- */

typedef struct ocr_nd ocr_nd;

/* NdGraph::new (src/nd.rs:505-817): any ONNX graph of the reference's N-D operator set, with its
 * load-time fusions. stop_before_softmax: the run returns the logits a final Softmax would read
 * (the arg-max needs no Softmax). */
ocr_nd *ocr_nd_new(ocr_ctx *ctx, const char *onnx_path, int stop_before_softmax);
/* NdGraph::new(&Gpu, &Onnx, stop_before_softmax) (src/nd.rs:505) from a graph the host has parsed. */
ocr_nd *ocr_nd_new_onnx(ocr_ctx *ctx, const ocr_onnx *graph, int stop_before_softmax);
void ocr_nd_free(ocr_nd *g);
/* The fusion plan NdGraph::new makes for an ONNX file (the operator contract of src/nd.rs:505-817),
 * as text, without a GPU: one line a launch, "<kind> <op>@<node> [<nodes>] [act=<a>] [bias=<n>]
 * [bn@<node>] [residual=<value>] [in_scale=<value>] -> <output>", in the order they run (node
 * indices after Identity nodes and unused nodes are dropped). Writes at most cap bytes, NUL
 * included, into buf (which may be NULL); *len receives the length without the NUL. */
int ocr_nd_plan(const char *onnx_path, int stop_before_softmax, char *buf, uint32_t cap, uint32_t *len);
/* Output shape (rank <= 6) for an input shape, without running the graph. */
int ocr_nd_dims(ocr_nd *g, const int64_t *in_shape, uint32_t rank, int64_t *out_shape, uint32_t *out_rank);
/* NdGraph::run (src/nd.rs:834-1195) on a row-major float input (host); out receives the output
 * (its size from ocr_nd_dims). */
int ocr_nd_run(ocr_nd *g, const float *in, const int64_t *in_shape, uint32_t rank, float *out);
/* The same with input and output in device memory, queued on the context's stream. */
int ocr_nd_run_device(ocr_nd *g, const float *d_in, const int64_t *in_shape, uint32_t rank, float *d_out);
/* NdGraph::argmax_record / argmax (src/nd.rs:1373-1392): the arg-max over the output's last axis
 * per row, the first index on ties (nd.rs:383); best has one entry per row. A graph that ends in
 * a Linear (the CTC head) never writes its logits: the GEMM keeps per-block maxima. */
int ocr_nd_argmax(ocr_nd *g, const float *in, const int64_t *in_shape, uint32_t rank, uint32_t *best);
int ocr_nd_argmax_device(ocr_nd *g, const float *d_in, const int64_t *in_shape, uint32_t rank, uint32_t *d_best);
/* NdGraph::det_input (src/nd.rs:1353-1369): the size of the PP-OCR detection input for a page
 * (long side at most max_side, sides rounded to multiples of 32) and the factors back to the
 * page (to_page may be NULL). */
int ocr_nd_det_input_dims(uint32_t w, uint32_t h, uint32_t max_side, uint32_t *ow, uint32_t *oh, float *to_page);
/* The detection input itself: rgb h x w x 3 bytes -> out [1][3][oh][ow] floats, bilinear
 * half-pixel, BGR, ImageNet mean and deviation. Host buffers; the _device form takes device
 * buffers and is queued on the context's stream. */
int ocr_nd_det_input(ocr_ctx *ctx, const uint8_t *rgb, uint32_t w, uint32_t h, uint32_t max_side, float *out);
int ocr_nd_det_input_device(ocr_ctx *ctx, const uint8_t *d_rgb, uint32_t w, uint32_t h, uint32_t max_side,
                            float *d_out);
/* DB thresholding (the first step of ppdet::boxes, src/ppdet.rs:88) on the GPU: prob (h rows of
 * w floats) > thr as h rows of ceil(w / 32) bit words. */
int ocr_db_threshold(ocr_ctx *ctx, const float *prob, uint32_t w, uint32_t h, float thr, uint32_t *bits);
int ocr_db_threshold_device(ocr_ctx *ctx, const float *d_prob, uint32_t w, uint32_t h, float thr, uint32_t *d_bits);

/* ---- The PP-OCR page pipeline (src/bin/ocr-bench.rs with DET=ppocr REC=ppocr) --------------- */

typedef struct ocr_pp_pipeline ocr_pp_pipeline;

/* merge: pages per recognition pass (MERGE); thr: DB threshold (ppdet.rs:58; 0.3 here);
 * relv: box padding across (RELV, 0.1 with DET=ppocr, ocr-bench.rs:540); max_side: detection
 * input's long side (DETMAX); per_batch: lines per batch (PPBATCH); threads: host workers;
 * det_batch: same-size pages per detection pass; box_thresh, unclip_ratio, min_size: DB
 * post-processing (ppdet.rs:55-60). Zeros take the defaults 2, 0.3, 0.1, 960, 16, 0, 4, 0.45,
 * 1.4, 3. */
typedef struct ocr_pp_opts {
    uint32_t merge;
    float thr;
    float relv;
    uint32_t max_side;
    uint32_t per_batch;
    uint32_t threads;
    uint32_t det_batch;
    float box_thresh;
    float unclip_ratio;
    float min_size;
} ocr_pp_opts;

/* det: the DB detector; rec: the SVTR recogniser, best built with stop_before_softmax (its head
 * arg-max then never writes logits). Both from the same context. */
ocr_pp_pipeline *ocr_pp_pipeline_new(ocr_nd *det, ocr_nd *rec, const ocr_pp_opts *opts);
void ocr_pp_pipeline_free(ocr_pp_pipeline *pipe);
/* Every page: detection input and map on the GPU, DB boxes on the host, line images and
 * recognition on the GPU, CTC on the host, pages overlapped (ocr-bench.rs:186-284, 500-560).
 * RGB bytes (h x w x 3) in device memory; the second form takes host memory. */
int ocr_pp_pipeline_run_device(ocr_pp_pipeline *pipe, const uint8_t *const *d_rgb, const uint32_t *w, const uint32_t *h,
                               uint32_t npages);
int ocr_pp_pipeline_run(ocr_pp_pipeline *pipe, const uint8_t *const *rgb, const uint32_t *w, const uint32_t *h,
                        uint32_t npages);
int ocr_pp_pipeline_stats_get(ocr_pp_pipeline *pipe, ocr_pipeline_stats *out);
/* Lines (DB boxes) of a page of the last run, and the text of one (UTF-8; the synthetic
 * dictionary maps class k >= 1 to U+4E00 + k - 1 and the last class to a space). */
int ocr_pp_pipeline_page(ocr_pp_pipeline *pipe, uint32_t page, uint32_t *lines);
int ocr_pp_pipeline_line_text(ocr_pp_pipeline *pipe, uint32_t page, uint32_t line, char *buf, uint32_t cap,
                              uint32_t *len);

/* ppdet::boxes (src/ppdet.rs:87-132) on the host from a thresholded map (bits, h rows of
 * ceil(w / 32) words) and the map (prob, h x w): the boxes in page coordinates and reading order.
 * Zeros take the defaults 0.45, 1.4, 3. Writes at most cap boxes; *count receives the number. */
int ocr_db_boxes(const uint32_t *bits, const float *prob, uint32_t w, uint32_t h, float to_page_x, float to_page_y,
                 float box_thresh, float unclip_ratio, float min_size, ocr_rrect *out, uint32_t cap, uint32_t *count);
/* One box as a PP-OCR line image (ocr-bench.rs:538-555, ppocr.rs:42-53): out = {left, top,
 * width, height, resized width at height 48} on a page_w x page_h page. */
int ocr_pp_line_box(const ocr_rrect *box, float relv, uint32_t page_w, uint32_t page_h, int32_t *out);
/* ocrs' line images (prepare_recognition_input, called at src/bin/ocr-bench.rs:378, and the batch
 * assembly of ocr-bench.rs:388-404) on the GPU: count lines of an RGB page (host), lines = count x
 * {left, top, width, height, resized width, first row offset} with every line's (height + 1) span
 * offsets in row_off (indices into spans, pairs [x0, x1) of crop columns), into out
 * [count][64][wb] (host), black (-0.5) outside the polygon and past each line's width. */
int ocr_line_images(ocr_ctx *ctx, const uint8_t *rgb, uint32_t page_w, uint32_t page_h, const int32_t *lines,
                    uint32_t count, const int32_t *row_off, uint32_t n_row_off, const int32_t *spans, uint32_t n_spans,
                    uint32_t wb, float *out);
/* ppocr::line_input + ppocr::batch (src/ppocr.rs:42-78) on the GPU: count line images of an RGB
 * page (host), lines = count x {left, top, width, height, resized width}, into out
 * [count][3][48][wb] (host), zero past each line's width. */
int ocr_pp_line_images(ocr_ctx *ctx, const uint8_t *rgb, uint32_t page_w, uint32_t page_h, const int32_t *lines,
                       uint32_t count, uint32_t wb, float *out);

#ifdef __cplusplus
}
#endif

#endif /* OCRHIP_H */
