// Host geometry of the page pipeline: words from the detection mask, text lines, line padding
// and the line-image layout. The reference takes these from ocrs 0.13.1 and rten-imageproc
// 0.26.0 (src/bin/ocr-bench.rs:40-60, 516, 534-558, 366-408), which are not available here;
// this is the library's own restatement of the same steps (see each function).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace ocr {

// A rotated rectangle: centre, unit "up" axis (image coordinates, y down), width across the up
// axis and height along it (rten-imageproc's RotatedRect).
struct RRect {
    float cx = 0, cy = 0, ux = 0, uy = -1, w = 0, h = 0;
    float rx() const { return -uy; }  // the width axis: up rotated a quarter turn clockwise
    float ry() const { return ux; }
    void corners(float xs[4], float ys[4]) const;  // top-left, top-right, bottom-right, bottom-left
    void bbox(float &l, float &t, float &r, float &b) const;
    float area() const { return w * h; }
    bool upright() const;  // up axis closer to vertical (ocr-bench.rs:544)
    void resize(float nw, float nh) { w = nw; h = nh; }
};

// Priority of this thread's parallel loops (word boxes, line geometry) in the shared host loop
// pool: lower runs first.
void set_loop_priority(int prio);

// word_rects (ocr-bench.rs:40-60): the external 8-connected components of the mask (h rows of
// ceil(w/32) words; components inside a hole of another one are left out, as
// find_contours(RetrievalMode::External) does), each one's outer border (Suzuki-Abe border
// following) simplified by Douglas-Peucker with epsilon 2, its minimum-area rectangle grown by
// `expand` on every side, kept when its area is at least min_area; in raster order of the
// components' first pixels; on `threads` threads (the same result).
std::vector<RRect> word_rects(const uint32_t *bits, int w, int h, float expand = 3.f, float min_area = 100.f,
                              int threads = 1);

// The same rectangles from the mask's components as labelled on the GPU (kernels/ccl.hip):
// comps holds ncomps records {first run, top row, rows, first slot} in any order, and row slot
// i (of nslots) a component's leftmost and rightmost pixel xmin[i] .. xmax[i] in one row, its
// rows' slots consecutive from the top. The borders are traced in the mask bits from each
// component's first pixel (the leftmost of its top row).
std::vector<RRect> word_rects_from_rows(const uint32_t *bits, int w, int h, const int32_t *comps, int ncomps,
                                        const uint32_t *xmin, const uint32_t *xmax, int nslots, float expand = 3.f,
                                        float min_area = 100.f, int threads = 1);

// Text lines from words, left to right within a line, lines top to bottom (the role of ocrs'
// find_text_lines, ocr-bench.rs:516).
std::vector<std::vector<RRect>> find_text_lines(const std::vector<RRect> &words);

// Line padding (ocr-bench.rs:534-558): every word grows by relv * h across the line, the first
// and last by relend * h along it, h the line's median word height.
void pad_lines(std::vector<std::vector<RRect>> &lines, float relv, float relend);

// The image of one text line: the polygon of its words' top edges (left to right) and bottom
// edges (right to left), floored to pixels; its bounding box [left, left + bw) x [top, top + bh)
// on the page; the pixels inside it as spans per row (even-odd rule at pixel centres); and the
// width the 64-high line image is resized to (aspect ratio kept, clamped to [10, 800]).
struct LineGeom {
    int left = 0, top = 0, bw = 0, bh = 0, out_w = 0;
    std::vector<int32_t> row_off;  // bh + 1 offsets into spans
    std::vector<int32_t> spans;    // pairs [x0, x1) of crop columns
};
LineGeom line_geometry(const std::vector<RRect> &words);

constexpr int LINE_H = 64, LINE_MIN_W = 10, LINE_MAX_W = 800;

// ocrs batching (ocr-bench.rs:385-407): lines grouped by their width rounded up to 50, in order
// of that width, at most 20 a batch. Returns for every batch its line indices and width.
struct BatchPlan {
    std::vector<std::vector<int>> lines;
    std::vector<int> width;
};
BatchPlan plan_batches(const std::vector<int> &out_w, int round_to = 50, int per_batch = 20);

// ---- PP-OCR (DB detection, SVTR recognition) ----------------------------------------------
// DB post-processing parameters (ppdet.rs:48-61; the threshold itself runs on the GPU).
struct DbParams {
    float box_thresh = 0.45f, unclip_ratio = 1.4f, min_size = 3.f;
};

// ppdet::boxes (ppdet.rs:87-132) from the thresholded map (bits) and the map itself (prob, for
// the box scores), both w x h: each external component's rectangle as word_rects finds it (outer
// border, Douglas-Peucker with epsilon 2, minimum-area rectangle), kept when its shorter side is
// at least min_size and its mean probability (an f32 sum) at least box_thresh, grown by the DB
// unclip offset, scaled to the page and put in reading order.
std::vector<RRect> db_boxes(const uint32_t *bits, const float *prob, int w, int h, float to_page_x, float to_page_y,
                            const DbParams &db = DbParams{});

constexpr int PP_LINE_H = 48, PP_CLASSES = 18708;

// One PP-OCR line image: the page box [left, left + cw) x [top, top + ch) and the width it is
// resized to at height 48.
struct PpLine {
    int left = 0, top = 0, cw = 1, ch = 1, out_w = 8;
};
// A DB box as a line (ocr-bench.rs:538-555 with relv, relend 0) and its crop (ppocr.rs:42-53).
PpLine pp_line_box(const RRect &box, float relv, int page_w, int page_h);

// PP-OCR batching (ocr-bench.rs:330-345): sorted by width, per_batch a batch, each padded to its
// widest line rounded up to a multiple of 8.
BatchPlan plan_pp_batches(const std::vector<int> &out_w, int per_batch = 16);

// Greedy CTC for the PP-OCR head (ppocr.rs:23-33) with a synthetic dictionary: class k in
// [1, 18706] is code point U+4E00 + k - 1 (UTF-8), class 18707 the space, 0 the blank.
std::string pp_ctc_decode(const uint32_t *best, int steps);

// Greedy CTC over per-step arg-max classes (ocr-bench.rs:62-74): emit when best != 0,
// best != prev and t * 4 < width. Classes index the 96-character ocrs alphabet (class 0 blank).
std::string ctc_decode(const uint32_t *best, int steps, int stride, int width);
extern const char *const OCRS_ALPHABET;

}  // namespace ocr
