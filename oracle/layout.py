"""ORACLE (test infrastructure only): the page layout before recognition, restated apart from the
product's host code, as the oracle of the page pipeline.

- Words: src/bin/ocr-bench.rs:40-60 (ocrs' find_connected_component_rects) through contours.c:
  external contours (Suzuki-Abe), Douglas-Peucker with epsilon 2, minimum-area rectangle, grown by
  3 px, area at least 100.
- DB boxes: src/ppdet.rs:63-132 (contours, simplification and rectangle as above, score in f32,
  unclip, reading order).
- Line padding: src/bin/ocr-bench.rs:534-558. Batches: src/bin/ocr-bench.rs:385-407.
- Text lines and line-image geometry: ocrs 0.13.1's find_text_lines and
  prepare_recognition_input (called at ocr-bench.rs:516 and 378) are not available here (the crate
  is not vendored and no Rust toolchain exists). What is restated is the library's own documented
  rule for them (a word joins the line whose last word ends nearest before it when they overlap
  vertically by half the smaller height and the gap is at most twice the taller height; the line
  polygon of the words' top and bottom edges, floored, filled by the even-odd rule at pixel
  centres, resized to height 64 keeping the aspect ratio, width clamped to [10, 800]). The lines
  are pinned against ocrs's own lines on the reference's four 300-dpi pages
  (results/texts-245k/ocrs_0..3.txt; tests/test_ocrs_lines.py): the same line counts, reading
  order and line extents. The rule's word-level decisions beyond those pages stay unpinned.

Arithmetic is float32 in the order the restated steps give it, so results are comparable bit for
bit.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import graph

F32 = np.float32
LINE_H, LINE_MIN_W, LINE_MAX_W = 64, 10, 800


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _bits(bits):
    return np.ascontiguousarray(bits, np.uint32)


# ---- contours, simplification, rectangles (contours.c) --------------------------------------
def find_contours(bits: np.ndarray, w: int):
    """Every border of the mask: a list of (type, parent, points [n, 2] as x, y), type 1 outer,
    2 hole, parent the list index of the enclosing border or -1 for the frame."""
    bits = _bits(bits)
    L = graph.lib()
    c = L.orc_find_contours(_p(bits), w, bits.shape[0])
    try:
        n, npts = L.orc_contours_count(c), L.orc_contours_points(c)
        typ, par = np.zeros(n, np.int32), np.zeros(n, np.int32)
        off, xy = np.zeros(n + 1, np.int32), np.zeros((max(npts, 1), 2), np.int32)
        L.orc_contours_get(c, _p(typ), _p(par), _p(off), _p(xy))
    finally:
        L.orc_contours_free(c)
    return [(int(typ[k]), int(par[k]), xy[off[k]: off[k + 1]].copy()) for k in range(n)]


def external_contours(bits: np.ndarray, w: int):
    """RetrievalMode::External: the outer borders whose parent is the frame, as point arrays."""
    return [pts for t, p, pts in find_contours(bits, w) if t == 1 and p == -1]


def simplify_polygon(points, eps: float = 2.0) -> np.ndarray:
    pts = np.ascontiguousarray(points, np.float32).reshape(-1, 2)
    out = np.zeros_like(pts)
    m = graph.lib().orc_simplify_polygon(_p(pts), len(pts), eps, _p(out))
    return out[:m].copy()


def convex_hull(points) -> np.ndarray:
    pts = np.ascontiguousarray(points, np.float32).reshape(-1, 2)
    out = np.zeros_like(pts)
    m = graph.lib().orc_convex_hull(_p(pts), len(pts), _p(out))
    return out[:m].copy()


def min_area_rect(points):
    """{cx, cy, ux, uy, w, h} as a float32 array, or None."""
    pts = np.ascontiguousarray(points, np.float32).reshape(-1, 2)
    r = np.zeros(6, np.float32)
    return r if graph.lib().orc_min_area_rect(_p(pts), len(pts), _p(r)) else None


def word_rects(bits: np.ndarray, w: int, eps: float = 2.0, expand: float = 3.0, min_area: float = 100.0):
    """ocr-bench.rs:40-60: the words of a page mask as an [n, 6] float32 array (cx, cy, ux, uy,
    w, h), in the order of their contours (raster order of the contour start pixels)."""
    bits = _bits(bits)
    L = graph.lib()
    n = L.orc_word_rects(_p(bits), w, bits.shape[0], eps, expand, min_area, None, 0)
    out = np.zeros((max(n, 1), 6), np.float32)
    L.orc_word_rects(_p(bits), w, bits.shape[0], eps, expand, min_area, _p(out), n)
    return out[:n].copy()


# ---- rotated rectangles -----------------------------------------------------------------------
def corners(r):
    """Top-left, top-right, bottom-right, bottom-left of (cx, cy, ux, uy, w, h): centre plus or
    minus half the height along the up axis and half the width along the right axis (-uy, ux)."""
    cx, cy, ux, uy, w, h = (F32(v) for v in r)
    two = F32(2)
    hx, hy = ux * h / two, uy * h / two
    wx, wy = (-uy) * w / two, ux * w / two
    return ((cx + hx - wx, cy + hy - wy), (cx + hx + wx, cy + hy + wy),
            (cx - hx + wx, cy - hy + wy), (cx - hx - wx, cy - hy - wy))


def bbox(r):
    c = corners(r)
    xs, ys = [p[0] for p in c], [p[1] for p in c]
    return min(xs), min(ys), max(xs), max(ys)


def upright(r) -> bool:
    """ocr-bench.rs:544: the up axis closer to vertical."""
    return abs(F32(r[3])) >= abs(F32(r[2]))


# ---- text lines, padding, geometry, batches ---------------------------------------------------
def find_text_lines(words):
    """Lines of word rects (left to right), lines in reading order (see the module docstring)."""
    boxes = sorted(((bbox(r), i) for i, r in enumerate(words)), key=lambda bi: bi[0][0])
    lines, last = [], []
    half, two = F32(0.5), F32(2)
    for (l, t, r, b), i in boxes:
        best, best_gap = -1, F32(np.inf)
        hb = b - t
        for k, (al, at, ar, ab) in enumerate(last):
            ha = ab - at
            overlap = min(ab, b) - max(at, t)
            gap = l - ar
            if overlap < half * min(ha, hb) or gap > two * max(ha, hb) or gap < -half * min(ha, hb):
                continue
            if gap < best_gap:
                best, best_gap = k, gap
        if best < 0:
            lines.append([i])
            last.append((l, t, r, b))
        else:
            lines[best].append(i)
            last[best] = (l, t, r, b)
    def key(line):
        l, t, _, _ = bbox(words[line[0]])
        return (t, l)
    return [[np.array(words[i], np.float32) for i in line] for line in sorted(lines, key=key)]


def pad_lines(lines, relv: float, relend: float):
    """ocr-bench.rs:534-558: every word grows by relv times the line's median word height
    across the line, the first and last also by relend times it along the line."""
    relv, relend = F32(relv), F32(relend)
    if relv <= 0 and relend <= 0:
        return lines
    out = []
    two = F32(2)
    for line in lines:
        hs = sorted(F32(r[5]) if upright(r) else F32(r[4]) for r in line)
        h = hs[len(hs) // 2] if hs else F32(0)
        n = len(line)
        new = []
        for i, r in enumerate(line):
            r = np.array(r, np.float32)
            along = relend * h if (i == 0 or i + 1 == n) else F32(0)
            across = relv * h
            if upright(r):
                r[4], r[5] = r[4] + two * along, r[5] + two * across
            else:
                r[4], r[5] = r[4] + two * across, r[5] + two * along
            new.append(r)
        out.append(new)
    return out


def line_geometry(words):
    """A line's crop: (box [left, top, bw, bh, out_w], row_off [bh + 1], spans [n, 2]): the polygon
    of the words' top edges left to right and bottom edges right to left, floored; its bounding
    box; per row the spans [x0, x1) of crop columns whose pixel centre lies inside (even-odd), row
    r's from index row_off[r] to row_off[r + 1] of the flattened span ends; the width at height
    64."""
    poly = []
    for r in words:
        c = corners(r)
        poly += [(np.floor(c[0][0]), np.floor(c[0][1])), (np.floor(c[1][0]), np.floor(c[1][1]))]
    for r in reversed(words):
        c = corners(r)
        poly += [(np.floor(c[2][0]), np.floor(c[2][1])), (np.floor(c[3][0]), np.floor(c[3][1]))]
    xs_all, ys_all = [p[0] for p in poly], [p[1] for p in poly]
    l, r_, t, b = min(xs_all), max(xs_all), min(ys_all), max(ys_all)
    left, top = int(l), int(t)
    bw, bh = max(1, int(r_ - l)), max(1, int(b - t))
    aspect = F32(bw) / F32(bh)
    out_w = int(min(max(F32(LINE_H) * aspect, F32(LINE_MIN_W)), F32(LINE_MAX_W)))
    row_off, spans = [], []
    half = F32(0.5)
    for cy in range(bh):
        row_off.append(2 * len(spans))
        Y = F32(top + cy) + half
        xs = []
        for i in range(len(poly)):
            (ax, ay), (cx, cy2) = poly[i], poly[(i + 1) % len(poly)]
            if (ay <= Y and cy2 > Y) or (cy2 <= Y and ay > Y):
                xs.append(ax + (Y - ay) * (cx - ax) / (cy2 - ay))
        xs.sort()
        for k in range(0, len(xs) - 1, 2):
            x0 = max(0, int(np.ceil(xs[k] - half)) - left)
            x1 = min(bw, int(np.ceil(xs[k + 1] - half)) - left)
            if x1 > x0:
                spans.append((x0, x1))
    row_off.append(2 * len(spans))
    box = np.array([left, top, bw, bh, out_w], np.int32)
    return box, np.array(row_off, np.int32), np.array(spans, np.int32).reshape(-1, 2)


def plan_batches(out_w, round_to: int = 50, per_batch: int = 20):
    """ocr-bench.rs:385-407: lines keyed by their width rounded up to a multiple of round_to
    (BTreeMap: keys ascending, members in line order), cut into chunks of per_batch. Returns
    [(width, [line indices])]."""
    groups: dict[int, list[int]] = {}
    for i, w in enumerate(out_w):
        groups.setdefault(-(-int(w) // round_to) * round_to, []).append(i)
    return [(key, groups[key][c: c + per_batch]) for key in sorted(groups)
            for c in range(0, len(groups[key]), per_batch)]


class Layout:
    """The oracle's layout of one page: the same interface as the product's ocrhip.Layout
    (words, nlines, nbatches, line(i) -> (box, row_off, spans), batch(i) -> (width, members))."""

    def __init__(self, bits: np.ndarray, w: int, relv: float = 0.15, relend: float = 0.1):
        self.rects = word_rects(bits, w)
        self.words = len(self.rects)
        self.lines = pad_lines(find_text_lines(list(self.rects)), relv, relend)
        self.geoms = [line_geometry(line) for line in self.lines]
        self.nlines = len(self.lines)
        self.batches = plan_batches([g[0][4] for g in self.geoms])
        self.nbatches = len(self.batches)

    def line(self, i: int):
        return self.geoms[i]

    def batch(self, i: int):
        return self.batches[i]


# ---- PP-OCR DB boxes (ppdet.rs:63-132) ---------------------------------------------------------
def db_score(prob: np.ndarray, w: int, h: int, r) -> np.float32:
    """ppdet.rs:65-85: the mean probability (f32 sum, in row-major order) of the pixels whose
    position lies inside r, scanning r's bounding box."""
    l, t, rr, b = bbox(r)
    x0, y0 = int(max(np.floor(l), F32(0))), int(max(np.floor(t), F32(0)))
    x1, y1 = min(int(np.ceil(rr)), w - 1), min(int(np.ceil(b)), h - 1)
    cx, cy, ux, uy, rw, rh = (F32(v) for v in r)
    hw, hh = rw / F32(2), rh / F32(2)
    s, n = F32(0), 0
    for y in range(y0, y1 + 1):
        for x in range(x0, x1 + 1):
            dx, dy = F32(x) - cx, F32(y) - cy
            along = dx * ux + dy * uy
            across = dx * -uy + dy * ux
            if abs(along) <= hh and abs(across) <= hw:
                s = F32(s + prob[y, x])
                n += 1
    return F32(0) if n == 0 else F32(s / F32(n))


def db_boxes(bits: np.ndarray, prob: np.ndarray, w: int, h: int, to_page, box_thresh=0.45, unclip_ratio=1.4,
             min_size=3.0):
    """ppdet::boxes from the thresholded map (bits) and the map (prob [h, w]): boxes in page
    coordinates, reading order, as an [n, 6] float32 array."""
    box_thresh, unclip, min_size = F32(box_thresh), F32(unclip_ratio), F32(min_size)
    out = []
    two = F32(2)
    for pts in external_contours(bits, w):
        r = min_area_rect(simplify_polygon(pts.astype(np.float32), 2.0))
        if r is None:
            continue
        if min(r[4], r[5]) < min_size or db_score(prob, w, h, r) < box_thresh:
            continue
        rw, rh = r[4], r[5]
        d = rw * rh * unclip / max(two * (rw + rh), F32(1e-6))
        nw, nh = rw + two * d, rh + two * d
        if min(nw, nh) < min_size + two:
            continue
        s = (F32(to_page[0]) + F32(to_page[1])) / two
        out.append(np.array([r[0] * F32(to_page[0]), r[1] * F32(to_page[1]), r[2], r[3], nw * s, nh * s], np.float32))
    out.sort(key=lambda r: bbox(r)[1])
    for i in range(len(out)):
        j = i
        while j > 0:
            a, b = bbox(out[j - 1]), bbox(out[j])
            if abs(b[1] - a[1]) < F32(10) and b[0] < a[0]:
                out[j - 1], out[j] = out[j], out[j - 1]
                j -= 1
            else:
                break
    return np.array(out, np.float32).reshape(-1, 6)


def pp_line_box(box, relv: float, page_w: int, page_h: int):
    """A DB box as a PP-OCR line: grown by relv times its height across (ocr-bench.rs:538-555 with
    one box a line and relend 0), its bounding rectangle clamped to the page as ppocr::line_input
    does (ppocr.rs:42-45, at least 1 x 1), and the width at height 48 (ppocr.rs:53). Returns
    (left, top, cw, ch, out_w)."""
    (r,), = pad_lines([[np.asarray(box, np.float32)]], relv, 0.0)
    l, t, rr, b = bbox(r)

    def clampf(v, hi):
        return int(min(max(v, F32(0)), F32(hi)))
    left, top, right, bottom = clampf(l, page_w), clampf(t, page_h), clampf(rr, page_w), clampf(b, page_h)
    cw, ch = max(right - left, 1), max(bottom - top, 1)
    out_w = min(max(int(np.ceil(F32(48) * F32(cw) / F32(ch))), 8), 3200)
    return (left, top, cw, ch, out_w)
