"""The oracle's page layout (oracle/contours.c, oracle/layout.py), pinned by what fixes it apart
from the product, then the product's host layout against it.

Pins of the oracle:
- border following (Suzuki-Abe): every border's pixel set is exactly the pixels of its
  8-connected component that touch, 4-connectedly, the 0-component on its side (scipy labelling);
  its start is the raster-first such pixel; consecutive points are 8-neighbours; hand-built chains
  (rectangle, line, L shape, lone pixel) in the published visiting order;
- external retrieval: exactly the components that touch the background reaching the frame;
- Douglas-Peucker: hand-built polylines, and on random polygons the defining guarantee (every
  dropped point within epsilon of the kept segment that spans it);
- convex hull: scipy's (qhull) vertex set; minimum-area rectangle: an angle sweep never finds a
  smaller enclosing rectangle and the rectangle encloses every point;
- batching (ocr-bench.rs:385-407) and line padding (ocr-bench.rs:534-558): hand-computed cases.
"""
import numpy as np
import pytest
from scipy import ndimage
from scipy.spatial import ConvexHull

import ocrhip
from ocrhip import synth
from oracle import layout as ol


def pack(mask: np.ndarray) -> np.ndarray:
    h, w = mask.shape
    padded = np.zeros((h, (w + 31) // 32 * 32), bool)
    padded[:, :w] = mask
    return np.packbits(padded, axis=1, bitorder="little").view(np.uint32).copy()


def random_masks(seed=0, count=40):
    rng = np.random.default_rng(seed)
    for it in range(count):
        h, w = int(rng.integers(4, 60)), int(rng.integers(4, 90))
        if it % 2:
            m = rng.random((h, w)) < rng.uniform(0.1, 0.7)
        else:
            m = np.zeros((h, w), bool)
            for _ in range(int(rng.integers(1, 9))):
                y0, x0 = int(rng.integers(0, h)), int(rng.integers(0, w))
                m[y0: y0 + int(rng.integers(1, 25)), x0: x0 + int(rng.integers(1, 50))] ^= True
        yield m


def rings_mask():
    m = np.zeros((120, 160), bool)
    for r in range(4, 55, 5):  # concentric square rings
        m[60 - r: 60 + r + 1, 80 - r] = m[60 - r: 60 + r + 1, 80 + r] = True
        m[60 - r, 80 - r: 80 + r + 1] = m[60 + r, 80 - r: 80 + r + 1] = True
    m[58:63, 78:83] = True  # a blob in the innermost hole
    return m


# ---- border following --------------------------------------------------------------------------
def test_border_sets_match_scipy_labelling():
    eight = np.ones((3, 3), int)
    four = ndimage.generate_binary_structure(2, 1)
    for m in list(random_masks()) + [rings_mask()]:
        h, w = m.shape
        pad = np.pad(m, 1)
        fg, _ = ndimage.label(pad, structure=eight)
        bg, _ = ndimage.label(~pad, structure=four)
        for typ, _, pts in ol.find_contours(pack(m), w):
            x0, y0 = pts[0]
            # the 0-component on the border's side: west of an outer start, east of a hole start
            side = bg[y0 + 1, x0] if typ == 1 else bg[y0 + 1, x0 + 2]
            comp = fg[y0 + 1, x0 + 1]
            touch = np.zeros_like(pad)
            near = bg == side
            touch[1:, :] |= near[:-1, :]
            touch[:-1, :] |= near[1:, :]
            touch[:, 1:] |= near[:, :-1]
            touch[:, :-1] |= near[:, 1:]
            want = {(x - 1, y - 1) for y, x in zip(*np.nonzero(touch & (fg == comp)))}
            got = {(int(x), int(y)) for x, y in pts}
            assert got == want
            # the start: an outer border's at its component's raster-first pixel, a hole border's
            # at the raster-first pixel of its component whose east neighbour lies in the hole
            if typ == 1:
                start = fg == comp
            else:
                start = np.zeros_like(pad)
                start[:, :-1] = (fg[:, :-1] == comp) & (bg[:, 1:] == side)
            ys, xs = np.nonzero(start)
            assert (int(x0), int(y0)) == (xs[0] - 1, ys[0] - 1)
            # a closed chain of 8-neighbours
            if len(pts) > 1:
                step = np.abs(np.diff(np.vstack([pts, pts[:1]]), axis=0))
                assert step.max() <= 1 and (step.sum(axis=1) > 0).all()


def test_external_selection_matches_frame_background():
    eight = np.ones((3, 3), int)
    four = ndimage.generate_binary_structure(2, 1)
    for m in list(random_masks(1)) + [rings_mask()]:
        w = m.shape[1]
        pad = np.pad(m, 1)
        fg, n = ndimage.label(pad, structure=eight)
        bg, _ = ndimage.label(~pad, structure=four)
        frame = ndimage.binary_dilation(bg == bg[0, 0], structure=four)
        want = sorted({int(c) for c in np.unique(fg[frame & (fg > 0)])})
        got = sorted(int(fg[p[0][1] + 1, p[0][0] + 1]) for p in ol.external_contours(pack(m), w))
        assert got == want
    # rings: only the outermost ring is external; the inner ones and the blob are not
    assert len(ol.external_contours(pack(rings_mask()), 160)) == 1


def test_border_chains_hand_built():
    m = np.zeros((6, 7), bool)
    m[1:4, 2:5] = True  # 3 x 3 square: down the left side, along the bottom, up, back along the top
    (t, p, pts), = ol.find_contours(pack(m), 7)
    assert (t, p) == (1, -1)
    assert pts.tolist() == [[2, 1], [2, 2], [2, 3], [3, 3], [4, 3], [4, 2], [4, 1], [3, 1]]
    m = np.zeros((3, 6), bool)
    m[1, 1:5] = True  # a line is walked out and back
    assert ol.external_contours(pack(m), 6)[0].tolist() == [[1, 1], [2, 1], [3, 1], [4, 1], [3, 1], [2, 1]]
    m = np.zeros((5, 5), bool)
    m[1:4, 1] = True
    m[3, 2:4] = True  # an L
    assert ol.external_contours(pack(m), 5)[0].tolist() == [[1, 1], [1, 2], [1, 3], [2, 3], [3, 3], [2, 3], [1, 2]]
    m = np.zeros((3, 3), bool)
    m[1, 1] = True
    assert ol.external_contours(pack(m), 3)[0].tolist() == [[1, 1]]
    # a ring with a blob inside: outer border, hole border (child), blob (child of the hole)
    m = np.zeros((7, 7), bool)
    m[1:6, 1:6] = True
    m[2:5, 2:5] = False
    m[3, 3] = True
    assert [(t, p) for t, p, _ in ol.find_contours(pack(m), 7)] == [(1, -1), (2, 0), (1, 1)]


# ---- Douglas-Peucker -----------------------------------------------------------------------------
def test_simplify_hand_built():
    sq = [[0, 0], [0, 5], [0, 10], [5, 10], [10, 10], [10, 5], [10, 0], [5, 0]]
    # first split at the farthest point from (0, 0): (10, 10); then the corners stay
    assert ol.simplify_polygon(sq).tolist() == [[0, 0], [0, 10], [10, 10], [10, 0]]
    bump = [[0, 0], [5, 1], [10, 0], [10, 20], [0, 20]]  # the 1-pixel bump is dropped at eps 2
    assert ol.simplify_polygon(bump).tolist() == [[0, 0], [10, 0], [10, 20], [0, 20]]
    big = [[0, 0], [5, 3], [10, 0], [10, 20], [0, 20]]  # a 3-pixel bump stays
    assert ol.simplify_polygon(big).tolist() == big
    # equally far points: the last one splits (5, 10) rather than (-5, 10)
    tie = [[0, 0], [-5, 10], [0, 1], [5, 10]]
    assert ol.simplify_polygon(tie, 2.0).tolist() == [[0, 0], [-5, 10], [0, 1], [5, 10]]
    assert ol.simplify_polygon([[3, 4]]).tolist() == [[3, 4]]


def _seg_dist(a, b, p):
    a, b, p = (np.asarray(v, np.float64) for v in (a, b, p))
    ab = b - a
    if not ab.any():
        return np.hypot(*(p - a))
    t = np.clip(np.dot(p - a, ab) / np.dot(ab, ab), 0, 1)
    return np.hypot(*(p - (a + t * ab)))


def test_simplify_guarantee_on_random_polygons():
    rng = np.random.default_rng(3)
    for _ in range(60):
        n = int(rng.integers(3, 60))
        ang = np.sort(rng.uniform(0, 2 * np.pi, n))
        rad = rng.uniform(5, 40, n)
        pts = np.round(np.stack([rad * np.cos(ang), rad * np.sin(ang)], 1)).astype(np.float32)
        eps = float(rng.choice([1.0, 2.0, 4.0]))
        out = ol.simplify_polygon(pts, eps)
        # kept points are input points in order, the first one among them
        idx = []
        for q in out:
            k = next(k for k in range(idx[-1] + 1 if idx else 0, n) if (pts[k] == q).all())
            idx.append(k)
        assert idx[0] == 0
        ring = idx + [n]
        closed = np.vstack([pts, pts[:1]])
        for a, b in zip(ring, ring[1:]):
            for k in range(a + 1, b):
                assert _seg_dist(closed[a], closed[b], closed[k]) <= eps + 1e-4


# ---- hull and minimum-area rectangle -------------------------------------------------------------
def test_hull_matches_qhull():
    rng = np.random.default_rng(4)
    for _ in range(50):
        pts = rng.integers(0, 60, (int(rng.integers(3, 40)), 2)).astype(np.float32)
        if np.linalg.matrix_rank(pts - pts[0]) < 2:
            continue
        want = {tuple(p) for p in pts[ConvexHull(pts).vertices]}
        got = ol.convex_hull(pts)
        assert {tuple(p) for p in got} == want
        # counter-clockwise (cross > 0) from the smallest (x, y)
        assert tuple(got[0]) == min(want)
        e1, e2 = np.roll(got, -1, 0) - got, np.roll(got, -2, 0) - np.roll(got, -1, 0)
        c = e1[:, 0] * e2[:, 1] - e1[:, 1] * e2[:, 0]
        assert (c > 0).all()


def _corners(r):
    cx, cy, ux, uy, w, h = (float(v) for v in r)
    rx, ry = -uy, ux
    return np.array([[cx + s * ux * h / 2 + t * rx * w / 2, cy + s * uy * h / 2 + t * ry * w / 2]
                     for s in (1, -1) for t in (1, -1)])


def test_min_area_rect_angle_sweep():
    rng = np.random.default_rng(5)
    angles = np.linspace(0, np.pi / 2, 2000, endpoint=False)
    for _ in range(40):
        pts = rng.integers(0, 50, (int(rng.integers(3, 25)), 2)).astype(np.float64)
        r = ol.min_area_rect(pts)
        assert r is not None
        area = float(r[4] * r[5])
        # encloses every point
        cx, cy, ux, uy, w, h = (float(v) for v in r)
        d = pts - [cx, cy]
        assert np.all(np.abs(d @ [ux, uy]) <= h / 2 + 1e-3) and np.all(np.abs(d @ [-uy, ux]) <= w / 2 + 1e-3)
        # no rotation does better
        c, s = np.cos(angles), np.sin(angles)
        px, py = pts[:, 0][:, None], pts[:, 1][:, None]
        a = px * c + py * s
        b = -px * s + py * c
        sweep = (a.max(0) - a.min(0)) * (b.max(0) - b.min(0))
        assert area <= sweep.min() * (1 + 1e-5) + 1e-3
        # the up axis points most towards -y of the four turns
        assert -uy >= max(ux, -ux, uy) - 1e-6
    # hand-built: an axis-aligned 10 x 3 box; a diagonal segment
    assert ol.min_area_rect([[0, 0], [10, 0], [10, 3], [0, 3]]).tolist() == [5, 1.5, 0, -1, 10, 3]
    r = ol.min_area_rect([[0, 0], [10, 10]])
    assert r[4] == 0 and abs(r[5] - np.hypot(10, 10)) < 1e-4
    assert ol.min_area_rect([[2, 2], [2, 2]]) is None


def test_word_rects_hand_built():
    m = np.zeros((30, 50), bool)
    m[3:13, 5:25] = True  # 20 x 10 pixels: corners (5, 3) .. (24, 12), grown by 3
    r = ol.word_rects(pack(m), 50)
    assert r.tolist() == [[14.5, 7.5, 0, -1, 25, 15]]
    m = np.zeros((30, 50), bool)
    m[5, 5:16] = True  # 11 pixels: 10 x 0 -> 16 x 6 = 96 < 100, dropped; 12 pixels kept
    assert len(ol.word_rects(pack(m), 50)) == 0
    m[5, 16] = True
    assert ol.word_rects(pack(m), 50).tolist() == [[10.5, 5, 0, -1, 17, 6]]
    # a ring holding a blob: one rectangle (the blob is inside the ring's hole)
    assert len(ol.word_rects(pack(rings_mask()), 160)) == 1


# ---- batching and padding (ocr-bench.rs) ----------------------------------------------------------
def test_plan_batches_rule():
    widths = [49, 50, 51, 100, 800, 10, 101] + [120] * 45
    plan = ol.plan_batches(widths)
    assert plan[0] == (50, [0, 1, 5])
    assert plan[1] == (100, [2, 3])
    assert plan[2] == (150, [6] + list(range(7, 26)))
    assert plan[3] == (150, list(range(26, 46)))
    assert plan[4] == (150, list(range(46, 52)))
    assert plan[5] == (800, [4])


def test_pad_lines_rule():
    up = np.array([10, 10, 0, -1, 40, 20], np.float32)
    side = np.array([50, 10, 1, 0, 30, 12], np.float32)  # up axis horizontal: width is the height
    lines = ol.pad_lines([[up, side, up]], 0.15, 0.1)
    # median of the heights 20, 30, 20 is 20
    a, b, c = lines[0]
    assert a[4] == np.float32(40) + 2 * np.float32(0.1) * 20 and a[5] == np.float32(20) + 2 * np.float32(0.15) * 20
    assert b[4] == np.float32(30) + 2 * np.float32(0.15) * 20 and b[5] == 12
    assert c[4] == a[4] and c[5] == a[5]


# ---- the product against the oracle -------------------------------------------------------------
def product_masks():
    yield from random_masks(7, 60)
    yield rings_mask()
    m = np.zeros((64, 2048), bool)
    m[::3] = True
    m[:, 1000] = True
    yield m
    yield np.eye(120, 130, dtype=bool) | np.eye(120, 130, k=7, dtype=bool)[:, ::-1]
    rng = np.random.default_rng(11)
    yield rng.random((300, 517)) < 0.45
    _, blocks = synth.page(2, with_blocks=True)
    noisy = blocks[:900].copy()
    noisy[rng.random(noisy.shape) < 0.02] ^= True
    yield noisy


def test_product_word_rects_match_oracle():
    for m in product_masks():
        b, w = pack(m), m.shape[1]
        want = ol.word_rects(b, w)
        for t in (1, 4):
            got = ocrhip.word_rects(b, w, threads=t)
            assert got.shape == want.shape
            np.testing.assert_array_equal(got, want)


def test_product_layout_matches_oracle():
    for seed in (0, 1):
        _, blocks = synth.page(seed, with_blocks=True)
        rng = np.random.default_rng(seed)
        m = blocks.copy()
        m[rng.random(m.shape) < 0.002] = True
        b, w = pack(m), m.shape[1]
        got, want = ocrhip.Layout(b, w), ol.Layout(b, w)
        assert (got.words, got.nlines, got.nbatches) == (want.words, want.nlines, want.nbatches)
        for i in range(want.nlines):
            g, o = got.line(i), want.line(i)
            for a, c in zip(g, o):
                np.testing.assert_array_equal(np.asarray(a).reshape(-1), np.asarray(c).reshape(-1))
        for i in range(want.nbatches):
            assert tuple(got.batch(i)[0:1]) == (want.batch(i)[0],)
            assert list(got.batch(i)[1]) == list(want.batch(i)[1])


def test_ground_truth_blocks_give_the_generated_lines():
    # The generator's own word blocks (no detector): every page's 36 text lines are found.
    for seed in (0, 3):
        _, blocks = synth.page(seed, with_blocks=True)
        b, w = pack(blocks), blocks.shape[1]
        assert ocrhip.Layout(b, w).nlines == 36
        assert ol.Layout(b, w).nlines == 36


def test_product_db_boxes_match_oracle():
    rng = np.random.default_rng(13)
    h, w = 240, 320
    prob = (0.1 * rng.random((h, w))).astype(np.float32)
    for y0 in range(10, 230, 24):  # text bands of varying strength, some broken into words
        x = 20
        while x < 290:
            x1 = min(x + int(rng.integers(15, 90)), 300)
            prob[y0: y0 + int(rng.integers(3, 10)), x: x1] = rng.uniform(0.32, 0.95, (1, x1 - x))
            x = x1 + int(rng.integers(3, 12))
    prob[rng.random((h, w)) < 0.01] = 0.9  # specks
    bits = pack(prob > 0.3)
    want = ol.db_boxes(bits, prob, w, h, (2.5, 2.75))
    got = ocrhip.db_boxes(bits, prob, (2.5, 2.75))
    assert len(want) > 5
    np.testing.assert_array_equal(got, want)


def test_product_pp_line_box_matches_oracle():
    rng = np.random.default_rng(17)
    for _ in range(200):
        ang = rng.uniform(-0.3, 0.3) + (np.pi / 2 if rng.random() < 0.2 else 0.0)
        box = np.array([rng.uniform(-50, 1300), rng.uniform(-30, 900), np.sin(ang), -np.cos(ang),
                        rng.uniform(1, 600), rng.uniform(1, 60)], np.float32)
        want = ol.pp_line_box(box, 0.1, 1200, 850)
        got = ocrhip.pp_line_box(box, 0.1, 1200, 850)
        assert tuple(int(v) for v in got) == want
