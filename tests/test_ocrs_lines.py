"""The page layout's text lines against the lines ocrs 0.13.1 itself found on the reference's four
300-dpi benchmark pages (results/texts-245k/ocrs_0..3.txt for data/pages/A_300/Text_page_1..4.png;
ocrs `find_text_lines` and `prepare_recognition_input`, called at src/bin/ocr-bench.rs:516 and 378).

The fixture (tests/golden/ocrs_lines.npz, written by tests/golden/make_ocrs_lines.py) holds word
masks of the pages from a stand-in for ocrs's trained detector (ink dilated into word blobs) and
the character count of every line ocrs recognised, in ocrs's reading order. On those masks the
product's layout (words, line grouping, padding, crop geometry) must give:
- exactly as many text lines as ocrs: 43, 42, 42 and 17;
- the lines in reading order, top to bottom;
- line k of the layout the same page line as ocrs's line k: every line's crop width over the
  character count of ocrs's text for it is within 6 % of the page's median (20.2-21.9 px a
  character here), so a line split in two, two lines merged or lines out of order would fail;
- the oracle's independent restatement of the layout: the same boxes, bit for bit.
Where the reference tree is present, ocr_png_decode's pixels of the PNG pages, through the
stand-in, give the fixture's masks exactly. The GPU test labels the masks on the GPU
(ocr_word_rects_gpu) and must give the host's word rectangles and so the same lines.

What this leaves unpinned: the masks come from the stand-in, not from ocrs's detector, so the
word boxes differ from the ones ocrs grouped; the pin is on the line structure ocrs produced.
"""
import importlib.util
import os

import numpy as np
import pytest

import ocrhip
from oracle import layout as ol

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
OCRS_LINES = (43, 42, 42, 17)


def _fixture():
    z = np.load(os.path.join(HERE, "golden", "ocrs_lines.npz"))
    return [(z[f"bits_{k}"], int(z[f"w_{k}"]), z[f"chars_{k}"]) for k in range(4)]


PAGES = _fixture()


def _boxes(lay):
    return np.array([lay.line(i)[0] for i in range(lay.nlines)], np.int64).reshape(-1, 5)


def _check_against_ocrs(boxes, chars, k):
    assert len(boxes) == len(chars) == OCRS_LINES[k], (k, len(boxes), len(chars))
    tops = boxes[:, 1]
    assert np.all(np.diff(tops) > 0), f"page {k + 1}: lines not top to bottom: {tops}"
    ratio = boxes[:, 2] / chars
    dev = np.abs(ratio / np.median(ratio) - 1)
    assert dev.max() < 0.06, f"page {k + 1}: line {int(dev.argmax())} width {boxes[dev.argmax(), 2]} for " \
                             f"{chars[dev.argmax()]} characters of ocrs's text"


@pytest.mark.parametrize("k", range(4))
def test_layout_lines_match_ocrs(k):
    bits, w, chars = PAGES[k]
    print(f"ocrs lines: page {k + 1}", flush=True)
    lay = ocrhip.Layout(bits, w)
    boxes = _boxes(lay)
    _check_against_ocrs(boxes, chars, k)
    want = ol.Layout(bits, w)
    assert want.nlines == lay.nlines
    np.testing.assert_array_equal(boxes, _boxes(want))


def test_fixture_masks_from_the_reference_pngs():
    pngs = [os.path.join(REF, "data", "pages", "A_300", f"Text_page_{k + 1}.png") for k in range(4)]
    if not all(os.path.exists(p) for p in pngs):
        pytest.skip("the reference's page PNGs are not on this machine")
    spec = importlib.util.spec_from_file_location("make_ocrs_lines", os.path.join(HERE, "golden", "make_ocrs_lines.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    for k, p in enumerate(pngs):
        rgb = ocrhip.decode_png(p)
        bits, w, chars = PAGES[k]
        assert rgb.shape[1] == w
        np.testing.assert_array_equal(mk.word_mask(rgb), bits, err_msg=f"page {k + 1}")
        np.testing.assert_array_equal(mk.ocrs_line_lengths(REF, k), chars)


@pytest.mark.gpu
def test_gpu_labelled_words_give_ocrs_lines(ctx):
    for k, (bits, w, chars) in enumerate(PAGES):
        print(f"ocrs lines on the GPU: page {k + 1}", flush=True)
        got = ocrhip.word_rects_gpu(ctx, bits, w)
        want = ocrhip.word_rects(bits, w)
        np.testing.assert_array_equal(got, want)
        assert len(got) > 200
        _check_against_ocrs(_boxes(ocrhip.Layout(bits, w)), chars, k)


def _grouping(words, overlap=0.5, overlap_of=min, max_gap=2.0, order=lambda l, t: (t, l)):
    """The layout's line rule with its constants as knobs (defaults: the rule itself), for the
    planted mistakes below."""
    boxes = sorted(((ol.bbox(r), i) for i, r in enumerate(words)), key=lambda bi: bi[0][0])
    lines, last = [], []
    for (l, t, r, b), i in boxes:
        best, best_gap = -1, np.float32(np.inf)
        for j, (al, at, ar, ab) in enumerate(last):
            ha, hb = ab - at, b - t
            ov, gap = min(ab, b) - max(at, t), l - ar
            if ov < np.float32(overlap) * overlap_of(ha, hb) or gap > np.float32(max_gap) * max(ha, hb) or \
                    gap < np.float32(-0.5) * min(ha, hb):
                continue
            if gap < best_gap:
                best, best_gap = j, gap
        if best < 0:
            lines.append([i])
            last.append((l, t, r, b))
        else:
            lines[best].append(i)
            last[best] = (l, t, r, b)
    lines.sort(key=lambda line: order(*ol.bbox(words[line[0]])[:2]))
    grouped = ol.pad_lines([[np.array(words[i], np.float32) for i in line] for line in lines], 0.15, 0.1)
    return np.array([ol.line_geometry(line)[0] for line in grouped], np.int64).reshape(-1, 5)


@pytest.mark.parametrize("mistake", ["none", "whole taller height overlapping", "most of the smaller height",
                                     "no gap between words", "lines by left edge", "lines bottom to top"])
def test_planted_grouping_mistakes_fail_the_ocrs_check(mistake):
    # Each planted mistake in the rule (in the oracle's terms, on the CPU) must fail the check
    # against ocrs's lines on both pages tried; the rule itself must pass and equal the oracle.
    knobs = {"none": {}, "whole taller height overlapping": {"overlap": 1.0, "overlap_of": max},
             "most of the smaller height": {"overlap": 0.9}, "no gap between words": {"max_gap": 0.0},
             "lines by left edge": {"order": lambda l, t: (l, t)}, "lines bottom to top": {"order": lambda l, t: (-t, l)}}
    failed = 0
    for k in (0, 3):
        bits, w, chars = PAGES[k]
        boxes = _grouping(list(ol.word_rects(bits, w)), **knobs[mistake])
        if mistake == "none":
            np.testing.assert_array_equal(boxes, _boxes(ol.Layout(bits, w)))
        try:
            _check_against_ocrs(boxes, chars, k)
        except AssertionError:
            failed += 1
    assert failed == (0 if mistake == "none" else 2), f"{mistake}: {failed} of 2 pages failed the check"
