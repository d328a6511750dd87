"""The whole-page pipeline on the GPU (ocr-bench.rs:133-310, 458-585) against the same pipeline
on the CPU: oracle detection, line images and recognition on the same host layout. Text must be
identical line by line (the arg-max parity of the recogniser, carried through the GPU line
crops and the host CTC)."""
import numpy as np
import pytest

import ocrhip
from ocrhip import synth
from oracle import graph as og
from oracle import layout as ol

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pipeline(detector, recognizer):
    return ocrhip.Pipeline(detector, recognizer, merge=2)


def layout_of(bits, w):
    """The oracle's layout (words, lines, padding, crops, batches), restated apart from the
    product's host code."""
    return ol.Layout(bits, w)


def test_pipeline_text_matches_cpu(pipeline, detector, det_oracle, rec_oracle):
    page = synth.page(3)
    print("pipeline page 3", flush=True)
    pipeline.run([page])
    texts, words = pipeline.texts(0)
    st = pipeline.stats()
    assert st["pages"] == 1 and st["lines"] == len(texts) > 20
    # The page mask must agree with the oracle (band excepted); the CPU pipeline then runs on
    # the GPU's mask so that both use one layout.
    bits = detector.detect_page(page, 0.5)
    want_bits, prob, _ = og.detect_page(det_oracle, page, 0.5)
    diff = np.unpackbits((bits ^ want_bits).view(np.uint8), bitorder="little").reshape(bits.shape[0], -1)
    diff = diff[:, : page.shape[1]].astype(bool)
    assert np.all(np.abs(prob[diff] - 0.5) < 1e-4)
    cpu_texts, cpu_words, _ = og.page_pipeline(det_oracle, rec_oracle, page, 0.5, lambda b, w: layout_of(bits, w))
    assert words == cpu_words
    assert texts == cpu_texts
    assert sum(len(t) for t in texts) > 0


def test_bench_configuration_text_matches_cpu(detector, recognizer, det_oracle, rec_oracle):
    # The benchmark's workload and plan (bench.py's defaults): 12 pages from host memory, merge 6
    # (recognition passes of 3, 4 and 5 pages), detection groups of 3 (the first pass's pages one
    # a group, as pages from host memory are), the recurrences and each pass's tail on their own
    # stream. Every page's text equals the CPU pipeline's (oracle detection, layout, line images,
    # recognition, CTC) on the same mask; detection groups of 2, 4 and 6 give the same text.
    pages = [synth.page(i) for i in range(12)]
    p = ocrhip.Pipeline(detector, recognizer, merge=6, det_batch=3)
    print("bench configuration: 12 pages, merge 6, detection groups of 3", flush=True)
    p.run(pages)
    others = []
    for db in (2, 4, 6):
        q = ocrhip.Pipeline(detector, recognizer, merge=6, det_batch=db)
        print(f"bench configuration: detection groups of {db}", flush=True)
        q.run(pages)
        others.append(q)
    for k, page in enumerate(pages):
        print(f"bench configuration: page {k} against the oracle", flush=True)
        texts, words = p.texts(k)
        for q in others:
            assert q.texts(k) == (texts, words)
        bits = detector.detect_page(page, 0.5)
        want_bits, prob, _ = og.detect_page(det_oracle, page, 0.5)
        diff = np.unpackbits((bits ^ want_bits).view(np.uint8), bitorder="little").reshape(bits.shape[0], -1)
        assert np.all(np.abs(prob[diff[:, : page.shape[1]].astype(bool)] - 0.5) < 1e-4)
        cpu_texts, cpu_words, _ = og.page_pipeline(det_oracle, rec_oracle, page, 0.5, lambda b, w: layout_of(bits, w))
        assert (texts, words) == (cpu_texts, cpu_words)


def test_line_images_match_oracle(detector, ctx):
    # Every line of a page's layout: the GPU line image (one launch for all lines, batch width
    # 800) equals the oracle's line crop bit for bit, black past each line's width.
    page = synth.page(5)
    bits = detector.detect_page(page, 0.5)
    lay = layout_of(bits, page.shape[1])
    lines = [lay.line(i) for i in range(lay.nlines)]
    assert len(lines) > 20
    print(f"line images: {len(lines)} lines", flush=True)
    got = ocrhip.line_images(ctx, page, lines, 800)
    for k, (box, row_off, spans) in enumerate(lines):
        want = og.line_crop(page, box, row_off, spans, 800)
        np.testing.assert_array_equal(got[k], want, err_msg=f"line {k} box {list(box)}")


def test_line_images_edge_boxes(ctx):
    # Boxes that leave the page, tall crops shrunk many times (the kernel narrows its tiles to
    # keep the source window in LDS), a wide crop squeezed to 800 columns, rows with two spans or
    # none, a 1 x 1 crop: bit for bit the oracle's line crop.
    rng = np.random.Generator(np.random.PCG64(17))
    page = rng.integers(0, 256, (700, 2600, 3), dtype=np.uint8)
    ph, pw = page.shape[:2]

    def full(bw, bh):
        return list(range(0, 2 * bh + 1, 2)), [v for _ in range(bh) for v in (0, bw)]

    def two_spans(bw, bh):
        row_off, spans = [0], []
        for r in range(bh):
            if r % 3 != 2:
                spans += [r % 7, bw // 3, bw // 2 + r % 5, bw - r % 4]
            row_off.append(len(spans))
        return row_off, spans

    boxes = [((-30, -10, 300, 40, 480), full), ((100, 20, 120, 680, 12), full), ((50, 300, 2400, 50, 800), full),
             ((400, 100, 200, 60, 213), two_spans), ((pw - 50, ph - 20, 100, 40, 160), full),
             ((7, 9, 1, 1, 1), full), ((900, 200, 700, 130, 345), two_spans), ((1300, 5, 37, 300, 8), full)]
    lines = []
    for box, spans_of in boxes:
        row_off, spans = spans_of(box[2], box[3])
        lines.append((box, row_off, spans))
    print(f"line images: {len(lines)} edge boxes", flush=True)
    got = ocrhip.line_images(ctx, page, lines, 800)
    for k, (box, row_off, spans) in enumerate(lines):
        want = og.line_crop(page, box, row_off, spans, 800)
        np.testing.assert_array_equal(got[k], want, err_msg=f"box {box}")


def _pack_bits(mask):
    """[h][w] bool -> [h][ceil(w / 32)] uint32, bit x % 32 of word x / 32."""
    h, w = mask.shape
    padded = np.zeros((h, (w + 31) // 32 * 32), np.uint8)
    padded[:, :w] = mask
    return np.packbits(padded, axis=1, bitorder="little").view(np.uint32).copy()


def test_word_rects_gpu_labelling_identical(detector, ctx):
    # Components labelled on the GPU give the oracle's rectangles bit for bit, in the same order:
    # a detector mask, noise with many tiny and diagonal-only components, nested rings, full
    # rows, an empty mask, widths inside a word.
    rng = np.random.Generator(np.random.PCG64(23))
    masks = []
    page = synth.page(3)
    masks.append((detector.detect_page(page, 0.5), page.shape[1]))
    for h, w, p in ((300, 517, 0.45), (97, 33, 0.6), (64, 2048, 0.15)):
        masks.append((_pack_bits(rng.random((h, w)) < p), w))
    rings = np.zeros((200, 300), bool)
    for r in range(5, 95, 6):
        rings[100 - r: 100 + r + 1, 150 - r] = rings[100 - r: 100 + r + 1, 150 + r] = True
        rings[100 - r, 150 - r: 150 + r + 1] = rings[100 + r, 150 - r: 150 + r + 1] = True
    masks.append((_pack_bits(rings), 300))
    full = np.zeros((50, 70), bool)
    full[::3] = True
    full[:, 35] = True
    masks.append((_pack_bits(full), 70))
    masks.append((_pack_bits(np.zeros((10, 40), bool)), 40))
    diag = np.eye(120, 130, dtype=bool) | np.eye(120, 130, k=7, dtype=bool)[:, ::-1]
    masks.append((_pack_bits(diag), 130))
    # 5000 runs a row on both sides of a 32-row band edge (more than a row's runs staged in LDS),
    # joined diagonally into one component, over sparse noise.
    wide = rng.random((40, 10000)) < 0.05
    wide[31], wide[32] = False, False
    wide[31, 0::2] = True
    wide[32, 1::2] = True
    masks.append((_pack_bits(wide), 10000))
    for bits, w in masks:
        print(f"word rects of a {bits.shape[0]} x {w} mask", flush=True)
        want = ol.word_rects(bits, w)
        got = ocrhip.word_rects_gpu(ctx, bits, w)
        assert got.shape == want.shape
        np.testing.assert_array_equal(got, want)
    # nested rings: only the outermost ring is an external contour (ocr-bench.rs:52)
    assert len(ocrhip.word_rects_gpu(ctx, masks[4][0], 300)) == 1


def test_detect_mask_words_at_odd_widths(detector, det_oracle):
    # Page widths that end inside a 64-pixel group and inside a 32-bit word.
    for w in (2549, 97):
        page = np.ascontiguousarray(synth.page(2)[:1100, :w])
        print(f"mask width {w}", flush=True)
        bits = detector.detect_page(page, 0.5)
        want_bits, prob, _ = og.detect_page(det_oracle, page, 0.5)
        diff = np.unpackbits((bits ^ want_bits).view(np.uint8), bitorder="little").reshape(bits.shape[0], -1)
        assert not diff[:, w:].any(), "bits past the page width"
        diff = diff[:, :w].astype(bool)
        assert np.all(np.abs(prob[diff] - 0.5) < 1e-4)


def test_pipeline_merge_and_device_entry(detector, recognizer, ctx):
    pages = [synth.page(s) for s in (4, 5, 6)]
    a = ocrhip.Pipeline(detector, recognizer, merge=1, det_batch=1)
    a.run(pages)
    b = ocrhip.Pipeline(detector, recognizer, merge=3, det_batch=2)
    d_pages = []
    for p in pages:
        buf = ctx.alloc(p.nbytes)
        buf.upload(p)
        d_pages.append(buf)
    b.run_device(d_pages, [p.shape[1] for p in pages], [p.shape[0] for p in pages])
    for k in range(3):
        assert a.texts(k) == b.texts(k)
    assert a.stats()["lines"] == b.stats()["lines"]


def test_pipeline_words_match_host_labelling(detector, recognizer):
    # Eight full pages in one detection pass label their masks on the GPU concurrently; every
    # page's word count equals the oracle's words of the same mask (a component split, merged or
    # given a wrong bottom row by a race would change it, or fail the run's own row checks).
    pages = [synth.page(s) for s in range(20, 28)]
    p = ocrhip.Pipeline(detector, recognizer, merge=8, det_batch=8)
    p.run(pages)
    for k, page in enumerate(pages):
        print(f"page {k}", flush=True)
        want = ol.word_rects(detector.detect_page(page, 0.5), page.shape[1])
        assert p.texts(k)[1] == len(want)


def test_pipeline_label_capacity_fallback(detector, recognizer):
    # Labelling capacities too small for a full page's mask: those pages are labelled on the
    # host from their bits, the small page beside them in the same detection group still on the
    # GPU, and every page's text equals the run with the default capacities.
    pages = [synth.page(30), np.ascontiguousarray(synth.page(31)[150:400, 100:900]), synth.page(32)]
    base = ocrhip.Pipeline(detector, recognizer, merge=2, det_batch=2)
    print("label fallback: default capacities", flush=True)
    base.run(pages)
    assert base.stats()["host_labelled"] == 0
    want = [base.texts(k) for k in range(3)]
    assert want[0][1] > 200 and want[2][1] > 200 and 0 < want[1][1] < 100
    for caps in ({"label_comps": 200}, {"label_runs": 4000, "label_slots": 4000}):
        print(f"label fallback: {caps}", flush=True)
        p = ocrhip.Pipeline(detector, recognizer, merge=2, det_batch=2, **caps)
        p.run(pages)
        assert [p.texts(k) for k in range(3)] == want
        n = p.stats()["host_labelled"]
        assert n == 2 if "label_comps" in caps else n >= 2


def test_pipeline_blank_and_small_pages(detector, recognizer):
    blank = np.full((3300, 2550, 3), 255, np.uint8)
    small = np.ascontiguousarray(synth.page(7)[150:400, 100:900])
    p = ocrhip.Pipeline(detector, recognizer)
    p.run([blank, small])
    t0, w0 = p.texts(0)
    assert t0 == [] and w0 == 0
    t1, _ = p.texts(1)
    assert isinstance(t1, list)


def test_pipeline_rejects_empty_page(detector, recognizer):
    p = ocrhip.Pipeline(detector, recognizer)
    with pytest.raises(ocrhip.OcrError):
        p.run([np.zeros((0, 10, 3), np.uint8)])


def test_pipeline_host_pinned_and_device_pages_agree(detector, recognizer, ctx):
    # The same pages from pageable host memory (pinned staging ring, upload stream overlapped
    # with detection), from page-locked host memory (uploaded straight from it) and resident in
    # device memory: identical text. Two page sets alternate, so pooled page buffers written on
    # the upload stream were last used by the compute stream in the run before.
    sets = [[synth.page(s) for s in (30, 31, 32, 33)], [synth.page(s) for s in (34, 35, 36)]]
    p = ocrhip.Pipeline(detector, recognizer, merge=2, det_batch=2)
    want = []
    for pages in sets:
        d = []
        for pg in pages:
            b = ctx.alloc(pg.nbytes)
            b.upload(pg)
            d.append(b)
        p.run_device(d, [pg.shape[1] for pg in pages], [pg.shape[0] for pg in pages])
        want.append([p.texts(k) for k in range(len(pages))])
    for rep in range(2):
        for i, pages in enumerate(sets):
            print(f"host pages, set {i}, repeat {rep}", flush=True)
            p.run(pages)
            assert [p.texts(k) for k in range(len(pages))] == want[i]
            assert all(p.page_error(k) == "" for k in range(len(pages)))
    pinned = []
    for pg in sets[0]:
        a = ctx.host_array(pg.shape)
        a.array[...] = pg
        pinned.append(a)
    print("pinned host pages", flush=True)
    p.run([a.array for a in pinned])
    assert [p.texts(k) for k in range(len(sets[0]))] == want[0]


def test_pipeline_from_png_pages(detector, recognizer, ctx):
    # Pages as PNG files (the reference decodes them with image::open(p)?.into_rgb8() before its
    # timed run, ocr-bench.rs:421-428): decoded by the library on host threads straight into
    # page-locked memory, then run; the text is that of the same pixels given as arrays. One page
    # is greyscale (decoded to R = G = B).
    import io
    Image = pytest.importorskip("PIL.Image")
    pages = [synth.page(s) for s in (40, 41)]
    pages.append(np.repeat(synth.page(42)[:, :, 1:2], 3, axis=2))
    pngs = []
    for i, pg in enumerate(pages):
        buf = io.BytesIO()
        (Image.fromarray(pg[:, :, 0], "L") if i == 2 else Image.fromarray(pg, "RGB")).save(buf, "PNG")
        pngs.append(buf.getvalue())
    p = ocrhip.Pipeline(detector, recognizer, merge=2, det_batch=2)
    p.run(pages)
    want = [p.texts(k) for k in range(len(pages))]
    pinned = [ctx.host_array(ocrhip.png_dims(b)[::-1] + (3,)) for b in pngs]
    import concurrent.futures as cf
    with cf.ThreadPoolExecutor(3) as ex:
        decoded = list(ex.map(lambda a: ocrhip.decode_png(a[0], out=a[1].array), zip(pngs, pinned)))
    for d, pg in zip(decoded, pages):
        np.testing.assert_array_equal(d, pg)
    print("pages decoded from PNG into pinned memory", flush=True)
    p.run([a.array for a in pinned])
    assert [p.texts(k) for k in range(len(pages))] == want
    assert sum(len(t[0]) for t in want) > 40


def test_pipeline_page_error_other_pages_finish(detector, recognizer, monkeypatch):
    # A page whose layout fails reports its error; the other pages of its recognition pass and
    # of the other passes finish with the text of a clean run (ocr-bench.rs:277-281, 303-307).
    pages = [synth.page(s) for s in (40, 41, 42, 43)]
    p = ocrhip.Pipeline(detector, recognizer, merge=2, det_batch=2)
    p.run(pages)
    clean = [p.texts(k) for k in range(4)]
    monkeypatch.setenv("OCR_PIPE_FAIL_LAYOUT", "1")
    print("layout of page 1 fails", flush=True)
    with pytest.raises(ocrhip.OcrError, match="1 of 4 pages failed"):
        p.run(pages)
    assert "injected" in p.page_error(1)
    assert p.texts(1) == ([], 0)
    for k in (0, 2, 3):
        assert p.page_error(k) == ""
        assert p.texts(k) == clean[k]
    monkeypatch.delenv("OCR_PIPE_FAIL_LAYOUT")
    p.run(pages)
    assert [p.texts(k) for k in range(4)] == clean


def test_pool_at_cap_same_results(rec_model_path, recognizer):
    # A context whose scratch pool keeps at most 1 MB frees almost every buffer it is given back
    # (hipFree) instead of keeping it: the recognition results are the same bits.
    lines = synth.rec_lines(12, seed=9, wmin=200, wmax=600)
    batches, _, _ = synth.batch_lines(lines)
    want_logits, want_lens, want_best = recognizer.recognize(batches)
    small = ocrhip.Context(pool_mb=1)
    try:
        rec = ocrhip.Recognizer(small, rec_model_path)
        for rep in range(2):
            print(f"pool at cap, repeat {rep}", flush=True)
            logits, lens, best = rec.recognize(batches)
            np.testing.assert_array_equal(lens, want_lens)
            for k, T in enumerate(lens):  # rows past a line's length are not defined
                np.testing.assert_array_equal(best[:T, k], want_best[:T, k])
                np.testing.assert_array_equal(logits[:T, k], want_logits[:T, k])
        del rec
    finally:
        small.close()
