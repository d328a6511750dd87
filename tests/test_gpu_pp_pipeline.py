"""The PP-OCR page pipeline (DB detection at long side 960, threshold 0.3, host boxes, SVTR
recognition, CTC) on the GPU against the oracle, through the C ABI: line images, then whole pages.
The oracle side takes its boxes from the oracle's own restatement of ppdet::boxes and of the
line boxes (oracle/layout.py)."""
import numpy as np
import pytest

from ocrhip import synth, synth_pp
from oracle import graph as og
from oracle import layout as ol
from oracle import onnx_read

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pp_models(ctx):
    import ocrhip
    det_path, rec_path = synth_pp.model_path("det"), synth_pp.model_path("rec")
    det = ocrhip.NdGraph(ctx, det_path)
    rec = ocrhip.NdGraph(ctx, rec_path, stop_before_softmax=True)
    return det, rec, onnx_read.load(det_path), onnx_read.load(rec_path)


def boxes_of(bits, prob, to_page, page_w, page_h):
    """The oracle's line boxes of a thresholded DB map."""
    h, w = prob.shape
    return [ol.pp_line_box(b, 0.1, page_w, page_h) for b in ol.db_boxes(bits, prob, w, h, to_page)]


def test_pp_line_images_match_oracle(ctx):
    import ocrhip
    page = np.ascontiguousarray(synth.page(2)[:600, :900])
    lines = [(100, 200, 300, 36, 400), (0, 0, 5, 40, 8), (850, 580, 80, 30, 128), (10, 10, 700, 20, 1680)]
    wb = 1680
    got = ocrhip.pp_line_images(ctx, page, lines, wb)
    for k, ln in enumerate(lines):
        want = og.pp_line_input(page, ln, wb)
        np.testing.assert_array_equal(got[k], want, err_msg=f"line {ln}")


def test_pp_page_text_matches_oracle(ctx, pp_models):
    """One page: the GPU pipeline's text equals the oracle pipeline's on every line whose box
    both sides found (they all are when the two thresholded maps agree)."""
    import ocrhip
    det, rec, det_o, rec_o = pp_models
    page = synth.page(4)
    h, w = page.shape[:2]
    pipe = ocrhip.PpPipeline(det, rec, merge=1)
    pipe.run([page])
    got = pipe.texts(0)
    want, lines, bits_o, prob_o = og.pp_page_pipeline(det_o, rec_o, page,
                                                      lambda b, p, tp: boxes_of(b, p, tp, w, h))
    x = ocrhip.det_input(ctx, page, 960)
    prob = det.run(x)[0, 0]
    bits = ocrhip.db_threshold(ctx, prob, 0.3)
    assert np.abs(prob - prob_o).max() <= 1e-4
    band = np.abs(prob_o - 0.3) < 1e-4
    assert np.array_equal((prob > 0.3)[~band], (prob_o > 0.3)[~band])
    print(f"page: {len(got)} lines on the GPU, {len(want)} in the oracle", flush=True)
    assert len(got) > 20
    if np.array_equal(bits, bits_o):
        assert got == want
    else:  # a pixel in the band flipped: compare the lines both sides found
        gpu_lines = boxes_of(bits, prob, (w / x.shape[3], h / x.shape[2]), w, h)
        common = [i for i, ln in enumerate(lines) if ln in gpu_lines]
        assert len(common) >= len(lines) - 2
        for i in common:
            assert got[gpu_lines.index(lines[i])] == want[i]


def test_pp_pipeline_merge_batching_and_device_entry(ctx, pp_models):
    import ocrhip
    det, rec, _, _ = pp_models
    pages = [synth.page(s) for s in (5, 6, 7)]
    one = ocrhip.PpPipeline(det, rec, merge=1, det_batch=1)
    one.run(pages)
    two = ocrhip.PpPipeline(det, rec, merge=2, det_batch=4)
    bufs = []
    for p in pages:
        b = ctx.alloc(p.nbytes)
        b.upload(p)
        bufs.append(b)
    two.run_device(bufs, [p.shape[1] for p in pages], [p.shape[0] for p in pages])
    for k in range(3):
        assert one.texts(k) == two.texts(k)
    st = two.stats()
    assert st["pages"] == 3 and st["rec_passes"] == 2 and st["lines"] > 60
    # From host memory with uploads between the detection passes (one page a pass), twice in a
    # row on one pipeline (its uploader and staging slots reused): the same text.
    three = ocrhip.PpPipeline(det, rec, merge=2, det_batch=1)
    for _ in range(2):
        three.run(pages)
        for k in range(3):
            assert three.texts(k) == one.texts(k)


def test_pp_pipeline_blank_small_and_empty_pages(ctx, pp_models):
    import ocrhip
    det, rec, _, _ = pp_models
    pipe = ocrhip.PpPipeline(det, rec)
    blank = np.full((500, 400, 3), 255, np.uint8)
    small = np.ascontiguousarray(synth.page(8)[150:260, 140:900])
    pipe.run([blank, small])
    assert pipe.stats()["pages"] == 2
    with pytest.raises(ocrhip.OcrError):
        pipe.run([np.zeros((0, 10, 3), np.uint8)])
