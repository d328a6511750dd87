"""The detector and recogniser on the GPU against the oracle, through the C ABI, on the
benchmark's synthetic inputs (configs: ocrs recognition of 36 lines; ocrs detection of an
800 x 600 image; whole synthetic 300-dpi pages).

Parity bar (from the reference's own checks, stages.rs:129-147 and ppocr-bench.rs:94-125):
- recognition: the same arg-max class at every valid CTC step, softmax probabilities within
  1e-3, identical decoded strings;
- detection: probability map within 1e-4 (the reference reports < 1e-5 vs rten, README:79),
  page masks bit-exact except pixels whose pre-threshold probability is within 1e-4 of the
  threshold."""
import numpy as np
import pytest

from ocrhip import synth
from oracle import graph as og

pytestmark = pytest.mark.gpu


def softmax(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def check_recognition(recognizer, rec_oracle, batches, widths):
    print(f"recognize {[(n, w) for _, n, w in batches]}", flush=True)
    logits, lens, best = recognizer.recognize([(d, n, w) for d, n, w in batches])
    ref = og.rec_logits(rec_oracle, batches)
    k0 = 0
    steps = 0
    for (d, n, w), rl in zip(batches, ref):
        T = rl.shape[0]
        assert np.all(lens[k0: k0 + n] == T)
        g = logits[:T, k0: k0 + n]
        # arg-max identical at every step (last index on ties, ocr-bench.rs:67)
        want_best = rl.shape[2] - 1 - np.argmax(rl[..., ::-1], axis=2)
        assert np.array_equal(best[:T, k0: k0 + n], want_best)
        np.testing.assert_array_less(np.abs(softmax(g) - softmax(rl)), 1e-3)
        for j in range(n):
            s_gpu, _ = og.ctc_decode(g[:, j], widths[k0 + j])
            s_ref, _ = og.ctc_decode(rl[:, j], widths[k0 + j])
            assert s_gpu == s_ref
        steps += T * n
        k0 += n
    return steps


def test_recognition_config1(recognizer, rec_oracle):
    lines = synth.rec_lines(36, seed=0)
    batches, order, widths = synth.batch_lines(lines)
    assert check_recognition(recognizer, rec_oracle, batches, widths) > 36 * 50


@pytest.mark.parametrize("f16", ["0", None])
def test_recognition_config1_float32_weights(ctx, f16):
    """Config 1 with float32 weights that are not float16 values (a trained model's). The trunk,
    projections and output layer run the fast kernels with remainder slices. With F16=0 the
    recurrence keeps R in float32 (gru_recurrence_f32), as the reference does with F16 off
    (gpu.rs:858, 1476-1486); by default R is rounded to float16, as the reference does with F16 on.
    Both must meet the bar against the float32 oracle."""
    import os

    import ocrhip
    from oracle import onnx_read
    path = synth.model_path("rec_f32")
    old = os.environ.pop("F16", None)
    try:
        if f16 is not None:
            os.environ["F16"] = f16
        rec = ocrhip.Recognizer(ctx, path)
    finally:
        os.environ.pop("F16", None)
        if old is not None:
            os.environ["F16"] = old
    lines = synth.rec_lines(36, seed=0, wmin=200, wmax=800)
    batches, _, widths = synth.batch_lines(lines)
    fams = ("conv3x3_dma", "gemm_dma", "conv_igemm", "conv_mfma", "gru")
    for f in fams:
        ocrhip.probe_start(f)
    check_recognition(rec, onnx_read.load(path), batches, widths)
    calls = {f: ocrhip.probe_stop(f)["calls"] for f in fams}
    assert calls["conv3x3_dma"] >= 1 and calls["gemm_dma"] >= 1 and calls["conv_mfma"] == 0, calls


def test_recognition_edge_shapes(recognizer, rec_oracle):
    # one narrow line (T = 2), a width not a multiple of 4, and a single-line batch
    rng = np.random.Generator(np.random.PCG64(9))
    batches = [(rng.uniform(-0.5, 0.5, (1, 64, 8)).astype(np.float32), 1, 8),
               (rng.uniform(-0.5, 0.5, (3, 64, 37)).astype(np.float32), 3, 37),
               (rng.uniform(-0.5, 0.5, (9, 64, 203)).astype(np.float32), 9, 203)]
    check_recognition(recognizer, rec_oracle, batches, [8, 37, 37, 37] + [203] * 9)


def test_recognition_batches_together_match_separate(recognizer):
    # The trunk layers of a pass run once over all width batches (more batches than one launch
    # takes, widths from 8 to 301, one to three lines each): every line's logits are the same
    # bits as when its batch is recognised alone.
    rng = np.random.Generator(np.random.PCG64(21))
    batches = []
    for i in range(35):
        w = int(rng.integers(8, 302))
        n = 1 + i % 3
        batches.append((rng.uniform(-0.5, 0.5, (n, 64, w)).astype(np.float32), n, w))
    print(f"recognize {len(batches)} batches together", flush=True)
    logits, lens, best = recognizer.recognize(batches)
    k0 = 0
    for d, n, w in batches:
        one, lens1, best1 = recognizer.recognize([(d, n, w)])
        T = int(lens1[0])
        assert np.all(lens[k0: k0 + n] == T)
        assert np.array_equal(logits[:T, k0: k0 + n], one[:T]), (n, w)
        assert np.array_equal(best[:T, k0: k0 + n], best1[:T])
        k0 += n


@pytest.mark.parametrize("tied", [(7, 40, 96), (3, 60), (0, 1)])
def test_recognition_argmax_ties(ctx, tied):
    """Tied maxima at every step: output-layer columns made identical, with a bias well above
    the others, give bit-identical logits, and the arg-max is the last tied index (the
    reference's rule, ocr-bench.rs:67), also where the last class (96) is one of them and where
    the tie sits in the first lanes of a row."""
    import ocrhip
    from oracle import onnx_read
    m = onnx_read.load(synth.model_path("rec"))
    weights = dict(m.weights)
    w, b = weights["output.w"].copy(), weights["output.b"].copy()
    for c in tied:
        w[:, c] = w[:, tied[0]]
        b[c] = 50.0
    weights["output.w"], weights["output.b"] = w, b
    nodes = [(n.op, n.inputs, n.outputs, n.attrs) for n in m.nodes]
    rec = ocrhip.Recognizer(ctx, ocrhip.ParsedGraph(nodes, weights, m.ints, m.input, m.output))
    batches, _, _ = synth.batch_lines(synth.rec_lines(12, seed=4, wmin=120, wmax=700))
    print(f"arg-max ties {tied}: {[(n, wd) for _, n, wd in batches]}", flush=True)
    logits, lens, best = rec.recognize(batches)
    k0 = 0
    for _, n, _ in batches:
        for j in range(k0, k0 + n):
            T = int(lens[j])
            assert np.all(logits[:T, j][:, list(tied)] == logits[:T, j, tied[0]][:, None])
            assert np.all(best[:T, j] == max(tied)), (tied, j)
        k0 += n


def test_recognition_empty_batch_is_an_error(recognizer):
    import ocrhip
    with pytest.raises(ocrhip.OcrError):
        recognizer.recognize([(np.zeros((0, 64, 50), np.float32), 0, 50)])


def test_detection_config2(detector, det_oracle):
    img = synth.det_input()
    got = detector.detect(img)
    want, _ = og.run(det_oracle, img.reshape(1, 1, 800, 600))
    want = want.reshape(800, 600)
    assert np.abs(got - want).max() <= 1e-4
    band = np.abs(want - 0.5) < 1e-4
    assert np.array_equal((got > 0.5)[~band], (want > 0.5)[~band])


@pytest.mark.parametrize("h,w", [(3300, 2550), (1000, 700), (500, 420), (1100, 97)])
def test_mask_up_bit_exact_on_the_gpu_map(detector, h, w):
    # The page mask from the GPU's own probability map: detect() on the oracle's grey resize
    # (gpu.rs:530-561, bit-exact) runs the same graph on the same input as detect_page() does,
    # so detect_page()'s bits must equal the oracle's upsampling and threshold of that map
    # (gpu.rs:563-593) bit for bit: for a page larger than the map (rows interpolated once per
    # wavefront) and for smaller ones (taps read per output row).
    page = np.ascontiguousarray(synth.page(1)[:h, :w])
    print(f"mask_up {h}x{w}", flush=True)
    bits = detector.detect_page(page, 0.5)
    m = detector.detect(og.grey_resize(page, w, h))
    want = og.pack_bits(og.mask_up_prob(m, w, h), 0.5)
    np.testing.assert_array_equal(bits, want)


@pytest.mark.parametrize("h,w", [(3300, 2550), (1000, 700), (500, 420)])
def test_detect_page_mask(detector, det_oracle, h, w):
    page = synth.page(1)
    if (h, w) != page.shape[:2]:
        page = np.ascontiguousarray(page[:h, :w])
    print(f"detect_page {h}x{w}", flush=True)
    bits = detector.detect_page(page, 0.5)
    want_bits, prob, _ = og.detect_page(det_oracle, page, 0.5)
    ys, xs = np.nonzero(bits != want_bits)
    # Unpack the differing words: every differing pixel must lie in the 1e-4 band.
    for y, wx in zip(ys, xs):
        diff = int(bits[y, wx]) ^ int(want_bits[y, wx])
        for b in range(32):
            if diff >> b & 1:
                assert abs(prob[y, wx * 32 + b] - 0.5) < 1e-4
