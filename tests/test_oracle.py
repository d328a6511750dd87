"""The oracle pinned: each operator against the golden vectors (torch-CPU, tests/golden) and the
closed forms of the reference's own formulas. CPU only."""
import os

import numpy as np
import pytest

from oracle import graph, onnx_read

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def cases(name):
    z = np.load(os.path.join(GOLD, f"{name}.npz"))
    out = {}
    for k in z.files:
        c, f = k.split("__")
        out.setdefault(c, {})[f] = z[k]
    return out


@pytest.mark.parametrize("case", sorted(cases("conv")))
def test_conv2d_golden(case):
    c = cases("conv")[case]
    y = graph.conv2d(c["x"], c["w"], c["b"], tuple(int(v) for v in c["pads"]), tuple(int(v) for v in c["strides"]),
                     int(c["group"]))
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=2e-5)


def test_conv2d_activation_and_residual():
    c = cases("conv")["c3x3"]
    res = np.random.Generator(np.random.PCG64(3)).standard_normal(c["y"].shape).astype(np.float32)
    y = graph.conv2d(c["x"], c["w"], c["b"], (1, 1, 1, 1), (1, 1), 1, act=1, res=res)
    np.testing.assert_allclose(y, np.maximum(c["y"], 0) + res, rtol=1e-5, atol=2e-5)
    y = graph.conv2d(c["x"], c["w"], c["b"], (1, 1, 1, 1), (1, 1), 1, act=2)
    np.testing.assert_allclose(y, 1 / (1 + np.exp(-c["y"].astype(np.float64))), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("case", sorted(cases("convt")))
def test_conv_transpose_golden(case):
    c = cases("convt")[case]
    s = int(c["stride"])
    y = graph.conv_transpose2d(c["x"], c["w"], c["b"], (s, s))
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=2e-5)


@pytest.mark.parametrize("case", sorted(cases("pool")))
def test_pool_golden(case):
    c = cases("pool")[case]
    k = tuple(int(v) for v in c["k"])
    y = graph.pool2d(c["x"], k, k, avg=case.startswith("avg"))
    np.testing.assert_allclose(y, c["y"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("case", sorted(cases("gru")))
def test_gru_golden(case):
    c = cases("gru")[case]
    y = graph.gru(c["x"], c["W"], c["R"], c["B"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=3e-6)


def test_gru_lengths_match_truncated_runs():
    """A line with length L gives what a run over its first L steps gives (the backward
    direction starting at its own end, gpu.rs:692), and zeros past L."""
    c = cases("gru")["g_small"]
    T = c["x"].shape[0]
    lens = np.array([T, 4, 1], np.int32)
    y = graph.gru(c["x"], c["W"], c["R"], c["B"], lens)
    for n, L in enumerate(lens):
        ref = graph.gru(c["x"][:L, n: n + 1], c["W"], c["R"], c["B"])
        np.testing.assert_allclose(y[:L, :, n: n + 1], ref, rtol=1e-6, atol=1e-7)
        assert np.all(y[L:, :, n] == 0)


@pytest.mark.parametrize("case", sorted(cases("resize")))
def test_grey_resize_golden(case):
    c = cases("resize")[case]
    rgb = c["rgb"]
    h, w = rgb.shape[:2]
    y = graph.grey_resize(rgb, w, h, int(c["mh"]), int(c["mw"]))
    np.testing.assert_allclose(y, c["model_in"], rtol=0, atol=2e-6)


@pytest.mark.parametrize("case", sorted(cases("resize")))
def test_mask_up_golden(case):
    c = cases("resize")[case]
    h, w = c["rgb"].shape[:2]
    prob = graph.mask_up_prob(c["m"], w, h, int(c["mh"]), int(c["mw"]))
    np.testing.assert_allclose(prob, c["prob"], rtol=0, atol=2e-6)


@pytest.mark.parametrize("case", sorted(cases("line_crop")))
def test_line_crop_golden(case):
    c = cases("line_crop")[case]
    y = graph.line_crop(c["rgb"], c["box"], c["row_off"], c["spans"], int(c["wb"]))
    # torch interpolates as a + (b - a) t, the reference's mix as a (1 - t) + b t: a few ulp apart.
    np.testing.assert_allclose(y, c["y"], rtol=0, atol=1e-5)


def test_logsoftmax_golden():
    c = cases("logsoftmax")["ls"]
    m = onnx_read.Model([onnx_read.Node("LogSoftmax", ["x"], ["y"], {"axis": 2})], {}, {}, "x", "y")
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-6, atol=1e-5)


def test_valid_region_closed_form():
    # gpu.rs:1414: vh = mh - (ph - h) * mh / ph with ph = max(h, mh) (integer arithmetic).
    assert graph.valid_region(600, 800) == (800, 600)  # exactly the model size: all valid
    assert graph.valid_region(2550, 3300) == (800, 600)  # larger than the model: no padding
    assert graph.valid_region(300, 400) == (400, 300)  # half the size: half the rows and columns
    assert graph.valid_region(600, 100) == (100, 600)
    assert graph.valid_region(599, 799) == (799, 599)


def test_pack_bits_layout():
    rng = np.random.Generator(np.random.PCG64(5))
    prob = rng.uniform(0, 1, (7, 70)).astype(np.float32)
    bits = graph.pack_bits(prob, 0.5)
    assert bits.shape == (7, 3)
    for y in range(7):
        for x in range(70):
            assert ((int(bits[y, x // 32]) >> (x % 32)) & 1) == int(prob[y, x] > 0.5)
    # padding bits of the last word stay 0
    assert np.all((bits[:, 2] >> 6) == 0)


def test_ctc_decode_rules():
    # ocr-bench.rs:62-74: repeats merged, blanks dropped, nothing at or past t * 4 >= width,
    # arg-max ties take the LAST class (Rust max_by).
    C = 5
    def rows(seq):
        x = np.zeros((len(seq), C), np.float32)
        for t, c in enumerate(seq):
            x[t, c] = 1.0
        return x
    out, _ = graph.ctc_decode(rows([0, 1, 1, 0, 1, 2, 2, 3]), width=100, classes=C)
    assert out == [1, 1, 2, 3]
    out, _ = graph.ctc_decode(rows([1, 2, 3, 4]), width=9, classes=C)  # t = 0, 1, 2 have t * 4 < 9
    assert out == [1, 2, 3]
    tie = np.zeros((1, C), np.float32)
    tie[0, 1] = tie[0, 3] = 2.0
    out, best = graph.ctc_decode(tie, width=100, classes=C)
    assert best[0] == 3 and out == [3]


def test_planted_mistake_is_caught():
    """A plausible oracle mistake (gates z and r swapped) breaks the GRU golden check."""
    c = cases("gru")["g_small"]
    W, R, B = c["W"].copy(), c["R"].copy(), c["B"].copy()
    H = R.shape[2]
    for a in (W, R):
        a[:, :H], a[:, H:2 * H] = a[:, H:2 * H].copy(), a[:, :H].copy()
    B[:, :H], B[:, H:2 * H] = B[:, H:2 * H].copy(), B[:, :H].copy()
    y = graph.gru(c["x"], W, R, B)
    assert np.abs(y - c["y"]).max() > 1e-2
