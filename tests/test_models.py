"""Synthetic models and the ONNX writer/reader, and the C ABI's exported symbols. CPU only."""
import ctypes
import os
import re

import numpy as np

from ocrhip import onnx_write as ow
from ocrhip import synth
from oracle import onnx_read

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_onnx_roundtrip(tmp_path):
    g = ow.Graph("t")
    w = g.init("w", np.arange(24, dtype=np.float32).reshape(2, 3, 2, 2))
    s = g.init("s", np.array([0, -1, 5], np.int64))
    y = g.add("Conv", ["x", w], kernel_shape=[2, 2], pads=[0, 1, 0, 1], alpha=0.5, mode="m")
    p = tmp_path / "t.onnx"
    p.write_bytes(g.model("x", [1, 3, 4, 4], y, [1, 2, 3, 5]))
    m = onnx_read.load(str(p))
    assert m.input == "x" and m.output == y
    assert [n.op for n in m.nodes] == ["Conv"]
    a = m.nodes[0].attrs
    assert a["kernel_shape"] == [2, 2] and a["pads"] == [0, 1, 0, 1] and a["mode"] == "m"
    assert abs(a["alpha"] - 0.5) < 1e-7
    np.testing.assert_array_equal(m.weights["w"], np.arange(24, dtype=np.float32).reshape(2, 3, 2, 2))
    np.testing.assert_array_equal(m.ints["s"], [0, -1, 5])


def test_rec_model_structure(rec_oracle):
    ops = [n.op for n in rec_oracle.nodes]
    assert ops.count("GRU") == 2 and ops.count("Conv") == 5 and ops[-1] == "LogSoftmax"
    for n in rec_oracle.nodes:
        if n.op == "GRU":
            assert n.attrs["hidden_size"] == 256 and n.attrs["linear_before_reset"] == 1
            assert n.attrs["direction"] == "bidirectional"
    mm = next(n for n in rec_oracle.nodes if n.op == "MatMul")
    assert rec_oracle.weights[mm.inputs[1]].shape == (512, 97)


def test_weights_are_float16_exact(rec_oracle, det_oracle):
    for m in (rec_oracle, det_oracle):
        for k, v in m.weights.items():
            assert np.array_equal(v.astype(np.float16).astype(np.float32), v), k


def test_models_are_deterministic():
    assert synth.rec_model(0) == synth.rec_model(0)
    assert synth.rec_model(0) != synth.rec_model(1)


def test_inputs_are_deterministic():
    a, b = synth.rec_lines(4), synth.rec_lines(4)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    assert all(200 <= x.shape[1] <= 800 and x.shape[0] == 64 for x in a)


def test_batching_rule():
    # ocr-bench.rs:385-407: widths rounded up to 50, at most 20 lines a batch, pad -0.5.
    lines = [np.zeros((64, w), np.float32) for w in [120, 101, 149, 150, 151] + [60] * 25]
    batches, order, widths = synth.batch_lines(lines)
    assert [(n, w) for _, n, w in batches] == [(20, 100), (5, 100), (4, 150), (1, 200)]
    assert sorted(order) == list(range(len(lines)))
    assert widths[order.index(1)] == 101
    k = order[25:29].index(2)  # the 149-wide line in the 150-wide batch
    assert np.all(batches[2][0][k, :, 149:] == -0.5) and np.all(batches[2][0][k, :, :149] == 0)


def _header_functions():
    src = open(os.path.join(ROOT, "include", "ocrhip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ocr_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = os.path.join(ROOT, "wgpu-ocr_amd", "ocrhip", "libocrhip.so")
    assert os.path.exists(lib), "libocrhip.so not built"
    L = ctypes.CDLL(lib)
    names = _header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n


def test_binding_covers_the_header():
    import ocrhip
    assert sorted(ocrhip.SIGNATURES) == _header_functions()


def test_word_rects_threads_identical():
    # The page cut into row bands on several threads: the same rectangles, in the same order, as
    # one thread (components that cross a cut in U shapes, combs and diagonals included).
    import ocrhip
    rng = np.random.Generator(np.random.PCG64(11))
    for trial in range(12):
        h, w = int(rng.integers(64, 900)), int(rng.integers(40, 700))
        yy, xx = np.mgrid[0:h, 0:w]
        kind = trial % 4
        if kind == 0:
            m = rng.random((h, w)) < 0.35
        elif kind == 1:
            m = ((xx // 7) % 3 == 0) | (yy % 97 < 2)
        elif kind == 2:
            m = ((xx + yy) % 23 < 3) | ((xx - yy + 10000) % 31 < 2)
        else:
            m = ((xx % 50 < 20) & (yy % 60 < 40)) | (rng.random((h, w)) < 0.003)
        words = (w + 31) // 32
        padded = np.zeros((h, words * 32), bool)
        padded[:, :w] = m
        bits = np.packbits(padded, axis=1, bitorder="little").view(np.uint32).reshape(h, words)
        want = ocrhip.word_rects(bits, w)
        for t in (2, 3, 5):
            got = ocrhip.word_rects(bits, w, threads=t)
            np.testing.assert_array_equal(got, want, err_msg=f"trial {trial} threads {t}")
