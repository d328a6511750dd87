"""The oracle's N-D operators (the PP-OCR graphs) pinned against torch-CPU golden vectors in
tests/golden/nd.npz: each golden is a library routine (F.layer_norm, scaled-dot-product
attention, F.batch_norm, F.gelu, F.silu, F.interpolate, padded pools, a strided depthwise conv)
and the oracle runs the ONNX node chain the exporter writes for it. CPU only."""
import os

import numpy as np
import pytest

from oracle import graph, onnx_read

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
N = onnx_read.Node


def nd(name):
    z = np.load(os.path.join(GOLD, "nd.npz"))
    return {k.split("__")[1]: z[k] for k in z.files if k.startswith(name + "__")}


def model(nodes, weights=None, ints=None, out="y"):
    return onnx_read.Model(nodes, {k: np.asarray(v, np.float32) for k, v in (weights or {}).items()},
                           {k: np.asarray(v, np.int64) for k, v in (ints or {}).items()}, "x", out)


def f32(v):
    return np.array([v], np.float32)


def test_layer_norm_chain():
    c = nd("ln")
    m = model([N("ReduceMean", ["x"], ["m"], {"axes": [-1], "keepdims": 1}), N("Sub", ["x", "m"], ["d"], {}),
               N("Pow", ["d", "two"], ["p"], {}), N("ReduceMean", ["p"], ["v"], {"axes": [-1], "keepdims": 1}),
               N("Add", ["v", "eps"], ["a"], {}), N("Sqrt", ["a"], ["s"], {}), N("Div", ["d", "s"], ["n"], {}),
               N("Mul", ["n", "g"], ["o"], {}), N("Add", ["o", "b"], ["y"], {})],
              {"two": f32(2.0), "eps": f32(1e-6), "g": c["g"], "b": c["b"]})
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=1e-5)


def test_attention_chain():
    c = nd("attn")
    x = np.stack([c["q"], c["k"], c["v"]])  # [3, n, 8, T, 15]
    nodes = []
    for i, nm in enumerate("qkv"):
        nodes += [N("Slice", ["x", f"s{i}", f"e{i}", "a0"], [f"{nm}5"], {}), N("Squeeze", [f"{nm}5", "a0"], [nm], {})]
    nodes += [N("Mul", ["q", "scale"], ["qs"], {}), N("Transpose", ["k"], ["kt"], {"perm": [0, 1, 3, 2]}),
              N("MatMul", ["qs", "kt"], ["s"], {}), N("Softmax", ["s"], ["p"], {"axis": -1}),
              N("MatMul", ["p", "v"], ["y"], {})]
    ints = {"a0": [0]}
    for i in range(3):
        ints[f"s{i}"], ints[f"e{i}"] = [i], [i + 1]
    y, _ = graph.run(model(nodes, {"scale": f32(15 ** -0.5)}, ints), x)
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=1e-6)


def test_batch_norm():
    c = nd("bn")
    m = model([N("BatchNormalization", ["x", "g", "b", "m", "v"], ["y"], {"epsilon": 1e-5})],
              {k: c[k] for k in ("g", "b", "m", "v")})
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=1e-6)


def test_gelu_chain_and_silu():
    c = nd("gelu")
    m = model([N("Div", ["x", "r2"], ["d"], {}), N("Erf", ["d"], ["e"], {}), N("Add", ["e", "one"], ["a"], {}),
               N("Mul", ["x", "a"], ["m"], {}), N("Mul", ["m", "half"], ["y"], {})],
              {"r2": f32(np.sqrt(2.0)), "one": f32(1.0), "half": f32(0.5)})
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-6, atol=1e-6)
    s = nd("silu")
    m = model([N("Sigmoid", ["x"], ["s"], {}), N("Mul", ["x", "s"], ["y"], {})])
    y, _ = graph.run(m, s["x"])
    np.testing.assert_allclose(y, s["y"], rtol=1e-6, atol=1e-6)


def test_hardsigmoid_attributes():
    # F.hardsigmoid is HardSigmoid with alpha 1/6 and beta 0.5: the node's attributes, not ONNX's
    # defaults (0.2, 0.5), must reach the arithmetic.
    c = nd("hardsigmoid")
    m = model([N("HardSigmoid", ["x"], ["y"], {"alpha": 1.0 / 6.0, "beta": 0.5})])
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-6, atol=1e-7)
    assert c["y"].min() == 0 and c["y"].max() == 1  # both clamps reached


def test_resize_nearest_x2():
    c = nd("resize2")
    m = model([N("Resize", ["x", "", "sc"], ["y"], {"mode": "nearest", "coordinate_transformation_mode": "asymmetric",
                                                  "nearest_mode": "floor"})],
              {"sc": np.array([1, 1, 2, 2], np.float32)})
    y, _ = graph.run(m, c["x"])
    np.testing.assert_array_equal(y, c["y"])


@pytest.mark.parametrize("op,case", [("AveragePool", "avgpool_pad"), ("MaxPool", "maxpool_pad")])
def test_padded_strided_pools(op, case):
    c = nd(case)
    m = model([N(op, ["x"], ["y"], {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]})])
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-6, atol=1e-6)


def test_depthwise_stride_2_1():
    c = nd("dw_s21")
    m = model([N("Conv", ["x", "w"], ["y"], {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "strides": [2, 1],
                                              "group": 6})], {"w": c["w"]})
    y, _ = graph.run(m, c["x"])
    np.testing.assert_allclose(y, c["y"], rtol=1e-5, atol=1e-5)


def test_det_prep_golden():
    c = nd("det_prep")
    y = graph.det_prep(c["rgb"], int(c["max_side"]))
    assert y.shape == c["y"].shape
    # torch interpolates as a + (b - a) t, the reference's mix as a (1 - t) + b t.
    np.testing.assert_allclose(y, c["y"], rtol=0, atol=2e-5)


def test_det_input_size_rule():
    # nd.rs:1356-1358 on a 300-dpi US Letter page: 2550 x 3300 with long side 960 -> 736 x 960.
    assert graph.det_input_size(2550, 3300, 960) == (736, 960)
    assert graph.det_input_size(100, 50, 960) == (96, 64)   # no down-scaling; 50 / 32 rounds to 2
    assert graph.det_input_size(10, 10, 960) == (32, 32)    # at least 32
    assert graph.det_input_size(48, 16, 960) == (64, 32)    # 1.5 rounds away from zero


def test_shape_arithmetic_on_integers():
    m = model([N("Shape", ["x"], ["s"], {}), N("Gather", ["s", "i01"], ["nt"], {"axis": 0}),
               N("Concat", ["nt", "tail"], ["shape"], {"axis": 0}), N("Reshape", ["x", "shape"], ["y"], {})],
              ints={"i01": [0, 1], "tail": [3, 2, 2]})
    x = np.arange(2 * 5 * 12, dtype=np.float32).reshape(2, 5, 12)
    y, _ = graph.run(m, x)
    np.testing.assert_array_equal(y, x.reshape(2, 5, 3, 2, 2))


def test_planted_layer_norm_mistake_is_caught():
    """Dividing by the variance instead of its square root breaks the LayerNorm golden."""
    c = nd("ln")
    m = model([N("ReduceMean", ["x"], ["m"], {"axes": [-1], "keepdims": 1}), N("Sub", ["x", "m"], ["d"], {}),
               N("Pow", ["d", "two"], ["p"], {}), N("ReduceMean", ["p"], ["v"], {"axes": [-1], "keepdims": 1}),
               N("Add", ["v", "eps"], ["a"], {}), N("Div", ["d", "a"], ["n"], {}),
               N("Mul", ["n", "g"], ["o"], {}), N("Add", ["o", "b"], ["y"], {})],
              {"two": f32(2.0), "eps": f32(1e-6), "g": c["g"], "b": c["b"]})
    y, _ = graph.run(m, c["x"])
    assert np.abs(y - c["y"]).max() > 1e-2


@pytest.mark.parametrize("case", ["pp_line_in", "pp_line_edge"])
def test_pp_line_input_golden(case):
    c = nd(case)
    y = graph.pp_line_input(c["rgb"], c["line"], int(c["wb"]))
    d = np.abs(y - c["y"])
    # Both round the interpolated value to a byte; a value within an ulp of .5 may round to the
    # neighbouring byte (2 / 255 after normalisation) on one side only.
    assert d.max() <= 2 / 255 + 1e-6
    assert (d > 1e-6).mean() < 0.005


def test_pp_decode_rules():
    assert graph.pp_decode([0, 5, 5, 0, 5, 18707, 18707, 1]) == "\u4e04\u4e04 \u4e00"
    assert graph.pp_decode([]) == ""
