"""The N-D executor's fusion plan (csrc/nd_plan.cpp, through ocr_nd_plan; no GPU): which ONNX nodes
run as one launch, against the operator contract of the reference's NdGraph::new
(src/nd.rs:505-817): Identity nodes dropped, a final Softmax cut on request, the squeeze-excitation
gate as a conv's input scale, the exporter's LayerNorm chain as one op, Conv + bias + BN + ReLU or
GELU + residual, MatMul + bias + SiLU (+ a residual Add), ConvTranspose + bias + ReLU or Sigmoid, a
lone BN as a channel affine, and the exporter's multi-head self-attention chain as one step. Chains are matched over def-use edges, so operand order (Add, Mul) and unrelated
nodes in between do not matter, and a value some other node still reads is never fused away.
The numerics of every fused launch are checked on the GPU (tests/test_gpu_nd.py)."""
import re

import numpy as np
import pytest

import ocrhip
from ocrhip import onnx_write as ow
from ocrhip import synth_pp

RNG = np.random.Generator(np.random.PCG64(3))


def plan(tmp_path, name, fn, in_shape, stop=False):
    g = ow.Graph(name)
    out = fn(g, "x")
    p = tmp_path / f"{name}.onnx"
    p.write_bytes(g.model("x", list(in_shape), out, ["a"]))
    return ocrhip.nd_plan(str(p), stop), out


def steps(lines):
    """[(kind, op, nodes, attrs dict, output)]"""
    out = []
    for line in lines:
        m = re.match(r"(\w+) (\w+)@(\d+) \[([\d,]*)\](.*) -> (\S+)$", line)
        assert m, line
        attrs = dict(kv.split("=", 1) if "=" in kv else (kv, True) for kv in m.group(5).split())
        out.append((m.group(1), m.group(2), [int(v) for v in m.group(4).split(",") if v], attrs, m.group(6)))
    return out


def w(g, shape):
    return g.init(g.fresh("w"), RNG.standard_normal(shape).astype(np.float32))


def const(g, v):
    return g.init(g.fresh("c"), np.array([v], np.float32))


def conv(g, x, cin, cout, bias=True):
    ins = [x, w(g, (cout, cin, 3, 3))] + ([w(g, (cout,))] if bias else [])
    return g.add("Conv", ins, kernel_shape=[3, 3], pads=[1, 1, 1, 1])


def test_pp_recognizer_plan():
    s = steps(ocrhip.nd_plan(synth_pp.model_path("rec"), True))
    kinds = [k for k, *_ in s]
    assert kinds.count("layer_norm") == 5  # two blocks of two, and the final one
    assert sum(1 for k, _, _, a, _ in s if k == "linear" and a.get("act") == "silu") == 2
    assert sum(1 for k, _, _, a, _ in s if k == "conv" and "in_scale" in a) == 1
    assert sum(1 for k, _, _, a, _ in s if k == "conv" and a.get("act") == "gelu" and "residual" in a) == 1
    assert s[-1][0] == "linear" and not any(op == "Softmax" and i == len(s) - 1 for i, (_, op, *_r) in enumerate(s))
    assert not any(op == "Identity" for _, op, *_ in s)
    # Every node of the graph is in exactly one step.
    nodes = sorted(n for _, _, ns, _, _ in s for n in ns)
    assert nodes == list(range(len(nodes)))
    full = steps(ocrhip.nd_plan(synth_pp.model_path("rec"), False))
    assert full[-1][1] == "Softmax" and len(full) == len(s) + 1


def test_pp_recognizer_attention_and_linear_residuals():
    s = steps(ocrhip.nd_plan(synth_pp.model_path("rec"), True))
    att = [(nodes, out) for k, _, nodes, _, out in s if k == "attention"]
    assert len(att) == 2 and all(len(nodes) == 15 for nodes, _ in att)
    # attention projection and second MLP layer of each block take the block's residual Add
    assert sum(1 for k, _, _, a, _ in s if k == "linear" and "residual" in a) == 4
    assert not any(op in ("Softmax", "Slice") for k, op, *_ in s if k == "node")


def _attention_graph(g, x, perm=(2, 0, 3, 1, 4), k_first=False, scale_first=False):
    qkv = g.add("MatMul", [x, w(g, (24, 72))])
    s5 = g.init(g.fresh("s"), np.array([0, 0, 3, 4, 6], np.int64))
    t5 = g.add("Transpose", [g.add("Reshape", [qkv, s5])], perm=list(perm))
    parts = {}
    for i in ((1, 0, 2) if k_first else (0, 1, 2)):
        ii = lambda v: g.init(g.fresh("i"), np.array(v, np.int64))  # noqa: E731
        sl = g.add("Slice", [t5, ii([i]), ii([i + 1]), ii([0])])
        parts[i] = g.add("Squeeze", [sl, ii([0])])
    sc = const(g, 6 ** -0.5)
    q = g.add("Mul", [sc, parts[0]] if scale_first else [parts[0], sc])
    att = g.add("Softmax", [g.add("MatMul", [q, g.add("Transpose", [parts[1]], perm=[0, 1, 3, 2])])], axis=-1)
    o = g.add("Transpose", [g.add("MatMul", [att, parts[2]])], perm=[0, 2, 1, 3])
    return g.add("Reshape", [o, g.init(g.fresh("r"), np.array([0, 0, 24], np.int64))]), att


def test_attention_chain_in_any_slice_order(tmp_path):
    for k_first, scale_first in ((False, False), (True, True)):
        lines, _ = plan(tmp_path, "att", lambda g, x: _attention_graph(g, x, k_first=k_first,
                                                                       scale_first=scale_first)[0], (2, 5, 24))
        s = steps(lines)
        assert [k for k, *_ in s] == ["linear", "attention"], lines


def test_attention_chain_with_another_layout_is_not_fused(tmp_path):
    lines, _ = plan(tmp_path, "att2", lambda g, x: _attention_graph(g, x, perm=(2, 0, 1, 3, 4))[0], (2, 5, 24))
    assert not any(k == "attention" for k, *_ in steps(lines))


def test_attention_chain_with_a_value_read_elsewhere_is_not_fused(tmp_path):
    def fn(g, x):
        y, sm = _attention_graph(g, x)
        # the softmax probabilities also leave the chain: nothing may be fused away
        return g.add("Add", [y, g.add("ReduceMean", [g.add("Reshape", [sm, g.init("r2", np.array([2, 5, -1], np.int64))])],
                                     axes=[-1], keepdims=1)])
    lines, _ = plan(tmp_path, "att3", fn, (2, 5, 24))
    assert not any(k == "attention" for k, *_ in steps(lines))


def test_pp_detector_plan():
    s = steps(ocrhip.nd_plan(synth_pp.model_path("det")))
    assert sum(1 for k, *_ in s if k == "conv_transpose") == 2
    assert s[-1][3].get("act") == "sigmoid"
    # Every conv with a ReLU in the backbone and the head has its BatchNormalization folded in.
    assert all(any(key.startswith("bn@") for key in a) for k, _, _, a, _ in s if k == "conv" and a.get("act") == "relu")


def test_bias_found_past_unrelated_nodes_and_in_either_order(tmp_path):
    def fn(g, x):
        c = conv(g, x, 4, 8, bias=False)
        side = g.add("Relu", [x])  # a node between the conv and its bias Add
        y = g.add("Add", [w(g, (1, 8, 1, 1)), c])  # bias first
        y = g.add("Relu", [y])
        return g.add("Add", [y, g.add("Conv", [side, w(g, (8, 4, 1, 1))], kernel_shape=[1, 1])])
    s = steps(plan(tmp_path, "bias", fn, (1, 4, 6, 6))[0])
    fused = [t for t in s if t[0] == "conv" and t[1] == "Conv" and t[3].get("bias") == "1"]
    assert len(fused) == 1 and fused[0][3]["act"] == "relu" and "residual" in fused[0][3]
    assert fused[0][2] == [0, 2, 3, 5] and s[-1] is fused[0]  # runs at the residual Add's place


def test_value_read_elsewhere_is_not_fused(tmp_path):
    def fn(g, x):
        c = conv(g, x, 4, 4)
        r = g.add("Relu", [c])
        return g.add("Add", [r, c])  # the conv's output has two readers
    s = steps(plan(tmp_path, "two", fn, (1, 4, 5, 5))[0])
    assert [k for k, *_ in s] == ["conv", "node", "node"] and "act" not in s[0][3]


def test_layer_norm_chain_any_operand_order(tmp_path):
    def ln(g, x, gamma_first):
        m = g.add("ReduceMean", [x], axes=[-1])
        d = g.add("Sub", [x, m])
        p = g.add("Pow", [d, const(g, 2.0)])
        v = g.add("ReduceMean", [p], axes=[-1])
        other = g.add("Relu", [x])  # an unrelated node inside the chain
        e = g.add("Add", [const(g, 1e-6), v])
        q = g.add("Sqrt", [e])
        n = g.add("Div", [d, q])
        gm = w(g, (6,))
        y = g.add("Mul", [gm, n] if gamma_first else [n, gm])
        y = g.add("Add", [y, w(g, (6,))])
        return g.add("Add", [y, other])
    for gamma_first in (False, True):
        s = steps(plan(tmp_path, f"ln{int(gamma_first)}", lambda g, x: ln(g, x, gamma_first), (3, 6))[0])
        lns = [t for t in s if t[0] == "layer_norm"]
        assert len(lns) == 1 and len(lns[0][2]) == 9


def test_layer_norm_chain_with_a_shared_middle_is_not_fused(tmp_path):
    def fn(g, x):
        m = g.add("ReduceMean", [x], axes=[-1])
        d = g.add("Sub", [x, m])
        p = g.add("Pow", [d, const(g, 2.0)])
        v = g.add("ReduceMean", [p], axes=[-1])
        e = g.add("Add", [v, const(g, 1e-5)])
        q = g.add("Sqrt", [e])
        n = g.add("Div", [d, q])
        y = g.add("Add", [g.add("Mul", [n, w(g, (6,))]), w(g, (6,))])
        return g.add("Add", [y, v])  # the variance is read outside the chain
    s = steps(plan(tmp_path, "lnshared", fn, (3, 6))[0])
    assert not any(k == "layer_norm" for k, *_ in s)


def test_gelu_chain_and_se_gate(tmp_path):
    def fn(g, x):
        gate = g.add("HardSigmoid", [g.add("GlobalAveragePool", [x])])
        y = conv(g, g.add("Mul", [gate, x]), 4, 4)  # gate first
        h = g.add("Erf", [g.add("Div", [y, const(g, 1.4142135)])])
        a = g.add("Add", [const(g, 1.0), h])
        return g.add("Mul", [const(g, 0.5), g.add("Mul", [a, y])])
    s = steps(plan(tmp_path, "gelu", fn, (2, 4, 5, 5))[0])
    c = [t for t in s if t[0] == "conv"]
    assert len(c) == 1 and c[0][3]["act"] == "gelu" and c[0][3]["in_scale"].startswith("hardsigmoid")
    assert len(c[0][2]) == 1 + 1 + 5  # the conv, the gating Mul, the five GELU nodes


def test_identity_and_dead_nodes_dropped(tmp_path):
    def fn(g, x):
        i = g.add("Identity", [g.add("Identity", [x])])
        g.add("Sigmoid", [x])  # read by nothing
        return g.add("Relu", [i])
    s = steps(plan(tmp_path, "ident", fn, (2, 3))[0])
    assert [(k, op) for k, op, *_ in s] == [("node", "Relu")]


def test_linear_silu_and_conv_transpose_epilogues(tmp_path):
    def fn(g, x):
        y = g.add("MatMul", [x, w(g, (6, 8))])
        y = g.add("Add", [y, w(g, (8,))])
        y = g.add("Mul", [g.add("Sigmoid", [y]), y])
        y = g.add("Reshape", [y, g.init("shp", np.array([1, 8, 2, 1], np.int64))])
        y = g.add("ConvTranspose", [y, w(g, (8, 2, 2, 2))], strides=[2, 2], kernel_shape=[2, 2])
        return g.add("Sigmoid", [g.add("Add", [y, w(g, (1, 2, 1, 1))])])
    s = steps(plan(tmp_path, "lin", fn, (2, 6))[0])
    assert (s[0][0], s[0][3].get("act"), s[0][3].get("bias")) == ("linear", "silu", "1")
    assert (s[-1][0], s[-1][3].get("act"), s[-1][3].get("bias")) == ("conv_transpose", "sigmoid", "1")


def test_bias_of_the_wrong_size_is_left_alone(tmp_path):
    def fn(g, x):
        return g.add("Add", [conv(g, x, 4, 8), w(g, (1, 1, 1, 5))])  # broadcast over width, not channels
    s = steps(plan(tmp_path, "badbias", fn, (1, 4, 5, 5))[0])
    assert [k for k, *_ in s] == ["conv", "node"]


def test_plan_of_a_missing_file_raises():
    with pytest.raises(ocrhip.OcrError):
        ocrhip.nd_plan("/nonexistent.onnx")
