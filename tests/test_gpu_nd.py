"""The N-D executor (NdGraph, src/nd.rs) on the GPU against the oracle, through the C ABI
(ocr_nd_*): every fusion pattern and operator on small graphs, then the PP-OCRv6-architecture
recogniser (36 lines, widths in [160, 960]) and the DB detector's front end and map.

Tolerances: float32 activations go through the matrix cores as float16 hi + lo (about 2^-22
relative), so results agree with the float32 oracle to float32 rounding:
|gpu - oracle| <= 1e-4 * (1 + |oracle|) per operator. Recognition: the identical arg-max at every
CTC step and probabilities within 1e-3. Detection: probabilities within 1e-4, so the thresholded
mask is bit-exact outside the 1e-4 band around the threshold."""
import numpy as np
import pytest

from ocrhip import onnx_write as ow
from ocrhip import synth_pp
from oracle import graph as og
from oracle import onnx_read

pytestmark = pytest.mark.gpu
RNG = np.random.Generator(np.random.PCG64(91))


def f16x(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def build(tmp_path, name, fn, in_shape):
    g = ow.Graph(name)
    out = fn(g, "x")
    p = tmp_path / f"{name}.onnx"
    p.write_bytes(g.model("x", list(in_shape), out, ["a"] * 1))
    return str(p)


def check(ctx, path, x, tol=1e-4, stop=False):
    import ocrhip
    print(f"nd graph {path} input {x.shape}", flush=True)
    got = ocrhip.NdGraph(ctx, path, stop).run(x)
    want, _ = og.run(onnx_read.load(path), x)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want) / (1 + np.abs(want))
    assert err.max() <= tol, f"max rel err {err.max()}"
    return got, want


def w(g, shape, fan, exact=True):
    a = RNG.standard_normal(shape).astype(np.float32) * np.float32(np.sqrt(2 / fan))
    return g.init(g.fresh("w"), f16x(a) if exact else a)


def conv(g, x, cin, cout, k=3, stride=(1, 1), group=1, bias=True, exact=True):
    ins = [x, w(g, (cout, cin // group, k, k), cin // group * k * k, exact)]
    if bias:
        ins.append(g.init(g.fresh("b"), (RNG.standard_normal(cout) * 0.1).astype(np.float32)))
    return g.add("Conv", ins, kernel_shape=[k, k], pads=[k // 2] * 4, strides=list(stride), group=group)


def bn(g, x, c):
    vals = [RNG.uniform(0.8, 1.2, c), RNG.uniform(-.1, .1, c), RNG.uniform(-.1, .1, c), RNG.uniform(.5, 1.5, c)]
    return g.add("BatchNormalization", [x] + [g.init(g.fresh("bn"), v.astype(np.float32)) for v in vals], epsilon=1e-5)


def const(g, v):
    return g.init(g.fresh("c"), np.array([v], np.float32))


def ints(g, v):
    return g.init(g.fresh("i"), np.array(v, np.int64))


def test_conv_bn_relu_nchw_mfma(ctx, tmp_path):
    p = build(tmp_path, "cbr", lambda g, x: g.add("Relu", [bn(g, conv(g, x, 24, 40, bias=False), 40)]), (2, 24, 11, 29))
    check(ctx, p, RNG.standard_normal((2, 24, 11, 29)).astype(np.float32))


def test_conv_bias_add_and_1x1(ctx, tmp_path):
    def fn(g, x):
        y = conv(g, x, 16, 32, k=1, bias=False)
        y = g.add("Add", [y, g.init("ab", (RNG.standard_normal((1, 32, 1, 1)) * 0.1).astype(np.float32))])
        return g.add("Relu", [y])
    p = build(tmp_path, "cba", fn, (1, 16, 6, 45))
    check(ctx, p, RNG.standard_normal((1, 16, 6, 45)).astype(np.float32))


def test_strided_and_depthwise_convs(ctx, tmp_path):
    def fn(g, x):
        y = g.add("Relu", [bn(g, conv(g, x, 3, 16, stride=(2, 2), bias=False), 16)])
        y = g.add("Relu", [conv(g, y, 16, 16, group=16)])
        return g.add("Relu", [bn(g, conv(g, y, 16, 16, stride=(2, 1), group=16, bias=False), 16)])
    p = build(tmp_path, "sd", fn, (2, 3, 24, 40))
    check(ctx, p, RNG.standard_normal((2, 3, 24, 40)).astype(np.float32))


def test_se_gate_gelu_residual(ctx, tmp_path):
    def fn(g, x):
        se = g.add("GlobalAveragePool", [x])
        se = g.add("Relu", [conv(g, se, 32, 8, k=1)])
        se = g.add("HardSigmoid", [conv(g, se, 8, 32, k=1)], alpha=0.2, beta=0.5)
        y = g.add("Mul", [x, se])
        y = conv(g, y, 32, 32, k=1)
        d = g.add("Div", [y, const(g, np.float32(np.sqrt(2.0)))])
        e = g.add("Erf", [d])
        a = g.add("Add", [e, const(g, 1.0)])
        m = g.add("Mul", [y, a])
        y = g.add("Mul", [m, const(g, 0.5)])
        return g.add("Add", [y, x])
    p = build(tmp_path, "seg", fn, (2, 32, 3, 17))
    check(ctx, p, RNG.standard_normal((2, 32, 3, 17)).astype(np.float32))


def test_hardsigmoid_non_default_attributes(ctx, tmp_path):
    # The SE gate with torch's hardsigmoid constants (alpha 1/6) and a standalone HardSigmoid with
    # alpha 0.3, beta 0.4: the attributes, not ONNX's defaults, reach the kernels.
    def fn(g, x):
        se = g.add("GlobalAveragePool", [x])
        se = g.add("HardSigmoid", [conv(g, se, 32, 32, k=1)], alpha=1.0 / 6.0, beta=0.5)
        y = conv(g, g.add("Mul", [x, se]), 32, 32, k=1)
        return g.add("HardSigmoid", [y], alpha=0.3, beta=0.4)
    p = build(tmp_path, "hsig", fn, (2, 32, 3, 17))
    check(ctx, p, (3 * RNG.standard_normal((2, 32, 3, 17))).astype(np.float32))


def test_linear_silu_and_inexact_weights(ctx, tmp_path):
    def fn(g, x):
        y = g.add("MatMul", [x, w(g, (120, 240), 120)])
        y = g.add("Add", [y, g.init("lb", (RNG.standard_normal(240) * 0.1).astype(np.float32))])
        s = g.add("Sigmoid", [y])
        y = g.add("Mul", [y, s])
        return g.add("MatMul", [y, w(g, (240, 50), 240, exact=False)])
    p = build(tmp_path, "lin", fn, (3, 37, 120))
    check(ctx, p, RNG.standard_normal((3, 37, 120)).astype(np.float32))


def test_layer_norm_and_attention(ctx, tmp_path):
    def fn(g, x):
        b = synth_pp._B("t", 5)
        b.g = g
        return synth_pp._svtr_block(b, x)
    p = build(tmp_path, "svtr", fn, (2, 23, 120))
    check(ctx, p, RNG.standard_normal((2, 23, 120)).astype(np.float32))


def test_pools_resize_convt_concat(ctx, tmp_path):
    def fn(g, x):
        a = g.add("AveragePool", [x], kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
        m = g.add("MaxPool", [x], kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
        y = g.add("Concat", [a, m], axis=1)
        y = g.add("Resize", [y, "", g.init("sc", np.array([1, 1, 2, 2], np.float32))], mode="nearest",
                  coordinate_transformation_mode="asymmetric", nearest_mode="floor")
        t = g.add("ConvTranspose", [y, w(g, (12, 5, 2, 2), 12), g.init("tb", np.full(5, 0.05, np.float32))],
                  kernel_shape=[2, 2], strides=[2, 2])
        t = g.add("Sigmoid", [t])
        r = g.add("ReduceMean", [t], axes=[2, 3], keepdims=0)
        return g.add("Concat", [r, g.add("Sqrt", [g.add("Mul", [r, r])])], axis=1)
    p = build(tmp_path, "prc", fn, (2, 6, 9, 10))
    check(ctx, p, RNG.standard_normal((2, 6, 9, 10)).astype(np.float32))


def test_binary_broadcast_and_shape_ops(ctx, tmp_path):
    def fn(g, x):
        sh = g.add("Shape", [x])
        nt = g.add("Gather", [sh, ints(g, [0, 1])], axis=0)
        s5 = g.add("Concat", [nt, ints(g, [2, 3])], axis=0)
        y = g.add("Reshape", [x, s5])                       # [2, 5, 2, 3]
        y = g.add("Transpose", [y], perm=[0, 2, 1, 3])      # [2, 2, 5, 3]
        z = g.add("Sub", [y, g.init("row", RNG.standard_normal(3).astype(np.float32))])
        z = g.add("Div", [z, g.init("col", (RNG.uniform(1, 2, (1, 2, 5, 1))).astype(np.float32))])
        z = g.add("Pow", [z, const(g, 2.0)])
        z = g.add("Slice", [z, ints(g, [1, 0]), ints(g, [4, 2]), ints(g, [2, 3])])
        return g.add("Unsqueeze", [g.add("Squeeze", [g.add("Unsqueeze", [z, ints(g, [0])]), ints(g, [0])]), ints(g, [1])])
    p = build(tmp_path, "bin", fn, (2, 5, 6))
    check(ctx, p, RNG.standard_normal((2, 5, 6)).astype(np.float32))


def test_fusions_across_unrelated_nodes_and_operand_orders(ctx, tmp_path):
    # Chains the plan matches over def-use edges rather than node order: a bias Add given first
    # and placed after an unrelated node, a residual produced after the conv, the LayerNorm's
    # gamma Mul with its operands swapped and an unrelated node inside the chain, GELU with its
    # constants first. Each runs fused and must equal the unfused oracle.
    def fn(g, x):
        c = conv(g, x, 8, 16, bias=False)
        side = g.add("Relu", [x])
        y = g.add("Add", [g.init("b0", (RNG.standard_normal((1, 16, 1, 1)) * 0.1).astype(np.float32)), c])
        h = g.add("Erf", [g.add("Div", [y, const(g, 1.4142135)])])
        y = g.add("Mul", [const(g, 0.5), g.add("Mul", [g.add("Add", [const(g, 1.0), h]), y])])
        y = g.add("Add", [conv(g, side, 8, 16), y])
        t = g.add("Reshape", [y, ints(g, [2, 16, -1])])
        m = g.add("ReduceMean", [t], axes=[-1])
        d = g.add("Sub", [t, m])
        v = g.add("ReduceMean", [g.add("Pow", [d, const(g, 2.0)])], axes=[-1])
        other = g.add("Sigmoid", [t])
        n = g.add("Div", [d, g.add("Sqrt", [g.add("Add", [const(g, 1e-5), v])])])
        width = 11 * 13
        n = g.add("Mul", [g.init("gm", RNG.uniform(0.5, 1.5, width).astype(np.float32)), n])
        n = g.add("Add", [n, g.init("bt", RNG.uniform(-.1, .1, width).astype(np.float32))])
        return g.add("Add", [n, other])
    p = build(tmp_path, "defuse", fn, (2, 8, 11, 13))
    import ocrhip
    kinds = [line.split()[0] for line in ocrhip.nd_plan(p)]
    assert kinds.count("layer_norm") == 1 and any("act=gelu" in line and "residual" in line
                                                  for line in ocrhip.nd_plan(p))
    check(ctx, p, RNG.standard_normal((2, 8, 11, 13)).astype(np.float32))


# ---- the N-D convolution and row-GEMM kernels at the PP-OCR shapes --------------------------------
@pytest.mark.parametrize("shape,stride,k", [((2, 32, 24, 70), (1, 1), 3), ((2, 64, 24, 70), (2, 2), 3),
                                            ((3, 128, 12, 37), (2, 1), 3), ((1, 16, 9, 8), (1, 2), 3),
                                            ((2, 24, 13, 29), (2, 2), 5)])
def test_depthwise_shapes(ctx, tmp_path, shape, stride, k):
    c = shape[1]
    p = build(tmp_path, "dw", lambda g, x: g.add("Relu", [bn(g, conv(g, x, c, c, k=k, stride=stride, group=c,
                                                                       bias=False), c)]), shape)
    check(ctx, p, RNG.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("cin,cout,h,wd,exact", [(32, 64, 24, 73, True), (64, 128, 12, 37, False),
                                                  (256, 256, 3, 109, True), (120, 256, 1, 61, True),
                                                  (30, 20, 5, 7, True), (128, 32, 1, 1, False)])
def test_1x1_nchw_shapes(ctx, tmp_path, cin, cout, h, wd, exact):
    shape = (3, cin, h, wd)
    p = build(tmp_path, "pw", lambda g, x: g.add("Relu", [bn(g, conv(g, x, cin, cout, k=1, bias=False, exact=exact),
                                                               cout)]), shape)
    check(ctx, p, RNG.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("n,cin,cout,h,wd,exact", [(4, 256, 32, 1, 109, True), (3, 512, 32, 1, 61, False),
                                                    (2, 64, 16, 20, 45, True), (2, 40, 24, 7, 130, False),
                                                    (16, 64, 64, 1, 9, True), (2, 960, 64, 1, 49, True),
                                                    (1, 480, 60, 1, 120, False), (5, 960, 48, 1, 37, False)])
def test_3x3_nchw_shapes(ctx, tmp_path, n, cin, cout, h, wd, exact):
    # One-row inputs (the SVTR neck's convs: two of the three kernel rows read padding only, and
    # few tiles make the wavefronts of a workgroup share the K steps, up to 16 of them for a long
    # K: 960 -> 64 and 960 -> 48) and two-dimensional ones.
    shape = (n, cin, h, wd)
    p = build(tmp_path, "c3", lambda g, x: g.add("Relu", [conv(g, x, cin, cout, k=3, exact=exact)]), shape)
    check(ctx, p, RNG.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("n,cin,cout,wd,exact", [(2, 1024, 64, 40, True), (3, 1024, 32, 21, False),
                                                 (1, 1200, 16, 300, True)])
def test_1x1_nchw_long_k(ctx, tmp_path, n, cin, cout, wd, exact):
    # 1 x 1 convs with a long K over few pixels: the K steps shared by up to 16 wavefronts of a
    # workgroup, their partial sums added in a fixed order.
    import ocrhip
    shape = (n, cin, 1, wd)
    p = build(tmp_path, "c1k", lambda g, x: conv(g, x, cin, cout, k=1, exact=exact), shape)
    x = RNG.standard_normal(shape).astype(np.float32)
    got, _ = check(ctx, p, x)
    np.testing.assert_array_equal(ocrhip.NdGraph(ctx, p).run(x), got)  # the same bits on a rerun


def test_se_gate_and_gelu_residual_at_pp_shapes(ctx, tmp_path):
    def fn(g, x):
        se = g.add("GlobalAveragePool", [x])
        se = g.add("Relu", [conv(g, se, 128, 32, k=1)])
        se = g.add("HardSigmoid", [conv(g, se, 32, 128, k=1)], alpha=0.2, beta=0.5)
        y = g.add("Relu", [conv(g, g.add("Mul", [x, se]), 128, 256, k=1)])
        z = conv(g, y, 256, 256, k=1)
        d = g.add("Div", [z, const(g, np.float32(np.sqrt(2.0)))])
        m = g.add("Mul", [z, g.add("Add", [g.add("Erf", [d]), const(g, 1.0)])])
        return g.add("Add", [g.add("Mul", [m, const(g, 0.5)]), y])
    p = build(tmp_path, "se2", fn, (3, 128, 6, 45))
    check(ctx, p, RNG.standard_normal((3, 128, 6, 45)).astype(np.float32))


@pytest.mark.parametrize("cin,cout,shape,stride", [(3, 32, (2, 3, 48, 97), (2, 2)), (1, 16, (3, 1, 21, 40), (1, 1)),
                                                    (3, 48, (1, 3, 33, 35), (2, 1))])
def test_stem_convs(ctx, tmp_path, cin, cout, shape, stride):
    p = build(tmp_path, "stem", lambda g, x: g.add("Relu", [bn(g, conv(g, x, cin, cout, stride=stride, bias=False),
                                                                 cout)]), shape)
    check(ctx, p, RNG.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("shape,k,n,exact", [((16, 109, 120), 120, 360, True), ((64, 200, 120), 120, 240, False),
                                             ((2, 21, 30), 30, 7, True), ((5, 33, 240), 240, 120, True)])
def test_linear_row_gemm_shapes(ctx, tmp_path, shape, k, n, exact):
    def fn(g, x):
        y = g.add("MatMul", [x, w(g, (k, n), k, exact=exact)])
        return g.add("Add", [y, g.init("lb", (RNG.standard_normal(n) * 0.1).astype(np.float32))])
    p = build(tmp_path, "rows", fn, shape)
    check(ctx, p, RNG.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("k,n,exact", [(120, 200, True), (256, 300, False), (64, 1000, True)])
def test_head_argmax_first_index_on_ties(ctx, tmp_path, k, n, exact):
    """The fused head: classes come in pairs with the same weights and bias, so every row's
    maximum is a tie; the first index of the pair must win (nd.rs:383), as in the oracle's
    logits."""
    import ocrhip

    def fn(g, x):
        a = RNG.standard_normal((k, n // 2)).astype(np.float32) * np.float32(np.sqrt(2 / k))
        a = f16x(a) if exact else a
        wt = np.repeat(a, 2, axis=1)
        bias = np.repeat((RNG.standard_normal(n // 2) * 0.1).astype(np.float32), 2)
        y = g.add("MatMul", [x, g.init("hw", wt)])
        y = g.add("Add", [y, g.init("hb", bias)])
        return g.add("Softmax", [y], axis=-1)
    shape = (3, 41, k)
    p = build(tmp_path, "head", fn, shape)
    x = RNG.standard_normal(shape).astype(np.float32)
    head = ocrhip.NdGraph(ctx, p, stop_before_softmax=True)
    got = head.argmax(x)
    probs, _ = og.run(onnx_read.load(p), x)
    want = np.argmax(probs, axis=-1)  # equal logits give equal probabilities: the first index
    assert np.all(want % 2 == 0)
    assert np.all(got % 2 == 0), "a tie went to the second index"
    assert np.array_equal(got, want)
    assert np.array_equal(got, np.argmax(head.run(x), axis=-1))


@pytest.mark.parametrize("cin,cout,k,s,act", [(16, 16, 2, 2, "Relu"), (16, 1, 2, 2, "Sigmoid"), (8, 5, 3, 3, "Relu"),
                                             (6, 4, 3, 2, "Sigmoid"), (5, 7, 4, 4, None)])
def test_conv_transpose_nchw_shapes(ctx, tmp_path, cin, cout, k, s, act):
    # kernel = stride (each input pixel alone makes its s x s outputs) and an overlapping one
    def fn(g, x):
        y = g.add("ConvTranspose", [x, w(g, (cin, cout, k, k), cin), g.init("tb", (RNG.standard_normal(cout) * 0.1)
                                                                          .astype(np.float32))],
                  kernel_shape=[k, k], strides=[s, s])
        return g.add(act, [y]) if act else y
    shape = (2, cin, 23, 37)
    p = build(tmp_path, "convt", fn, shape)
    check(ctx, p, RNG.standard_normal(shape).astype(np.float32))


def _attention(g, x, dim, heads):
    hd = dim // heads
    qkv = g.add("MatMul", [x, w(g, (dim, 3 * dim), dim)])
    t5 = g.add("Transpose", [g.add("Reshape", [qkv, ints(g, [0, 0, 3, heads, hd])])], perm=[2, 0, 3, 1, 4])
    parts = [g.add("Squeeze", [g.add("Slice", [t5, ints(g, [i]), ints(g, [i + 1]), ints(g, [0])]), ints(g, [0])])
             for i in range(3)]
    q = g.add("Mul", [parts[0], const(g, np.float32(hd ** -0.5))])
    att = g.add("Softmax", [g.add("MatMul", [q, g.add("Transpose", [parts[1]], perm=[0, 1, 3, 2])])], axis=-1)
    o = g.add("Transpose", [g.add("MatMul", [att, parts[2]])], perm=[0, 2, 1, 3])
    return g.add("Reshape", [o, ints(g, [0, 0, dim])])


@pytest.mark.parametrize("n,t,dim,heads", [(3, 37, 120, 8), (2, 300, 120, 8), (2, 77, 64, 2), (1, 150, 128, 2),
                                           (4, 1, 48, 4)])
def test_fused_attention_shapes(ctx, tmp_path, n, t, dim, heads):
    # Heads of 15, 32 and 64 values; 300 and 150 keys take several LDS tiles (the running softmax
    # rescaled between them); one query alone.
    import ocrhip
    p = build(tmp_path, "attn", lambda g, x: _attention(g, x, dim, heads), (n, t, dim))
    assert any(line.startswith("attention") for line in ocrhip.nd_plan(p))
    check(ctx, p, RNG.standard_normal((n, t, dim)).astype(np.float32))


def test_unsupported_and_bad_shapes_raise(ctx, tmp_path):
    import ocrhip
    p = build(tmp_path, "bad", lambda g, x: g.add("Tanh", [x]), (1, 4))
    g = ocrhip.NdGraph(ctx, p)
    with pytest.raises(ocrhip.OcrError, match="unsupported op Tanh"):
        g.run(np.zeros((1, 4), np.float32))
    p = build(tmp_path, "c", lambda g, x: conv(g, x, 8, 8), (1, 8, 5, 5))
    with pytest.raises(ocrhip.OcrError, match="channels"):
        ocrhip.NdGraph(ctx, p).run(np.zeros((1, 6, 5, 5), np.float32))


# ---- the PP-OCRv6-architecture models ------------------------------------------------------------
@pytest.fixture(scope="module")
def pp_rec_path():
    return synth_pp.model_path("rec")


@pytest.fixture(scope="module")
def pp_lines():
    return synth_pp.batch_lines(synth_pp.rec_lines(36))


def test_pp_recognition_config4(ctx, pp_rec_path, pp_lines):
    """36 lines, widths in [160, 960], batches sorted by width (16 a batch): the GPU's softmax
    within 1e-3 of the oracle's and the identical arg-max (the fused head) at every step."""
    import ocrhip
    full = ocrhip.NdGraph(ctx, pp_rec_path)
    head = ocrhip.NdGraph(ctx, pp_rec_path, stop_before_softmax=True)
    model = onnx_read.load(pp_rec_path)
    batches, _ = pp_lines
    steps = 0
    for data, n, wd in batches:
        print(f"pp rec batch n={n} w={wd}", flush=True)
        want, _ = og.run(model, data)
        got = full.run(data)
        assert got.shape == want.shape == (n, wd // 8, synth_pp.PP_CLASSES)
        assert np.abs(got - want).max() <= 1e-3
        best = head.argmax(data)
        want_best = np.argmax(want, axis=-1)  # first index on ties, as nd.rs:383
        assert np.array_equal(best, want_best), f"{int((best != want_best).sum())} steps differ"
        steps += best.size
    assert steps == sum(n * wd // 8 for _, n, wd in batches)


def test_pp_head_argmax_matches_materialised_logits(ctx, pp_rec_path, pp_lines):
    """The fused head arg-max equals the arg-max over the head's own logits on the GPU."""
    import ocrhip
    head = ocrhip.NdGraph(ctx, pp_rec_path, stop_before_softmax=True)
    data, n, wd = pp_lines[0][0]
    logits = head.run(data)
    assert np.array_equal(head.argmax(data), np.argmax(logits, axis=-1))


def test_pp_det_input_matches_oracle(ctx):
    import ocrhip
    from ocrhip import synth
    page = np.ascontiguousarray(synth.page(1)[:1700, :1300])
    got = ocrhip.det_input(ctx, page, synth_pp.DET_MAX_SIDE)
    want = og.det_prep(page, synth_pp.DET_MAX_SIDE)
    assert got.shape == want.shape
    # The same float32 operations in the same order, none fused, on both sides: bit-exact.
    np.testing.assert_array_equal(got, want)


def test_pp_detection_map_and_threshold(ctx):
    """The DB detector on a 960 x 736 input: probabilities within 1e-4 of the oracle; the GPU
    threshold (0.3) bit-exact against the oracle's on the same map."""
    import ocrhip
    path = synth_pp.model_path("det")
    x = RNG.standard_normal((1, 3, 960, 736)).astype(np.float32)
    got, want = check(ctx, path, x)
    assert np.abs(got - want).max() <= 1e-4
    bits = ocrhip.db_threshold(ctx, got[0, 0], 0.3)
    assert np.array_equal(bits, og.threshold_bits(got[0, 0], 0.3))
    band = np.abs(want[0, 0] - 0.3) < 1e-4
    assert np.array_equal((got[0, 0] > 0.3)[~band], (want[0, 0] > 0.3)[~band])
