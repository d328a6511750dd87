"""Every graph operator and kernel path on the GPU against the oracle, through the C ABI
(ocr_graph_run), on small seeded inputs. Tolerance: the matrix-core path splits float32
activations into float16 hi + lo (about 2^-22 relative) and accumulates in float32, so results
agree with the float32 oracle to float32 rounding: |gpu - oracle| <= 1e-4 * (1 + |oracle|)."""
import numpy as np
import pytest

from ocrhip import onnx_write as ow
from oracle import graph as oracle_graph
from oracle import onnx_read

pytestmark = pytest.mark.gpu
RNG = np.random.Generator(np.random.PCG64(77))


def f16x(a):
    return a.astype(np.float16).astype(np.float32)


def build(tmp_path, name, nodes_fn, in_shape):
    g = ow.Graph(name)
    out = nodes_fn(g, "x")
    p = tmp_path / f"{name}.onnx"
    p.write_bytes(g.model("x", list(in_shape), out, ["n", "c", "h", "w"]))
    return str(p)


def check(ctx, path, x, tol=1e-4):
    import ocrhip
    print(f"graph {path} input {x.shape}", flush=True)
    got = ocrhip.Graph(ctx, path).run(x)
    want, _ = oracle_graph.run(onnx_read.load(path), x)
    assert got.shape == want.shape
    err = np.abs(got - want) / (1 + np.abs(want))
    assert err.max() <= tol, f"max rel err {err.max()}"
    return got, want


def conv(g, x, cin, cout, k=(3, 3), pads=(1, 1, 1, 1), strides=(1, 1), group=1, exact=True, act=None):
    w = RNG.standard_normal((cout, cin // group, *k)).astype(np.float32) * np.float32(np.sqrt(2 / (cin * k[0] * k[1] / group)))
    if exact:
        w = f16x(w)
    b = (RNG.standard_normal(cout) * 0.1).astype(np.float32)
    y = g.add("Conv", [x, g.init(g.fresh("w"), w), g.init(g.fresh("b"), b)], kernel_shape=list(k), pads=list(pads),
              strides=list(strides), group=group)
    return g.add(act, [y]) if act else y


@pytest.mark.parametrize("cin,cout,h,w", [(5, 7, 9, 11), (16, 32, 20, 33), (40, 70, 6, 21), (64, 64, 8, 50),
                                          (128, 256, 4, 37), (32, 16, 33, 17), (64, 32, 19, 41), (48, 20, 12, 35)])
def test_conv3x3_mfma(ctx, tmp_path, cin, cout, h, w):
    p = build(tmp_path, "c", lambda g, x: conv(g, x, cin, cout, act="Relu"), (2, cin, h, w))
    check(ctx, p, RNG.standard_normal((2, cin, h, w)).astype(np.float32))


@pytest.mark.parametrize("cin,cout,h,w,act", [(256, 1536, 1, 700, None), (512, 97, 3, 301, None), (160, 70, 5, 61, "Relu"),
                                              (512, 256, 2, 1031, "Sigmoid"), (132, 40, 1, 300, None)])
def test_conv1x1_gemm(ctx, tmp_path, cin, cout, h, w, act):
    # The GEMM path: row tails (M % 256), column tails (N % 16, N % 4), K % 32 != 0.
    p = build(tmp_path, "g", lambda g, x: conv(g, x, cin, cout, k=(1, 1), pads=(0, 0, 0, 0), act=act), (1, cin, h, w))
    check(ctx, p, RNG.standard_normal((1, cin, h, w)).astype(np.float32))


def test_conv1x1_and_sigmoid(ctx, tmp_path):
    p = build(tmp_path, "c1", lambda g, x: conv(g, x, 16, 3, k=(1, 1), pads=(0, 0, 0, 0), act="Sigmoid"), (1, 16, 7, 130))
    check(ctx, p, RNG.standard_normal((1, 16, 7, 130)).astype(np.float32))


def test_conv_inexact_weights_third_pass(ctx, tmp_path):
    # Weights that are not float16 values take the x_hi * w_lo pass as well.
    p = build(tmp_path, "ci", lambda g, x: conv(g, x, 24, 40, exact=False), (1, 24, 10, 19))
    check(ctx, p, RNG.standard_normal((1, 24, 10, 19)).astype(np.float32))


def _ran(families, fn):
    """Runs fn with the kernel families probed; returns {family: launches}."""
    import ocrhip
    for f in families:
        ocrhip.probe_start(f)
    out = fn()
    calls = {f: ocrhip.probe_stop(f)["calls"] for f in families}
    return out, calls


FAST = ("conv3x3_dma", "gemm_dma", "conv_igemm", "conv_mfma")


@pytest.mark.parametrize("cin,cout,h,w,pool", [(128, 128, 8, 61, (2, 1)), (128, 256, 4, 37, (2, 1)),
                                               (64, 128, 16, 45, (2, 1)), (32, 64, 32, 41, (2, 2)),
                                               (32, 16, 33, 17, None), (16, 32, 20, 33, None)])
def test_conv3x3_dma_inexact_weights(ctx, tmp_path, cin, cout, h, w, pool):
    # Float32 weights that are not float16 values (as a trained model's are) on the DMA-fed 3 x 3
    # kernel: the remainder slices are a second walk over the input; float32-class results.
    def fn(g, x):
        y = conv(g, x, cin, cout, exact=False, act="Relu")
        return g.add("MaxPool", [y], kernel_shape=list(pool), strides=list(pool)) if pool else y
    p = build(tmp_path, "c3i", fn, (2, cin, h, w))
    x = RNG.standard_normal((2, cin, h, w)).astype(np.float32)
    _, calls = _ran(FAST, lambda: check(ctx, p, x))
    assert calls["conv3x3_dma"] >= 1 and calls["conv_mfma"] == 0, calls


@pytest.mark.parametrize("cin,cout,h,w,fam", [(512, 1536, 1, 700, "gemm_dma"), (256, 97, 3, 301, "gemm_dma"),
                                              (40, 24, 7, 53, "gemm_dma"), (20, 24, 7, 53, "conv_igemm")])
def test_conv1x1_inexact_weights(ctx, tmp_path, cin, cout, h, w, fam):
    # The GRU input projection's shape (512 -> 1536), the output layer's (-> 97) and narrow 1 x 1
    # convs (K of 40 is 4 weight slices with its remainders: the DMA GEMM; K of 20 only 2: the
    # implicit GEMM), all with float32 weights that are not float16 values.
    p = build(tmp_path, "g1i", lambda g, x: conv(g, x, cin, cout, k=(1, 1), pads=(0, 0, 0, 0), exact=False),
              (1, cin, h, w))
    x = RNG.standard_normal((1, cin, h, w)).astype(np.float32)
    _, calls = _ran(FAST, lambda: check(ctx, p, x))
    assert calls[fam] >= 1 and calls["conv_mfma"] == 0, calls


def test_conv_asymmetric_pads(ctx, tmp_path):
    p = build(tmp_path, "ca", lambda g, x: conv(g, x, 8, 12, k=(3, 2), pads=(0, 1, 2, 0)), (1, 8, 9, 10))
    check(ctx, p, RNG.standard_normal((1, 8, 9, 10)).astype(np.float32))


def test_conv_strided_generic(ctx, tmp_path):
    p = build(tmp_path, "cs", lambda g, x: conv(g, x, 6, 5, strides=(2, 2), exact=False), (1, 6, 11, 12))
    check(ctx, p, RNG.standard_normal((1, 6, 11, 12)).astype(np.float32))


def test_depthwise(ctx, tmp_path):
    p = build(tmp_path, "dw", lambda g, x: conv(g, x, 6, 6, group=6, act="Relu"), (2, 6, 9, 8))
    check(ctx, p, RNG.standard_normal((2, 6, 9, 8)).astype(np.float32))


@pytest.mark.parametrize("pool", [(2, 2), (2, 1)])
def test_direct_conv_fused_pool(ctx, tmp_path, pool):
    def net(g, x):
        y = conv(g, x, 1, 32, act="Relu")
        return g.add("MaxPool", [y], kernel_shape=list(pool), strides=list(pool))
    p = build(tmp_path, "dp", net, (3, 1, 64, 37))
    check(ctx, p, RNG.uniform(-0.5, 0.5, (3, 1, 64, 37)).astype(np.float32))


@pytest.mark.parametrize("cout,act,pool", [(48, "Sigmoid", None), (64, "Relu", (2, 2)), (16, None, (2, 2)),
                                          (32, "Sigmoid", (2, 2))])
def test_direct_conv_matrix_cores(ctx, tmp_path, cout, act, pool):
    # The one-channel 3 x 3 conv on the matrix cores: tile edges (50 x 131), 1-4 channel tiles.
    def net(g, x):
        y = conv(g, x, 1, cout, act=act)
        return g.add("MaxPool", [y], kernel_shape=list(pool), strides=list(pool)) if pool else y
    p = build(tmp_path, "d1", net, (2, 1, 50, 131))
    check(ctx, p, RNG.uniform(-0.5, 0.5, (2, 1, 50, 131)).astype(np.float32))


def test_direct_conv_full_and_pooled_outputs(ctx, tmp_path):
    # e0 read by a 2 x 2 MaxPool and a Concat (16-aligned channel slice): one pass writes the
    # full output into the Concat and the pooled one (the detector's first level).
    def net(g, x):
        e0 = conv(g, x, 1, 16, act="Relu")
        p0 = g.add("MaxPool", [e0], kernel_shape=[2, 2], strides=[2, 2])
        e1 = conv(g, p0, 16, 16, act="Relu")
        wt = f16x(RNG.standard_normal((16, 16, 2, 2)).astype(np.float32) * 0.25)
        u = g.add("ConvTranspose", [e1, g.init("ut", wt), g.init("ub", np.zeros(16, np.float32) + 0.05)],
                  kernel_shape=[2, 2], strides=[2, 2])
        u = g.add("Relu", [u])
        c = g.add("Concat", [u, e0], axis=1)
        return conv(g, c, 32, 8, act="Relu")
    p = build(tmp_path, "fp", net, (2, 1, 40, 52))
    check(ctx, p, RNG.uniform(-0.5, 0.5, (2, 1, 40, 52)).astype(np.float32))


def test_direct_conv_two_readers_and_concat(ctx, tmp_path):
    # e0 is read by a MaxPool and a Concat (no fusion); the Concat takes the ConvTranspose output
    # and the skip in its channel range, plus the graph input (a copy, not an alias).
    def net(g, x):
        e0 = conv(g, x, 1, 16, act="Relu")
        p0 = g.add("MaxPool", [e0], kernel_shape=[2, 2], strides=[2, 2])
        e1 = conv(g, p0, 16, 32, act="Relu")
        wt = f16x(RNG.standard_normal((32, 16, 2, 2)).astype(np.float32) * 0.25)
        u = g.add("ConvTranspose", [e1, g.init("ut", wt), g.init("ub", np.zeros(16, np.float32) + 0.05)],
                  kernel_shape=[2, 2], strides=[2, 2])
        u = g.add("Relu", [u])
        c = g.add("Concat", [u, e0, x], axis=1)
        return conv(g, c, 33, 8, act="Relu")
    p = build(tmp_path, "cc", net, (1, 1, 24, 30))
    check(ctx, p, RNG.uniform(-0.5, 0.5, (1, 1, 24, 30)).astype(np.float32))


def test_conv_transpose_2x3(ctx, tmp_path):
    def net(g, x):
        wt = RNG.standard_normal((20, 9, 2, 3)).astype(np.float32) * 0.3
        y = g.add("ConvTranspose", [x, g.init("w", wt), g.init("b", RNG.standard_normal(9).astype(np.float32))],
                  kernel_shape=[2, 3], strides=[2, 2])
        return g.add("Sigmoid", [y])
    p = build(tmp_path, "t", net, (2, 20, 5, 7))
    check(ctx, p, RNG.standard_normal((2, 20, 5, 7)).astype(np.float32))


@pytest.mark.parametrize("k,stride,cin,cout,hw,exact", [((3, 3), 1, 8, 5, (6, 9), False),
                                                        ((2, 2), 2, 40, 16, (6, 9), False),
                                                        ((3, 3), 2, 12, 7, (6, 9), False),
                                                        ((1, 1), 2, 6, 4, (6, 9), False),
                                                        ((2, 2), 2, 40, 16, (6, 9), True),
                                                        ((2, 2), 2, 64, 32, (13, 37), True),
                                                        ((2, 2), 2, 32, 48, (1, 1), True),
                                                        ((2, 2), 2, 128, 64, (5, 7), True),
                                                        ((2, 2), 2, 256, 48, (3, 10), False),
                                                        ((3, 3), 3, 16, 16, (5, 4), True),
                                                        ((3, 3), 2, 16, 16, (5, 7), True),
                                                        ((2, 3), 2, 32, 16, (4, 5), True),
                                                        ((2, 3), 2, 256, 128, (5, 7), True),
                                                        ((3, 3), 2, 128, 32, (4, 6), True)])
def test_conv_transpose_phases(ctx, tmp_path, k, stride, cin, cout, hw, exact):
    """Sub-pixel phases on the matrix cores (any kernel at least the stride; kernel = stride with
    float16-exact weights as one GEMM over the input pixels), the scalar kernel when a phase has
    no taps (1 x 1 with stride 2); the detector's 2 x 3 upsampler at 256 -> 128 and a 3 x 3 kernel
    with stride 2 (up to four taps on one output) among them."""
    def net(g, x):
        wt = RNG.standard_normal((cin, cout, *k)).astype(np.float32) * 0.3
        if exact:
            wt = f16x(wt)
        y = g.add("ConvTranspose", [x, g.init("w", wt), g.init("b", RNG.standard_normal(cout).astype(np.float32))],
                  kernel_shape=list(k), strides=[stride, stride])
        return g.add("Relu", [y])
    p = build(tmp_path, "tp", net, (2, cin, *hw))
    check(ctx, p, RNG.standard_normal((2, cin, *hw)).astype(np.float32))


@pytest.mark.parametrize("cin,cout,hw,stride,act,exact", [(32, 16, (37, 29), 2, "Relu", True),
                                                          (64, 48, (11, 13), 2, "Sigmoid", False),
                                                          (24, 32, (7, 9), 3, "Relu", True),
                                                          (16, 8, (9, 10), 2, "Relu", True)])
def test_conv_transpose_into_concat_slice(ctx, tmp_path, cin, cout, hw, stride, act, exact):
    """Kernel = stride ConvTranspose writing its phases into a channel slice of a Concat (the
    U-Net's skip joins), as one matrix-core GEMM over the input pixels when the phases are packed
    (output channels a multiple of 16), else the float32 or general paths."""
    def net(g, x):
        wt = RNG.standard_normal((cin, cout, stride, stride)).astype(np.float32) * 0.3
        if exact:
            wt = f16x(wt)
        up = g.add("ConvTranspose", [x, g.init("w", wt), g.init("b", RNG.standard_normal(cout).astype(np.float32))],
                   kernel_shape=[stride, stride], strides=[stride, stride])
        up = g.add(act, [up])
        side = g.add("Relu", [g.add("ConvTranspose", [x, g.init("w2", f16x(RNG.standard_normal(
            (cin, 16, stride, stride)).astype(np.float32) * 0.3))], kernel_shape=[stride, stride],
            strides=[stride, stride])])
        return g.add("Concat", [side, up], axis=1)
    p = build(tmp_path, "tcat", net, (2, cin, *hw))
    check(ctx, p, RNG.standard_normal((2, cin, *hw)).astype(np.float32))


def test_conv_pool_fusion_single_and_dual(ctx, tmp_path):
    """A MaxPool after a 3 x 3 conv runs in its epilogue: alone, and next to the full output
    when a Concat also reads the conv."""
    def net(g, x):
        a = conv(g, x, 16, 32, act="Relu")
        pa = g.add("MaxPool", [a], kernel_shape=[2, 2], strides=[2, 2])
        b = conv(g, pa, 32, 32, act="Relu")
        pb = g.add("MaxPool", [b], kernel_shape=[2, 2], strides=[2, 2])
        up = g.add("ConvTranspose", [pb, g.init("wu", RNG.standard_normal((32, 32, 2, 3)).astype(np.float32) * 0.2)],
                   kernel_shape=[2, 3], strides=[2, 2])
        return g.add("Concat", [up, b], axis=1)
    p = build(tmp_path, "pf", net, (2, 16, 20, 34))
    check(ctx, p, RNG.standard_normal((2, 16, 20, 34)).astype(np.float32))


def test_maxpool_slice_pad(ctx, tmp_path):
    def net(g, x):
        y = g.add("MaxPool", [x], kernel_shape=[2, 1], strides=[2, 1])
        y = g.add("Pad", [y, g.init("pads", np.zeros(8, np.int64))])
        return g.add("Slice", [y, g.init("st", np.array([1, 2], np.int64)), g.init("en", np.array([-1, 100], np.int64)),
                               g.init("ax", np.array([2, 3], np.int64))])
    p = build(tmp_path, "mp", net, (2, 6, 13, 9))
    check(ctx, p, RNG.standard_normal((2, 6, 13, 9)).astype(np.float32), tol=0)


def test_unsupported_op_is_an_error(ctx, tmp_path):
    import ocrhip
    p = build(tmp_path, "bad", lambda g, x: g.add("Tanh", [x]), (1, 1, 4, 4))
    with pytest.raises(ocrhip.OcrError, match="unsupported op Tanh"):
        ocrhip.Graph(ctx, p)


def test_shape_errors(ctx, tmp_path):
    import ocrhip
    p = build(tmp_path, "cs", lambda g, x: conv(g, x, 4, 4), (1, 4, 5, 5))
    gr = ocrhip.Graph(ctx, p)
    with pytest.raises(ocrhip.OcrError):
        gr.run(np.zeros((1, 3, 5, 5), np.float32))  # wrong channel count


@pytest.mark.parametrize("cin,cout,h,w,pool,two", [(32, 64, 17, 45, (2, 2), False), (64, 128, 16, 37, (2, 1), False),
                                                   (128, 256, 4, 53, (2, 1), False), (16, 97, 9, 23, (2, 1), True),
                                                   (256, 128, 13, 19, (2, 2), True), (20, 48, 31, 70, (2, 2), False),
                                                   (64, 32, 15, 29, (2, 2), True)])
def test_conv_pool_fusion_shapes(ctx, tmp_path, cin, cout, h, w, pool, two):
    """MaxPool fused into the conv epilogue over odd sizes, several channel blocks (cout not a
    multiple of the block), several input slices and partial slices; `two`: the full output is
    read as well (by a Concat), so both are written."""
    h2, w2 = h // pool[0] * pool[0], w // pool[1] * pool[1]

    def crop(g, y, name):
        return g.add("Slice", [y, g.init(f"{name}0", np.array([0, 0], np.int64)),
                               g.init(f"{name}1", np.array([h2, w2], np.int64)),
                               g.init(f"{name}2", np.array([2, 3], np.int64))])

    def net(g, x):
        a = conv(g, x, cin, cout, act="Relu")
        pa = g.add("MaxPool", [a], kernel_shape=list(pool), strides=list(pool))
        if not two:
            return pa
        wu = f16x(RNG.standard_normal((cout, 8, 2, 2)).astype(np.float32) * 0.1)
        up = g.add("ConvTranspose", [pa, g.init("wu", wu)], kernel_shape=[2, 2], strides=[2, 2])
        return g.add("Concat", [crop(g, up, "cu"), crop(g, a, "ca")], axis=1)

    p = build(tmp_path, "pfs", net, (2, cin, h, w))
    check(ctx, p, RNG.standard_normal((2, cin, h, w)).astype(np.float32))
