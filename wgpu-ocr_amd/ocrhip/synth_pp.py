"""Synthetic PP-OCRv6-architecture models and inputs (random-init; no model files exist offline).

The layer lists are this library's own, built from the operator patterns the reference's N-D
executor accepts and fuses (src/nd.rs:505-817): BatchNormalization, a separate bias Add after a
Conv or MatMul, Relu, the exporter's GELU chain (Div by sqrt 2, Erf, Add 1, Mul, Mul 0.5), a
residual Add, squeeze-excitation (HardSigmoid gate Mul read by a dense Conv), the 9-node
LayerNorm chain, MatMul + bias + SiLU (Sigmoid, Mul), ConvTranspose + bias + Relu / Sigmoid,
nearest Resize, and shape arithmetic kept on the host (Shape, Gather, Concat of integers).

Recogniser (the PP-OCR text-line configuration): [n, 3, 48, W] -> a CNN backbone (stride-2 stem, depthwise +
pointwise blocks, one SE block, one GELU residual block, AveragePool (3, 1)) to [n, 256, 1, W/8]
-> an SVTR neck (3x3 and 1x1 convs to dim 120, 2 transformer blocks with 8 heads and MLP ratio
2, LayerNorm, then back to channels, concat with the shortcut, 3x3 and 1x1 convs) -> a linear
CTC head over 18 708 classes -> Softmax.

Detector (the PP-OCR page configuration): [1, 3, H, W] (multiples of 32) -> stem + 4 depthwise/pointwise
stages (strides 4, 8, 16, 32; 32-256 channels) -> a DB FPN (1x1 laterals to 64, nearest x2
top-down adds, 3x3 convs to 16, nearest upsampling to H/4, Concat) -> the DB head (3x3 conv,
BatchNormalization, Relu, ConvTranspose x2 with Relu, ConvTranspose x2 with Sigmoid) -> the
probability map [1, 1, H, W]. Its last layer is fitted so the map follows the ink (det_model).

Every weight is Kaiming-normal from a seeded PCG64 stream, rounded to a float16 value.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np

from . import onnx_write as ow
from .synth import _f16_exact, kaiming, uniform_bias

REC_H = 48
PP_CLASSES = 18708
DIM, HEADS, MLP = 120, 8, 2
DET_MAX_SIDE = 960


class _B:
    """Graph builder helpers for the patterns above."""

    def __init__(self, name: str, seed: int):
        self.g = ow.Graph(name)
        self.rng = np.random.Generator(np.random.PCG64(seed))
        self.k = 0

    def name(self, stem):
        self.k += 1
        return f"{stem}{self.k}"

    def w(self, stem, arr):
        return self.g.init(self.name(stem), arr)

    def const(self, stem, value):
        return self.w(stem, np.asarray(value, np.float32).reshape(1) if np.ndim(value) == 0 else
                      np.asarray(value, np.float32))

    def ints(self, stem, vals):
        return self.g.init(self.name(stem), np.asarray(vals, np.int64))

    def conv(self, x, cin, cout, k=3, stride=(1, 1), group=1, bias=True, pads=None):
        kh, kw = (k, k) if isinstance(k, int) else k
        fan = cin // group * kh * kw
        w = self.w("cw", kaiming(self.rng, (cout, cin // group, kh, kw), fan))
        if pads is None:
            pads = [kh // 2, kw // 2, kh // 2, kw // 2]
        ins = [x, w] + ([self.w("cb", uniform_bias(self.rng, cout, fan))] if bias else [])
        return self.g.add("Conv", ins, kernel_shape=[kh, kw], pads=list(pads), strides=list(stride), group=group)

    def bn(self, x, c):
        gamma = _f16_exact(self.rng.uniform(0.8, 1.2, c).astype(np.float32))
        beta = _f16_exact(self.rng.uniform(-0.1, 0.1, c).astype(np.float32))
        mean = _f16_exact(self.rng.uniform(-0.1, 0.1, c).astype(np.float32))
        var = _f16_exact(self.rng.uniform(0.5, 1.5, c).astype(np.float32))
        ins = [x] + [self.w(s, v) for s, v in (("g", gamma), ("b", beta), ("m", mean), ("v", var))]
        return self.g.add("BatchNormalization", ins, epsilon=1e-5)

    def relu(self, x):
        return self.g.add("Relu", [x])

    def gelu(self, x):
        d = self.g.add("Div", [x, self.const("sqrt2", np.float32(np.sqrt(2.0)))])
        e = self.g.add("Erf", [d])
        a = self.g.add("Add", [e, self.const("one", 1.0)])
        m = self.g.add("Mul", [x, a])
        return self.g.add("Mul", [m, self.const("half", 0.5)])

    def linear(self, x, k, n, silu=False):
        w = self.w("lw", kaiming(self.rng, (k, n), k))
        y = self.g.add("MatMul", [x, w])
        y = self.g.add("Add", [y, self.w("lb", uniform_bias(self.rng, n, k))])
        if silu:
            s = self.g.add("Sigmoid", [y])
            y = self.g.add("Mul", [y, s])
        return y

    def layer_norm(self, x, c, eps=1e-6):
        gamma = _f16_exact(self.rng.uniform(0.8, 1.2, c).astype(np.float32))
        beta = _f16_exact(self.rng.uniform(-0.1, 0.1, c).astype(np.float32))
        m = self.g.add("ReduceMean", [x], axes=[-1], keepdims=1)
        d = self.g.add("Sub", [x, m])
        p = self.g.add("Pow", [d, self.const("two", 2.0)])
        v = self.g.add("ReduceMean", [p], axes=[-1], keepdims=1)
        a = self.g.add("Add", [v, self.const("eps", np.float32(eps))])
        s = self.g.add("Sqrt", [a])
        n = self.g.add("Div", [d, s])
        y = self.g.add("Mul", [n, self.w("lng", gamma)])
        return self.g.add("Add", [y, self.w("lnb", beta)])

    def resize(self, x, f):
        sc = self.w("sc", np.array([1.0, 1.0, f, f], np.float32))
        return self.g.add("Resize", [x, "", sc], mode="nearest", coordinate_transformation_mode="asymmetric",
                          nearest_mode="floor")


# ---------------------------------------------------------------------------------------------
# Recogniser
# ---------------------------------------------------------------------------------------------
def _svtr_block(b: _B, x):
    """x [n, T, 120]: x + proj(attention(LN(x))), then x + fc2(SiLU(fc1(LN(x))))."""
    hd = DIM // HEADS
    h = b.layer_norm(x, DIM)
    qkv = b.linear(h, DIM, 3 * DIM)
    # The head layout through shape arithmetic on the host: [n, T] from Shape + Gather.
    shp = b.g.add("Shape", [qkv])
    nt = b.g.add("Gather", [shp, b.ints("i01", [0, 1])], axis=0)
    s5 = b.g.add("Concat", [nt, b.ints("h", [3, HEADS, hd])], axis=0)
    q5 = b.g.add("Reshape", [qkv, s5])                              # [n, T, 3, 8, 15]
    t5 = b.g.add("Transpose", [q5], perm=[2, 0, 3, 1, 4])         # [3, n, 8, T, 15]
    parts = []
    for i in range(3):
        s = b.g.add("Slice", [t5, b.ints("s", [i]), b.ints("e", [i + 1]), b.ints("a", [0])])
        parts.append(b.g.add("Squeeze", [s, b.ints("ax", [0])]))   # [n, 8, T, 15]
    q, k, v = parts
    q = b.g.add("Mul", [q, b.const("scale", np.float32(hd ** -0.5))])
    kt = b.g.add("Transpose", [k], perm=[0, 1, 3, 2])              # [n, 8, 15, T]
    att = b.g.add("MatMul", [q, kt])                               # [n, 8, T, T]
    att = b.g.add("Softmax", [att], axis=-1)
    o = b.g.add("MatMul", [att, v])                                # [n, 8, T, 15]
    o = b.g.add("Transpose", [o], perm=[0, 2, 1, 3])               # [n, T, 8, 15]
    o = b.g.add("Reshape", [o, b.ints("r", [0, 0, DIM])])
    x = b.g.add("Add", [x, b.linear(o, DIM, DIM)])
    h = b.layer_norm(x, DIM)
    h = b.linear(h, DIM, MLP * DIM, silu=True)
    return b.g.add("Add", [x, b.linear(h, MLP * DIM, DIM)])


def rec_model(seed: int = 0, classes: int = PP_CLASSES) -> bytes:
    b = _B("ppocr_rec_synth", seed + 500)
    x = "pp_lines"
    # Backbone
    x = b.relu(b.bn(b.conv(x, 3, 32, stride=(2, 2), bias=False), 32))                    # 24 x W/2
    x = b.relu(b.conv(x, 32, 32, group=32))
    x = b.relu(b.g.add("Add", [b.conv(x, 32, 64, k=1, bias=False), b.w("ab", uniform_bias(b.rng, 64, 32).reshape(1, 64, 1, 1))]))
    x = b.relu(b.bn(b.conv(x, 64, 64, stride=(2, 2), group=64, bias=False), 64))         # 12 x W/4
    x = b.relu(b.bn(b.conv(x, 64, 128, k=1, bias=False), 128))
    x = b.relu(b.bn(b.conv(x, 128, 128, stride=(2, 1), group=128, bias=False), 128))     # 6 x W/4
    se = b.g.add("GlobalAveragePool", [x])
    se = b.relu(b.conv(se, 128, 32, k=1))
    se = b.g.add("HardSigmoid", [b.conv(se, 32, 128, k=1)], alpha=0.2, beta=0.5)
    x = b.g.add("Mul", [x, se])
    x = b.relu(b.conv(x, 128, 256, k=1))
    x = b.relu(b.bn(b.conv(x, 256, 256, stride=(2, 2), group=256, bias=False), 256))     # 3 x W/8
    x = b.g.add("Add", [b.gelu(b.conv(x, 256, 256, k=1)), x])
    x = b.g.add("AveragePool", [x], kernel_shape=[3, 1], strides=[3, 1])                 # 1 x W/8
    shortcut = x
    # Neck (SVTR)
    x = b.relu(b.conv(x, 256, 32, k=3))
    x = b.relu(b.conv(x, 32, DIM, k=1))
    x = b.g.add("Squeeze", [x, b.ints("ax", [2])])
    x = b.g.add("Transpose", [x], perm=[0, 2, 1])                                       # [n, T, 120]
    for _ in range(2):
        x = _svtr_block(b, x)
    x = b.layer_norm(x, DIM)
    x = b.g.add("Transpose", [x], perm=[0, 2, 1])
    x = b.g.add("Unsqueeze", [x, b.ints("ax", [2])])                                    # [n, 120, 1, T]
    x = b.relu(b.conv(x, DIM, 256, k=1))
    x = b.g.add("Concat", [shortcut, x], axis=1)
    x = b.relu(b.conv(x, 512, 32, k=3))
    x = b.relu(b.conv(x, 32, DIM, k=1))
    x = b.g.add("Squeeze", [x, b.ints("ax", [2])])
    x = b.g.add("Transpose", [x], perm=[0, 2, 1])
    # Head
    x = b.linear(x, DIM, classes)
    out = b.g.add("Softmax", [x], axis=2)
    return b.g.model("pp_lines", ["batch", 3, REC_H, "width"], out, ["batch", "steps", classes])


# ---------------------------------------------------------------------------------------------
# DB detector
# ---------------------------------------------------------------------------------------------
class _Eager:
    """numpy evaluation of the detector's layers, for the calibration of its last layer only."""

    @staticmethod
    def conv(x, w, b, stride, group):
        n, c, h, wd = x.shape
        cout, cin_g, kh, kw = w.shape
        xp = np.pad(x, ((0, 0), (0, 0), (kh // 2, kh // 2), (kw // 2, kw // 2)))
        oh, ow = (h + 2 * (kh // 2) - kh) // stride[0] + 1, (wd + 2 * (kw // 2) - kw) // stride[1] + 1
        taps = [xp[:, :, ky: ky + stride[0] * (oh - 1) + 1: stride[0], kx: kx + stride[1] * (ow - 1) + 1: stride[1]]
                for ky in range(kh) for kx in range(kw)]
        if group == c and cin_g == 1:  # depthwise
            y = sum(t * w[:, 0, k // kw, k % kw][None, :, None, None] for k, t in enumerate(taps))
        else:
            cols = np.stack(taps, axis=2).reshape(n, c * kh * kw, oh * ow)  # channel-major like w
            y = np.einsum("ok,nkp->nop", w.reshape(cout, -1), cols).reshape(n, cout, oh, ow)
        return (y + (0 if b is None else b[None, :, None, None])).astype(np.float32)

    @staticmethod
    def bn(x, g, b, m, v, eps=1e-5):
        s = g / np.sqrt(v + eps)
        return (x * s[None, :, None, None] + (b - m * s)[None, :, None, None]).astype(np.float32)

    @staticmethod
    def up(x, f):
        f = int(f)
        return np.repeat(np.repeat(x, f, axis=2), f, axis=3)

    @staticmethod
    def convt2(x, w, b):
        n, c, h, wd = x.shape
        y = np.zeros((n, w.shape[1], 2 * h, 2 * wd), np.float32)
        for dy in range(2):
            for dx in range(2):
                y[:, :, dy::2, dx::2] = np.einsum("co,nchw->nohw", w[:, :, dy, dx], x)
        return y + b[None, :, None, None]


def _det_layers(b: _B, x_name: str, x_val):
    """The detector up to the features the last ConvTranspose reads: graph nodes into b, and the
    same layers evaluated with numpy on x_val (None: graph only). Returns (name, value)."""
    E = _Eager
    v = x_val

    def cbr(x, v, cin, cout, k=3, stride=(1, 1), group=1, blur=False, signed=False):
        fan = cin // group * k * k
        wt = kaiming(b.rng, (cout, cin // group, k, k), fan)
        if blur or signed:
            # Random positive kernels normalised to sum 1 (a random blur), with a random sign per
            # output channel for the stem: the features keep how dark each region is.
            wt = np.abs(wt) / np.abs(wt).reshape(cout, -1).sum(axis=1)[:, None, None, None]
            if signed:
                wt *= np.where(b.rng.random(cout) < 0.5, -1.0, 1.0).astype(np.float32)[:, None, None, None] * 4
            wt = _f16_exact(wt)
        gamma = _f16_exact(b.rng.uniform(0.8, 1.2, cout).astype(np.float32))
        beta = _f16_exact(b.rng.uniform(-0.1, 0.1, cout).astype(np.float32))
        mean = _f16_exact(b.rng.uniform(-0.1, 0.1, cout).astype(np.float32))
        var = _f16_exact(b.rng.uniform(0.5, 1.5, cout).astype(np.float32))
        y = b.g.add("Conv", [x, b.w("cw", wt)], kernel_shape=[k, k], pads=[k // 2] * 4, strides=list(stride),
                    group=group)
        y = b.g.add("BatchNormalization", [y] + [b.w(nm, a) for nm, a in
                                                 (("g", gamma), ("b", beta), ("m", mean), ("v", var))], epsilon=1e-5)
        y = b.relu(y)
        if v is not None:
            v = np.maximum(E.bn(E.conv(v, wt, None, stride, group), gamma, beta, mean, var), 0)
        return y, v

    def conv(x, v, cin, cout, k):
        wt = kaiming(b.rng, (cout, cin, k, k), cin * k * k)
        y = b.g.add("Conv", [x, b.w("cw", wt)], kernel_shape=[k, k], pads=[k // 2] * 4, strides=[1, 1])
        return y, (None if v is None else E.conv(v, wt, None, (1, 1), 1))

    def add(a, va, c, vc):
        return b.g.add("Add", [a, c]), (None if va is None else va + vc)

    def up(x, vx, f):
        return b.resize(x, float(f)), (None if vx is None else E.up(vx, f))

    x, v = cbr(x_name, v, 3, 16, stride=(2, 2), signed=True)                             # /2
    feats = []
    cin = 16
    for cout in (32, 64, 128, 256):                                                      # /4 .. /32
        x, v = cbr(x, v, cin, cin, stride=(2, 2), group=cin, blur=True)
        x, v = cbr(x, v, cin, cout, k=1)
        feats.append((x, v, cout))
        cin = cout
    lat = [conv(f, fv, c, 64, 1) for f, fv, c in feats]
    (in2, v2), (in3, v3), (in4, v4), (in5, v5) = lat
    out4 = add(in4, v4, *up(in5, v5, 2))
    out3 = add(in3, v3, *up(*out4, 2))
    out2 = add(in2, v2, *up(*out3, 2))
    p5 = up(*conv(in5, v5, 64, 16, 3), 8)
    p4 = up(*conv(*out4, 64, 16, 3), 4)
    p3 = up(*conv(*out3, 64, 16, 3), 2)
    p2 = conv(*out2, 64, 16, 3)
    fuse = b.g.add("Concat", [p5[0], p4[0], p3[0], p2[0]], axis=1)                       # [1, 64, H/4, W/4]
    fv = None if v is None else np.concatenate([p5[1], p4[1], p3[1], p2[1]], axis=1)
    x, v = cbr(fuse, fv, 64, 16)
    w1 = kaiming(b.rng, (16, 16, 2, 2), 16)
    b1 = uniform_bias(b.rng, 16, 16)
    x = b.g.add("ConvTranspose", [x, b.w("tw", w1), b.w("tb", b1)], kernel_shape=[2, 2], strides=[2, 2])
    x = b.relu(x)
    if v is not None:
        v = np.maximum(E.convt2(v, w1, b1), 0)
    return x, v


def _det_calibration_input(seed: int = 999):
    """A synthetic page as the detector sees it (about [1, 3, 960, 736]: page pixels sampled at
    the resize's source positions, BGR, ImageNet-normalised) and its word-block mask at H/2."""
    from . import synth
    rgb, blocks = synth.page(seed, with_blocks=True)
    h, w = rgb.shape[:2]
    ow, oh = 736, 960
    ys = np.minimum(((np.arange(oh) + 0.5) * h / oh).astype(int), h - 1)
    xs = np.minimum(((np.arange(ow) + 0.5) * w / ow).astype(int), w - 1)
    small = rgb[np.ix_(ys, xs)].astype(np.float32)[..., ::-1]
    mean, dev = np.array([0.485, 0.456, 0.406], np.float32), np.array([0.229, 0.224, 0.225], np.float32)
    x = ((small / 255.0 - mean) / dev).transpose(2, 0, 1)[None].astype(np.float32)
    label = blocks[np.ix_(ys[1::2], xs[1::2])]
    return x, label


def det_model(seed: int = 0) -> bytes:
    """The DB detector. Its last layer (ConvTranspose 16 -> 1 with Sigmoid) is not random: its
    four taps share one weight vector (a 1 x 1 projection upsampled by 2, as the ocrs synthetic
    detector's heads are tied) fitted by least squares on a held-out synthetic page (seed 999)
    against its word blocks, so that the probability map follows the ink."""
    x_in, label = _det_calibration_input()
    b = _B("ppocr_det_synth", seed + 700)
    x, feats = _det_layers(b, "pp_page", x_in)
    f = feats[0].reshape(16, -1).T.astype(np.float64)                                    # [pixels, 16]
    a = np.concatenate([f, np.ones((f.shape[0], 1))], axis=1)
    y = np.where(label.reshape(-1), 1.0, -1.0)
    wt = np.sqrt(np.where(label, 0.5 / label.mean(), 0.5 / (1 - label.mean()))).reshape(-1)
    sol = np.linalg.lstsq(a * wt[:, None], y * wt, rcond=None)[0]
    # Logits of about +-4; the bias puts 10 % of the fit page's paper pixels (most of them next to
    # the ink) above 0.3.
    sol *= 4.0
    paper = (f @ sol[:-1])[~label.reshape(-1)]
    sol[-1] = np.log(0.3 / 0.7) - np.quantile(paper, 0.90)
    w2 = np.repeat(np.repeat(sol[:-1].reshape(16, 1, 1, 1), 2, axis=2), 2, axis=3).astype(np.float32)
    x = b.g.add("ConvTranspose", [x, b.w("tw", _f16_exact(w2))], kernel_shape=[2, 2], strides=[2, 2])
    x = b.g.add("Add", [x, b.w("tb", _f16_exact(np.array([sol[-1]], np.float32)))])
    out = b.g.add("Sigmoid", [x])
    return b.g.model("pp_page", [1, 3, "height", "width"], out, [1, 1, "height", "width"])


def model_path(kind: str, seed: int = 0, directory: str | None = None) -> str:
    """Write (once) and return the path of a synthetic PP-OCR model: kind 'rec' or 'det'."""
    from . import synth

    directory = directory or os.environ.get("OCRHIP_MODELS") or os.path.join(
        os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))), ".models")
    os.makedirs(directory, exist_ok=True)
    src = open(__file__, "rb").read() + open(ow.__file__, "rb").read() + open(synth.__file__, "rb").read()
    tag = hashlib.sha256(src + kind.encode() + str(seed).encode()).hexdigest()[:12]
    path = os.path.join(directory, f"pp_{kind}_s{seed}_{tag}.onnx")
    if not os.path.exists(path):
        data = rec_model(seed) if kind == "rec" else det_model(seed)
        tmp = f"{path}.{os.getpid()}.tmp"
        with open(tmp, "wb") as f:
            f.write(data)
        os.replace(tmp, path)
    return path


# ---------------------------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------------------------
def rec_lines(n: int = 36, seed: int = 0, wmin: int = 160, wmax: int = 960):
    """RGB line images [3, 48, W] in [-1, 1]: a light background with dark strokes."""
    rng = np.random.Generator(np.random.PCG64(seed + 4000))
    out = []
    for _ in range(n):
        w = int(rng.integers(wmin, wmax + 1))
        img = np.full((3, REC_H, w), 0.9, np.float32) + rng.uniform(-0.05, 0.05, (3, 1, 1)).astype(np.float32)
        x = int(rng.integers(0, 12))
        while x < w - 4:
            sw, sh = int(rng.integers(2, 7)), int(rng.integers(14, 34))
            y0 = int(rng.integers(4, REC_H - sh))
            img[:, y0: y0 + sh, x: x + sw] = rng.uniform(-1.0, -0.5)
            x += sw + int(rng.integers(1, 9))
        out.append(np.clip(img, -1, 1).astype(np.float32))
    return out


def batch_lines(lines, per_batch: int = 16):
    """The reference's PP-OCR batching (src/bin/ocr-bench.rs:330-345): lines sorted by width,
    cut into batches of `per_batch`, each padded with 0 on the right to its widest line rounded
    up to a multiple of 8. Returns (batches as (array [n, 3, 48, W], n, W), order)."""
    order = sorted(range(len(lines)), key=lambda i: lines[i].shape[2])
    batches = []
    for c in range(0, len(order), per_batch):
        part = order[c: c + per_batch]
        width = -(-max(lines[i].shape[2] for i in part) // 8) * 8
        data = np.zeros((len(part), 3, REC_H, width), np.float32)
        for k, i in enumerate(part):
            data[k, :, :, : lines[i].shape[2]] = lines[i]
        batches.append((data, len(part), width))
    return batches, order
