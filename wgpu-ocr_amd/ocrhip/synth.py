"""Synthetic ocrs-architecture models and inputs (no model files exist offline).

Models are written as ONNX files with the same operator set the reference's loaders accept
(src/gpu.rs:1104-1240 for the convolutional graph, src/gpu.rs:1452-1506 for the recogniser).
Every weight is Kaiming-normal (std = sqrt(2 / fan_in)) from a seeded numpy PCG64 stream and
then rounded to the nearest float16 value (kept as float32 in the file): a float16 copy of a
weight is therefore exact, which the GPU kernels rely on for their f16 matrix-core operands.

The detector is random-init too, with two changes that make its mask follow the ink: each
ConvTranspose's random weights are tied across its stride taps (the resize-convolution
initialisation of Odena et al., "Deconvolution and Checkerboard Artifacts", 2016; a 3-wide kernel
gets half weight on its outer taps, i.e. linear interpolation), and the 16 weights and bias of
the 1x1 head are a least-squares fit on one held-out synthetic page (seed 999) against its word
blocks. An untrained U-Net's mask is otherwise unrelated to where the text is, and the page
pipeline would find no text lines.
"""
from __future__ import annotations

import hashlib
import os

import numpy as np

from . import onnx_write as ow

REC_HEIGHT = 64
CLASSES = 97
HIDDEN = 256
DET_H, DET_W = 800, 600
BLACK = -0.5

# ocr-bench.rs:31 - class k > 0 is ALPHABET[k - 1]; class 0 is the CTC blank.
ALPHABET = " 0123456789!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~EABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz"


def _f16_exact(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16).astype(np.float32)


def kaiming(rng: np.random.Generator, shape, fan_in: int, exact: bool = True) -> np.ndarray:
    std = np.float32(np.sqrt(2.0 / fan_in))
    w = rng.standard_normal(shape, dtype=np.float32) * std
    return _f16_exact(w) if exact else w


def uniform_bias(rng: np.random.Generator, n: int, fan_in: int, exact: bool = True) -> np.ndarray:
    b = np.float32(1.0 / np.sqrt(fan_in))
    v = rng.uniform(-b, b, n).astype(np.float32)
    return _f16_exact(v) if exact else v


# ---------------------------------------------------------------------------------------------
# Recogniser: 5 x (3x3 conv + ReLU + MaxPool) -> AveragePool (2,1) -> 2 x BiGRU(256) -> 512x97
# ---------------------------------------------------------------------------------------------
REC_CONVS = [(1, 32, (2, 2)), (32, 64, (2, 2)), (64, 128, (2, 1)), (128, 128, (2, 1)), (128, 256, (2, 1))]


def rec_model(seed: int = 0, exact: bool = True) -> bytes:
    """The recogniser with Kaiming-normal weights; exact=False keeps them float32 (not rounded to
    float16 values), as a trained model's are."""
    rng = np.random.Generator(np.random.PCG64(seed))
    kaiming_ = lambda *a: kaiming(*a, exact=exact)  # noqa: E731
    bias_ = lambda *a: uniform_bias(*a, exact=exact)  # noqa: E731
    g = ow.Graph("ocrs_rec_synth")
    x = "line_images"
    for i, (cin, cout, pool) in enumerate(REC_CONVS):
        w = g.init(f"conv{i}.w", kaiming_(rng, (cout, cin, 3, 3), cin * 9))
        b = g.init(f"conv{i}.b", bias_(rng, cout, cin * 9))
        x = g.add("Conv", [x, w, b], kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[1, 1])
        x = g.add("Relu", [x])
        x = g.add("MaxPool", [x], kernel_shape=list(pool), strides=list(pool))
    x = g.add("AveragePool", [x], kernel_shape=[2, 1], strides=[2, 1])
    x = g.add("Squeeze", [x, g.init("squeeze_axes", np.array([2], np.int64))])
    x = g.add("Transpose", [x], perm=[2, 0, 1])  # [T, N, 256]
    shape512 = g.init("shape_t_n_512", np.array([0, 0, 2 * HIDDEN], np.int64))
    inp = HIDDEN
    for layer in range(2):
        w = g.init(f"gru{layer}.W", kaiming_(rng, (2, 3 * HIDDEN, inp), inp))
        r = g.init(f"gru{layer}.R", kaiming_(rng, (2, 3 * HIDDEN, HIDDEN), HIDDEN))
        bb = np.concatenate([bias_(rng, 6 * HIDDEN, HIDDEN) for _ in range(2)]).reshape(2, 6 * HIDDEN)
        b = g.init(f"gru{layer}.B", bb)
        y, _ = g.add("GRU", [x, w, r, b], n_out=2, hidden_size=HIDDEN, direction="bidirectional",
                     linear_before_reset=1)
        y = g.add("Transpose", [y], perm=[0, 2, 1, 3])  # [T, N, 2, 256]
        x = g.add("Reshape", [y, shape512])
        inp = 2 * HIDDEN
    lw = g.init("output.w", kaiming_(rng, (2 * HIDDEN, CLASSES), 2 * HIDDEN))
    lb = g.init("output.b", bias_(rng, CLASSES, 2 * HIDDEN))
    x = g.add("MatMul", [x, lw])
    x = g.add("Add", [x, lb])
    out = g.add("LogSoftmax", [x], axis=2)
    return g.model("line_images", ["batch", 1, REC_HEIGHT, "width"], out, ["seq", "batch", CLASSES])


# ---------------------------------------------------------------------------------------------
# Detector: U-Net 16-32-64-128-256, ConvTranspose upsampling + Concat skips, 1x1 head + Sigmoid
# ---------------------------------------------------------------------------------------------
DET_ENC = [16, 32, 64, 128, 256]


def _det_weights(seed: int):
    rng = np.random.Generator(np.random.PCG64(seed + 1000))
    p = {}
    cin = 1
    for i, c in enumerate(DET_ENC):
        p[f"enc{i}.w"] = kaiming(rng, (c, cin, 3, 3), cin * 9)
        p[f"enc{i}.b"] = uniform_bias(rng, c, cin * 9)
        cin = c
    for lvl in (3, 2, 1, 0):
        cup, cskip = DET_ENC[lvl + 1], DET_ENC[lvl]
        kw = 3 if lvl == 3 else 2  # 37 -> 75 columns at the coarsest level of an 800x600 input
        base = kaiming(rng, (cup, cskip), cup)
        w = np.repeat(np.repeat(base[:, :, None, None], 2, axis=2), kw, axis=3)
        if kw == 3:  # even columns take taps 0 and 2 (half each), odd columns tap 1
            w[:, :, :, 0] *= np.float32(0.5)
            w[:, :, :, 2] *= np.float32(0.5)
        p[f"up{lvl}.w"] = _f16_exact(np.ascontiguousarray(w))
        p[f"up{lvl}.b"] = uniform_bias(rng, cskip, cup)
        p[f"dec{lvl}.w"] = kaiming(rng, (cskip, 2 * cskip, 3, 3), 2 * cskip * 9)
        p[f"dec{lvl}.b"] = uniform_bias(rng, cskip, 2 * cskip * 9)
    return p


def _np_conv3(x, w, b):
    """3x3 convolution, pad 1, NCHW with N = 1, for the head calibration only."""
    c, h, wd = x.shape
    xp = np.pad(x, ((0, 0), (1, 1), (1, 1)))
    cols = np.lib.stride_tricks.sliding_window_view(xp, (3, 3), axis=(1, 2))  # c h w 3 3
    cols = cols.transpose(1, 2, 0, 3, 4).reshape(h * wd, c * 9)
    y = cols @ w.reshape(w.shape[0], -1).T + b
    return np.maximum(y, 0).T.reshape(w.shape[0], h, wd)


def _np_pool(x):
    c, h, w = x.shape
    x = x[:, : h // 2 * 2, : w // 2 * 2]
    return x.reshape(c, h // 2, 2, w // 2, 2).max(axis=(2, 4))


def _np_convt(x, w, b):
    cin, h, wd = x.shape
    _, cout, kh, kw = w.shape
    y = np.zeros((cout, (h - 1) * 2 + kh, (wd - 1) * 2 + kw), np.float32)
    for ky in range(kh):
        for kx in range(kw):
            contrib = np.tensordot(w[:, :, ky, kx], x, axes=([0], [0]))  # cout h w
            y[:, ky: ky + 2 * h: 2, kx: kx + 2 * wd: 2] += contrib
    return np.maximum(y + b[:, None, None], 0)


def _det_features(p, img):
    """Features before the head (d0) on a [h, w] image; h % 16 == 0, w = 8 * odd."""
    skips = []
    x = img[None].astype(np.float32)
    for i in range(5):
        x = _np_conv3(x, p[f"enc{i}.w"], p[f"enc{i}.b"])
        if i < 4:
            skips.append(x)
            x = _np_pool(x)
    for lvl in (3, 2, 1, 0):
        x = _np_convt(x, p[f"up{lvl}.w"], p[f"up{lvl}.b"])
        x = np.concatenate([x, skips[lvl]], axis=0)
        x = _np_conv3(x, p[f"dec{lvl}.w"], p[f"dec{lvl}.b"])
    return x


def _page_grey_small(seed: int):
    """A synthetic page as the detector sees it (grey, about 800 x 600: 4x4 box mean sampled at
    the resize's source positions) and its word-block mask at that size."""
    rgb, blocks = page(seed, with_blocks=True)
    grey = (-0.5 + rgb[..., 0] * np.float32(0.299 / 255) + rgb[..., 1] * np.float32(0.587 / 255)
            + rgb[..., 2] * np.float32(0.114 / 255)).astype(np.float32)
    ys = (np.arange(DET_H) * PAGE_H / DET_H + PAGE_H / (2 * DET_H)).astype(int)
    xs = (np.arange(DET_W) * PAGE_W / DET_W + PAGE_W / (2 * DET_W)).astype(int)
    c = np.cumsum(np.cumsum(np.pad(grey.astype(np.float64), ((1, 0), (1, 0))), 0), 1)
    y0, x0 = np.clip(ys - 2, 0, PAGE_H - 4), np.clip(xs - 2, 0, PAGE_W - 4)
    s = c[np.ix_(y0 + 4, x0 + 4)] - c[np.ix_(y0, x0 + 4)] - c[np.ix_(y0 + 4, x0)] + c[np.ix_(y0, x0)]
    label = blocks[np.ix_(ys, xs)]
    return (s / 16).astype(np.float32), label


def det_model(seed: int = 0) -> bytes:
    p = _det_weights(seed)
    grey, label = _page_grey_small(999)
    feats = _det_features(p, grey).reshape(DET_ENC[0], -1).T.astype(np.float64)
    x = np.concatenate([feats, np.ones((feats.shape[0], 1))], axis=1)
    y = np.where(label.reshape(-1), 1.0, -1.0)
    wt = np.where(label, 0.5 / label.mean(), 0.5 / (1 - label.mean()))
    edge = np.zeros_like(label)
    edge[:4], edge[-4:], edge[:, :4], edge[:, -4:] = True, True, True, True
    wt = np.sqrt(np.where(edge, 50.0 * wt, wt)).reshape(-1)  # the zero-padded border is paper too
    sol = np.linalg.lstsq(x * wt[:, None], y * wt, rcond=None)[0]
    # Bias: at most 0.5 % of the paper pixels of the fit page above the threshold (logit 0).
    paper_logits = (x[:, :-1] @ sol[:-1])[~label.reshape(-1)]
    sol[-1] = -np.quantile(paper_logits, 0.995)
    sol *= 4.0  # logits of about +-4
    p["head.w"] = _f16_exact(sol[:-1].astype(np.float32).reshape(1, DET_ENC[0], 1, 1))
    p["head.b"] = _f16_exact(sol[-1:].astype(np.float32))

    g = ow.Graph("ocrs_det_synth")
    for k, v in p.items():
        g.init(k, v)
    x = "page_grey"
    skips = []
    for i in range(5):
        x = g.add("Conv", [x, f"enc{i}.w", f"enc{i}.b"], kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[1, 1])
        x = g.add("Relu", [x])
        if i < 4:
            skips.append(x)
            x = g.add("MaxPool", [x], kernel_shape=[2, 2], strides=[2, 2])
    for lvl in (3, 2, 1, 0):
        kw = 3 if lvl == 3 else 2
        x = g.add("ConvTranspose", [x, f"up{lvl}.w", f"up{lvl}.b"], kernel_shape=[2, kw], strides=[2, 2])
        x = g.add("Relu", [x])
        x = g.add("Concat", [x, skips[lvl]], axis=1)
        x = g.add("Conv", [x, f"dec{lvl}.w", f"dec{lvl}.b"], kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[1, 1])
        x = g.add("Relu", [x])
    x = g.add("Conv", [x, "head.w", "head.b"], kernel_shape=[1, 1])
    out = g.add("Sigmoid", [x])
    return g.model("page_grey", [1, 1, DET_H, DET_W], out, [1, 1, DET_H, DET_W])


def model_path(kind: str, seed: int = 0, directory: str | None = None) -> str:
    """Write (once) and return the path of a synthetic model: kind 'rec', 'det', or 'rec_f32'
    (the recogniser with float32 weights that are not float16 values)."""
    directory = directory or os.environ.get("OCRHIP_MODELS") or os.path.join(
        os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))), ".models")
    os.makedirs(directory, exist_ok=True)
    src = open(__file__, "rb").read() + open(ow.__file__, "rb").read()
    tag = hashlib.sha256(src + kind.encode() + str(seed).encode()).hexdigest()[:12]
    path = os.path.join(directory, f"{kind}_s{seed}_{tag}.onnx")
    if not os.path.exists(path):
        if kind not in ("rec", "det", "rec_f32"):
            raise ValueError(f"unknown synthetic model kind {kind!r}")
        data = rec_model(seed) if kind == "rec" else rec_model(seed, exact=False) if kind == "rec_f32" else det_model(seed)
        tmp = f"{path}.{os.getpid()}.tmp"
        with open(tmp, "wb") as f:
            f.write(data)
        os.replace(tmp, path)
    return path


# ---------------------------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------------------------
def rec_lines(n: int = 36, seed: int = 0, wmin: int = 200, wmax: int = 800, cover: float = 0.30):
    """Grey line images [64, W]: background 1.0, dark rectangles/strokes in [0, 0.3]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    lines = []
    for _ in range(n):
        w = int(rng.integers(wmin, wmax + 1))
        img = np.ones((REC_HEIGHT, w), np.float32)
        dark = np.zeros((REC_HEIGHT, w), bool)
        while dark.mean() < cover:
            rh, rw = int(rng.integers(3, 41)), int(rng.integers(2, 31))
            y0, x0 = int(rng.integers(0, REC_HEIGHT - rh + 1)), int(rng.integers(0, max(1, w - rw + 1)))
            img[y0: y0 + rh, x0: x0 + rw] = rng.uniform(0.0, 0.3)
            dark[y0: y0 + rh, x0: x0 + rw] = True
        lines.append(img)
    return lines


def batch_lines(lines, round_to: int = 50, per_batch: int = 20, pad: float = BLACK):
    """ocrs batching (ocr-bench.rs:385-407): group by width rounded up to `round_to`, at most
    `per_batch` lines a batch, padded on the right with `pad`. Returns (batches, order, widths)
    with batches as (array [n, 64, W], n, W)."""
    groups: dict[int, list[int]] = {}
    for i, img in enumerate(lines):
        wr = -(-img.shape[1] // round_to) * round_to
        groups.setdefault(wr, []).append(i)
    batches, order, widths = [], [], []
    for wr in sorted(groups):
        members = groups[wr]
        for c in range(0, len(members), per_batch):
            chunk = members[c: c + per_batch]
            data = np.full((len(chunk), REC_HEIGHT, wr), pad, np.float32)
            for k, i in enumerate(chunk):
                data[k, :, : lines[i].shape[1]] = lines[i]
                order.append(i)
                widths.append(lines[i].shape[1])
            batches.append((data, len(chunk), wr))
    return batches, order, widths


def det_input(seed: int = 0, bands: int = 40):
    """[800, 600] grey: background 1.0 and ~40 horizontal dark text-like bands 8-20 px tall."""
    rng = np.random.Generator(np.random.PCG64(seed + 2000))
    img = np.ones((DET_H, DET_W), np.float32)
    for _ in range(bands):
        bh = int(rng.integers(8, 21))
        y0 = int(rng.integers(0, DET_H - bh))
        x = int(rng.integers(0, 80))
        xend = int(rng.integers(300, DET_W + 1))
        while x < xend:
            ww = int(rng.integers(10, 70))
            img[y0: y0 + bh, x: min(x + ww, xend)] = rng.uniform(0.0, 0.3)
            x += ww + int(rng.integers(4, 12))
    return img


PAGE_W, PAGE_H = 2550, 3300  # US Letter at 300 dpi


def page(seed: int, lines: int = 36, noise: float = 4.0, with_blocks: bool = False):
    """One synthetic page: RGB u8 [3300, 2550, 3], white, ~36 text lines made of word blocks
    of vertical ink strokes, plus Gaussian noise (sigma 4), clamped to [0, 255]. With
    with_blocks, also the [3300, 2550] bool mask of the word blocks."""
    rng = np.random.Generator(np.random.PCG64(seed + 3000))
    grey = np.full((PAGE_H, PAGE_W), 255.0, np.float32)
    blocks = np.zeros((PAGE_H, PAGE_W), bool) if with_blocks else None
    top, bottom, left = 180, PAGE_H - 180, 150
    pitch = (bottom - top) / lines
    for i in range(lines):
        lh = int(rng.integers(24, 37))
        y0 = int(top + i * pitch + rng.integers(0, max(1, int(pitch) - lh)))
        x = left + int(rng.integers(0, 60))
        xend = PAGE_W - 150 - int(rng.integers(0, 900))
        while x < xend:
            ww = int(rng.integers(40, 320))
            x1 = min(x + ww, xend)
            ink = float(rng.uniform(0, 60))
            sx = x
            while sx < x1:  # vertical strokes 4-9 px wide, gaps 1-2 px
                s = int(rng.integers(4, 10))
                grey[y0: y0 + lh, sx: min(sx + s, x1)] = ink
                sx += s + int(rng.integers(1, 3))
            if with_blocks:
                blocks[y0: y0 + lh, x: x1] = True
            x = x1 + int(rng.integers(22, 40))
    rgb = grey[:, :, None] + rng.normal(0.0, noise, (PAGE_H, PAGE_W, 3)).astype(np.float32)
    rgb = np.clip(np.rint(rgb), 0, 255).astype(np.uint8)
    return (rgb, blocks) if with_blocks else rgb
