"""ORACLE (test infrastructure only): runs an ONNX graph on the CPU in float32 with the C
restatement in oracle.c for the heavy operators and numpy for the shape operators. Only tests,
the smoke check and bench.py's cpu_baseline leg use it, always as the oracle results are compared with.

ONNX operator semantics as rten (the reference's CPU engine, rten 0.26.0) implements them; the
ocrs front and back ends follow the reference's GPU code where ocrs itself is not available:
Detector::detect_page (src/gpu.rs:1393-1422) and the greedy CTC of src/bin/ocr-bench.rs:62-74.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import onnx_read

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
SOURCES = ("oracle.c", "contours.c")
_lib = None


def build() -> str:
    """Compile oracle.c (gcc, OpenMP) into oracle/_build/liboracle.so."""
    os.makedirs(os.path.dirname(LIB_PATH), exist_ok=True)
    tmp = LIB_PATH + f".tmp{os.getpid()}"
    subprocess.run(["gcc", "-O3", "-march=x86-64-v2", "-fopenmp", "-fPIC", "-shared", "-ffp-contract=off",
                    "-o", tmp, *(os.path.join(HERE, f) for f in SOURCES), "-lm"], check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or any(os.path.getmtime(LIB_PATH) < os.path.getmtime(os.path.join(HERE, f))
                                               for f in SOURCES):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.orc_conv2d.argtypes = [P, I, I, I, I, P, I, I, I, P, I, I, I, I, I, I, I, I, P, P]
        L.orc_conv_transpose2d.argtypes = [P, I, I, I, I, P, I, I, I, P, I, I, I, P]
        L.orc_pool2d.argtypes = [P, I, I, I, I, I, I, I, I, P]
        L.orc_gru.argtypes = [P, I, I, I, P, P, P, I, I, P, P]
        L.orc_grey_resize.argtypes = [P, I, I, I, I, I, I, F, F, P]
        L.orc_mask_up_prob.argtypes = [P, I, I, I, I, I, F, F, P]
        L.orc_pack_bits.argtypes = [P, I, I, F, P]
        L.orc_line_crop.argtypes = [P, I, I, I, I, I, I, I, P, P, I, P]
        L.orc_det_prep.argtypes = [P, I, I, I, I, P]
        L.orc_pp_line_input.argtypes = [P, I, I, I, I, I, I, I, I, P]
        L.orc_activate.argtypes = [F, I]
        L.orc_activate.restype = F
        L.orc_find_contours.argtypes = [P, I, I]
        L.orc_find_contours.restype = P
        L.orc_contours_free.argtypes = [P]
        L.orc_contours_count.argtypes = [P]
        L.orc_contours_points.argtypes = [P]
        L.orc_contours_get.argtypes = [P, P, P, P, P]
        L.orc_simplify_polygon.argtypes = [P, I, F, P]
        L.orc_convex_hull.argtypes = [P, I, P]
        L.orc_min_area_rect.argtypes = [P, I, P]
        L.orc_word_rects.argtypes = [P, I, I, F, F, F, P, I]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype=np.float32):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------------------------------
# Operators (NCHW float32)
# ------------------------------------------------------------------------------------------
def conv2d(x, w, b=None, pads=(0, 0, 0, 0), strides=(1, 1), group=1, act=0, res=None):
    x, w = _c(x), _c(w)
    n, cin, h, wd = x.shape
    cout, _, kh, kw = w.shape
    pt, pl, pb, pr = pads
    oh, ow = (h + pt + pb - kh) // strides[0] + 1, (wd + pl + pr - kw) // strides[1] + 1
    y = np.empty((n, cout, oh, ow), np.float32)
    b = None if b is None else _c(b)
    res = None if res is None else _c(res)
    lib().orc_conv2d(_p(x), n, cin, h, wd, _p(w), cout, kh, kw, _p(b), pt, pl, pb, pr, strides[0], strides[1],
                     group, act, _p(res), _p(y))
    return y


def conv_transpose2d(x, w, b=None, strides=(2, 2), act=0):
    x, w = _c(x), _c(w)
    n, cin, h, wd = x.shape
    _, cout, kh, kw = w.shape
    y = np.empty((n, cout, (h - 1) * strides[0] + kh, (wd - 1) * strides[1] + kw), np.float32)
    b = None if b is None else _c(b)
    lib().orc_conv_transpose2d(_p(x), n, cin, h, wd, _p(w), cout, kh, kw, _p(b), strides[0], strides[1], act, _p(y))
    return y


def pool2d(x, kernel, strides, avg=False):
    x = _c(x)
    n, c, h, w = x.shape
    oh, ow = (h - kernel[0]) // strides[0] + 1, (w - kernel[1]) // strides[1] + 1
    y = np.empty((n, c, oh, ow), np.float32)
    lib().orc_pool2d(_p(x), n * c, h, w, kernel[0], kernel[1], strides[0], strides[1], int(avg), _p(y))
    return y


def pool2d_padded(x, kernel, strides, pads, avg=False):
    """Max / average pool with leading and trailing padding that is never counted (ONNX with
    count_include_pad = 0), numpy."""
    x = np.asarray(x, np.float32)
    n, c, h, w = x.shape
    pt, pl, pb, pr = pads
    oh, ow = (h + pt + pb - kernel[0]) // strides[0] + 1, (w + pl + pr - kernel[1]) // strides[1] + 1
    y = np.empty((n, c, oh, ow), np.float32)
    for oy in range(oh):
        y0, y1 = max(oy * strides[0] - pt, 0), min(oy * strides[0] - pt + kernel[0], h)
        for ox in range(ow):
            x0, x1 = max(ox * strides[1] - pl, 0), min(ox * strides[1] - pl + kernel[1], w)
            win = x[:, :, y0:y1, x0:x1].astype(np.float64)
            y[:, :, oy, ox] = win.mean(axis=(2, 3)) if avg else win.max(axis=(2, 3))
    return y


def gru(X, W, R, B, lens=None):
    X, W, R, B = _c(X), _c(W), _c(R), _c(B)
    T, N, I = X.shape
    D, H3, _ = W.shape
    H = H3 // 3
    Y = np.empty((T, D, N, H), np.float32)
    lens_a = None if lens is None else _c(lens, np.int32)
    lib().orc_gru(_p(X), T, N, I, _p(W), _p(R), _p(B), H, D, _p(lens_a), _p(Y))
    return Y


def activate(x, act):
    f = {0: lambda v: v, 1: lambda v: np.maximum(v, np.float32(0)),
         2: lambda v: np.float32(1) / (np.float32(1) + np.exp(-v))}
    return f[act](np.asarray(x, np.float32)).astype(np.float32)


# ------------------------------------------------------------------------------------------
# Graph walker
# ------------------------------------------------------------------------------------------
def _attr(node, name, default=None):
    return node.attrs.get(name, default)


def _is_int(a):
    return isinstance(a, np.ndarray) and np.issubdtype(a.dtype, np.integer)


def _erf(v):
    """The error function in float64 (scipy's, else the math module's, element by element)."""
    try:
        from scipy.special import erf
        return erf(v)
    except ImportError:  # pragma: no cover
        import math
        return np.vectorize(math.erf)(v)


def run(model: onnx_read.Model, x: np.ndarray, want=()):
    """Run the whole graph on input x; returns (output, {name: value for name in want})."""
    vals = {model.input: np.asarray(x, np.float32)}
    W, I = model.weights, model.ints

    def get(name):
        if name in vals:
            return vals[name]
        if name in W:
            return W[name]
        if name in I:
            return I[name]
        raise KeyError(name)

    for nd in model.nodes:
        ins = [get(i) if i else None for i in nd.inputs]
        op = nd.op
        if op == "Conv":
            w = ins[1]
            if _attr(nd, "auto_pad", "NOTSET") not in ("NOTSET", b"NOTSET"):
                raise ValueError("Conv auto_pad")
            pads = _attr(nd, "pads", [0, 0, 0, 0])
            pads = (pads[0], pads[1], pads[2], pads[3])
            if any(d != 1 for d in _attr(nd, "dilations", [1, 1])):
                raise ValueError("dilated conv")
            y = conv2d(ins[0], w, ins[2] if len(ins) > 2 else None, pads, tuple(_attr(nd, "strides", [1, 1])),
                       _attr(nd, "group", 1))
        elif op == "ConvTranspose":
            if any(_attr(nd, "pads", [0]) ) or any(_attr(nd, "output_padding", [0])) or _attr(nd, "group", 1) != 1:
                raise ValueError("unsupported ConvTranspose")
            y = conv_transpose2d(ins[0], ins[1], ins[2] if len(ins) > 2 else None, tuple(_attr(nd, "strides", [1, 1])))
        elif op in ("MaxPool", "AveragePool"):
            k = _attr(nd, "kernel_shape")
            s = _attr(nd, "strides", [1] * len(k))
            pads = _attr(nd, "pads", [0, 0, 0, 0])
            if _attr(nd, "ceil_mode", 0) or _attr(nd, "count_include_pad", 0) or \
                    _attr(nd, "auto_pad", "NOTSET") not in ("NOTSET", b"NOTSET"):
                raise ValueError("ceil_mode / count_include_pad / auto_pad pool")
            if any(pads):
                y = pool2d_padded(ins[0], k, s, pads, avg=(op == "AveragePool"))
            else:
                y = pool2d(ins[0], k, s, avg=(op == "AveragePool"))
        elif op == "Relu":
            y = activate(ins[0], 1)
        elif op == "Sigmoid":
            y = (1.0 / (1.0 + np.exp(-ins[0].astype(np.float64)))).astype(np.float32)
        elif op == "HardSigmoid":
            a, b = _attr(nd, "alpha", 0.2), _attr(nd, "beta", 0.5)
            y = np.clip(np.float32(a) * ins[0] + np.float32(b), 0, 1).astype(np.float32)
        elif op == "Erf":
            y = _erf(ins[0].astype(np.float64)).astype(np.float32)
        elif op == "Sqrt":
            y = np.sqrt(ins[0]).astype(np.float32)
        elif op in ("Add", "Sub", "Mul", "Div", "Pow"):
            a, b = ins
            if _is_int(a) and _is_int(b):
                y = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply,
                     "Div": lambda u, v: np.where(v == 0, 0, u // np.where(v == 0, 1, v)),
                     "Pow": lambda u, v: u}[op](a, b).astype(np.int64)
            else:
                a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
                if op == "Pow":
                    y = (a * a) if (b.size == 1 and float(b.reshape(-1)[0]) == 2.0) else np.power(a, b)
                else:
                    y = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide}[op](a, b)
                y = y.astype(np.float32)
        elif op == "BatchNormalization":
            g, b, m, v = (np.asarray(t, np.float64) for t in ins[1:5])
            eps = _attr(nd, "epsilon", 1e-5)
            sh = (1, -1) + (1,) * (ins[0].ndim - 2)
            y = ((ins[0] - m.reshape(sh)) / np.sqrt(v.reshape(sh) + eps) * g.reshape(sh) + b.reshape(sh)).astype(np.float32)
        elif op in ("ReduceMean", "GlobalAveragePool"):
            xv = ins[0].astype(np.float64)
            axes = tuple(range(2, xv.ndim)) if op == "GlobalAveragePool" else \
                tuple(int(a) % xv.ndim for a in _attr(nd, "axes", range(xv.ndim)))
            keep = op == "GlobalAveragePool" or bool(_attr(nd, "keepdims", 1))
            y = xv.mean(axis=axes, keepdims=keep).astype(np.float32)
        elif op == "Softmax":
            ax = _attr(nd, "axis", -1)
            v = ins[0].astype(np.float64)
            e = np.exp(v - v.max(axis=ax, keepdims=True))
            y = (e / e.sum(axis=ax, keepdims=True)).astype(np.float32)
        elif op == "Resize":
            if _attr(nd, "mode") != "nearest" or _attr(nd, "coordinate_transformation_mode") != "asymmetric":
                raise ValueError("Resize other than nearest / asymmetric")
            sc = np.asarray(ins[2], np.float32)
            xv = ins[0]
            oh, ow = int(np.floor(xv.shape[2] * sc[2])), int(np.floor(xv.shape[3] * sc[3]))
            iy = np.minimum(np.floor(np.arange(oh, dtype=np.float32) / sc[2]).astype(int), xv.shape[2] - 1)
            ix = np.minimum(np.floor(np.arange(ow, dtype=np.float32) / sc[3]).astype(int), xv.shape[3] - 1)
            y = np.ascontiguousarray(xv[:, :, iy][:, :, :, ix])
        elif op == "Concat":
            if all(_is_int(t) for t in ins):
                y = np.concatenate([np.asarray(t, np.int64).reshape(-1) for t in ins])
            else:
                y = np.concatenate(ins, axis=_attr(nd, "axis"))
        elif op in ("Squeeze", "Unsqueeze"):
            axes = _attr(nd, "axes") if _attr(nd, "axes") is not None else [int(a) for a in ins[1]]
            if op == "Squeeze":
                y = np.squeeze(ins[0], axis=tuple(int(a) % ins[0].ndim for a in axes))
            else:
                y = ins[0]
                r = y.ndim + len(axes)
                for a in sorted(int(a) % r for a in axes):
                    y = np.expand_dims(y, a)
        elif op == "Transpose":
            y = np.ascontiguousarray(np.transpose(ins[0], _attr(nd, "perm")))
        elif op == "Reshape":
            target = [int(v) for v in ins[1]]
            shape = [ins[0].shape[i] if s == 0 else s for i, s in enumerate(target)]
            y = ins[0].reshape(shape)
        elif op == "Shape":
            y = np.array(np.shape(ins[0]), np.int64)
        elif op == "Gather":
            if _attr(nd, "axis", 0) != 0 or not _is_int(ins[0]):
                raise ValueError("Gather other than of integers on axis 0")
            y = np.asarray(ins[0], np.int64)[np.asarray(ins[1], np.int64)]
        elif op == "GRU":
            if _attr(nd, "linear_before_reset", 0) != 1:
                raise ValueError("GRU linear_before_reset=0")
            d = 2 if _attr(nd, "direction", "forward") == "bidirectional" else 1
            assert ins[1].shape[0] == d
            y = gru(ins[0], ins[1], ins[2], ins[3])
            vals[nd.outputs[0]] = y
            if len(nd.outputs) > 1 and nd.outputs[1]:
                vals[nd.outputs[1]] = None
            continue
        elif op == "MatMul":
            y = np.matmul(ins[0].astype(np.float64), np.asarray(ins[1], np.float64)).astype(np.float32)
        elif op == "LogSoftmax":
            ax = _attr(nd, "axis", -1)
            v = ins[0].astype(np.float64)
            m = v.max(axis=ax, keepdims=True)
            y = (v - m - np.log(np.exp(v - m).sum(axis=ax, keepdims=True))).astype(np.float32)
        elif op == "Pad":
            if np.any(np.asarray(ins[1]) != 0):
                raise ValueError("non-zero Pad")
            y = ins[0]
        elif op == "Slice":
            y = ins[0]
            if len(ins) > 4 and ins[4] is not None and np.any(np.asarray(ins[4]) != 1):
                raise ValueError("Slice with steps")
            axes = ins[3] if len(ins) > 3 and ins[3] is not None else range(len(ins[1]))
            sl = [slice(None)] * y.ndim
            for st, en, ax in zip(ins[1], ins[2], axes):
                sl[int(ax)] = slice(int(st), int(en))
            y = np.ascontiguousarray(y[tuple(sl)])
        elif op in ("Cast", "Identity"):
            y = ins[0]
        else:
            raise ValueError(f"oracle: unsupported op {op}")
        vals[nd.outputs[0]] = y
    return vals[model.output], {k: vals[k] for k in want}


def gru_nodes(model):
    return [n for n in model.nodes if n.op == "GRU"]


def rec_logits(model, batches):
    """Per batch, the raw logits (the MatMul + bias Add output, before LogSoftmax) [T][n][C],
    as rten computes them for each batch on its own (gpu.rs:1510-1602 returns these)."""
    add = next(n for n in model.nodes if n.op == "Add")
    out = []
    for data, n, w in batches:
        _, got = run(model, np.asarray(data, np.float32).reshape(n, 1, 64, w), want=[add.outputs[0]])
        out.append(got[add.outputs[0]])
    return out


# ------------------------------------------------------------------------------------------
# Detector front/back end (gpu.rs:1393-1422) and CTC (ocr-bench.rs:62-74)
# ------------------------------------------------------------------------------------------
MODEL_H, MODEL_W = 800, 600


def grey_resize(rgb, w, h, mh=MODEL_H, mw=MODEL_W):
    ph, pw = max(h, mh), max(w, mw)
    y = np.empty((mh, mw), np.float32)
    rgb = _c(rgb, np.uint8)
    lib().orc_grey_resize(_p(rgb), w, h, pw, ph, mw, mh, np.float32(pw) / np.float32(mw),
                          np.float32(ph) / np.float32(mh), _p(y))
    return y


def valid_region(w, h, mh=MODEL_H, mw=MODEL_W):
    """gpu.rs:1414: the part of the model output that covers the page, not its padding."""
    ph, pw = max(h, mh), max(w, mw)
    return mh - (ph - h) * mh // ph, mw - (pw - w) * mw // pw


def mask_up_prob(m, w, h, mh=MODEL_H, mw=MODEL_W):
    vh, vw = valid_region(w, h, mh, mw)
    prob = np.empty((h, w), np.float32)
    m = _c(m)
    lib().orc_mask_up_prob(_p(m), mw, vw, vh, w, h, np.float32(vw) / np.float32(w), np.float32(vh) / np.float32(h),
                           _p(prob))
    return prob


def pack_bits(prob, thr):
    h, w = prob.shape
    bits = np.empty((h, (w + 31) // 32), np.uint32)
    lib().orc_pack_bits(_p(_c(prob)), w, h, np.float32(thr), _p(bits))
    return bits


def detect_page(model, rgb, thr):
    """Returns (bits [h][ceil(w/32)], pre-threshold prob [h][w], model output [800][600])."""
    h, w = rgb.shape[:2]
    inp = grey_resize(rgb, w, h)
    out, _ = run(model, inp.reshape(1, 1, MODEL_H, MODEL_W))
    m = out.reshape(MODEL_H, MODEL_W)
    prob = mask_up_prob(m, w, h)
    return pack_bits(prob, thr), prob, m


def ctc_decode(logits_line, width, classes=97):
    """ocr-bench.rs:62-74 on one line's [T][C] rows: arg-max with the LAST index on ties (Rust
    `max_by`), emit when best != 0, best != prev and t * 4 < width."""
    from_right = logits_line[:, ::-1]
    best = classes - 1 - np.argmax(from_right, axis=1)
    out, prev = [], 0
    for t, b in enumerate(best):
        if b != 0 and b != prev and t * 4 < width:
            out.append(int(b))
        prev = b
    return out, best


def line_crop(rgb, box, row_off, spans, wb):
    """One line image [64][wb] (see orc_line_crop); box = (left, top, bw, bh, out_w)."""
    rgb = _c(rgb, np.uint8)
    h, w = rgb.shape[:2]
    out = np.empty((64, wb), np.float32)
    ro = _c(row_off, np.int32)
    sp = _c(np.asarray(spans).reshape(-1), np.int32)
    if sp.size == 0:
        sp = np.zeros(2, np.int32)
    lib().orc_line_crop(_p(rgb), w, h, int(box[0]), int(box[1]), int(box[2]), int(box[3]), int(box[4]), _p(ro),
                        _p(sp), wb, _p(out))
    return out


def page_pipeline(det_model, rec_model, page, thr, layout_of):
    """The whole page on the CPU: detection (oracle), the layout (given: layout_of(bits, w)
    returns an object with nlines, nbatches, line(i) and batch(i) as the product's host layout
    does), line images (oracle), recognition (oracle), greedy CTC. Returns (texts by line,
    words, bits)."""
    bits, _, _ = detect_page(det_model, page, thr)
    lay = layout_of(bits, page.shape[1])
    texts = [""] * lay.nlines
    for b in range(lay.nbatches):
        wb, members = lay.batch(b)
        data = np.stack([line_crop(page, *lay.line(i), wb) for i in members])
        (logits,) = rec_logits(rec_model, [(data, len(members), wb)])
        for k, i in enumerate(members):
            out_w = int(lay.line(i)[0][4])
            cls, _ = ctc_decode(logits[:, k], out_w)
            texts[i] = "".join(ALPHABET[c - 1] for c in cls)
    return texts, lay.words, bits


# ocr-bench.rs:31: class k > 0 is ALPHABET[k - 1].
ALPHABET = " 0123456789!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~EABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz"


# ------------------------------------------------------------------------------------------
# PP-OCR front and back ends (src/nd.rs:1353-1369, src/ppdet.rs:29-44, 87-132)
# ------------------------------------------------------------------------------------------
def det_input_size(w, h, max_side):
    """nd.rs:1356-1358: long side at most max_side, each side rounded to the nearest multiple of
    32 (at least 32; halves away from zero, as Rust's f32::round)."""
    ratio = np.float32(max_side) / np.float32(max(w, h)) if max(w, h) > max_side else np.float32(1.0)
    def round32(v):
        q = np.float32(v) / np.float32(32.0)
        return max(int(np.floor(q + np.float32(0.5))) * 32, 32)
    return round32(np.float32(w) * ratio), round32(np.float32(h) * ratio)


def det_prep(rgb, max_side):
    """The detection input [1, 3, oh, ow] (see orc_det_prep)."""
    rgb = _c(rgb, np.uint8)
    h, w = rgb.shape[:2]
    ow, oh = det_input_size(w, h, max_side)
    y = np.empty((1, 3, oh, ow), np.float32)
    lib().orc_det_prep(_p(rgb), w, h, ow, oh, _p(y))
    return y


def threshold_bits(prob, thr):
    """ppdet.rs:88 as bit rows: prob [h, w] > thr, bit x % 32 of word x / 32."""
    return pack_bits(np.asarray(prob, np.float32), thr)


PP_H = 48


def pp_line_input(rgb, line, wb):
    """One PP-OCR line image [3, 48, wb] (see orc_pp_line_input); line = (left, top, cw, ch, out_w)."""
    rgb = _c(rgb, np.uint8)
    ph, pw = rgb.shape[:2]
    out = np.empty((3, PP_H, wb), np.float32)
    lib().orc_pp_line_input(_p(rgb), pw, ph, *[int(v) for v in line], wb, _p(out))
    return out


def pp_batches(lines, per_batch=16):
    """ocr-bench.rs:330-345: line indices sorted by resized width (stable), per_batch a batch,
    each as wide as its widest line rounded up to a multiple of 8."""
    order = sorted(range(len(lines)), key=lambda i: lines[i][4])
    out = []
    for c in range(0, len(order), per_batch):
        part = order[c: c + per_batch]
        out.append((part, -(-max(max(lines[i][4] for i in part), 8) // 8) * 8))
    return out


def pp_decode(best):
    """ppocr.rs:23-33 with the synthetic dictionary: class k in [1, 18706] is U+4E00 + k - 1,
    class 18707 a space, 0 the blank; repeats merged, blanks dropped."""
    out, prev = [], 0
    for c in best:
        c = int(c)
        if c != 0 and c != prev:
            out.append(" " if c == 18707 else chr(0x4E00 + c - 1))
        prev = c
    return "".join(out)


def pp_page_pipeline(det_model, rec_model, page, boxes_of, thr=0.3, max_side=960, per_batch=16):
    """The PP-OCR page on the CPU: detection input, DB map and threshold (oracle); the boxes and
    their line geometry (given: boxes_of(bits, prob, to_page) returns (left, top, cw, ch, out_w)
    per line in reading order, as the product's host code does); line images, recognition and
    CTC (oracle). Returns (texts by line, lines, bits, prob)."""
    h, w = page.shape[:2]
    x = det_prep(page, max_side)
    prob, _ = run(det_model, x)
    prob = prob[0, 0]
    bits = pack_bits(prob, thr)
    ow, oh = x.shape[3], x.shape[2]
    lines = boxes_of(bits, prob, (np.float32(w) / np.float32(ow), np.float32(h) / np.float32(oh)))
    texts = [""] * len(lines)
    for part, wb in pp_batches(lines, per_batch):
        data = np.stack([pp_line_input(page, lines[i], wb) for i in part])
        y, _ = run(rec_model, data)
        best = np.argmax(y, axis=-1)  # the first index on ties (nd.rs:383)
        for k, i in enumerate(part):
            texts[i] = pp_decode(best[k])
    return texts, lines, bits, prob
