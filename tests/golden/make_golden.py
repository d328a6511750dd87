"""Writes the golden vectors in tests/golden/*.npz with torch on the CPU as the library routine.

The reference has no tests or golden tensors of its own, and its CPU engine (rten 0.26.0) is a
Rust crate that is not available here. These vectors pin the oracle's operators against
PyTorch's independent implementations of the same ONNX semantics:
  conv2d (pads, strides, groups), conv_transpose2d (kernel (2, 3), stride 2), max_pool2d and
  avg_pool2d (kernel = stride), GRU (linear_before_reset = 1 is torch's GRU; torch orders gates
  r, z, n and ONNX z, r, h, so the rows are reordered), bilinear resize with half-pixel centres
  (F.interpolate, align_corners=False), log_softmax.
Run from the repository root: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.dirname(os.path.abspath(__file__))
torch.manual_seed(0)
rng = np.random.Generator(np.random.PCG64(1234))


def f32(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def conv_cases():
    cases = {}
    specs = [  # name: (n, cin, h, w, cout, kh, kw, pads(t,l,b,r), strides, group)
        ("c3x3", (2, 5, 9, 11, 7, 3, 3, (1, 1, 1, 1), (1, 1), 1)),
        ("c1x1", (1, 16, 4, 6, 3, 1, 1, (0, 0, 0, 0), (1, 1), 1)),
        ("c_stride", (1, 4, 10, 9, 6, 3, 3, (1, 1, 1, 1), (2, 2), 1)),
        ("c_asym", (1, 3, 7, 8, 4, 3, 2, (0, 1, 2, 1), (1, 2), 1)),
        ("c_dw", (1, 6, 8, 8, 6, 3, 3, (1, 1, 1, 1), (1, 1), 6)),
        ("c_cin1", (2, 1, 12, 13, 8, 3, 3, (1, 1, 1, 1), (1, 1), 1)),
        ("c_wide", (1, 40, 6, 21, 70, 3, 3, (1, 1, 1, 1), (1, 1), 1)),
    ]
    for name, (n, cin, h, w, cout, kh, kw, pads, st, g) in specs:
        x, wt, b = f32(n, cin, h, w), f32(cout, cin // g, kh, kw, scale=0.3), f32(cout, scale=0.1)
        xp = F.pad(t(x), (pads[1], pads[3], pads[0], pads[2]))
        y = F.conv2d(xp, t(wt), t(b), stride=st, groups=g).numpy()
        cases[name] = dict(x=x, w=wt, b=b, pads=np.array(pads), strides=np.array(st), group=np.array(g), y=y)
    return cases


def convt_cases():
    cases = {}
    for name, (n, cin, h, w, cout, kh, kw, s) in [("t22", (1, 6, 5, 4, 3, 2, 2, 2)), ("t23", (2, 4, 3, 5, 5, 2, 3, 2)),
                                                  ("t33s1", (1, 3, 4, 4, 2, 3, 3, 1))]:
        x, wt, b = f32(n, cin, h, w), f32(cin, cout, kh, kw, scale=0.3), f32(cout, scale=0.1)
        y = F.conv_transpose2d(t(x), t(wt), t(b), stride=s).numpy()
        cases[name] = dict(x=x, w=wt, b=b, stride=np.array(s), y=y)
    return cases


def pool_cases():
    x = f32(2, 3, 9, 13)
    return {
        "max22": dict(x=x, k=np.array([2, 2]), y=F.max_pool2d(t(x), (2, 2), (2, 2)).numpy()),
        "max21": dict(x=x, k=np.array([2, 1]), y=F.max_pool2d(t(x), (2, 1), (2, 1)).numpy()),
        "avg21": dict(x=x, k=np.array([2, 1]), y=F.avg_pool2d(t(x), (2, 1), (2, 1)).numpy()),
    }


def gru_cases():
    cases = {}
    for name, (T, N, I, H) in [("g_small", (7, 3, 10, 8)), ("g_wide", (5, 2, 24, 16))]:
        g = torch.nn.GRU(I, H, bidirectional=True)
        with torch.no_grad():
            for p in g.parameters():
                p.copy_(t(f32(*p.shape, scale=0.4)))
        x = f32(T, N, I)
        y, _ = g(t(x))  # [T, N, 2H]
        y = y.detach().numpy().reshape(T, N, 2, H).transpose(0, 2, 1, 3)  # ONNX Y [T][D][N][H]

        def onnx_order(m):  # torch (r, z, n) -> ONNX (z, r, h)
            r, z, n = np.split(m, 3, axis=0)
            return np.concatenate([z, r, n], axis=0)

        W, R, B = [], [], []
        for sfx in ("", "_reverse"):
            W.append(onnx_order(getattr(g, f"weight_ih_l0{sfx}").detach().numpy()))
            R.append(onnx_order(getattr(g, f"weight_hh_l0{sfx}").detach().numpy()))
            B.append(np.concatenate([onnx_order(getattr(g, f"bias_ih_l0{sfx}").detach().numpy()),
                                     onnx_order(getattr(g, f"bias_hh_l0{sfx}").detach().numpy())]))
        cases[name] = dict(x=x, W=np.stack(W), R=np.stack(R), B=np.stack(B), y=np.ascontiguousarray(y))
    return cases


def resize_cases():
    """Bilinear half-pixel resizes: the ocrs grey front end (page padded with black, resized to the
    model size) and the mask back end (model output cut to the valid part, resized to the page)."""
    cases = {}
    for name, (h, w, mh, mw) in [("down", (97, 61, 40, 30)), ("up_pad", (23, 19, 40, 30)), ("mixed", (53, 17, 40, 30))]:
        rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
        grey = (-0.5 + rgb[..., 0].astype(np.float32) * np.float32(0.299 / 255)
                + rgb[..., 1].astype(np.float32) * np.float32(0.587 / 255)
                + rgb[..., 2].astype(np.float32) * np.float32(0.114 / 255)).astype(np.float32)
        ph, pw = max(h, mh), max(w, mw)
        padded = np.full((ph, pw), -0.5, np.float32)
        padded[:h, :w] = grey
        model_in = F.interpolate(t(padded)[None, None], size=(mh, mw), mode="bilinear", align_corners=False)[0, 0]
        m = rng.uniform(0, 1, (mh, mw)).astype(np.float32)
        vh, vw = mh - (ph - h) * mh // ph, mw - (pw - w) * mw // pw
        prob = F.interpolate(t(m[:vh, :vw].copy())[None, None], size=(h, w), mode="bilinear", align_corners=False)[0, 0]
        cases[name] = dict(rgb=rgb, mh=np.array(mh), mw=np.array(mw), model_in=model_in.numpy(), m=m,
                           prob=prob.numpy())
    return cases


def line_crop_cases():
    """Line images: the ocrs grey value inside the line polygon (row spans), black (-0.5) outside
    it and off the page, resized to 64 rows x out_w columns (F.interpolate, half-pixel), padded
    on the right to the batch width wb with black."""
    cases = {}
    for name, (ph, pw, left, top, bh, bw, out_w, wb) in [("inside", (40, 90, 5, 3, 30, 70, 150, 200)),
                                                         ("edge", (30, 50, -4, 20, 16, 60, 240, 250))]:
        rgb = rng.integers(0, 256, (ph, pw, 3), dtype=np.uint8)
        grey = (-0.5 + rgb[..., 0].astype(np.float32) * np.float32(0.299 / 255)
                + rgb[..., 1].astype(np.float32) * np.float32(0.587 / 255)
                + rgb[..., 2].astype(np.float32) * np.float32(0.114 / 255)).astype(np.float32)
        row_off, spans = [0], []
        crop = np.full((bh, bw), -0.5, np.float32)
        for cy in range(bh):
            a = int(rng.integers(0, bw // 3))
            b = int(rng.integers(bw // 2, bw + 1))
            runs = [(a, b)] if cy % 3 else [(a, a + (b - a) // 3), (a + (b - a) // 2, b)]
            for x0, x1 in runs:
                spans += [x0, x1]
                for cx in range(x0, x1):
                    x, y = left + cx, top + cy
                    if 0 <= x < pw and 0 <= y < ph:
                        crop[cy, cx] = grey[y, x]
            row_off.append(len(spans))
        img = F.interpolate(t(crop)[None, None], size=(64, out_w), mode="bilinear", align_corners=False)[0, 0]
        out = np.full((64, wb), -0.5, np.float32)
        out[:, :out_w] = img.numpy()
        cases[name] = dict(rgb=rgb, box=np.array([left, top, bw, bh, out_w]), row_off=np.array(row_off, np.int32),
                           spans=np.array(spans, np.int32), wb=np.array(wb), y=out)
    return cases


def softmax_cases():
    x = f32(4, 3, 97, scale=3.0)
    return {"ls": dict(x=x, y=F.log_softmax(t(x), dim=2).numpy())}


def nd_cases():
    """Operators of the N-D (PP-OCR) graphs: LayerNorm, attention, BatchNormalization, GELU, SiLU,
    nearest resize x2, padded strided pools, a depthwise conv with stride (2, 1) and the PP-OCR
    detection input (bilinear half-pixel of the page's bytes, BGR, ImageNet normalisation)."""
    c = {}
    x = f32(3, 7, 120)
    g, b = f32(120, scale=0.2) + 1, f32(120, scale=0.1)
    c["ln"] = dict(x=x, g=g, b=b, y=F.layer_norm(t(x), (120,), t(g), t(b), eps=1e-6).numpy())
    q, k, v = f32(2, 8, 9, 15), f32(2, 8, 9, 15), f32(2, 8, 9, 15)
    att = torch.softmax((t(q) * 15 ** -0.5) @ t(k).transpose(2, 3).contiguous(), dim=-1)
    c["attn"] = dict(q=q, k=k, v=v, y=(att @ t(v)).numpy())
    x = f32(2, 5, 6, 7)
    gm, bt, mu, var = f32(5, scale=0.2) + 1, f32(5, scale=0.1), f32(5, scale=0.1), np.abs(f32(5)) + 0.5
    c["bn"] = dict(x=x, g=gm, b=bt, m=mu, v=var,
                   y=F.batch_norm(t(x), t(mu), t(var), t(gm), t(bt), training=False, eps=1e-5).numpy())
    x = f32(4, 33, scale=2.0)
    c["gelu"] = dict(x=x, y=F.gelu(t(x)).numpy())
    c["silu"] = dict(x=x, y=F.silu(t(x)).numpy())
    x = f32(1, 3, 5, 7)
    c["resize2"] = dict(x=x, y=F.interpolate(t(x), scale_factor=2.0, mode="nearest").numpy())
    x = f32(2, 3, 9, 10)
    c["avgpool_pad"] = dict(x=x, y=F.avg_pool2d(t(x), 3, 2, padding=1, count_include_pad=False).numpy())
    c["maxpool_pad"] = dict(x=x, y=F.max_pool2d(t(x), 3, 2, padding=1).numpy())
    x, wd = f32(1, 6, 9, 8), f32(6, 1, 3, 3, scale=0.3)
    c["dw_s21"] = dict(x=x, w=wd, y=F.conv2d(F.pad(t(x), (1, 1, 1, 1)), t(wd), stride=(2, 1), groups=6).numpy())
    rgb = rng.integers(0, 256, (53, 70, 3), dtype=np.uint8)
    bgr = t(rgb[..., ::-1].astype(np.float32).transpose(2, 0, 1).copy())[None]
    ow, oh = 64, 64  # 70 x 53 with max side 64: ratio 64 / 70 gives 64 x 48.5, rounded to multiples of 32
    img = F.interpolate(bgr, size=(oh, ow), mode="bilinear", align_corners=False)[0]
    mean = torch.tensor([0.485, 0.456, 0.406]).reshape(3, 1, 1)
    dev = torch.tensor([0.229, 0.224, 0.225]).reshape(3, 1, 1)
    c["det_prep"] = dict(rgb=rgb, max_side=np.array(64), y=((img / 255.0 - mean) / dev).numpy()[None])
    # PP-OCR line images: page boxes (one reaching past the page's right and bottom edges, where
    # pixels read 0) resized to 48 rows, rounded to bytes, (v / 255 - 0.5) / 0.5, padded to wb.
    page = rng.integers(0, 256, (40, 90, 3), dtype=np.uint8)
    for name, (left, top, cw, ch, out_w, wb) in [("pp_line_in", (7, 5, 60, 22, 131, 136)),
                                                 ("pp_line_edge", (70, 30, 25, 14, 86, 88))]:
        crop = np.zeros((ch, cw, 3), np.float32)
        sub = page[top: top + ch, left: left + cw].astype(np.float32)
        crop[: sub.shape[0], : sub.shape[1]] = sub
        img = F.interpolate(t(crop.transpose(2, 0, 1).copy())[None], size=(48, out_w), mode="bilinear",
                            align_corners=False)[0].numpy()
        q = np.floor(img + 0.5)
        y = np.zeros((3, 48, wb), np.float32)
        y[:, :, :out_w] = (q / 255.0 - 0.5) / 0.5
        c[name] = dict(rgb=page, line=np.array([left, top, cw, ch, out_w]), wb=np.array(wb), y=y)
    # torch's hardsigmoid is ONNX HardSigmoid with alpha 1/6, beta 0.5 (ONNX's defaults are 0.2, 0.5)
    x = np.concatenate([f32(200, scale=3.0), np.array([-3.0, 3.0, 0.0, -6.0, 6.0], np.float32)])
    c["hardsigmoid"] = dict(x=x, y=F.hardsigmoid(t(x)).numpy())
    return c


def save(name, cases):
    flat = {f"{c}__{k}": v for c, d in cases.items() for k, v in d.items()}
    np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **flat)


if __name__ == "__main__":
    save("conv", conv_cases())
    save("convt", convt_cases())
    save("pool", pool_cases())
    save("gru", gru_cases())
    save("resize", resize_cases())
    save("logsoftmax", softmax_cases())
    save("line_crop", line_crop_cases())
    save("nd", nd_cases())
    print("written to", OUT)
