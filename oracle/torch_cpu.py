"""CPU baseline (measurement infrastructure only): the ocrs-architecture detection and recognition
graphs executed by PyTorch on the host cores, the stand-in for the reference's rten CPU path
(rten 0.26.0 is a Rust crate that is not available here). The graph is walked node by node as
rten walks it (one library call per ONNX node: conv2d, conv_transpose2d, pools, GRU, matmul), in
float32, on torch's intra-op threads. The whole-page loop around it (grey resize, mask, layout,
line crops, CTC) is the oracle's, page by page as the reference's CPU loop runs
(src/bin/ocr-bench.rs:431-444). Only bench.py's cpu_baseline leg uses this file.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import graph as og
from . import onnx_read


def _attr(node, name, default=None):
    return node.attrs.get(name, default)


class TorchGraph:
    """An ONNX graph (the op set of the ocrs models) on torch-CPU, weights converted once."""

    def __init__(self, model: onnx_read.Model):
        self.model = model
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v, np.float32)) for k, v in model.weights.items()}
        self.ints = dict(model.ints)
        self.gru = {}
        for nd in model.nodes:
            if nd.op == "GRU":
                self.gru[nd.outputs[0]] = self._gru_module(nd)

    def _gru_module(self, nd):
        # ONNX gate rows z, r, h; torch's r, z, n (linear_before_reset = 1 is torch's GRU).
        W, R, B = (self.model.weights[nd.inputs[i]] for i in (1, 2, 3))
        D, H3, I = W.shape
        H = H3 // 3
        g = torch.nn.GRU(I, H, bidirectional=D == 2)

        def reorder(a):
            z, r, h = a[:H], a[H: 2 * H], a[2 * H:]
            return torch.from_numpy(np.ascontiguousarray(np.concatenate([r, z, h]), np.float32))
        with torch.no_grad():
            for d in range(D):
                sfx = "_reverse" if d else ""
                getattr(g, "weight_ih_l0" + sfx).copy_(reorder(W[d]))
                getattr(g, "weight_hh_l0" + sfx).copy_(reorder(R[d]))
                getattr(g, "bias_ih_l0" + sfx).copy_(reorder(B[d][:H3]))
                getattr(g, "bias_hh_l0" + sfx).copy_(reorder(B[d][H3:]))
        return g.eval()

    @torch.no_grad()
    def run(self, x: np.ndarray) -> np.ndarray:
        vals = {self.model.input: torch.from_numpy(np.ascontiguousarray(x, np.float32))}

        def get(name):
            if name in vals:
                return vals[name]
            if name in self.w:
                return self.w[name]
            return self.ints[name]

        for nd in self.model.nodes:
            ins = [get(i) if i else None for i in nd.inputs]
            op = nd.op
            if op == "Conv":
                p = _attr(nd, "pads", [0, 0, 0, 0])
                xin = ins[0]
                if p[0] != p[2] or p[1] != p[3]:
                    xin = F.pad(xin, (p[1], p[3], p[0], p[2]))
                    pad = 0
                else:
                    pad = (p[0], p[1])
                y = F.conv2d(xin, ins[1], ins[2] if len(ins) > 2 else None, stride=tuple(_attr(nd, "strides", [1, 1])),
                             padding=pad, groups=_attr(nd, "group", 1))
            elif op == "ConvTranspose":
                y = F.conv_transpose2d(ins[0], ins[1], ins[2] if len(ins) > 2 else None,
                                       stride=tuple(_attr(nd, "strides", [1, 1])))
            elif op == "MaxPool":
                k = _attr(nd, "kernel_shape")
                y = F.max_pool2d(ins[0], k, _attr(nd, "strides", k))
            elif op == "AveragePool":
                k = _attr(nd, "kernel_shape")
                y = F.avg_pool2d(ins[0], k, _attr(nd, "strides", k))
            elif op == "Relu":
                y = torch.relu(ins[0])
            elif op == "Sigmoid":
                y = torch.sigmoid(ins[0])
            elif op == "Concat":
                y = torch.cat(ins, dim=_attr(nd, "axis"))
            elif op == "Add":
                y = ins[0] + ins[1]
            elif op == "MatMul":
                y = torch.matmul(ins[0], ins[1])
            elif op == "LogSoftmax":
                y = torch.log_softmax(ins[0], dim=_attr(nd, "axis", -1))
            elif op == "Squeeze":
                axes = _attr(nd, "axes") if _attr(nd, "axes") is not None else [int(a) for a in ins[1]]
                y = ins[0]
                for a in sorted((int(a) % y.dim() for a in axes), reverse=True):
                    y = y.squeeze(a)
            elif op == "Transpose":
                y = ins[0].permute(*_attr(nd, "perm")).contiguous()
            elif op == "Reshape":
                target = [int(v) for v in np.asarray(ins[1]).reshape(-1)]
                y = ins[0].reshape([ins[0].shape[i] if s == 0 else s for i, s in enumerate(target)])
            elif op == "GRU":
                out, _ = self.gru[nd.outputs[0]](ins[0])
                T, N, _ = out.shape
                D = 2 if _attr(nd, "direction", "forward") == "bidirectional" else 1
                y = out.reshape(T, N, D, -1).permute(0, 2, 1, 3).contiguous()  # ONNX Y [T, D, N, H]
                vals[nd.outputs[0]] = y
                continue
            else:
                raise ValueError(f"torch CPU baseline: unsupported op {op}")
            vals[nd.outputs[0]] = y
        return vals[self.model.output].numpy()


def page_pipeline(det: TorchGraph, rec: TorchGraph, page, thr, layout_of):
    """One page on the CPU: detection with torch (grey resize and mask as the oracle's), the
    layout, line crops, recognition with torch, greedy CTC. Returns the texts by line."""
    h, w = page.shape[:2]
    inp = og.grey_resize(page, w, h)
    m = det.run(inp.reshape(1, 1, og.MODEL_H, og.MODEL_W)).reshape(og.MODEL_H, og.MODEL_W)
    bits = og.pack_bits(og.mask_up_prob(m, w, h), thr)
    lay = layout_of(bits, w)
    texts = [""] * lay.nlines
    for b in range(lay.nbatches):
        wb, members = lay.batch(b)
        data = np.stack([og.line_crop(page, *lay.line(i), wb) for i in members])
        logits = rec.run(data.reshape(len(members), 1, 64, wb))
        for k, i in enumerate(members):
            cls, _ = og.ctc_decode(logits[:, k], int(lay.line(i)[0][4]))
            texts[i] = "".join(og.ALPHABET[c - 1] for c in cls)
    return texts
