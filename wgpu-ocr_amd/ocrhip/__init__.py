"""ocrhip: Python binding (ctypes) of libocrhip.so, the HIP path for AMD MI355X (gfx950).

The binding is a thin host-side mirror of the reference's public API (src/gpu.rs: Gpu,
Detector, Recognizer) over the C ABI declared in include/ocrhip.h. There is no CPU fallback:
if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libocrhip.so")

_lib = None


class OcrError(RuntimeError):
    pass


class ocr_opts(ctypes.Structure):
    _fields_ = [("lines", ctypes.c_uint32), ("pool_mb", ctypes.c_uint32), ("device", ctypes.c_int32)]


class ocr_batch(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("n", ctypes.c_uint32), ("w", ctypes.c_uint32)]


# Every symbol include/ocrhip.h declares, with (restype, argtypes).
P, U32, I32, F32, SZ = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int32, ctypes.c_float, ctypes.c_size_t
PU32 = ctypes.POINTER(ctypes.c_uint32)
SIGNATURES = {
    "ocr_last_error": (ctypes.c_char_p, []),
    "ocr_version": (ctypes.c_char_p, []),
    "ocr_create": (P, [ctypes.POINTER(ocr_opts)]),
    "ocr_destroy": (None, [P]),
    "ocr_synchronize": (ctypes.c_int, [P]),
    "ocr_device_alloc": (P, [P, SZ]),
    "ocr_device_free": (ctypes.c_int, [P, P]),
    "ocr_memcpy_h2d": (ctypes.c_int, [P, P, P, SZ]),
    "ocr_memcpy_d2h": (ctypes.c_int, [P, P, P, SZ]),
    "ocr_detector_new": (P, [P, ctypes.c_char_p]),
    "ocr_detector_free": (None, [P]),
    "ocr_detect_page": (ctypes.c_int, [P, P, U32, U32, F32, P]),
    "ocr_detect_pages_device": (ctypes.c_int, [P, P, P, P, U32, F32, P]),
    "ocr_detect": (ctypes.c_int, [P, P, U32, U32, P]),
    "ocr_graph_new": (P, [P, ctypes.c_char_p, ctypes.c_char_p]),
    "ocr_graph_free": (None, [P]),
    "ocr_graph_dims": (ctypes.c_int, [P, U32, U32, U32, U32, P]),
    "ocr_graph_run": (ctypes.c_int, [P, P, U32, U32, U32, U32, P]),
    "ocr_recognizer_new": (P, [P, ctypes.c_char_p, U32]),
    "ocr_recognizer_free": (None, [P]),
    "ocr_recognize_dims": (ctypes.c_int, [P, P, U32, PU32, PU32, PU32]),
    "ocr_recognize": (ctypes.c_int, [P, P, U32, P, P, P]),
    "ocr_recognize_device": (ctypes.c_int, [P, P, U32, P, P, P]),
}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OcrError(f"{LIB_PATH} is not built (run __graft_entry__.build() or python -m ocrhip.build)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise OcrError(lib().ocr_last_error().decode())


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class DeviceBuffer:
    """Device memory of a context (ocr_device_alloc), freed with the object."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.ptr = lib().ocr_device_alloc(ctx.handle, self.nbytes)
        if not self.ptr:
            raise OcrError(lib().ocr_last_error().decode())

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib().ocr_memcpy_h2d(self.ctx.handle, self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, count) -> np.ndarray:
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        _check(lib().ocr_memcpy_d2h(self.ctx.handle, _ptr(out), self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib().ocr_device_free(self.ctx.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """Gpu::new (src/gpu.rs:850): device, stream and scratch pool."""

    def __init__(self, lines: int = 8, pool_mb: int = 8192, device: int = 0):
        opts = ocr_opts(lines, pool_mb, device)
        self.handle = lib().ocr_create(ctypes.byref(opts))
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    def synchronize(self):
        _check(lib().ocr_synchronize(self.handle))

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def close(self):
        if self.handle:
            lib().ocr_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Detector:
    """Detector (src/gpu.rs:1380-1431)."""

    def __init__(self, ctx: Context, onnx_path: str):
        self.ctx = ctx
        self.handle = lib().ocr_detector_new(ctx.handle, onnx_path.encode())
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    def detect_page(self, rgb: np.ndarray, thr: float) -> np.ndarray:
        """RGB u8 [h, w, 3] -> bits u32 [h, ceil(w / 32)]."""
        rgb = np.ascontiguousarray(rgb, np.uint8)
        h, w = rgb.shape[:2]
        bits = np.empty((h, (w + 31) // 32), np.uint32)
        _check(lib().ocr_detect_page(self.handle, _ptr(rgb), w, h, thr, _ptr(bits)))
        return bits

    def detect_pages_device(self, d_rgb, ws, hs, thr: float, d_bits):
        n = len(d_rgb)
        arr_rgb = (ctypes.c_void_p * n)(*[b.ptr for b in d_rgb])
        arr_bits = (ctypes.c_void_p * n)(*[b.ptr for b in d_bits])
        w = np.asarray(ws, np.uint32)
        h = np.asarray(hs, np.uint32)
        _check(lib().ocr_detect_pages_device(self.handle, arr_rgb, _ptr(w), _ptr(h), n, thr, arr_bits))

    def detect(self, image: np.ndarray) -> np.ndarray:
        """[h, w] float input -> [h, w] probability map."""
        image = np.ascontiguousarray(image, np.float32)
        h, w = image.shape
        prob = np.empty((h, w), np.float32)
        _check(lib().ocr_detect(self.handle, _ptr(image), h, w, _ptr(prob)))
        return prob

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_detector_free(self.handle)
                self.handle = None
        except Exception:
            pass


class Graph:
    """Graph (src/gpu.rs:1077-1378): a convolutional ONNX graph on the GPU."""

    def __init__(self, ctx: Context, onnx_path: str, stop_op: str | None = None):
        self.ctx = ctx
        self.handle = lib().ocr_graph_new(ctx.handle, onnx_path.encode(), stop_op.encode() if stop_op else None)
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    def dims(self, shape):
        out = np.empty(4, np.uint32)
        _check(lib().ocr_graph_dims(self.handle, *[int(v) for v in shape], _ptr(out)))
        return tuple(int(v) for v in out)

    def run(self, x: np.ndarray) -> np.ndarray:
        """NCHW float input -> NCHW float output."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(self.dims(x.shape), np.float32)
        _check(lib().ocr_graph_run(self.handle, _ptr(x), *[int(v) for v in x.shape], _ptr(y)))
        return y

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_graph_free(self.handle)
                self.handle = None
        except Exception:
            pass


class Recognizer:
    """Recognizer (src/gpu.rs:1441-1603)."""

    def __init__(self, ctx: Context, onnx_path: str, lines: int = 8):
        self.ctx = ctx
        self.handle = lib().ocr_recognizer_new(ctx.handle, onnx_path.encode(), lines)
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    @staticmethod
    def _batches(batches):
        arr = (ocr_batch * len(batches))()
        for i, (data, n, w) in enumerate(batches):
            ptr = data.ptr if isinstance(data, DeviceBuffer) else data.ctypes.data
            arr[i] = ocr_batch(ptr, n, w)
        return arr

    def dims(self, batches):
        arr = self._batches(batches)
        t, n, c = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().ocr_recognize_dims(self.handle, arr, len(batches), ctypes.byref(t), ctypes.byref(n),
                                        ctypes.byref(c)))
        return t.value, n.value, c.value

    def recognize(self, batches, want_logits: bool = True):
        """batches: [(float32 [n, 64, w], n, w)]. Returns (logits [tmax, ntot, classes] or None,
        lens [ntot], best [tmax, ntot])."""
        batches = [(np.ascontiguousarray(d, np.float32), n, w) for d, n, w in batches]
        tmax, ntot, classes = self.dims(batches)
        arr = self._batches(batches)
        logits = np.empty((tmax, ntot, classes), np.float32) if want_logits else None
        lens = np.empty(ntot, np.uint32)
        best = np.empty((tmax, ntot), np.uint32)
        _check(lib().ocr_recognize(self.handle, arr, len(batches), None if logits is None else _ptr(logits),
                                   _ptr(lens), _ptr(best)))
        return logits, lens, best

    def recognize_device(self, d_batches, d_logits=None, d_best=None):
        arr = self._batches(d_batches)
        _, ntot, _ = self.dims(d_batches)
        lens = np.empty(ntot, np.uint32)
        _check(lib().ocr_recognize_device(self.handle, arr, len(d_batches), d_logits.ptr if d_logits else None,
                                          d_best.ptr if d_best else None, _ptr(lens)))
        return lens

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_recognizer_free(self.handle)
                self.handle = None
        except Exception:
            pass
