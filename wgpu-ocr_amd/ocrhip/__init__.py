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
    "ocr_host_alloc": (P, [P, SZ]),
    "ocr_host_free": (ctypes.c_int, [P, P]),
    "ocr_memory_stats": (ctypes.c_int, [P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "ocr_png_dims": (ctypes.c_int, [P, SZ, PU32, PU32]),
    "ocr_png_decode": (ctypes.c_int, [P, SZ, P, SZ, PU32, PU32]),
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
    "ocr_probe_start": (ctypes.c_int, [ctypes.c_char_p]),
    "ocr_probe_stop": (ctypes.c_int, [ctypes.c_char_p, PU32, P, P, P]),
    "ocr_detector_new_onnx": (P, [P, P]),
    "ocr_graph_new_onnx": (P, [P, P, ctypes.c_char_p]),
    "ocr_recognizer_new_onnx": (P, [P, P, U32]),
    "ocr_nd_new_onnx": (P, [P, P, ctypes.c_int]),
    "ocr_word_rects": (ctypes.c_int, [P, U32, U32, P, U32, PU32]),
    "ocr_word_rects_mt": (ctypes.c_int, [P, U32, U32, U32, P, U32, PU32]),
    "ocr_word_rects_gpu": (ctypes.c_int, [P, P, U32, U32, P, U32, PU32]),
    "ocr_word_rects_gpu_noalloc": (ctypes.c_int, [P, P, U32, U32, P, U32, PU32]),
    "ocr_layout_page": (P, [P, U32, U32, F32, F32]),
    "ocr_layout_free": (None, [P]),
    "ocr_layout_counts": (ctypes.c_int, [P, PU32, PU32, PU32]),
    "ocr_layout_line": (ctypes.c_int, [P, U32, P, P, P, PU32]),
    "ocr_layout_batch": (ctypes.c_int, [P, U32, PU32, P, PU32]),
    "ocr_pipeline_new": (P, [P, P, P]),
    "ocr_pipeline_free": (None, [P]),
    "ocr_pipeline_run_device": (ctypes.c_int, [P, P, P, P, U32]),
    "ocr_pipeline_run": (ctypes.c_int, [P, P, P, P, U32]),
    "ocr_pipeline_stats_get": (ctypes.c_int, [P, P]),
    "ocr_pipeline_page": (ctypes.c_int, [P, U32, PU32, PU32]),
    "ocr_pipeline_line_text": (ctypes.c_int, [P, U32, U32, ctypes.c_char_p, U32, PU32]),
    "ocr_pipeline_page_error": (ctypes.c_int, [P, U32, ctypes.c_char_p, U32, PU32]),
    "ocr_nd_new": (P, [P, ctypes.c_char_p, ctypes.c_int]),
    "ocr_nd_plan": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p, U32, PU32]),
    "ocr_nd_free": (None, [P]),
    "ocr_nd_dims": (ctypes.c_int, [P, P, U32, P, PU32]),
    "ocr_nd_run": (ctypes.c_int, [P, P, P, U32, P]),
    "ocr_nd_run_device": (ctypes.c_int, [P, P, P, U32, P]),
    "ocr_nd_argmax": (ctypes.c_int, [P, P, P, U32, P]),
    "ocr_nd_argmax_device": (ctypes.c_int, [P, P, P, U32, P]),
    "ocr_nd_det_input_dims": (ctypes.c_int, [U32, U32, U32, PU32, PU32, P]),
    "ocr_nd_det_input": (ctypes.c_int, [P, P, U32, U32, U32, P]),
    "ocr_nd_det_input_device": (ctypes.c_int, [P, P, U32, U32, U32, P]),
    "ocr_db_threshold": (ctypes.c_int, [P, P, U32, U32, F32, P]),
    "ocr_db_threshold_device": (ctypes.c_int, [P, P, U32, U32, F32, P]),
    "ocr_pp_pipeline_new": (P, [P, P, P]),
    "ocr_pp_pipeline_free": (None, [P]),
    "ocr_pp_pipeline_run_device": (ctypes.c_int, [P, P, P, P, U32]),
    "ocr_pp_pipeline_run": (ctypes.c_int, [P, P, P, P, U32]),
    "ocr_pp_pipeline_stats_get": (ctypes.c_int, [P, P]),
    "ocr_pp_pipeline_page": (ctypes.c_int, [P, U32, PU32]),
    "ocr_pp_pipeline_line_text": (ctypes.c_int, [P, U32, U32, ctypes.c_char_p, U32, PU32]),
    "ocr_db_boxes": (ctypes.c_int, [P, P, U32, U32, F32, F32, F32, F32, F32, P, U32, PU32]),
    "ocr_pp_line_box": (ctypes.c_int, [P, F32, U32, U32, P]),
    "ocr_pp_line_images": (ctypes.c_int, [P, P, U32, U32, P, U32, U32, P]),
    "ocr_line_images": (ctypes.c_int, [P, P, U32, U32, P, U32, P, U32, P, U32, U32, P]),
}


class ocr_onnx_attr(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("f", ctypes.c_float), ("i", ctypes.c_int64),
                ("s", ctypes.c_char_p), ("floats", ctypes.c_void_p), ("ints", ctypes.c_void_p), ("count", ctypes.c_uint32)]


class ocr_onnx_node(ctypes.Structure):
    _fields_ = [("op", ctypes.c_char_p), ("inputs", ctypes.c_void_p), ("ninputs", ctypes.c_uint32),
                ("outputs", ctypes.c_void_p), ("noutputs", ctypes.c_uint32), ("attrs", ctypes.c_void_p),
                ("nattrs", ctypes.c_uint32)]


class ocr_onnx_tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dims", ctypes.c_void_p), ("rank", ctypes.c_uint32),
                ("data", ctypes.c_void_p), ("ints", ctypes.c_void_p), ("count", ctypes.c_uint64)]


class ocr_onnx(ctypes.Structure):
    _fields_ = [("nodes", ctypes.c_void_p), ("nnodes", ctypes.c_uint32), ("tensors", ctypes.c_void_p),
                ("ntensors", ctypes.c_uint32), ("input", ctypes.c_char_p), ("output", ctypes.c_char_p)]


class ParsedGraph:
    """A graph the host has parsed (the reference's Onnx, src/onnx.rs:44-56) as the C ABI's
    ocr_onnx: nodes = [(op, inputs, outputs, {attribute: value})] (value a float, int, str or a
    list of ints or floats), weights = {name: float32 array}, ints = {name: int64 array}. Keeps
    every buffer alive for as long as the object lives."""

    def __init__(self, nodes, weights, ints, input_name: str, output_name: str):
        keep = self._keep = []

        def cstr(v):
            b = v.encode()
            keep.append(b)
            return b

        def strs(names):
            arr = (ctypes.c_char_p * max(len(names), 1))(*[cstr(n) for n in names])
            keep.append(arr)
            return ctypes.cast(arr, ctypes.c_void_p)

        cnodes = (ocr_onnx_node * max(len(nodes), 1))()
        for k, (op, ins, outs, attrs) in enumerate(nodes):
            attrs = {k: v for k, v in attrs.items() if v is not None}
            catt = (ocr_onnx_attr * max(len(attrs), 1))()
            for j, (name, v) in enumerate(attrs.items()):
                a = catt[j]
                a.name = cstr(name)
                if isinstance(v, bool) or isinstance(v, (int, np.integer)):
                    a.type, a.i = 2, int(v)
                elif isinstance(v, (float, np.floating)):
                    a.type, a.f = 1, float(v)
                elif isinstance(v, (str, bytes)):
                    a.type, a.s = 3, cstr(v if isinstance(v, str) else v.decode())
                else:
                    vals = list(np.asarray(v).reshape(-1))
                    if vals and all(isinstance(x, (float, np.floating)) for x in vals):
                        arr = np.ascontiguousarray(vals, np.float32)
                        a.type, a.floats = 6, arr.ctypes.data
                    else:
                        arr = np.ascontiguousarray(vals, np.int64)
                        a.type, a.ints = 7, arr.ctypes.data
                    keep.append(arr)
                    a.count = len(vals)
            keep.append(catt)
            cnodes[k] = ocr_onnx_node(cstr(op), strs(list(ins)), len(ins), strs(list(outs)), len(outs),
                                      ctypes.cast(catt, ctypes.c_void_p), len(attrs))
        keep.append(cnodes)
        tensors = []
        for name, arr in weights.items():
            a = np.ascontiguousarray(arr, np.float32)
            d = np.ascontiguousarray(a.shape, np.int64)
            keep += [a, d]
            tensors.append(ocr_onnx_tensor(cstr(name), d.ctypes.data, a.ndim, a.ctypes.data, None, a.size))
        for name, arr in ints.items():
            a = np.ascontiguousarray(arr, np.int64).reshape(-1)
            d = np.ascontiguousarray([a.size], np.int64)
            keep += [a, d]
            tensors.append(ocr_onnx_tensor(cstr(name), d.ctypes.data, 1, None, a.ctypes.data, a.size))
        ctens = (ocr_onnx_tensor * max(len(tensors), 1))(*tensors)
        keep.append(ctens)
        self.struct = ocr_onnx(ctypes.cast(cnodes, ctypes.c_void_p), len(nodes), ctypes.cast(ctens, ctypes.c_void_p),
                               len(tensors), cstr(input_name), cstr(output_name))

    def ref(self):
        return ctypes.byref(self.struct)


class ocr_pipeline_opts(ctypes.Structure):
    _fields_ = [("merge", ctypes.c_uint32), ("relv", ctypes.c_float), ("relend", ctypes.c_float),
                ("thr", ctypes.c_float), ("threads", ctypes.c_uint32), ("det_batch", ctypes.c_uint32),
                ("label_runs", ctypes.c_uint32), ("label_comps", ctypes.c_uint32), ("label_slots", ctypes.c_uint32)]


class ocr_pipeline_stats(ctypes.Structure):
    _fields_ = [("ms", ctypes.c_double), ("cpu_busy_ms", ctypes.c_double), ("pages", ctypes.c_uint32),
                ("lines", ctypes.c_uint32), ("words", ctypes.c_uint32), ("batches", ctypes.c_uint32),
                ("rec_passes", ctypes.c_uint32), ("rec_steps", ctypes.c_uint64), ("host_labelled", ctypes.c_uint32)]


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


class HostArray:
    """Page-locked host memory of a context (ocr_host_alloc) as a numpy array (.array); freed
    with the object."""

    def __init__(self, ctx: "Context", shape, dtype=np.uint8):
        self.ctx = ctx
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape)) * dtype.itemsize
        self.ptr = lib().ocr_host_alloc(ctx.handle, max(nbytes, 1))
        if not self.ptr:
            raise OcrError(lib().ocr_last_error().decode())
        buf = (ctypes.c_uint8 * max(nbytes, 1)).from_address(self.ptr)
        self.array = np.frombuffer(buf, dtype=dtype, count=int(np.prod(shape))).reshape(shape)

    def free(self):
        if self.ptr:
            self.array = None
            lib().ocr_host_free(self.ctx.handle, self.ptr)
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

    def host_array(self, shape, dtype=np.uint8) -> "HostArray":
        """A numpy array in page-locked host memory (ocr_host_alloc)."""
        return HostArray(self, shape, dtype)

    def memory_stats(self) -> dict:
        """The library's allocation counts (process-wide) and this context's pool bytes."""
        v = [ctypes.c_uint64() for _ in range(4)]
        _check(lib().ocr_memory_stats(self.handle, *[ctypes.byref(x) for x in v]))
        return dict(zip(("device_allocs", "host_allocs", "pool_live", "pool_held"), (x.value for x in v)))

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

    def __init__(self, ctx: Context, onnx_path: "str | ParsedGraph"):
        self.ctx = ctx
        if isinstance(onnx_path, ParsedGraph):
            self.handle = lib().ocr_detector_new_onnx(ctx.handle, onnx_path.ref())
        else:
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

    def __init__(self, ctx: Context, onnx_path: "str | ParsedGraph", stop_op: str | None = None):
        self.ctx = ctx
        stop = stop_op.encode() if stop_op else None
        if isinstance(onnx_path, ParsedGraph):
            self.handle = lib().ocr_graph_new_onnx(ctx.handle, onnx_path.ref(), stop)
        else:
            self.handle = lib().ocr_graph_new(ctx.handle, onnx_path.encode(), stop)
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


def nd_plan(onnx_path: str, stop_before_softmax: bool = False) -> list:
    """The N-D executor's fusion plan for an ONNX file (no GPU needed): one text line a launch."""
    n = ctypes.c_uint32()
    _check(lib().ocr_nd_plan(onnx_path.encode(), int(bool(stop_before_softmax)), None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(n.value + 1)
    _check(lib().ocr_nd_plan(onnx_path.encode(), int(bool(stop_before_softmax)), buf, n.value + 1, ctypes.byref(n)))
    return buf.value.decode().splitlines()


class NdGraph:
    """NdGraph (src/nd.rs:428-1394): an ONNX graph of the N-D operator set on the GPU."""

    def __init__(self, ctx: Context, onnx_path: "str | ParsedGraph", stop_before_softmax: bool = False):
        self.ctx = ctx
        if isinstance(onnx_path, ParsedGraph):
            self.handle = lib().ocr_nd_new_onnx(ctx.handle, onnx_path.ref(), int(bool(stop_before_softmax)))
        else:
            self.handle = lib().ocr_nd_new(ctx.handle, onnx_path.encode(), int(bool(stop_before_softmax)))
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    def dims(self, shape):
        s = np.asarray(shape, np.int64)
        out = np.zeros(6, np.int64)
        rank = ctypes.c_uint32()
        _check(lib().ocr_nd_dims(self.handle, _ptr(s), len(s), _ptr(out), ctypes.byref(rank)))
        return tuple(int(v) for v in out[: rank.value])

    def run(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        s = np.asarray(x.shape, np.int64)
        y = np.empty(self.dims(x.shape), np.float32)
        _check(lib().ocr_nd_run(self.handle, _ptr(x), _ptr(s), len(s), _ptr(y)))
        return y

    def argmax(self, x: np.ndarray) -> np.ndarray:
        """Arg-max over the output's last axis (first index on ties), shape = output shape[:-1]."""
        x = np.ascontiguousarray(x, np.float32)
        s = np.asarray(x.shape, np.int64)
        shape = self.dims(x.shape)[:-1]
        best = np.empty(shape, np.uint32)
        _check(lib().ocr_nd_argmax(self.handle, _ptr(x), _ptr(s), len(s), _ptr(best)))
        return best

    def argmax_device(self, d_x: "DeviceBuffer", shape, d_best: "DeviceBuffer"):
        """argmax with input and output in device memory, queued on the context's stream."""
        s = np.asarray(shape, np.int64)
        _check(lib().ocr_nd_argmax_device(self.handle, ctypes.c_void_p(d_x.ptr), _ptr(s), len(s),
                                          ctypes.c_void_p(d_best.ptr)))

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_nd_free(self.handle)
                self.handle = None
        except Exception:
            pass


def det_input_dims(w: int, h: int, max_side: int):
    """(ow, oh, to_page) of the PP-OCR detection input (src/nd.rs:1356-1358)."""
    ow, oh = ctypes.c_uint32(), ctypes.c_uint32()
    tp = np.zeros(2, np.float32)
    _check(lib().ocr_nd_det_input_dims(w, h, max_side, ctypes.byref(ow), ctypes.byref(oh), _ptr(tp)))
    return ow.value, oh.value, (float(tp[0]), float(tp[1]))


def det_input(ctx: Context, rgb: np.ndarray, max_side: int) -> np.ndarray:
    """The PP-OCR detection input [1, 3, oh, ow] of an RGB page (src/nd.rs:1353-1369)."""
    rgb = np.ascontiguousarray(rgb, np.uint8)
    h, w = rgb.shape[:2]
    ow, oh, _ = det_input_dims(w, h, max_side)
    out = np.empty((1, 3, oh, ow), np.float32)
    _check(lib().ocr_nd_det_input(ctx.handle, _ptr(rgb), w, h, max_side, _ptr(out)))
    return out


def db_threshold(ctx: Context, prob: np.ndarray, thr: float) -> np.ndarray:
    """prob [h, w] > thr as [h, ceil(w / 32)] bit words (src/ppdet.rs:88)."""
    prob = np.ascontiguousarray(prob, np.float32)
    h, w = prob.shape
    bits = np.empty((h, (w + 31) // 32), np.uint32)
    _check(lib().ocr_db_threshold(ctx.handle, _ptr(prob), w, h, thr, _ptr(bits)))
    return bits


class Recognizer:
    """Recognizer (src/gpu.rs:1441-1603)."""

    def __init__(self, ctx: Context, onnx_path: "str | ParsedGraph", lines: int = 8):
        self.ctx = ctx
        if isinstance(onnx_path, ParsedGraph):
            self.handle = lib().ocr_recognizer_new_onnx(ctx.handle, onnx_path.ref(), lines)
        else:
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


FAMILIES = ("conv3x3_dma", "gemm_dma", "conv_narrow", "conv_igemm", "conv_mfma", "gru", "conv_transpose", "conv_direct", "conv_generic", "maxpool", "mask_up",
            "grey_resize", "line_crop", "avgpool_t", "argmax", "copy", "ccl")
ND_FAMILIES = ("conv3x3_dma", "gemm_dma", "conv_narrow", "conv_igemm", "conv_mfma", "nd_conv_nchw", "nd_conv_dw", "nd_conv_small",
               "nd_gemm_rows", "nd_head", "nd_attention", "nd_bgemm", "nd_conv_generic", "nd_conv_transpose", "nd_elementwise", "nd_copy",
               "nd_reduce", "nd_layer_norm", "nd_softmax", "nd_argmax", "nd_pool", "nd_resize", "nd_det_prep",
               "nd_threshold")


def probe_start(family: str):
    _check(lib().ocr_probe_start(family.encode()))


def probe_stop(family: str) -> dict:
    calls = ctypes.c_uint32()
    ms, flops, nbytes = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    _check(lib().ocr_probe_stop(family.encode(), ctypes.byref(calls), ctypes.byref(ms), ctypes.byref(flops),
                                ctypes.byref(nbytes)))
    return {"calls": calls.value, "ms": ms.value, "flops": flops.value, "bytes": nbytes.value}


# ---- page images (no GPU) ------------------------------------------------------------------
def _png_bytes(src) -> np.ndarray:
    if isinstance(src, (str, os.PathLike)):
        with open(src, "rb") as f:
            src = f.read()
    return np.frombuffer(src, np.uint8) if not isinstance(src, np.ndarray) else np.ascontiguousarray(src, np.uint8)


def png_dims(src) -> tuple:
    """(width, height) of a PNG (a path or its bytes) from its IHDR chunk (ocr_png_dims)."""
    data = _png_bytes(src)
    w, h = ctypes.c_uint32(), ctypes.c_uint32()
    _check(lib().ocr_png_dims(_ptr(data), data.size, ctypes.byref(w), ctypes.byref(h)))
    return w.value, h.value


def decode_png(src, out: np.ndarray | None = None) -> np.ndarray:
    """A PNG page (a path or its bytes) as an [h, w, 3] uint8 RGB array, as the reference's
    image::open(p)?.into_rgb8() (ocr-bench.rs:424). out, if given, is a C-contiguous uint8 array
    of at least w * h * 3 bytes (page-locked memory from Context.host_array suits the pipeline);
    the result is then a view of it."""
    data = _png_bytes(src)
    w, h = png_dims(data)
    if out is None:
        out = np.empty((h, w, 3), np.uint8)
    if out.dtype != np.uint8 or not out.flags.c_contiguous:
        raise OcrError("decode_png: out must be a C-contiguous uint8 array")
    _check(lib().ocr_png_decode(_ptr(data), data.size, _ptr(out), out.nbytes, None, None))
    return out.reshape(-1)[: w * h * 3].reshape(h, w, 3)


def decode_pngs(srcs, threads: int = 8) -> list:
    """Several PNG pages decoded side by side on host threads (the decode releases the GIL)."""
    import concurrent.futures as cf
    with cf.ThreadPoolExecutor(max(1, threads)) as ex:
        return list(ex.map(decode_png, srcs))


# ---- host geometry (no GPU) -----------------------------------------------------------------
def word_rects(bits: np.ndarray, w: int, threads: int = 1):
    """Words of a page mask (ocr-bench.rs:40-60) as an [n, 6] array (cx, cy, ux, uy, w, h),
    computed on `threads` host threads."""
    bits = _mask_bits(bits, w)
    h = bits.shape[0]
    count = ctypes.c_uint32()
    _check(lib().ocr_word_rects_mt(_ptr(bits), w, h, threads, None, 0, ctypes.byref(count)))
    out = np.zeros((count.value, 6), np.float32)
    _check(lib().ocr_word_rects_mt(_ptr(bits), w, h, threads, _ptr(out), count.value, ctypes.byref(count)))
    return out


def _mask_bits(bits: np.ndarray, w: int) -> np.ndarray:
    """A page mask as the C ABI reads it: h rows of ceil(w / 32) 32-bit words."""
    bits = np.ascontiguousarray(bits, np.uint32)
    if bits.ndim != 2 or bits.shape[1] != (w + 31) // 32:
        raise OcrError(f"mask of shape {bits.shape} is not rows of ceil({w} / 32) = {(w + 31) // 32} words")
    return bits


def word_rects_gpu(ctx: "Context", bits: np.ndarray, w: int):
    """The same words with the mask's runs labelled on the GPU (the page pipeline's path)."""
    bits = _mask_bits(bits, w)
    h = bits.shape[0]
    count = ctypes.c_uint32()
    _check(lib().ocr_word_rects_gpu(ctx.handle, _ptr(bits), w, h, None, 0, ctypes.byref(count)))
    out = np.zeros((count.value, 6), np.float32)
    _check(lib().ocr_word_rects_gpu(ctx.handle, _ptr(bits), w, h, _ptr(out), count.value, ctypes.byref(count)))
    return out


def word_rects_gpu_noalloc(ctx: "Context", bits: np.ndarray, w: int):
    """word_rects_gpu with the labelling in the library's fixed device array (no allocation)."""
    bits = _mask_bits(bits, w)
    h = bits.shape[0]
    count = ctypes.c_uint32()
    _check(lib().ocr_word_rects_gpu_noalloc(ctx.handle, _ptr(bits), w, h, None, 0, ctypes.byref(count)))
    out = np.zeros((count.value, 6), np.float32)
    _check(lib().ocr_word_rects_gpu_noalloc(ctx.handle, _ptr(bits), w, h, _ptr(out), count.value,
                                            ctypes.byref(count)))
    return out


class Layout:
    """The layout of one page before recognition: words, lines, crop geometry, batches."""

    def __init__(self, bits: np.ndarray, w: int, relv: float = 0.15, relend: float = 0.1):
        bits = np.ascontiguousarray(bits, np.uint32)
        self.handle = lib().ocr_layout_page(_ptr(bits), w, bits.shape[0], relv, relend)
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())
        nw, nl, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().ocr_layout_counts(self.handle, ctypes.byref(nw), ctypes.byref(nl), ctypes.byref(nb)))
        self.words, self.nlines, self.nbatches = nw.value, nl.value, nb.value

    def line(self, i: int):
        """(box [left, top, bw, bh, out_w], row_off [bh + 1], spans [n, 2])"""
        box = np.zeros(5, np.int32)
        ns = ctypes.c_uint32()
        _check(lib().ocr_layout_line(self.handle, i, _ptr(box), None, None, ctypes.byref(ns)))
        row_off = np.zeros(box[3] + 1, np.int32)
        spans = np.zeros((ns.value, 2), np.int32)
        _check(lib().ocr_layout_line(self.handle, i, None, _ptr(row_off), _ptr(spans), ctypes.byref(ns)))
        return box, row_off, spans

    def batch(self, i: int):
        """(width, [line indices])"""
        w, n = ctypes.c_uint32(), ctypes.c_uint32()
        members = np.zeros(64, np.uint32)
        _check(lib().ocr_layout_batch(self.handle, i, ctypes.byref(w), _ptr(members), ctypes.byref(n)))
        return w.value, [int(v) for v in members[: n.value]]

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_layout_free(self.handle)
                self.handle = None
        except Exception:
            pass


class Pipeline:
    """The whole-page pipeline (ocr-bench.rs:133-310, 458-585)."""

    def __init__(self, det: Detector, rec: Recognizer, merge=2, relv=0.15, relend=0.1, thr=0.5, threads=0,
                 det_batch=3, label_runs=0, label_comps=0, label_slots=0):
        self.ctx = det.ctx
        self._keep = (det, rec)
        opts = ocr_pipeline_opts(merge, relv, relend, thr, threads, det_batch, label_runs, label_comps, label_slots)
        self.handle = lib().ocr_pipeline_new(det.handle, rec.handle, ctypes.byref(opts))
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    def run_device(self, d_pages, ws, hs):
        n = len(d_pages)
        arr = (ctypes.c_void_p * n)(*[b.ptr for b in d_pages])
        w, h = np.asarray(ws, np.uint32), np.asarray(hs, np.uint32)
        _check(lib().ocr_pipeline_run_device(self.handle, arr, _ptr(w), _ptr(h), n))

    def run(self, pages):
        """Pages in host memory (numpy [h, w, 3] uint8; pageable, or HostArray arrays)."""
        pages = [np.ascontiguousarray(p, np.uint8) for p in pages]
        n = len(pages)
        arr = (ctypes.c_void_p * n)(*[p.ctypes.data for p in pages])
        w = np.asarray([p.shape[1] for p in pages], np.uint32)
        h = np.asarray([p.shape[0] for p in pages], np.uint32)
        _check(lib().ocr_pipeline_run(self.handle, arr, _ptr(w), _ptr(h), n))

    def page_error(self, page: int) -> str:
        """Why a page of the last run failed ("" when it finished)."""
        buf = ctypes.create_string_buffer(4096)
        n = ctypes.c_uint32()
        _check(lib().ocr_pipeline_page_error(self.handle, page, buf, 4096, ctypes.byref(n)))
        return buf.value.decode()

    def stats(self) -> dict:
        s = ocr_pipeline_stats()
        _check(lib().ocr_pipeline_stats_get(self.handle, ctypes.byref(s)))
        return {k: getattr(s, k) for k, _ in ocr_pipeline_stats._fields_}

    def texts(self, page: int):
        nl, nw = ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().ocr_pipeline_page(self.handle, page, ctypes.byref(nl), ctypes.byref(nw)))
        out = []
        buf = ctypes.create_string_buffer(4096)
        n = ctypes.c_uint32()
        for i in range(nl.value):
            _check(lib().ocr_pipeline_line_text(self.handle, page, i, buf, 4096, ctypes.byref(n)))
            out.append(buf.value.decode())
        return out, nw.value

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_pipeline_free(self.handle)
                self.handle = None
        except Exception:
            pass


class ocr_pp_opts(ctypes.Structure):
    _fields_ = [("merge", ctypes.c_uint32), ("thr", ctypes.c_float), ("relv", ctypes.c_float),
                ("max_side", ctypes.c_uint32), ("per_batch", ctypes.c_uint32), ("threads", ctypes.c_uint32),
                ("det_batch", ctypes.c_uint32), ("box_thresh", ctypes.c_float), ("unclip_ratio", ctypes.c_float),
                ("min_size", ctypes.c_float)]


class PpPipeline:
    """The PP-OCR page pipeline (ocr-bench.rs with DET=ppocr REC=ppocr): DB detection, host boxes,
    SVTR recognition with the fused arg-max head, host CTC."""

    def __init__(self, det: NdGraph, rec: NdGraph, merge=2, thr=0.3, relv=0.1, max_side=960, per_batch=16,
                 threads=0, det_batch=4):
        self.ctx = det.ctx
        self._keep = (det, rec)
        opts = ocr_pp_opts(merge, thr, relv, max_side, per_batch, threads, det_batch, 0.0, 0.0, 0.0)
        self.handle = lib().ocr_pp_pipeline_new(det.handle, rec.handle, ctypes.byref(opts))
        if not self.handle:
            raise OcrError(lib().ocr_last_error().decode())

    def run_device(self, d_pages, ws, hs):
        n = len(d_pages)
        arr = (ctypes.c_void_p * n)(*[b.ptr for b in d_pages])
        w, h = np.asarray(ws, np.uint32), np.asarray(hs, np.uint32)
        _check(lib().ocr_pp_pipeline_run_device(self.handle, arr, _ptr(w), _ptr(h), n))

    def run(self, pages):
        pages = [np.ascontiguousarray(p, np.uint8) for p in pages]
        n = len(pages)
        arr = (ctypes.c_void_p * n)(*[p.ctypes.data for p in pages])
        w = np.asarray([p.shape[1] for p in pages], np.uint32)
        h = np.asarray([p.shape[0] for p in pages], np.uint32)
        _check(lib().ocr_pp_pipeline_run(self.handle, arr, _ptr(w), _ptr(h), n))

    def stats(self) -> dict:
        s = ocr_pipeline_stats()
        _check(lib().ocr_pp_pipeline_stats_get(self.handle, ctypes.byref(s)))
        return {k: getattr(s, k) for k, _ in ocr_pipeline_stats._fields_}

    def texts(self, page: int):
        nl = ctypes.c_uint32()
        _check(lib().ocr_pp_pipeline_page(self.handle, page, ctypes.byref(nl)))
        out = []
        buf = ctypes.create_string_buffer(1 << 16)
        n = ctypes.c_uint32()
        for i in range(nl.value):
            _check(lib().ocr_pp_pipeline_line_text(self.handle, page, i, buf, 1 << 16, ctypes.byref(n)))
            out.append(buf.value.decode())
        return out

    def __del__(self):
        try:
            if self.handle:
                lib().ocr_pp_pipeline_free(self.handle)
                self.handle = None
        except Exception:
            pass


def db_boxes(bits: np.ndarray, prob: np.ndarray, to_page=(1.0, 1.0), box_thresh=0.45, unclip_ratio=1.4,
             min_size=3.0):
    """ppdet::boxes (ppdet.rs:87-132) on the host: [n, 6] (cx, cy, ux, uy, w, h) in page units."""
    prob = np.ascontiguousarray(prob, np.float32)
    bits = np.ascontiguousarray(bits, np.uint32)
    h, w = prob.shape
    count = ctypes.c_uint32()
    _check(lib().ocr_db_boxes(_ptr(bits), _ptr(prob), w, h, to_page[0], to_page[1], box_thresh, unclip_ratio,
                              min_size, None, 0, ctypes.byref(count)))
    out = np.zeros((max(count.value, 1), 6), np.float32)
    _check(lib().ocr_db_boxes(_ptr(bits), _ptr(prob), w, h, to_page[0], to_page[1], box_thresh, unclip_ratio,
                              min_size, _ptr(out), count.value, ctypes.byref(count)))
    return out[: count.value]


def pp_line_box(box, relv: float, page_w: int, page_h: int):
    """(left, top, width, height, resized width) of a box's PP-OCR line image."""
    b = np.ascontiguousarray(box, np.float32)
    out = np.zeros(5, np.int32)
    _check(lib().ocr_pp_line_box(_ptr(b), relv, page_w, page_h, _ptr(out)))
    return tuple(int(v) for v in out)


def line_images(ctx: Context, rgb: np.ndarray, lines, wb: int) -> np.ndarray:
    """ocrs line images on the GPU: lines = [(box, row_off, spans)] with box = (left, top, width,
    height, resized width) as Layout.line gives them; returns [n][64][wb] float32."""
    rgb = np.ascontiguousarray(rgb, np.uint8)
    desc, ro, sp = [], [], []
    for box, row_off, spans in lines:
        base = len(sp)
        desc.append(list(box[:5]) + [len(ro)])
        ro.extend(int(o) + base for o in row_off)
        sp.extend(int(v) for v in np.asarray(spans).reshape(-1))
    d = np.ascontiguousarray(desc, np.int32).reshape(-1, 6)
    r = np.ascontiguousarray(ro, np.int32)
    s = np.ascontiguousarray(sp if sp else [0], np.int32)
    out = np.empty((len(lines), 64, wb), np.float32)
    _check(lib().ocr_line_images(ctx.handle, _ptr(rgb), rgb.shape[1], rgb.shape[0], _ptr(d), len(lines), _ptr(r),
                                 len(r), _ptr(s), len(sp), wb, _ptr(out)))
    return out


def pp_line_images(ctx: Context, rgb: np.ndarray, lines, wb: int) -> np.ndarray:
    """PP-OCR line images [n, 3, 48, wb] of an RGB page on the GPU (ppocr.rs:42-78)."""
    rgb = np.ascontiguousarray(rgb, np.uint8)
    ln = np.ascontiguousarray(np.asarray(lines, np.int32).reshape(-1, 5))
    out = np.empty((len(ln), 3, 48, wb), np.float32)
    _check(lib().ocr_pp_line_images(ctx.handle, _ptr(rgb), rgb.shape[1], rgb.shape[0], _ptr(ln), len(ln), wb,
                                    _ptr(out)))
    return out
