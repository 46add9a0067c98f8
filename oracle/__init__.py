"""ctypes front of the CPU oracle (engine.c).

TEST INFRASTRUCTURE ONLY: the reference the GPU backend is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline import it.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None

KINDS = [
    "conv", "dwconv", "add", "maxpool", "avgpool", "channelmul", "concatc",
    "layernorm", "attention", "mean", "ctchead", "ctcargmax", "upsample",
    "upsampleadd", "convtranspose",
]
FUSED = ["none", "relu", "sigmoid", "gelu", "swish", "hardsigmoid", "hardsigmoidfifth",
         "hardswish"]

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")


def build() -> None:
    subprocess.run(["make", "-B", "-C", str(HERE)], check=True, capture_output=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        sz, szp, vp = C.c_size_t, C.POINTER(C.c_size_t), C.c_void_p
        L.oracle_load.argtypes = [C.c_char_p, sz, C.POINTER(vp), C.c_char_p, sz]
        L.oracle_load.restype = C.c_int
        L.oracle_free.argtypes = [vp]
        L.oracle_set_size.argtypes = [vp, sz, sz, C.c_char_p, sz]
        L.oracle_set_size.restype = C.c_int
        L.oracle_input_shape.argtypes = [vp, szp]
        L.oracle_input.argtypes = [vp]
        L.oracle_input.restype = C.POINTER(C.c_float)
        L.oracle_output_count.argtypes = [vp]
        L.oracle_output_count.restype = sz
        L.oracle_output.argtypes = [vp, sz, szp]
        L.oracle_output.restype = C.POINTER(C.c_float)
        L.oracle_op_count.argtypes = [vp]
        L.oracle_op_count.restype = sz
        L.oracle_op_info.argtypes = [vp, sz, szp]
        L.oracle_pool_floats.argtypes = [vp, sz]
        L.oracle_pool_floats.restype = sz
        L.oracle_buffer.argtypes = [vp, sz]
        L.oracle_buffer.restype = C.POINTER(C.c_float)
        L.oracle_run.argtypes = [vp, C.c_int]
        L.oracle_run_ops.argtypes = [vp, sz, sz, C.c_int]
        L.oracle_exp_neg.argtypes = [C.c_float]
        L.oracle_exp_neg.restype = C.c_float
        L.oracle_act.argtypes = [C.c_float, C.c_int]
        L.oracle_act.restype = C.c_float
        L.oracle_add.argtypes = [F32P, F32P, F32P, sz, C.c_int]
        L.oracle_mul.argtypes = [F32P, F32P, F32P, sz]
        L.oracle_activation.argtypes = [F32P, F32P, sz, C.c_int]
        L.oracle_channel_mean.argtypes = [F32P, F32P, sz, sz]
        L.oracle_channel_mul.argtypes = [F32P, F32P, F32P, sz, sz]
        L.oracle_layer_norm.argtypes = [F32P, F32P, F32P, sz, sz]
        L.oracle_softmax_row.argtypes = [F32P, sz]
        L.oracle_row_argmax.argtypes = [F32P, F32P, sz, sz, C.c_int]
        L.oracle_max_threads.restype = C.c_int
        L.oracle_find_contours.argtypes = [C.POINTER(C.c_uint8), sz, sz, vp, sz, vp, sz, szp, szp]
        L.oracle_find_contours.restype = C.c_int
        _lib = L
    return _lib


def threads() -> int:
    return int(os.environ.get("ORACLE_THREADS", lib().oracle_max_threads()))


class OracleError(RuntimeError):
    pass


class OracleModel:
    """A plan on the CPU oracle, at one input size."""

    def __init__(self, plan: bytes):
        L = lib()
        self._h = C.c_void_p()
        err = C.create_string_buffer(512)
        if L.oracle_load(plan, len(plan), C.byref(self._h), err, 512):
            raise OracleError(err.value.decode())

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().oracle_free(self._h)
            self._h = C.c_void_p()

    def set_size(self, h: int, w: int) -> None:
        err = C.create_string_buffer(512)
        if lib().oracle_set_size(self._h, h, w, err, 512):
            raise OracleError(err.value.decode())

    def input_shape(self) -> tuple[int, int, int]:
        hwc = (C.c_size_t * 3)()
        lib().oracle_input_shape(self._h, hwc)
        return tuple(hwc)

    def ops(self) -> list[dict]:
        names = ["kind", "fused", "ih", "iw", "ic", "oh", "ow", "oc", "kh", "kw", "sh", "sw",
                 "n2", "x", "x2", "y"]
        out = []
        for i in range(lib().oracle_op_count(self._h)):
            f = (C.c_size_t * 16)()
            lib().oracle_op_info(self._h, i, f)
            d = dict(zip(names, list(f)))
            d["kind"] = KINDS[d["kind"]]
            d["fused"] = FUSED[d["fused"]]
            out.append(d)
        return out

    def pool(self, slot: int) -> int:
        return lib().oracle_pool_floats(self._h, slot)

    def buffer(self, slot: int, n: int) -> np.ndarray:
        p = lib().oracle_buffer(self._h, slot)
        return np.ctypeslib.as_array(p, shape=(n,)).copy()

    def run(self, image: np.ndarray, nthreads: int | None = None) -> list[np.ndarray]:
        h, w, c = self.input_shape()
        image = np.ascontiguousarray(image, np.float32).reshape(-1)
        assert image.size == h * w * c, (image.size, (h, w, c))
        p = lib().oracle_input(self._h)
        np.ctypeslib.as_array(p, shape=(image.size,))[:] = image
        lib().oracle_run(self._h, nthreads or threads())
        outs = []
        for k in range(lib().oracle_output_count(self._h)):
            n = C.c_size_t()
            q = lib().oracle_output(self._h, k, C.byref(n))
            outs.append(np.ctypeslib.as_array(q, shape=(n.value,)).copy())
        return outs


def exp_neg(z: float) -> float:
    return lib().oracle_exp_neg(z)


def act(v: np.ndarray, fused: str) -> np.ndarray:
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    y = np.empty_like(v)
    lib().oracle_activation(v, y, v.size, FUSED.index(fused))
    return y


def add(a, b, fused: str = "none"):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    y = np.empty_like(a)
    lib().oracle_add(a, b, y, a.size, FUSED.index(fused))
    return y


def mul(a, b):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    y = np.empty_like(a)
    lib().oracle_mul(a, b, y, a.size)
    return y


def channel_mean(x: np.ndarray, pixels: int, c: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.empty(c, np.float32)
    lib().oracle_channel_mean(x, y, pixels, c)
    return y


def channel_mul(x, g, pixels: int, c: int):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    g = np.ascontiguousarray(g, np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().oracle_channel_mul(x, g, y, pixels, c)
    return y


def layer_norm(x, w, rows: int, c: int):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().oracle_layer_norm(x, w, y, rows, c)
    return y


def softmax_row(v):
    v = np.ascontiguousarray(v, np.float32).reshape(-1).copy()
    lib().oracle_softmax_row(v, v.size)
    return v


def row_argmax(x, rows: int, cols: int, nthreads: int | None = None):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.empty(2 * rows, np.float32)
    lib().oracle_row_argmax(x, y, rows, cols, nthreads or threads())
    return y


# ---------------------------------------------------------------- image stages
# Restatements of the reference's image arithmetic (oracle/image.c); images
# are uint8 HxWx3 arrays.

def _u8p(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def _img(a) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint8)
    assert a.ndim == 3 and a.shape[2] == 3, a.shape
    return a


def resize_linear(image, width: int, height: int) -> np.ndarray:
    src = _img(image)
    out = np.empty((height, width, 3), np.uint8)
    L = lib()
    L.oracle_resize_linear.argtypes = [C.POINTER(C.c_uint8), C.c_size_t, C.c_size_t,
                                       C.POINTER(C.c_uint8), C.c_size_t, C.c_size_t]
    L.oracle_resize_linear(_u8p(src), src.shape[1], src.shape[0], _u8p(out), width, height)
    return out


def det_input(image, width: int, height: int, mean, std) -> np.ndarray:
    """HWC f32, height x width x 3."""
    src = _img(image)
    out = np.empty((height, width, 3), np.float32)
    m = (C.c_double * 3)(*mean)
    s = (C.c_double * 3)(*std)
    L = lib()
    L.oracle_det_input.argtypes = [C.POINTER(C.c_uint8), C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                   C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_float)]
    L.oracle_det_input(_u8p(src), src.shape[1], src.shape[0], width, height, m, s,
                       out.ctypes.data_as(C.POINTER(C.c_float)))
    return out


def rec_width(w: int, h: int) -> tuple[int, int]:
    """(tensor width, resized width) of a w x h crop."""
    L = lib()
    L.oracle_rec_width.argtypes = [C.c_size_t, C.c_size_t, C.POINTER(C.c_size_t)]
    L.oracle_rec_width.restype = C.c_size_t
    rw = C.c_size_t()
    width = L.oracle_rec_width(w, h, C.byref(rw))
    return width, rw.value


def rec_width_fit(w: int, h: int, max_width: int) -> tuple[int, int]:
    """(tensor width, resized width) with the tensor capped at max_width."""
    L = lib()
    L.oracle_rec_width_fit.argtypes = [C.c_size_t, C.c_size_t, C.c_size_t, C.POINTER(C.c_size_t)]
    L.oracle_rec_width_fit.restype = C.c_size_t
    rw = C.c_size_t()
    width = L.oracle_rec_width_fit(w, h, max_width, C.byref(rw))
    return width, rw.value


def rec_input(crop, max_width: int = 0) -> np.ndarray:
    """HWC f32, 48 x width x 3 (width capped at max_width unless 0)."""
    src = _img(crop)
    width, _ = rec_width_fit(src.shape[1], src.shape[0], max_width)
    out = np.empty((48, width, 3), np.float32)
    L = lib()
    L.oracle_rec_input_fit.argtypes = [C.POINTER(C.c_uint8), C.c_size_t, C.c_size_t, C.c_size_t,
                                       C.POINTER(C.c_float), C.c_size_t]
    L.oracle_rec_input_fit.restype = C.c_size_t
    got = L.oracle_rec_input_fit(_u8p(src), src.shape[1], src.shape[0], max_width,
                                 out.ctypes.data_as(C.POINTER(C.c_float)), out.size)
    assert got == width
    return out


def crop_text(image, quad) -> np.ndarray:
    src = _img(image)
    q = np.ascontiguousarray(np.asarray(quad, np.float32).reshape(8))
    L = lib()
    L.oracle_crop_size.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L.oracle_crop_text.argtypes = [C.POINTER(C.c_uint8), C.c_size_t, C.c_size_t, C.POINTER(C.c_float),
                                   C.POINTER(C.c_uint8), C.c_size_t, C.POINTER(C.c_size_t),
                                   C.POINTER(C.c_size_t)]
    qp = q.ctypes.data_as(C.POINTER(C.c_float))
    w, h = C.c_size_t(), C.c_size_t()
    L.oracle_crop_size(qp, C.byref(w), C.byref(h))
    out = np.empty(max(w.value * h.value * 3, 1), np.uint8)
    assert L.oracle_crop_text(_u8p(src), src.shape[1], src.shape[0], qp, _u8p(out), out.size,
                              C.byref(w), C.byref(h))
    return out[:w.value * h.value * 3].reshape(h.value, w.value, 3)


def find_contours(mask) -> list[list[list[int]]]:
    """Region borders of a 2-D mask (oracle_find_contours: src/contour.rs:44-140):
    each border's corners [x, y], in cv2.findContours's list order."""
    m = np.ascontiguousarray(np.asarray(mask) != 0, np.uint8)
    h, w = m.shape
    pcap, ccap = 4096, 1024
    while True:
        pts = np.zeros(2 * pcap, np.int32)
        lens = np.zeros(ccap, np.uint64)
        np_, nc = C.c_size_t(), C.c_size_t()
        rc = lib().oracle_find_contours(_u8p(m), w, h, pts.ctypes.data_as(C.c_void_p), pcap,
                                        lens.ctypes.data_as(C.c_void_p), ccap, C.byref(np_), C.byref(nc))
        if rc == 1:
            pcap, ccap = max(pcap, np_.value), max(ccap, nc.value)
            continue
        if rc:
            raise MemoryError("oracle_find_contours")
        out, k = [], 0
        for n in lens[:nc.value].astype(np.int64):
            out.append(pts[2 * k:2 * (k + n)].reshape(-1, 2).tolist())
            k += n
        return out
