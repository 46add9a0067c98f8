"""The image stages on the GPU, over the C ABI (ppocr_hip_resize_linear,
ppocr_hip_det_input, ppocr_hip_rec_input, ppocr_hip_crop_text): host arrays
in, host arrays out, with the reference's names and results
(src/image.rs:68-142, src/det.rs:228-289, src/rec.rs:19-43,
src/crop.rs:84-127). Images are uint8 H x W x 3; tensors HWC float32.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import GpuError, lib
from .devmem import DeviceArray, synchronize

MEAN = (0.485, 0.456, 0.406)
STD = (0.229, 0.224, 0.225)


def _sig():
    L = lib()
    vp, sz = C.c_void_p, C.c_size_t
    szp, fp, dp = C.POINTER(C.c_size_t), C.POINTER(C.c_float), C.POINTER(C.c_double)
    for name, args, res in [
        ("ppocr_hip_resize_linear", [vp, sz, sz, vp, sz, sz, vp], C.c_int),
        ("ppocr_hip_det_input", [vp, sz, sz, vp, sz, sz, dp, dp, vp], C.c_int),
        ("ppocr_rec_width", [sz, sz, szp], sz),
        ("ppocr_hip_rec_input", [vp, sz, sz, vp, sz, szp, vp], C.c_int),
        ("ppocr_rec_width_fit", [sz, sz, sz, szp], sz),
        ("ppocr_hip_rec_input_fit", [vp, sz, sz, sz, vp, sz, szp, vp], C.c_int),
        ("ppocr_hip_crop_rec_inputs", [vp, sz, sz, fp, sz, sz, C.POINTER(vp), szp, szp, vp], C.c_int),
        ("ppocr_crop_size", [fp, szp, szp], C.c_int),
        ("ppocr_hip_crop_text", [vp, sz, sz, fp, vp, sz, szp, szp, vp], C.c_int),
    ]:
        f = getattr(L, name)
        f.argtypes, f.restype = args, res
    return L


def _check(rc: int, what: str) -> None:
    if rc:
        raise GpuError(f"{what} failed with HIP error {rc}")


def _upload(image) -> tuple[DeviceArray, int, int]:
    a = np.ascontiguousarray(image, np.uint8)
    if a.ndim != 3 or a.shape[2] != 3:
        raise ValueError("an H x W x 3 image")
    return DeviceArray.of(a.reshape(-1)), a.shape[1], a.shape[0]


def resize_linear(image, width: int, height: int) -> np.ndarray:
    L = _sig()
    src, w, h = _upload(image)
    dst = DeviceArray(width * height * 3)
    _check(L.ppocr_hip_resize_linear(src.addr, w, h, dst.addr, width, height, None), "resize")
    synchronize()
    return dst.download(width * height * 3, np.uint8).reshape(height, width, 3)


def det_input(image, width: int, height: int, mean=MEAN, std=STD) -> np.ndarray:
    L = _sig()
    src, w, h = _upload(image)
    out = DeviceArray(4 * width * height * 3)
    m, s = (C.c_double * 3)(*mean), (C.c_double * 3)(*std)
    _check(L.ppocr_hip_det_input(src.addr, w, h, out.addr, width, height, m, s, None), "det_input")
    synchronize()
    return out.download(width * height * 3).reshape(height, width, 3)


def rec_width(w: int, h: int) -> tuple[int, int]:
    rw = C.c_size_t()
    return _sig().ppocr_rec_width(w, h, C.byref(rw)), rw.value


def rec_width_fit(w: int, h: int, max_width: int) -> tuple[int, int]:
    rw = C.c_size_t()
    return _sig().ppocr_rec_width_fit(w, h, max_width, C.byref(rw)), rw.value


def rec_input(crop, max_width: int = 0) -> np.ndarray:
    """The recogniser tensor of a crop; with `max_width` the tensor is at
    most that wide (wider crops squeezed), as the page pipeline feeds it."""
    L = _sig()
    src, w, h = _upload(crop)
    width, _ = rec_width_fit(w, h, max_width)
    out = DeviceArray(4 * 48 * width * 3)
    got = C.c_size_t()
    if max_width:
        rc = L.ppocr_hip_rec_input_fit(src.addr, w, h, max_width, out.addr, 48 * width * 3, C.byref(got), None)
    else:
        rc = L.ppocr_hip_rec_input(src.addr, w, h, out.addr, 48 * width * 3, C.byref(got), None)
    _check(rc, "rec_input")
    synchronize()
    return out.download(48 * width * 3).reshape(48, width, 3)


def crop_size(quad) -> tuple[int, int]:
    q = np.ascontiguousarray(np.asarray(quad, np.float32).reshape(8))
    w, h = C.c_size_t(), C.c_size_t()
    _sig().ppocr_crop_size(q.ctypes.data_as(C.POINTER(C.c_float)), C.byref(w), C.byref(h))
    return w.value, h.value


def crop_text(image, quad) -> np.ndarray:
    L = _sig()
    src, w, h = _upload(image)
    q = np.ascontiguousarray(np.asarray(quad, np.float32).reshape(8))
    cw, ch = crop_size(q)
    out = DeviceArray(max(cw * ch * 3, 1))
    ow, oh = C.c_size_t(), C.c_size_t()
    _check(L.ppocr_hip_crop_text(src.addr, w, h, q.ctypes.data_as(C.POINTER(C.c_float)), out.addr,
                                 cw * ch * 3, C.byref(ow), C.byref(oh), None), "crop_text")
    synchronize()
    return out.download(ow.value * oh.value * 3, np.uint8).reshape(oh.value, ow.value, 3)
