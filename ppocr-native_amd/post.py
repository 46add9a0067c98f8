"""The host stages either side of the GPU model, over the library's C ABI:
the recogniser's text (`Dictionary`, `ctc_decode`, src/rec.rs:45-161) and
the detector's text boxes (`find_contours`, `min_area_rect`, `unclip`,
`boxes_from_prob`, src/contour.rs, src/geometry.rs, src/det.rs:291-452),
with the reference's names, arguments and results.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import GpuError, lib

_ERR = 1024


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


class Dictionary:
    """Recogniser classes: blank, the model's characters, a space."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle

    @classmethod
    def from_metadata(cls, text: str) -> "Dictionary":
        raw = text.encode("utf-8")
        h, err = C.c_void_p(), C.create_string_buffer(_ERR)
        if lib().ppocr_dictionary_load(raw, len(raw), C.byref(h), err, _ERR):
            raise GpuError(err.value.decode())
        return cls(h)

    def __len__(self) -> int:
        return lib().ppocr_dictionary_len(self._h)

    def cls(self, index: int) -> str:
        n = C.c_size_t()
        p = lib().ppocr_dictionary_class(self._h, index, C.byref(n))
        if not p:
            raise IndexError(index)
        return C.string_at(p, n.value).decode("utf-8")

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().ppocr_dictionary_free(self._h)
            self._h = C.c_void_p()

    __del__ = close


def _decode(fn, *args) -> tuple[str, float]:
    cap = 256
    while True:
        buf, n, score = C.create_string_buffer(cap), C.c_size_t(), C.c_double()
        err = C.create_string_buffer(_ERR)
        rc = fn(*args, buf, cap, C.byref(n), C.byref(score), err, _ERR)
        if rc == 2:
            cap = n.value + 1
            continue
        if rc:
            raise GpuError(err.value.decode())
        return C.string_at(buf, n.value).decode("utf-8"), score.value


def ctc_decode(best, prob, dictionary: Dictionary) -> tuple[str, float]:
    """Text and score of a line from its per-step best class and probability."""
    b = np.ascontiguousarray(np.asarray(best, dtype=np.uint32))
    p = _f32(prob)
    if b.shape != p.shape:
        raise ValueError("one probability per timestep")
    return _decode(lib().ppocr_ctc_decode, dictionary._h, b.ctypes.data_as(C.POINTER(C.c_uint32)),
                   p.ctypes.data_as(C.POINTER(C.c_float)), b.size)


def ctc_decode_pairs(pairs, dictionary: Dictionary) -> tuple[str, float]:
    """The same from the model's [T][2] output (class as f32, probability)."""
    q = _f32(pairs).reshape(-1)
    return _decode(lib().ppocr_ctc_decode_pairs, dictionary._h, q.ctypes.data_as(C.POINTER(C.c_float)),
                   q.size // 2)


def find_contours(mask, width: int, height: int) -> list[list[list[int]]]:
    m = np.ascontiguousarray(np.asarray(mask, dtype=np.uint8).reshape(-1))
    if m.size != width * height:
        raise ValueError("mask size")
    npts, ncon = C.c_size_t(), C.c_size_t()
    lib().ppocr_find_contours(m.ctypes.data_as(C.c_void_p), width, height, None, 0, None, 0,
                              C.byref(npts), C.byref(ncon))
    pts = np.zeros(2 * npts.value, np.int32)
    lens = (C.c_size_t * max(ncon.value, 1))()
    rc = lib().ppocr_find_contours(m.ctypes.data_as(C.c_void_p), width, height,
                                   pts.ctypes.data_as(C.POINTER(C.c_int32)), npts.value, lens,
                                   ncon.value, C.byref(npts), C.byref(ncon))
    if rc:
        raise GpuError(f"ppocr_find_contours failed ({rc})")
    out, k = [], 0
    for i in range(ncon.value):
        n = lens[i]
        out.append(pts[2 * k:2 * (k + n)].reshape(n, 2).tolist())
        k += n
    return out


@dataclass
class RotatedRect:
    center: tuple[float, float]
    width: float
    height: float
    angle: float
    corners: np.ndarray  # cv2.boxPoints, f32 [4][2]

    def points(self) -> np.ndarray:
        return self.corners


def min_area_rect(points) -> RotatedRect:
    p = _i32(points).reshape(-1)
    rect, corners = (C.c_float * 5)(), np.zeros(8, np.float32)
    lib().ppocr_min_area_rect(p.ctypes.data_as(C.POINTER(C.c_int32)), p.size // 2, rect,
                              corners.ctypes.data_as(C.POINTER(C.c_float)))
    return RotatedRect((rect[0], rect[1]), rect[2], rect[3], rect[4], corners.reshape(4, 2))


def unclip(quad, ratio: float) -> list[list[int]]:
    q = _f32(quad).reshape(-1)
    n = C.c_size_t()
    lib().ppocr_unclip(q.ctypes.data_as(C.POINTER(C.c_float)), ratio, None, 0, C.byref(n))
    ring = np.zeros(2 * max(n.value, 1), np.int32)
    if lib().ppocr_unclip(q.ctypes.data_as(C.POINTER(C.c_float)), ratio,
                          ring.ctypes.data_as(C.POINTER(C.c_int32)), n.value, C.byref(n)):
        raise GpuError("ppocr_unclip failed")
    return ring[:2 * n.value].reshape(-1, 2).tolist()


class _DbOptions(C.Structure):
    _fields_ = [("thresh", C.c_float), ("box_thresh", C.c_double), ("unclip_ratio", C.c_double),
                ("max_candidates", C.c_size_t)]


@dataclass
class DbOptions:
    """The DB postprocess settings (src/det.rs:291-321), RapidOCR's defaults."""
    thresh: float = 0.3
    box_thresh: float = 0.5
    unclip_ratio: float = 1.5
    max_candidates: int = 1000


def boxes_from_prob(prob, map_w: int, map_h: int, dest_w: int, dest_h: int,
                    options: DbOptions | None = None, mask=None) -> np.ndarray:
    """Text boxes [n][4][2] (f32, page pixels, reading order) of a map."""
    o = options or DbOptions()
    opt = _DbOptions(o.thresh, o.box_thresh, o.unclip_ratio, o.max_candidates)
    p = _f32(prob).reshape(-1)
    if p.size != map_w * map_h:
        raise ValueError("map size")
    m = None if mask is None else np.ascontiguousarray(np.asarray(mask, dtype=np.uint8).reshape(-1))
    mp = None if m is None else m.ctypes.data_as(C.c_void_p)
    cap = 64
    while True:
        boxes, n, err = np.zeros(8 * cap, np.float32), C.c_size_t(), C.create_string_buffer(_ERR)
        rc = lib().ppocr_db_boxes(p.ctypes.data_as(C.POINTER(C.c_float)), mp, map_w, map_h, dest_w,
                                  dest_h, C.byref(opt), boxes.ctypes.data_as(C.POINTER(C.c_float)),
                                  cap, C.byref(n), err, _ERR)
        if rc == 2:
            cap = n.value
            continue
        if rc:
            raise GpuError(err.value.decode())
        return boxes[:8 * n.value].reshape(-1, 4, 2)


def boxes_from_bits(prob, bits, map_w: int, map_h: int, dest_w: int, dest_h: int,
                    options: DbOptions | None = None) -> np.ndarray:
    """`boxes_from_prob` with the threshold already taken as row bitmasks
    (map_h x words uint64, bit x % 64 of word x / 64 is prob > thresh), as
    the detector's run writes them (`GpuModel.set_db_mask`)."""
    o = options or DbOptions()
    opt = _DbOptions(o.thresh, o.box_thresh, o.unclip_ratio, o.max_candidates)
    p = _f32(prob).reshape(-1)
    b = np.ascontiguousarray(bits, np.uint64)
    if p.size != map_w * map_h or b.ndim != 2 or b.shape[0] != map_h or b.shape[1] * 64 < map_w:
        raise ValueError("map or bitmask size")
    cap = max(1, o.max_candidates)
    boxes, n, err = np.zeros(8 * cap, np.float32), C.c_size_t(), C.create_string_buffer(_ERR)
    rc = lib().ppocr_db_boxes_bits(p.ctypes.data_as(C.POINTER(C.c_float)), b.ctypes.data_as(C.c_void_p),
                                   b.shape[1], map_w, map_h, dest_w, dest_h, C.byref(opt),
                                   boxes.ctypes.data_as(C.POINTER(C.c_float)), cap, C.byref(n), err, _ERR)
    if rc:
        raise GpuError(err.value.decode())
    return boxes[:8 * n.value].reshape(-1, 4, 2)


def pack_rows(mask) -> np.ndarray:
    """Row bitmasks (rows x words, uint64) of a 2-D mask, bit x % 64 of word
    x / 64 set where mask[y][x] != 0."""
    m = np.asarray(mask) != 0
    h, w = m.shape
    words = (w + 63) // 64
    padded = np.zeros((h, words * 64), np.uint8)
    padded[:, :w] = m
    return np.ascontiguousarray(np.packbits(padded, axis=1, bitorder="little")).view("<u8").astype(np.uint64)
