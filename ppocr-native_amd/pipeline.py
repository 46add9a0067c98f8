"""The worker's page path on one GPU: a page in, its text lines out.

It follows the worker's `detect` and `read` (src/bin/ppocr-native/ocr.rs:
202-261) as the page benchmark states them: the page's long side limited to
960 (the `Limit::Max` rule of src/det.rs:166-193 with the side fixed at the
limit, `scaled_size` and `snap32` of src/det.rs:10-27), the detector input
made on the GPU from the uploaded page (`det_input_hwc`, src/det.rs:228-289)
straight into the detector's input, the detector and its map's DB threshold
as row bitmasks on the GPU (src/det.rs:438), the DB boxes on the host from
those bitmasks (`boxes_from_prob`, src/det.rs:291-452, reading order), then for each box
the perspective crop (`crop_text`, src/crop.rs:84-127) and the recogniser
input (`rec_input`, src/rec.rs:19-43, the tensor at most 320 wide: wider
crops are squeezed to 320) made on the GPU straight into the recogniser's
lanes, batches of 16 lanes (`recognise_all`, ocr.rs:436-530) on up to three
recogniser handles at once, and each lane's text and score (`ctc_decode`,
src/rec.rs:112-161). Over several pages the next page's detector runs while
the host finds this page's boxes, and the host finds the next page's boxes
while the GPU reads this page's lines.

Left out, as the benchmark leaves them out: RapidOCR's page fitting and
padding (`prepare_page`), the text-score filter, and the vertical re-read.
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field

import numpy as np

from . import GpuError, GpuModel, lib
from .devmem import DeviceArray
from .images import MEAN, STD, _check, _sig
from .post import DbOptions, Dictionary, boxes_from_bits, ctc_decode_pairs

REC_HEIGHT = 48


def _snap32(x: int) -> int:
    """Python's int(round(x / 32) * 32): halves to the even multiple."""
    return int(round(x / 32.0)) * 32


def det_size(width: int, height: int, limit: int = 960) -> tuple[int, int] | None:
    """The detector input (width, height) for a page: both sides scaled by
    limit / long side when the long side exceeds `limit`, truncated, then
    snapped to multiples of 32 (src/det.rs:16-27); None when a side would
    vanish."""
    if width == 0 or height == 0:
        return None
    long = max(width, height)
    ratio = limit / long if long > limit else 1.0
    w, h = _snap32(int(width * ratio)), _snap32(int(height * ratio))
    return (w, h) if w > 0 and h > 0 else None


def default_recognisers() -> int:
    """Recogniser handles a page pipeline runs at once: three when the
    process has a hardware queue for each of its streams (the detector's,
    the recognisers' and the null stream, which the model loads use), else
    two. HIP gives a process GPU_MAX_HW_QUEUES queues (four by default); two
    streams on one queue run their work in turn. Measured on a 44-line page:
    1.46 ms a page with three handles and eight queues, 1.67 with two
    handles and 1.76 with three on four queues."""
    import os
    try:
        queues = int(os.environ.get("GPU_MAX_HW_QUEUES", "4"))
    except ValueError:
        queues = 4
    return 3 if queues >= 5 else 2


@dataclass
class Line:
    quad: np.ndarray  # [4][2] f32, page pixels: top-left, top-right, bottom-right, bottom-left
    text: str
    score: float


@dataclass
class PageTimes:
    """Host wall time of each stage of the last page, milliseconds."""
    detect: float = 0.0    # detector input + detector forward + map to the host
    boxes: float = 0.0     # DB boxes on the host
    read: float = 0.0      # crops + recogniser inputs + recogniser forwards
    decode: float = 0.0    # CTC text on the host
    lines: int = 0
    batches: list[int] = field(default_factory=list)


class PagePipeline:
    """A detector and `recognisers` recogniser handles (PPOCRPL1 plans) on
    the GPU, and the dictionary of the recogniser's classes.

    A page's recogniser batches go to the handles in turn and run at the
    same time on their own streams; over several pages (`read_pages`) the
    next page's detector runs on the GPU while this page's boxes are found
    on the host."""

    def __init__(self, det_plan: bytes, rec_plan: bytes, dictionary: Dictionary, *, limit: int = 960,
                 batch: int = 16, max_width: int = 320, options: DbOptions | None = None,
                 recognisers: int | None = None):
        if recognisers is None:
            recognisers = default_recognisers()
        self.det = GpuModel.load(det_plan)
        self.recs = [GpuModel.load(rec_plan) for _ in range(max(1, recognisers))]
        self.rec = self.recs[0]
        self.dictionary = dictionary
        self.limit, self.batch, self.max_width = limit, batch, max_width
        self.options = options or DbOptions()
        # The detector's runs also write the map's DB threshold as row
        # bitmasks, which the host's border following starts from.
        self.det.set_db_mask(0, self.options.thresh)
        self._det_hw: tuple[int, int] | None = None
        self._rec_sizes: list[list[tuple[int, int]]] = [[] for _ in self.recs]
        self.times = PageTimes()
        L = _sig()
        self._L = L
        self._mean = (C.c_double * 3)(*MEAN)
        self._std = (C.c_double * 3)(*STD)

    def close(self) -> None:
        self.det.close()
        for r in self.recs:
            r.close()

    def read(self, page: np.ndarray) -> list[Line]:
        """The text lines of a uint8 H x W x 3 page on the host."""
        a = np.ascontiguousarray(page, np.uint8)
        if a.ndim != 3 or a.shape[2] != 3:
            raise ValueError("an H x W x 3 page")
        d = DeviceArray.of(a.reshape(-1))
        try:
            return self.read_device(d.addr, a.shape[1], a.shape[0])
        finally:
            d.free()

    def read_device(self, page: int, width: int, height: int) -> list[Line]:
        """The text lines of a page already on the device (uint8 HWC)."""
        return self.read_pages([(page, width, height)])[0]

    def read_pages(self, pages: list[tuple[int, int, int]]) -> list[list[Line]]:
        """The text lines of each page (device address, width, height), in
        order. While the GPU reads a page's lines, the host finds the next
        page's boxes (its detector queued meanwhile), and while it reads the
        next page's lines, the host decodes this page's text, so that host
        and GPU work overlap."""
        out: list[list[Line]] = []
        if not pages:
            return out
        self.times = PageTimes()
        sizes: list[tuple[int, int] | None] = [None] * len(pages)
        sizes[0] = self._detect(*pages[0])
        quads = self._boxes(0, pages, sizes)
        job = self._queue_page(*pages[0], quads)
        for k in range(len(pages)):
            following = self._boxes(k + 1, pages, sizes) if k + 1 < len(pages) else None
            pairs = self._finish_page(job)
            # The next page's lines go to the GPU before this page's text is
            # decoded on the host (its outputs are copies by now).
            if following is not None:
                job = self._queue_page(*pages[k + 1], following)
            t0 = time.perf_counter()
            out.append([Line(q, *ctc_decode_pairs(p, self.dictionary)) for q, p in zip(quads, pairs)])
            self.times.decode += (time.perf_counter() - t0) * 1e3
            self.times.lines += len(out[-1])
            quads = following
        return out

    def _boxes(self, k: int, pages: list[tuple[int, int, int]], sizes: list) -> np.ndarray:
        """Page k's boxes: waits for its detector, queues page k + 1's, then
        the DB boxes on the host (none for a page too thin)."""
        t0 = time.perf_counter()
        prob = bits = None
        if sizes[k] is not None:
            self.det.wait()
            prob = self.det.lane_output(0, 0)
            bits = self.det.lane_db_mask(0)
        if k + 1 < len(pages):
            sizes[k + 1] = self._detect(*pages[k + 1])
        t1 = time.perf_counter()
        self.times.detect += (t1 - t0) * 1e3
        if prob is None:
            return np.zeros((0, 4, 2), np.float32)
        w, h = sizes[k]
        _, width, height = pages[k]
        quads = boxes_from_bits(prob, bits, w, h, width, height, self.options)
        self.times.boxes += (time.perf_counter() - t1) * 1e3
        return quads

    def _queue_page(self, page: int, width: int, height: int, quads: np.ndarray) -> dict:
        """Queues the page's first recogniser batches, one per handle."""
        t0 = time.perf_counter()
        groups = [quads[s:s + self.batch] for s in range(0, len(quads), self.batch)]
        job = {"page": (page, width, height), "groups": groups, "next": 0, "busy": {},
               "out": [None] * len(quads)}
        while job["next"] < min(len(groups), len(self.recs)):
            self._queue_group(job)
        self.times.read += (time.perf_counter() - t0) * 1e3
        return job

    def _queue_group(self, job: dict) -> None:
        g = job["next"]
        r = g % len(self.recs)
        if r in job["busy"]:
            self._collect(job, r)
        group = job["groups"][g]
        self.times.batches.append(len(group))
        self._queue_batch(r, *job["page"], group)
        job["busy"][r] = (g * self.batch, len(group))
        job["next"] = g + 1

    def _collect(self, job: dict, r: int) -> None:
        first, n = job["busy"].pop(r)
        self.recs[r].wait()
        for i in range(n):
            job["out"][first + i] = self.recs[r].lane_output(i, 0)

    def _finish_page(self, job: dict) -> list[np.ndarray]:
        """The [T][2] recogniser output of each box: the page's remaining
        batches queued as handles come free, then every batch collected."""
        t0 = time.perf_counter()
        while job["next"] < len(job["groups"]):
            self._queue_group(job)
        for r in list(job["busy"]):
            self._collect(job, r)
        self.times.read += (time.perf_counter() - t0) * 1e3
        return job["out"]

    def _detect(self, page: int, width: int, height: int) -> tuple[int, int] | None:
        """Queues the page's detector input and forward on the detector's
        stream; the detector input size, or None for a page too thin."""
        size = det_size(width, height, self.limit)
        if size is None:
            return None
        w, h = size
        if self._det_hw != (h, w):
            self.det.set_input_size(h, w)
            self._det_hw = (h, w)
        dst, n = self.det.lane_input_device(0)
        assert n == w * h * 3
        _check(self._L.ppocr_hip_det_input(page, width, height, dst, w, h, self._mean, self._std,
                                           self.det.stream() or None), "det_input")
        self.det.run_device_async()
        return size

    def _queue_batch(self, r: int, page: int, width: int, height: int, quads: np.ndarray) -> None:
        """Recogniser handle r's lanes for one batch: 48 rows, the width
        `rec_input` gives the crop (capped); inputs and forward queued."""
        L, rec = self._L, self.recs[r]
        qs = [np.ascontiguousarray(q, np.float32).reshape(8) for q in quads]
        lanes = []
        for q in qs:
            cw, ch = C.c_size_t(), C.c_size_t()
            if L.ppocr_crop_size(q.ctypes.data_as(C.POINTER(C.c_float)), C.byref(cw), C.byref(ch)):
                raise GpuError("crop size")
            rw = C.c_size_t()
            tw = L.ppocr_rec_width_fit(cw.value, ch.value, self.max_width, C.byref(rw))
            if tw == 0:
                raise GpuError(f"an empty crop ({cw.value} x {ch.value})")
            lanes.append((REC_HEIGHT, tw))
        # A short last batch of lanes that all have one size keeps the full
        # batch's lanes (their extra lanes compute on stale inputs and are not
        # read: a lane's result does not depend on the others), so that the
        # lanes are not set again for it and again for the next page.
        if len(set(lanes)) == 1 and len(lanes) < self.batch:
            lanes = lanes + [lanes[0]] * (self.batch - len(lanes))
        if self._rec_sizes[r] != lanes:
            rec.set_sizes(lanes)
            self._rec_sizes[r] = lanes
        outs = (C.c_void_p * len(qs))()
        caps = (C.c_size_t * len(qs))()
        for lane in range(len(qs)):
            outs[lane], caps[lane] = rec.lane_input_device(lane)
        flat = np.ascontiguousarray(np.stack(qs), np.float32)
        got = (C.c_size_t * len(qs))()
        _check(L.ppocr_hip_crop_rec_inputs(page, width, height, flat.ctypes.data_as(C.POINTER(C.c_float)),
                                           len(qs), self.max_width, outs, caps, got,
                                           rec.stream() or None), "crop_rec_inputs")
        rec.run_device_async()
