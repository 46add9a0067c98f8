"""ppocr-native_amd: ppocr-native's GPU model on MI355X (gfx950), over the C ABI
of include/ppocr_hip.h (libppocr_hip.so, built from csrc/).

`GpuModel` mirrors the engine's `GpuModel` (src/engine/gpu/mod.rs:110-291):
``load``, ``device``, ``integrated``, ``set_input_size``, ``max_lanes``,
``set_sizes``, ``input_mut`` / ``lane_input_mut``, ``output`` /
``lane_output`` and ``run``, with the same meaning and the same error
behaviour: every failure raises ``GpuError`` with the library's message
where the Rust model returns ``Err(String)``; nothing falls back to the CPU.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libppocr_hip.so"
_lib = None


class GpuError(RuntimeError):
    """A plan the GPU refuses, a size it cannot take, or a HIP failure."""


def build() -> None:
    """Compile libppocr_hip.so for gfx950 (hipcc)."""
    r = subprocess.run(["make", "-B", "-j8", "-C", str(HERE / "csrc")], capture_output=True,
                       text=True)
    if r.returncode:
        raise RuntimeError("building libppocr_hip.so failed:\n" + r.stdout[-4000:] + r.stderr[-4000:])


def lib() -> C.CDLL:
    """The HIP library; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        raise GpuError(f"{LIB} is missing: build it first (ppocr_native_amd.build())")
    L = C.CDLL(str(LIB))
    vp, sz, szp, cp = C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t), C.c_char_p
    fp = C.POINTER(C.c_float)
    sig = {
        "ppocr_gpu_load": ([cp, C.POINTER(vp), cp, sz], C.c_int),
        "ppocr_gpu_load_bytes": ([cp, sz, C.POINTER(vp), cp, sz], C.c_int),
        "ppocr_gpu_free": ([vp], None),
        "ppocr_gpu_device": ([vp], cp),
        "ppocr_gpu_integrated": ([vp], C.c_int),
        "ppocr_gpu_set_input_size": ([vp, sz, sz, cp, sz], C.c_int),
        "ppocr_gpu_set_sizes": ([vp, szp, sz, cp, sz], C.c_int),
        "ppocr_gpu_max_lanes": ([vp], sz),
        "ppocr_gpu_lanes": ([vp], sz),
        "ppocr_gpu_lane_input": ([vp, sz, szp], fp),
        "ppocr_gpu_lane_output": ([vp, sz, sz, szp], fp),
        "ppocr_gpu_output_count": ([vp], sz),
        "ppocr_gpu_run": ([vp, cp, sz], C.c_int),
        "ppocr_gpu_upload": ([vp, cp, sz], C.c_int),
        "ppocr_gpu_run_resident": ([vp, C.c_int, fp, cp, sz], C.c_int),
        "ppocr_gpu_download": ([vp, cp, sz], C.c_int),
        "ppocr_gpu_stream": ([vp], vp),
        "ppocr_gpu_lane_input_device": ([vp, sz, szp], vp),
        "ppocr_gpu_run_device": ([vp, cp, sz], C.c_int),
        "ppocr_gpu_run_device_async": ([vp, cp, sz], C.c_int),
        "ppocr_gpu_wait": ([vp, cp, sz], C.c_int),
        "ppocr_gpu_set_graphs": ([vp, C.c_int], C.c_int),
        "ppocr_gpu_launch_count": ([vp], sz),
        "ppocr_gpu_launch_name": ([vp, sz, szp], cp),
        "ppocr_gpu_profile_launches": ([vp, C.c_int, fp, cp, sz], C.c_int),
        "ppocr_gpu_launch_work": ([vp, sz, C.POINTER(C.c_double), C.POINTER(C.c_double)], C.c_int),
        "ppocr_gpu_launch_ops": ([vp, sz, szp, sz], sz),
        "ppocr_hip_add": ([vp, vp, vp, sz, C.c_int, vp], C.c_int),
        "ppocr_hip_mul": ([vp, vp, vp, sz, vp], C.c_int),
        "ppocr_hip_activation": ([vp, vp, sz, C.c_int, vp], C.c_int),
        "ppocr_hip_copy_lds": ([vp, vp, sz, vp], C.c_int),
        "ppocr_hip_channel_mean": ([vp, vp, sz, sz, vp], C.c_int),
        "ppocr_hip_channel_mean_noalloc": ([vp, vp, sz, sz, vp, C.c_char_p, sz], C.c_int),
        "ppocr_hip_channel_mul": ([vp, vp, vp, sz, sz, vp], C.c_int),
        "ppocr_hip_layer_norm": ([vp, vp, vp, sz, sz, vp], C.c_int),
        "ppocr_hip_row_argmax": ([vp, vp, sz, sz, vp], C.c_int),
        "ppocr_hip_db_mask": ([vp, vp, sz, C.c_float, vp], C.c_int),
        "ppocr_dictionary_load": ([cp, sz, C.POINTER(vp), cp, sz], C.c_int),
        "ppocr_dictionary_free": ([vp], None),
        "ppocr_dictionary_len": ([vp], sz),
        "ppocr_dictionary_class": ([vp, sz, szp], C.POINTER(C.c_char)),
        "ppocr_ctc_decode": ([vp, C.POINTER(C.c_uint32), fp, sz, C.c_char_p, sz, szp,
                              C.POINTER(C.c_double), cp, sz], C.c_int),
        "ppocr_ctc_decode_pairs": ([vp, fp, sz, C.c_char_p, sz, szp, C.POINTER(C.c_double), cp, sz],
                                   C.c_int),
        "ppocr_find_contours": ([vp, sz, sz, C.POINTER(C.c_int32), sz, szp, sz, szp, szp], C.c_int),
        "ppocr_min_area_rect": ([C.POINTER(C.c_int32), sz, fp, fp], C.c_int),
        "ppocr_unclip": ([fp, C.c_double, C.POINTER(C.c_int32), sz, szp], C.c_int),
        "ppocr_db_boxes": ([fp, vp, sz, sz, sz, sz, vp, fp, sz, szp, cp, sz], C.c_int),
        "ppocr_db_boxes_bits": ([fp, vp, sz, sz, sz, sz, sz, vp, fp, sz, szp, cp, sz], C.c_int),
        "ppocr_gpu_set_db_mask": ([vp, C.c_long, C.c_float, cp, sz], C.c_int),
        "ppocr_gpu_lane_db_mask": ([vp, sz, szp, szp], vp),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def _call(fn, *args) -> None:
    err = C.create_string_buffer(1024)
    if fn(*args, err, 1024):
        raise GpuError(err.value.decode(errors="replace"))


class GpuModel:
    """A plan loaded onto the GPU, run over one or more lanes at a time."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle

    @classmethod
    def load(cls, plan: str | Path | bytes) -> "GpuModel":
        h = C.c_void_p()
        if isinstance(plan, (bytes, bytearray)):
            _call(lib().ppocr_gpu_load_bytes, bytes(plan), len(plan), C.byref(h))
        else:
            _call(lib().ppocr_gpu_load, str(plan).encode(), C.byref(h))
        return cls(h)

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().ppocr_gpu_free(self._h)
            self._h = C.c_void_p()

    __del__ = close

    def device(self) -> str:
        return lib().ppocr_gpu_device(self._h).decode()

    def integrated(self) -> bool:
        return bool(lib().ppocr_gpu_integrated(self._h))

    def set_input_size(self, height: int, width: int) -> None:
        _call(lib().ppocr_gpu_set_input_size, self._h, height, width)

    def set_sizes(self, sizes: list[tuple[int, int]]) -> None:
        flat = (C.c_size_t * (2 * len(sizes)))(*[v for hw in sizes for v in hw])
        _call(lib().ppocr_gpu_set_sizes, self._h, flat, len(sizes))

    def max_lanes(self) -> int:
        return lib().ppocr_gpu_max_lanes(self._h)

    def lanes(self) -> int:
        return lib().ppocr_gpu_lanes(self._h)

    def output_count(self) -> int:
        return lib().ppocr_gpu_output_count(self._h)

    def lane_input_mut(self, lane: int) -> np.ndarray:
        """Lane `lane`'s image, HWC f32, as a view of the model's pinned memory."""
        n = C.c_size_t()
        p = lib().ppocr_gpu_lane_input(self._h, lane, C.byref(n))
        if not p:
            raise GpuError(f"lane {lane} does not exist")
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def input_mut(self) -> np.ndarray:
        return self.lane_input_mut(0)

    def lane_output(self, lane: int, index: int = 0) -> np.ndarray:
        """Result `index` of lane `lane` from the last run (a copy)."""
        n = C.c_size_t()
        p = lib().ppocr_gpu_lane_output(self._h, lane, index, C.byref(n))
        if not p:
            raise GpuError(f"lane {lane} output {index} does not exist")
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy()

    def output(self, index: int = 0) -> np.ndarray:
        return self.lane_output(0, index)

    def run(self) -> None:
        _call(lib().ppocr_gpu_run, self._h)

    def lane_input_device(self, lane: int) -> tuple[int, int]:
        """(device address, floats) of lane `lane`'s input, for inputs
        prepared on the GPU in order on `stream()`; valid until set_sizes."""
        n = C.c_size_t()
        p = lib().ppocr_gpu_lane_input_device(self._h, lane, C.byref(n))
        if not p:
            raise GpuError(f"lane {lane} does not exist")
        return p, n.value

    def run_device(self) -> None:
        """`run` over inputs already written on the device."""
        _call(lib().ppocr_gpu_run_device, self._h)

    def set_db_mask(self, output: int = 0, thresh: float = 0.3) -> None:
        """From the next run on, also write output `output`'s DB threshold
        (prob > thresh) as row bitmasks; output < 0 stops it."""
        _call(lib().ppocr_gpu_set_db_mask, self._h, output, thresh)

    def lane_db_mask(self, lane: int = 0) -> np.ndarray:
        """Lane `lane`'s DB bitmasks from the last run (a copy): rows x words
        (uint64), bit x % 64 of word x / 64 set where the map exceeds the
        threshold."""
        wpr, rows = C.c_size_t(), C.c_size_t()
        p = lib().ppocr_gpu_lane_db_mask(self._h, lane, C.byref(wpr), C.byref(rows))
        if not p:
            raise GpuError(f"no DB mask for lane {lane}")
        n = wpr.value * rows.value
        return np.ctypeslib.as_array((C.c_uint64 * n).from_address(p)).reshape(rows.value, wpr.value).copy()

    def run_device_async(self) -> None:
        """`run_device` queued on the model's stream; `wait()` ends it."""
        _call(lib().ppocr_gpu_run_device_async, self._h)

    def wait(self) -> None:
        _call(lib().ppocr_gpu_wait, self._h)

    # Measurement helpers.
    def upload(self) -> None:
        _call(lib().ppocr_gpu_upload, self._h)

    def download(self) -> None:
        _call(lib().ppocr_gpu_download, self._h)

    def run_resident(self, repeats: int = 1) -> float:
        """Run `repeats` times on the inputs already on the device; device ms."""
        ms = C.c_float()
        _call(lib().ppocr_gpu_run_resident, self._h, repeats, C.byref(ms))
        return ms.value

    def stream(self) -> int:
        return lib().ppocr_gpu_stream(self._h) or 0

    def set_graphs(self, enable: bool) -> None:
        """Replay runs from a captured HIP graph (default) or launch eagerly."""
        lib().ppocr_gpu_set_graphs(self._h, int(enable))

    def launches(self) -> list[tuple[str, int]]:
        out = []
        for i in range(lib().ppocr_gpu_launch_count(self._h)):
            op = C.c_size_t()
            name = lib().ppocr_gpu_launch_name(self._h, i, C.byref(op))
            out.append((name.decode(), op.value))
        return out

    def launch_ops(self) -> list[list[int]]:
        """The plan operations each launch runs (several for a grouped launch)."""
        out = []
        for i in range(lib().ppocr_gpu_launch_count(self._h)):
            n = lib().ppocr_gpu_launch_ops(self._h, i, None, 0)
            buf = (C.c_size_t * max(n, 1))()
            lib().ppocr_gpu_launch_ops(self._h, i, buf, n)
            out.append([int(buf[k]) for k in range(n)])
        return out

    def launch_work(self) -> list[tuple[float, float]]:
        """(flops, bytes) of each launch: the layer's algorithmic work."""
        out = []
        for i in range(lib().ppocr_gpu_launch_count(self._h)):
            f, b = C.c_double(), C.c_double()
            lib().ppocr_gpu_launch_work(self._h, i, C.byref(f), C.byref(b))
            out.append((f.value, b.value))
        return out

    def profile_launches(self, repeats: int = 10) -> list[float]:
        n = lib().ppocr_gpu_launch_count(self._h)
        ms = (C.c_float * max(n, 1))()
        _call(lib().ppocr_gpu_profile_launches, self._h, repeats, ms)
        return list(ms)[:n]


def _check(rc: int, what: str) -> None:
    if rc:
        raise GpuError(f"{what} failed with HIP error {rc}")


def hip_add(a: int, b: int, y: int, n: int, act: int = 0, stream: int = 0) -> None:
    _check(lib().ppocr_hip_add(a, b, y, n, act, stream or None), "ppocr_hip_add")


def hip_mul(a: int, b: int, y: int, n: int, stream: int = 0) -> None:
    _check(lib().ppocr_hip_mul(a, b, y, n, stream or None), "ppocr_hip_mul")


def hip_activation(x: int, y: int, n: int, act: int, stream: int = 0) -> None:
    _check(lib().ppocr_hip_activation(x, y, n, act, stream or None), "ppocr_hip_activation")


def hip_copy_lds(x: int, y: int, n: int, stream: int = 0) -> None:
    """y = x through LDS by direct loads (the counters' calibration copy)."""
    _check(lib().ppocr_hip_copy_lds(x, y, n, stream or None), "ppocr_hip_copy_lds")


def hip_channel_mean(x: int, y: int, pixels: int, c: int, stream: int = 0) -> None:
    _check(lib().ppocr_hip_channel_mean(x, y, pixels, c, stream or None), "ppocr_hip_channel_mean")


def hip_channel_mean_noalloc(x: int, y: int, pixels: int, c: int, stream: int = 0) -> None:
    """ppocr_hip_channel_mean with its scratch in the library's device array
    (no allocation; at most 4096 channels)."""
    err = C.create_string_buffer(256)
    rc = lib().ppocr_hip_channel_mean_noalloc(x, y, pixels, c, stream or None, err, 256)
    if rc:
        raise RuntimeError(f"ppocr_hip_channel_mean_noalloc: {err.value.decode()} ({rc})")


def hip_channel_mul(x: int, g: int, y: int, pixels: int, c: int, stream: int = 0) -> None:
    _check(lib().ppocr_hip_channel_mul(x, g, y, pixels, c, stream or None), "ppocr_hip_channel_mul")


def hip_layer_norm(x: int, w: int, y: int, rows: int, c: int, stream: int = 0) -> None:
    _check(lib().ppocr_hip_layer_norm(x, w, y, rows, c, stream or None), "ppocr_hip_layer_norm")


def hip_row_argmax(x: int, y: int, rows: int, cols: int, stream: int = 0) -> None:
    _check(lib().ppocr_hip_row_argmax(x, y, rows, cols, stream or None), "ppocr_hip_row_argmax")
