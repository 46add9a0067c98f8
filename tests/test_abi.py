"""The C ABI: the library loads and exports every entry point the header
declares; calls that need no GPU behave (CPU-only)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from ppocr_native_amd import LIB, GpuError, GpuModel, lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "ppocr_hip.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ppocr_(?:gpu|hip)_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "ppocr_gpu_load" in names and "ppocr_gpu_run" in names
    assert len(names) >= 25


@pytest.mark.parametrize("name", declared())
def test_library_exports(name):
    assert LIB.exists()
    L = C.CDLL(str(LIB))
    assert hasattr(L, name), name


def test_null_handles_are_refused():
    L = lib()
    err = C.create_string_buffer(256)
    assert L.ppocr_gpu_run(None, err, 256) != 0 and err.value
    assert L.ppocr_gpu_lane_input(None, 0, None) is None or not L.ppocr_gpu_lane_input(None, 0, None)
    assert L.ppocr_gpu_max_lanes(None) == 0
    L.ppocr_gpu_free(None)


def test_missing_plan_file_is_an_error(tmp_path):
    with pytest.raises(GpuError, match="cannot open"):
        GpuModel.load(tmp_path / "absent.plan")
