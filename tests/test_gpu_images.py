"""The image stages on the GPU (ppocr_hip_resize_linear, _det_input,
_rec_input, _crop_text) against the oracle on seeded images at production
sizes, and against the reference's golden data. Bit-exact: every kernel
performs the reference's integer and IEEE f32 / f64 operations in its order.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from ppocr_native_amd import images

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
FX = json.loads((GOLD / "fixtures.json").read_text())
MEAN, STD = (0.485, 0.456, 0.406), (0.229, 0.224, 0.225)


def npy(name):
    return np.load(GOLD / name, allow_pickle=False)


def same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.flatnonzero(a.view(np.uint8) != b.view(np.uint8))
    assert bad.size == 0, f"{bad.size} bytes differ"


@pytest.mark.parametrize("case", FX["resize"], ids=[c["file"] for c in FX["resize"]])
def test_resize_golden(case):
    same(images.resize_linear(npy("noise.npy"), case["width"], case["height"]), npy(case["file"]))


@pytest.mark.parametrize("src,dst", [((3300, 2550), (960, 736)), ((480, 640), (1280, 960)),
                                     ((61, 97), (32, 32)), ((1, 5), (7, 3)), ((300, 300), (150, 150))])
def test_resize_against_oracle(oracle, src, dst):
    img = np.random.default_rng(sum(src)).integers(0, 256, (*src, 3), dtype=np.uint8)
    same(images.resize_linear(img, dst[1], dst[0]), oracle.resize_linear(img, dst[1], dst[0]))


def test_det_input_golden():
    want = npy(FX["det_input"]["file"])[0].transpose(1, 2, 0)
    same(images.det_input(npy("noise.npy"), 32, 32, FX["det_input"]["mean"], FX["det_input"]["std"]), want)


@pytest.mark.parametrize("src,dst", [((3300, 2550), (960, 736)), ((1100, 850), (960, 736)),
                                     ((700, 500), (704, 512))])
def test_det_input_against_oracle(oracle, src, dst):
    # A letter page at 300 dpi to the detector's 736 x 960 input, and others.
    img = np.random.default_rng(src[0]).integers(0, 256, (*src, 3), dtype=np.uint8)
    same(images.det_input(img, dst[1], dst[0], MEAN, STD), oracle.det_input(img, dst[1], dst[0], MEAN, STD))


@pytest.mark.parametrize("case", FX["rec_input"], ids=[c["crop"] for c in FX["rec_input"]])
def test_rec_input_golden(case):
    same(images.rec_input(npy(case["crop"])), npy(case["input"])[0].transpose(1, 2, 0))


@pytest.mark.parametrize("hw", [(20, 60), (10, 71), (31, 400), (48, 2000), (9, 3), (60, 20)])
def test_rec_input_against_oracle(oracle, hw):
    crop = np.random.default_rng(hw[1]).integers(0, 256, (*hw, 3), dtype=np.uint8)
    assert images.rec_width(hw[1], hw[0]) == oracle.rec_width(hw[1], hw[0])
    same(images.rec_input(crop), oracle.rec_input(crop))


@pytest.mark.parametrize("case", FX["crops"], ids=[c["file"] for c in FX["crops"]])
def test_crops_golden(oracle, case):
    page = npy("page.npy")
    got = images.crop_text(page, case["quad"])
    same(got, oracle.crop_text(page, case["quad"]))
    d = got.astype(np.int16) - npy(case["file"])
    assert np.abs(d).max() <= 1 and np.count_nonzero(d) * 100 <= d.size


def test_crops_against_oracle(oracle):
    # Seeded quads on a 1100 x 850 page: tilted, partly outside the page,
    # tall enough to turn, and degenerate.
    rng = np.random.default_rng(4)
    page = rng.integers(0, 256, (1100, 850, 3), dtype=np.uint8)
    quads = [[[-3, 100], [230, 98], [231, 125], [-2, 127]], [[30, 20], [52, 20], [52, 110], [30, 110]],
             [[800, 1050], [900, 1060], [895, 1120], [795, 1110]], [[5, 5], [5, 5], [5, 5], [5, 5]]]
    for _ in range(24):
        x, y = rng.uniform(0, 800), rng.uniform(0, 1050)
        w, h, t = rng.uniform(3, 400), rng.uniform(3, 120), rng.uniform(-0.3, 0.3)
        c, s = np.cos(t), np.sin(t)
        quads.append([[x, y], [x + w * c, y + w * s], [x + w * c - h * s, y + w * s + h * c],
                      [x - h * s, y + h * c]])
    for q in quads:
        q = np.asarray(q, np.float32)
        same(images.crop_text(page, q), oracle.crop_text(page, q))
