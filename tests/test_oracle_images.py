"""The oracle's image stages against the reference's golden data
(tests/golden/: OpenCV 5.0 and RapidOCR outputs, tests/parity.rs:47-211) and
against what the arithmetic fixes (identities of the resize and the crop)."""
import json
from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden"
FX = json.loads((GOLD / "fixtures.json").read_text())
MEAN, STD = (0.485, 0.456, 0.406), (0.229, 0.224, 0.225)


def npy(name):
    return np.load(GOLD / name, allow_pickle=False)


@pytest.mark.parametrize("case", FX["resize"], ids=[c["file"] for c in FX["resize"]])
def test_resize_matches_opencv(oracle, case):
    got = oracle.resize_linear(npy("noise.npy"), case["width"], case["height"])
    assert np.array_equal(got, npy(case["file"]))


def test_resize_identities(oracle):
    rng = np.random.default_rng(2)
    img = rng.integers(0, 256, (13, 17, 3), dtype=np.uint8)
    assert np.array_equal(oracle.resize_linear(img, 17, 13), img)  # same size: a copy
    flat = np.full((9, 11, 3), 77, np.uint8)
    assert np.all(oracle.resize_linear(flat, 40, 3) == 77)  # a constant stays constant


def test_det_input_matches_rapidocr(oracle):
    # 40x28 noise snaps to 32x32 (tests/parity.rs:67-80); fixture is 1x3x32x32.
    want = npy(FX["det_input"]["file"])[0].transpose(1, 2, 0)
    got = oracle.det_input(npy("noise.npy"), 32, 32, FX["det_input"]["mean"], FX["det_input"]["std"])
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(want).view(np.uint32))


@pytest.mark.parametrize("case", FX["rec_input"], ids=[c["crop"] for c in FX["rec_input"]])
def test_rec_input_matches_rapidocr(oracle, case):
    want = npy(case["input"])[0].transpose(1, 2, 0)
    got = oracle.rec_input(npy(case["crop"]))
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(want).view(np.uint32))


@pytest.mark.parametrize("case", FX["crops"], ids=[c["file"] for c in FX["crops"]])
def test_crops_match_opencv(oracle, case):
    # tests/parity.rs:155-189: OpenCV rounds some bicubic sums near a half its
    # own way: at most one level, on at most 1 % of the values.
    want = npy(case["file"])
    got = oracle.crop_text(npy("page.npy"), case["quad"])
    assert got.shape == want.shape
    d = got.astype(np.int16) - want
    assert np.abs(d).max() <= 1
    assert np.count_nonzero(d) * 100 <= d.size


def test_crop_of_an_upright_rectangle_is_the_subimage(oracle):
    # At whole-pixel samples the cubic weights are (0, 1, 0, 0).
    page = npy("page.npy")
    got = oracle.crop_text(page, [[6, 9], [200, 9], [200, 31], [6, 31]])
    assert np.array_equal(got, page[9:31, 6:200])


def test_tall_crops_turn(oracle):
    page = npy("page.npy")
    got = oracle.crop_text(page, [[30, 20], [52, 20], [52, 110], [30, 110]])
    assert got.shape == (22, 90, 3)
    assert np.array_equal(got, np.rot90(page[20:110, 30:52]))


def _taps(src, dst, corners):
    scale = 1.0 / (dst / src)
    d = np.arange(dst, dtype=np.float64)
    f = (d * scale if corners else (d + 0.5) * scale - 0.5).astype(np.float32)
    fl = np.floor(f)
    a = f - fl
    s = fl.astype(np.int64)
    near = np.clip(s, 0, src - 1)
    far = np.clip(s + 1, 0, src - 1)
    wf = np.rint(a * np.float32(2048)).astype(np.int64)
    wn = np.rint((np.float32(1) - a) * np.float32(2048)).astype(np.int64)
    return near, far, wn, wf


def _resize(img, w, h, sum_first=False, corners=False):
    """numpy restatement of the 8-bit bilinear resize, with two plausible
    mistakes available: rounding the vertical sum once instead of each row,
    and sampling at d * scale (no half-pixel centres)."""
    img = img.astype(np.int64)
    xn, xf, xwn, xwf = _taps(img.shape[1], w, corners)
    yn, yf, ywn, ywf = _taps(img.shape[0], h, corners)
    rows = img[:, xn] * xwn[None, :, None] + img[:, xf] * xwf[None, :, None]
    a, b = rows[yn], rows[yf]
    if sum_first:
        v = (a * ywn[:, None, None] + b * ywf[:, None, None] + (1 << 21)) >> 22
    else:
        v = (((a >> 4) * ywn[:, None, None]) >> 16) + (((b >> 4) * ywf[:, None, None]) >> 16)
        v = (v + 2) >> 2
    return np.clip(v, 0, 255).astype(np.uint8)


def test_checks_have_teeth():
    # The restatement passes every resize fixture; each planted mistake fails
    # at least one of them.
    noise = npy("noise.npy")
    cases = [(c["width"], c["height"], npy(c["file"])) for c in FX["resize"]]
    assert all(np.array_equal(_resize(noise, w, h), want) for w, h, want in cases)
    for kw in [{"sum_first": True}, {"corners": True}]:
        assert not all(np.array_equal(_resize(noise, w, h, **kw), want) for w, h, want in cases), kw


@pytest.mark.parametrize("i", range(len(FX["contours"])))
def test_oracle_contours_match_opencv(oracle, i):
    # The oracle's border following (src/contour.rs:44-140) gives
    # cv2.findContours's borders, corner for corner, in its list order.
    case = FX["contours"][i]
    assert oracle.find_contours(npy(case["file"])) == case["contours"]


def test_oracle_contours_of_small_cases(oracle):
    # A lone pixel is its own border; a 2 x 2 block has four corners; a ring
    # has an outer border and a hole border, the hole (found second) listed
    # first; pixels on the image edge count as border pixels.
    assert oracle.find_contours(np.array([[0, 0, 0], [0, 1, 0], [0, 0, 0]])) == [[[1, 1]]]
    assert oracle.find_contours(np.ones((2, 2))) == [[[0, 0], [0, 1], [1, 1], [1, 0]]]
    ring = np.ones((5, 5), np.uint8)
    ring[2, 2] = 0
    got = oracle.find_contours(ring)
    assert len(got) == 2 and got[1] == [[0, 0], [0, 4], [4, 4], [4, 0]]
    assert sorted(map(tuple, got[0])) == [(1, 2), (2, 1), (2, 3), (3, 2)]
