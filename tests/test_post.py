"""The host stages either side of the model against the reference's golden
data (tests/golden/, copied from the reference's fixtures by
copy_fixtures.py; written there from OpenCV 5.0, pyclipper 1.4, RapidOCR 3.9
and numpy). Bit-exact everywhere, as the reference's own tests demand
(tests/parity.rs:83-231). CPU only: these stages are host code.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from ppocr_native_amd import post

GOLD = Path(__file__).resolve().parent / "golden"
FX = json.loads((GOLD / "fixtures.json").read_text())


def npy(name):
    return np.load(GOLD / name, allow_pickle=False)


@pytest.fixture(scope="module")
def dictionary():
    return post.Dictionary.from_metadata((GOLD / "characters.txt").read_text(encoding="utf-8"))


def test_dictionary_size(dictionary):
    # tests/parity.rs:217: blank + 18708 characters + space.
    assert len(dictionary) == 18710
    assert dictionary.cls(0) == "blank" and dictionary.cls(18709) == " "


def test_dictionary_splits_like_python():
    # tests/parity.rs:234-238: str.splitlines, "\r\n" one break, no trailing class.
    d = post.Dictionary.from_metadata("a\nb\r\nc\r\n\nd\n")
    assert [d.cls(i) for i in range(len(d))] == ["blank", "a", "b", "c", "", "d", " "]
    d = post.Dictionary.from_metadata("x y\x85z")
    assert [d.cls(i) for i in range(len(d))] == ["blank", "x", "y", "z", " "]


@pytest.mark.parametrize("case", FX["ctc"], ids=[c["stem"] for c in FX["ctc"]])
def test_ctc_matches_rapidocr(dictionary, case):
    best = npy(case["stem"] + "_argmax.npy").astype(np.uint32)
    prob = npy(case["stem"] + "_maxprob.npy")
    text, score = post.ctc_decode(best, prob, dictionary)
    assert text == case["text"]
    assert score == case["score"]
    # The model's own [T][2] output gives the same.
    pairs = np.stack([best.astype(np.float32), prob], axis=1)
    assert post.ctc_decode_pairs(pairs, dictionary) == (text, score)


def test_ctc_rejects_classes_outside_the_dictionary():
    d = post.Dictionary.from_metadata("a\nb")
    with pytest.raises(Exception):
        post.ctc_decode([1, 9], [0.5, 0.5], d)


@pytest.mark.parametrize("i", range(len(FX["contours"])))
def test_contours_match_opencv(i):
    case = FX["contours"][i]
    mask = npy(case["file"])
    h, w = mask.shape
    assert post.find_contours(mask, w, h) == case["contours"]


def test_min_area_rect_matches_opencv():
    bad = []
    for case in FX["min_area_rect"]:
        got = post.min_area_rect(case["points"]).points()
        want = np.asarray(case["box"], np.float32)
        if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
            bad.append((case["points"][:4], got.tolist(), case["box"]))
    assert not bad, f"{len(bad)} of {len(FX['min_area_rect'])} differ, first {bad[0]}"


def test_unclip_matches_pyclipper():
    bad = [c["quad"] for c in FX["unclip"] if post.unclip(c["quad"], 1.5) != c["ring"]]
    assert not bad, f"{len(bad)} of {len(FX['unclip'])} differ, first {bad[0]}"


def test_db_boxes_match_rapidocr():
    case = FX["boxes"]
    prob = npy(case["file"])
    h, w = prob.shape
    dest_w, dest_h = case["dest"]
    got = post.boxes_from_prob(prob, w, h, dest_w, dest_h)
    want = np.asarray(case["boxes"], np.float32)
    assert got.shape == want.shape
    assert np.array_equal(got, want)
    # With the threshold mask given (as the GPU kernel makes it): the same.
    mask = (prob > np.float32(0.3)).astype(np.uint8)
    assert np.array_equal(post.boxes_from_prob(prob, w, h, dest_w, dest_h, mask=mask), want)


def test_db_boxes_of_an_empty_map():
    assert post.boxes_from_prob(np.zeros((32, 32), np.float32), 32, 32, 64, 64).shape == (0, 4, 2)


def _masks():
    """Seeded masks that exercise the border scan: noise at several
    densities, blobs with holes, single pixels and lines, widths on and
    either side of the 64-pixel words."""
    rng = np.random.default_rng(17)
    out = []
    for w in (1, 5, 63, 64, 65, 127, 130, 200):
        for h in (1, 7, 33):
            for density in (0.05, 0.5, 0.93):
                out.append((rng.random((h, w)) < density).astype(np.uint8))
    for _ in range(6):  # blobs with holes: thick rings and filled rectangles
        m = np.zeros((90, 150), np.uint8)
        for _ in range(12):
            y, x = rng.integers(0, 80), rng.integers(0, 140)
            hh, ww = rng.integers(3, 30), rng.integers(3, 60)
            m[y:y + hh, x:x + ww] = 1
            if hh > 6 and ww > 6:
                m[y + 2:y + hh - 2, x + 2:x + ww - 2] = rng.integers(0, 2)
        out.append(m)
    return out


def test_contours_equal_the_oracle_on_seeded_masks(oracle):
    # The product follows borders from where a row's bits change; the
    # oracle scans every pixel as the reference does (src/contour.rs:44-140).
    for m in _masks():
        h, w = m.shape
        assert post.find_contours(m, w, h) == oracle.find_contours(m), (h, w)


def test_db_boxes_from_bits_match_rapidocr():
    # The golden map's boxes from its threshold as row bitmasks (the form the
    # detector's run writes with set_db_mask): the same 11 boxes, bit for bit.
    case = FX["boxes"]
    prob = npy(case["file"])
    h, w = prob.shape
    dest_w, dest_h = case["dest"]
    bits = post.pack_rows(prob > np.float32(0.3))
    got = post.boxes_from_bits(prob, bits, w, h, dest_w, dest_h)
    assert np.array_equal(got, np.asarray(case["boxes"], np.float32))


def test_db_boxes_from_bits_equal_boxes_from_prob():
    # Seeded blob maps (text-line-like bands of high probability over noise):
    # every box equal whichever form the threshold comes in.
    rng = np.random.default_rng(23)
    for k in range(4):
        h, w = 96 + 32 * k, 160 + 64 * k
        prob = rng.uniform(0, 0.35, (h, w)).astype(np.float32)
        for _ in range(8):
            y, x = rng.integers(0, h - 12), rng.integers(0, w - 40)
            prob[y:y + rng.integers(6, 12), x:x + rng.integers(20, 40)] = rng.uniform(0.5, 1.0)
        want = post.boxes_from_prob(prob, w, h, 3 * w, 3 * h)
        got = post.boxes_from_bits(prob, post.pack_rows(prob > np.float32(0.3)), w, h, 3 * w, 3 * h)
        assert len(want) > 0 and np.array_equal(got, want)
