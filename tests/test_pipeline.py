"""The page pipeline's host rules (CPU only): the detector size of a page
(src/det.rs:10-27, 166-193 with the long side limited to 960) and the
oracle's recogniser input with the tensor width capped at 320."""
import numpy as np
import pytest

from ppocr_native_amd.pipeline import default_recognisers, det_size


def test_det_size_reference_cases():
    # tests/parity.rs:72-73: a 40 x 28 page snaps to 32 x 32.
    assert det_size(40, 28) == (32, 32)
    # tests/parity.rs:316-323: an empty side has no size.
    for w, h in [(100, 0), (0, 100), (0, 0)]:
        assert det_size(w, h) is None
    # det.rs:10-11: 2000 snaps to 1984 (ties to the even multiple).
    assert det_size(2000, 2000, limit=2000) == (1984, 1984)
    assert det_size(2016, 1000, limit=4096) == (2016, 992)  # 1000 / 32 = 31.25 -> 31


def test_det_size_letter_page():
    # A 2550 x 3300 page (300 dpi letter) at the long side 960: 736 x 960.
    assert det_size(2550, 3300) == (736, 960)
    assert det_size(3300, 2550) == (960, 736)
    # Pages at or under the limit keep their size, snapped.
    assert det_size(960, 640) == (960, 640)
    assert det_size(100, 50) == (96, 64)
    # A thin strip's short side vanishes.
    assert det_size(4096, 1) is None


def test_rec_input_capped_width(oracle):
    rng = np.random.default_rng(3)
    narrow = rng.integers(0, 256, (40, 200, 3), dtype=np.uint8)   # 48 * 5 = 240 -> padded to 320
    wide = rng.integers(0, 256, (31, 1400, 3), dtype=np.uint8)    # 48 * 45.2 -> 2168, capped
    # A crop the cap does not touch: the reference's tensor.
    assert np.array_equal(oracle.rec_input(narrow, 320), oracle.rec_input(narrow))
    assert oracle.rec_width_fit(200, 40, 320) == (320, 240)
    # A wider one: the reference's resize to exactly 320 x 48, then the same
    # scaling to [-1, 1]; nothing to the right.
    assert oracle.rec_width_fit(1400, 31, 320) == (320, 320)
    want = (oracle.resize_linear(wide, 320, 48).astype(np.float32) / np.float32(255.0) - np.float32(0.5)) \
        / np.float32(0.5)
    assert np.array_equal(oracle.rec_input(wide, 320), want)
    # No cap: the reference's width.
    assert oracle.rec_input(wide).shape == (48, 2167, 3)


@pytest.mark.parametrize("queues,want", [(None, 2), ("4", 2), ("5", 3), ("8", 3), ("junk", 2)])
def test_default_recognisers_follow_the_queue_count(monkeypatch, queues, want):
    # Three recogniser handles only when every stream of the page path (the
    # detector's, three recognisers' and the null stream) has a queue.
    if queues is None:
        monkeypatch.delenv("GPU_MAX_HW_QUEUES", raising=False)
    else:
        monkeypatch.setenv("GPU_MAX_HW_QUEUES", queues)
    assert default_recognisers() == want
