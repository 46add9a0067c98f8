"""The page pipeline on the GPU against the same pipeline on the CPU path.

The GPU side is `PagePipeline`: detector input, detector, crops, recogniser
inputs and recogniser on the GPU, boxes and text on the host. The CPU side
runs the oracle's restatements of the same stages (det_input_hwc,
the engine's forward, crop_text, rec_input) and the same host boxes and CTC
decode. The page is a seeded 2550 x 3300 letter page with 44 text lines; the
detector is the PP-OCR-style graph whose channel-0 path carries an ink
signal (nets.InkInit), so the DB boxes land on the lines; the recogniser is
the SVTR-style one with scaled seeded weights (18385 classes, T = 80).
Boxes (integer page coordinates) and text must be identical, scores within
1e-5 relative.
"""
from pathlib import Path

import numpy as np
import pytest

from ppocr_native_amd import GpuError, GpuModel, images, nets, post
from ppocr_native_amd.devmem import DeviceArray
from ppocr_native_amd.pipeline import PagePipeline, det_size

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
MEAN, STD = (0.485, 0.456, 0.406), (0.229, 0.224, 0.225)


@pytest.fixture(scope="module")
def dictionary():
    return post.Dictionary.from_metadata((GOLD / "characters.txt").read_text(encoding="utf-8"))


@pytest.mark.parametrize("shape", [(40, 200), (31, 1400), (48, 320), (20, 3000), (90, 400)])
def test_rec_input_capped_against_oracle(oracle, shape):
    crop = np.random.default_rng(shape[1]).integers(0, 256, (*shape, 3), dtype=np.uint8)
    got = images.rec_input(crop, 320)
    want = oracle.rec_input(crop, 320)
    assert got.shape == want.shape == (48, 320, 3)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_crop_rec_inputs_equal_crop_then_rec_input(oracle):
    # The batched, crop-free inputs equal crop_text then rec_input (capped
    # at 320), bit for bit, for 21 boxes (two launches): tilted lines, short
    # and long ones, a tall box that is turned, and one past the page edge.
    import ctypes as C
    rng = np.random.default_rng(8)
    page = rng.integers(0, 256, (900, 700, 3), dtype=np.uint8)
    quads = []
    for i in range(21):
        x, y, w, h, t = 20 + 9 * i, 30 + 40 * i, 80 + 37 * i, 18 + (i % 5) * 6, 0.03 * (i - 10)
        if i == 7:
            w, h = 30, 160  # tall: the crop is turned
        if i == 20:
            x, y = 650, 860  # runs past the right and bottom edges
        c, s_ = np.cos(t), np.sin(t)
        quads.append([[x, y], [x + w * c, y + w * s_], [x + w * c - h * s_, y + w * s_ + h * c],
                      [x - h * s_, y + h * c]])
    quads = np.asarray(quads, np.float32)
    L = images._sig()
    dpage = DeviceArray.of(page.reshape(-1))
    outs = [DeviceArray(4 * 48 * 320 * 3) for _ in quads]
    ptrs = (C.c_void_p * len(quads))(*[o.addr for o in outs])
    caps = (C.c_size_t * len(quads))(*([48 * 320 * 3] * len(quads)))
    widths = (C.c_size_t * len(quads))()
    rc = L.ppocr_hip_crop_rec_inputs(dpage.addr, 700, 900, quads.ctypes.data_as(C.POINTER(C.c_float)),
                                     len(quads), 320, ptrs, caps, widths, None)
    assert rc == 0
    from ppocr_native_amd.devmem import synchronize
    synchronize()
    for i, q in enumerate(quads):
        assert widths[i] == 320
        got = outs[i].download(48 * 320 * 3).reshape(48, 320, 3)
        crop = images.crop_text(page, q)
        assert np.array_equal(got.view(np.uint32), images.rec_input(crop, 320).view(np.uint32)), i
        want = oracle.rec_input(oracle.crop_text(page, q), 320)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
    turned = images.crop_size(quads[7])
    assert turned[0] > turned[1]  # 160 x 30 after the quarter turn


def test_device_input_run_equals_host_input_run():
    # The same detector input written by the GPU into the lane's device
    # input, or by the host into its pinned input: identical maps.
    page = nets.letter_page(lines=6, seed=2, width=640, height=480)
    w, h = det_size(640, 480)
    m = GpuModel.load(nets.detector_plan(h=h, w=w, init="ink"))
    m.set_input_size(h, w)
    m.input_mut()[:] = images.det_input(page, w, h, MEAN, STD).reshape(-1)
    m.run()
    host = m.output(0)
    d = DeviceArray.of(page.reshape(-1))
    dst, n = m.lane_input_device(0)
    assert n == w * h * 3
    import ctypes as C
    L = images._sig()
    rc = L.ppocr_hip_det_input(d.addr, 640, 480, dst, w, h, (C.c_double * 3)(*MEAN), (C.c_double * 3)(*STD),
                               m.stream() or None)
    assert rc == 0
    m.run_device()
    assert np.array_equal(m.output(0).view(np.uint32), host.view(np.uint32))
    m.close()


def cpu_page(oracle, page, det_plan, rec_plan, dictionary):
    """The CPU path: the oracle's stages and the host boxes and decode."""
    H, W = page.shape[:2]
    w, h = det_size(W, H)
    det = oracle.OracleModel(det_plan)
    det.set_size(h, w)
    prob = det.run(oracle.det_input(page, w, h, MEAN, STD))[0]
    quads = post.boxes_from_prob(prob, w, h, W, H)
    rec = oracle.OracleModel(rec_plan)
    rec.set_size(48, 320)
    lines = []
    for q in quads:
        x = oracle.rec_input(oracle.crop_text(page, q), 320)
        pairs = rec.run(x)[0]
        lines.append((q, *post.ctc_decode_pairs(pairs, dictionary)))
    return prob, lines


def test_page_pipeline_against_cpu_path(oracle, dictionary):
    page = nets.letter_page()
    H, W = page.shape[:2]
    w, h = det_size(W, H)
    det_plan = nets.detector_plan(h=h, w=w, init="ink")
    rec_plan = nets.recognizer_plan(init="scaled")
    pipe = PagePipeline(det_plan, rec_plan, dictionary)
    got = pipe.read(page)
    gpu_prob = pipe.det.output(0)
    prob, want = cpu_page(oracle, page, det_plan, rec_plan, dictionary)
    print(f"page {W}x{H} -> {w}x{h}: {len(got)} lines, batches {pipe.times.batches}", flush=True)
    assert np.max(np.abs(gpu_prob - prob)) <= 4e-5
    assert 40 <= len(want) <= 48  # one box per line of the 44
    assert len(got) == len(want)
    for g, (q, text, score) in zip(got, want):
        assert np.array_equal(g.quad, q), (g.quad, q)
        assert g.text == text
        assert g.score == pytest.approx(score, rel=1e-5, abs=1e-6)
    assert sum(len(t) for _, t, _ in want) > 0
    pipe.close()


def test_page_pipeline_again_and_other_sizes(dictionary):
    # A second page through the same pipeline (sizes cached, lanes reused)
    # reads as a fresh pipeline does; a smaller page changes the sizes.
    det_plan = nets.detector_plan(h=960, w=736, init="ink")
    rec_plan = nets.recognizer_plan(init="scaled")
    a = PagePipeline(det_plan, rec_plan, dictionary)
    p1, p2 = nets.letter_page(seed=5), nets.letter_page(lines=20, seed=9, width=2200, height=1700)
    first = a.read(p1)
    second = a.read(p2)
    again = a.read(p1)
    b = PagePipeline(det_plan, rec_plan, dictionary)
    fresh = b.read(p2)
    assert [(x.text, x.quad.tolist()) for x in first] == [(x.text, x.quad.tolist()) for x in again]
    assert [(x.text, x.quad.tolist()) for x in second] == [(x.text, x.quad.tolist()) for x in fresh]
    assert len(second) >= 15
    a.close()
    b.close()


def test_read_pages_equals_single_reads(dictionary):
    # Several pages through read_pages (each page's detector queued while
    # the page before is read, recogniser batches on three handles at once)
    # give what one read per page gives, through one recogniser handle.
    det_plan = nets.detector_plan(h=960, w=736, init="ink")
    rec_plan = nets.recognizer_plan(init="scaled")
    pages = [nets.letter_page(seed=5), nets.letter_page(lines=20, seed=9, width=2200, height=1700),
             nets.letter_page(lines=30, seed=13)]
    one = PagePipeline(det_plan, rec_plan, dictionary, recognisers=1)
    want = [one.read(p) for p in pages]
    many = PagePipeline(det_plan, rec_plan, dictionary)
    dev = [DeviceArray.of(p.reshape(-1)) for p in pages]
    got = many.read_pages([(d.addr, p.shape[1], p.shape[0]) for d, p in zip(dev, pages)])
    assert len(got) == 3
    for g, w in zip(got, want):
        assert [(x.text, x.quad.tolist(), x.score) for x in g] == [(x.text, x.quad.tolist(), x.score) for x in w]
    assert sum(len(g) for g in got) >= 80
    one.close()
    many.close()


def test_db_mask_written_by_the_detector_run():
    # The detector's runs write the map's threshold as row bitmasks (one
    # launch after the forward): equal to the host's threshold of the map the
    # same run returns, lane by lane, on the eager first run and the graph
    # replays after it; the boxes from them equal the boxes from the map.
    h, w = 960, 736
    m = GpuModel.load(nets.detector_plan(h=h, w=w, init="ink"))
    m.set_sizes([(h, w)] * 2)
    m.set_db_mask(0, 0.3)
    for run in range(3):
        for lane in range(2):
            page = nets.letter_page(seed=run * 2 + lane)
            m.lane_input_mut(lane)[:] = images.det_input(page, w, h, MEAN, STD).reshape(-1)
        m.run()
        for lane in range(2):
            prob = m.lane_output(lane, 0)
            bits = m.lane_db_mask(lane)
            assert bits.shape == (h, (w + 63) // 64)
            assert np.array_equal(bits, post.pack_rows(prob.reshape(h, w) > np.float32(0.3))), (run, lane)
            want = post.boxes_from_prob(prob, w, h, 2550, 3300)
            assert len(want) > 30 and np.array_equal(post.boxes_from_bits(prob, bits, w, h, 2550, 3300), want)
    m.set_db_mask(-1)
    m.run()
    with pytest.raises(GpuError):
        m.lane_db_mask(0)
    m.close()
