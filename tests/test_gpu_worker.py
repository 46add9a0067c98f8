"""The C++ page worker (`ppocr_hip_worker`, over the C ABI alone) against
the Python page pipeline and a restatement of the worker's vertical pass.

The worker follows src/bin/ppocr-native/ocr.rs: both plans loaded on the
GPU (ocr.rs:131-187), the detector per page (`Detector::run`, ocr.rs:60-91),
the lines in batches of up to 16 lanes (`read_on_gpu`, ocr.rs:513-530), and
the vertical pass that reads tall, unsure lines again turned half a turn on
one lane (`reorient`, ocr.rs:250-283; `rereads`, `reads_better`,
`rotate_half`, ocr.rs:590-612). Its boxes, text and scores must equal the
pipeline's exactly (the same kernels and host code through another
binding); the vertical pass's rule is pinned here by the reference's own
vectors (`vertical_pass_choices`, `half_turn_reverses_pixels`,
ocr.rs:627-659) and the worker's lines checked against it.
"""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ppocr_native_amd
from ppocr_native_amd import GpuModel, images, nets, post
from ppocr_native_amd.pipeline import PagePipeline

GOLD = Path(__file__).resolve().parent / "golden"
WORKER = Path(ppocr_native_amd.__file__).resolve().parent / "ppocr_hip_worker"
CONFIDENT, GAIN, ASPECT = 0.90, 0.05, 1.5  # ocr.rs:30-31, src/crop.rs:67


def rereads(quad, score) -> bool:
    """`rereads` (ocr.rs:590-600)."""
    q = np.asarray(quad, np.float64).reshape(4, 2)
    w, h = q[:, 0].max() - q[:, 0].min(), q[:, 1].max() - q[:, 1].min()
    return bool(w > 0.0 and h >= w * ASPECT and score < CONFIDENT)


def is_blank(text: str) -> bool:
    """`is_blank` (src/rec.rs:187-190)."""
    return all(c.isspace() or "\x1c" <= c <= "\x1f" for c in text)


def reads_better(score, text, new_score) -> bool:
    """`reads_better` (ocr.rs:603-605)."""
    return not is_blank(text) and new_score >= score + GAIN


def rotate_half(image: np.ndarray) -> np.ndarray:
    """`rotate_half` (ocr.rs:608-612): the pixels in reverse order."""
    return np.ascontiguousarray(image[::-1, ::-1])


def test_vertical_pass_rule_against_reference_vectors():
    # ocr.rs:627-651: (width, height, score) -> rereads; then reads_better.
    for w, h, score, want in [(40.0, 10.0, 0.5, False), (10.0, 40.0, 0.5, True), (10.0, 15.0, 0.5, True),
                              (10.0, 14.9, 0.5, False), (0.0, 40.0, 0.5, False), (10.0, 40.0, 0.9, False)]:
        quad = np.array([[0, 0], [w, 0], [w, h], [0, h]], np.float32)
        assert rereads(quad, score) is want, (w, h, score)
    for text, score, want in [("abd", 0.55, True), ("abd", 0.54, False), (" \x1c", 0.99, False)]:
        assert reads_better(0.5, text, score) is want, (text, score)
    image = np.arange(12, dtype=np.uint8).reshape(2, 2, 3)
    assert rotate_half(image).reshape(-1).tolist() == [9, 10, 11, 6, 7, 8, 3, 4, 5, 0, 1, 2]


def test_worker_usage_errors():
    # No GPU call: the flags are checked first.
    if not WORKER.exists():
        pytest.skip("the worker is not built")
    r = subprocess.run([str(WORKER), "--det", "a", "--rec", "b", "--dict", "c"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 2 and "pass --gpu" in r.stderr
    r = subprocess.run([str(WORKER), "--gpu", "--det", "a"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "--det, --rec and --dict are needed" in r.stderr
    r = subprocess.run([str(WORKER), "--gpu", "--det", "a", "--rec", "b", "--dict", "c", "--batch", "0"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "positive whole number" in r.stderr


def write_ppm(path: Path, page: np.ndarray) -> None:
    h, w, _ = page.shape
    path.write_bytes(b"P6\n# page\n%d %d\n255\n" % (w, h) + np.ascontiguousarray(page, np.uint8).tobytes())


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("worker")
    det_plan = nets.detector_plan(h=960, w=736, init="ink")
    rec_plan = nets.recognizer_plan(init="scaled")
    (d / "det.plan").write_bytes(det_plan)
    (d / "rec.plan").write_bytes(rec_plan)
    (d / "characters.txt").write_bytes((GOLD / "characters.txt").read_bytes())
    pages = {
        "letter": nets.letter_page(seed=5),
        "wide": nets.letter_page(lines=20, seed=9, width=2200, height=1700),
        # A quarter-turned page: its lines stand upright, tall and unsure.
        "upright": np.ascontiguousarray(np.rot90(nets.letter_page(lines=8, seed=3, width=900, height=700))),
    }
    for name, page in pages.items():
        write_ppm(d / f"{name}.ppm", page)
    return d, det_plan, rec_plan, pages


def run_worker(d: Path, names: list[str]) -> list[dict]:
    args = [str(WORKER), "--gpu", "--det", str(d / "det.plan"), "--rec", str(d / "rec.plan"), "--dict",
            str(d / "characters.txt"), *[str(d / f"{n}.ppm") for n in names]]
    print("worker:", " ".join(names), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, encoding="utf-8", timeout=180)
    assert r.returncode == 0, r.stderr
    assert "ppocr-native: running on" in r.stderr
    return [json.loads(line) for line in r.stdout.splitlines()]


@pytest.mark.gpu
def test_worker_equals_page_pipeline_and_vertical_pass(files):
    if not WORKER.exists():
        pytest.fail(f"{WORKER} is missing: build the package first")
    d, det_plan, rec_plan, pages = files
    dictionary = post.Dictionary.from_metadata((d / "characters.txt").read_text(encoding="utf-8"))
    names = list(pages)
    got = run_worker(d, names)
    assert [g["page"] for g in got] == [str(d / f"{n}.ppm") for n in names]
    pipe = PagePipeline(det_plan, rec_plan, dictionary, recognisers=1)
    rec = GpuModel.load(rec_plan)
    total_reread = 0
    try:
        for name, g in zip(names, got):
            page = pages[name]
            lines = pipe.read(page)
            assert len(g["lines"]) == len(lines) > 0, name
            replaced = 0
            for k, (gl, line) in enumerate(zip(g["lines"], lines)):
                quad = np.asarray(gl["quad"], np.float32).reshape(4, 2)
                assert np.array_equal(quad, line.quad), (name, k)
                text, score = line.text, line.score
                if rereads(line.quad, score):
                    total_reread += 1
                    turned = rotate_half(images.crop_text(page, line.quad))
                    x = images.rec_input(turned, 320)
                    rec.set_sizes([(48, x.shape[1])])
                    rec.lane_input_mut(0)[:] = x.reshape(-1)
                    rec.run()
                    t2, s2 = post.ctc_decode_pairs(rec.lane_output(0, 0), dictionary)
                    if reads_better(score, t2, s2):
                        text, score = t2, s2
                        replaced += 1
                assert gl["text"] == text and gl["score"] == score, (name, k, gl["text"], text)
            assert g["reoriented"] == replaced, name
    finally:
        pipe.close()
        rec.close()
    assert total_reread > 0  # the upright page exercises the vertical pass
