"""The three synthetic networks on the GPU against the CPU oracle.

Tolerances are the benchmark's: detector probabilities within 4e-5
absolute; recogniser probabilities within 1e-5 relative plus 1e-5 absolute;
CTC argmax classes bit-exact. The fused block is checked within
1e-5 * |y| + 1e-5. The recogniser also repeats the
reference's lane checks (tests/gpu.rs:39-84): lanes of different widths in
one run, and a lane run alone bit-identical to the same lane run beside
others.
"""
import numpy as np
import pytest

from ppocr_native_amd import GpuModel, nets

pytestmark = pytest.mark.gpu


def gpu_run(plan, images, sizes=None):
    g = GpuModel.load(plan)
    sizes = sizes or [im.shape[:2] for im in images]
    g.set_sizes(sizes)
    for i, im in enumerate(images):
        g.lane_input_mut(i)[:] = im.reshape(-1)
    g.run()
    out = [g.lane_output(i) for i in range(len(images))]
    g.close()
    return out


@pytest.mark.parametrize("init", ["baseline", "scaled"])
def test_fused_block(oracle, init):
    plan = nets.fused_block_plan(init=init)
    x = np.random.default_rng(5).uniform(-1, 1, (160, 160, 96)).astype(np.float32)
    got = gpu_run(plan, [x])[0]
    want = oracle.OracleModel(plan).run(x)[0]
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 1e-5 * np.abs(want) + 1e-5), err.max()


@pytest.mark.parametrize("init,h,w", [("scaled", 960, 960), ("baseline", 960, 960),
                                      ("scaled", 960, 736), ("scaled", 96, 2016)])
def test_detector(oracle, init, h, w):
    plan = nets.detector_plan(h=h, w=w, init=init)
    img = nets.page_image(h, w)
    got = gpu_run(plan, [img])[0]
    want = oracle.OracleModel(plan).run(img)[0]
    err = np.abs(got.astype(np.float64) - want)
    print(f"det {init} {h}x{w}: max |dp| {err.max():.3g}, mean p {want.mean():.4f}")
    assert got.shape == (h * w,)
    assert err.max() <= 4e-5


def check_rec(got, want):
    g, o = got.reshape(-1, 2), want.reshape(-1, 2)
    assert np.array_equal(g[:, 0], o[:, 0]), np.flatnonzero(g[:, 0] != o[:, 0])
    np.testing.assert_allclose(g[:, 1], o[:, 1], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("init,vocab", [("scaled", 18385), ("baseline", 18385),
                                         ("scaled", 18710)])
def test_recognizer_batch(oracle, init, vocab):
    # 18385 classes as benchmarked; 18710 is the shipped dictionary's count
    # (tests/parity.rs:217).
    plan = nets.recognizer_plan(init=init, vocab=vocab)
    lines = nets.line_images(16)
    got = gpu_run(plan, list(lines))
    m = oracle.OracleModel(plan)
    for i in range(16):
        check_rec(got[i], m.run(lines[i])[0])


@pytest.mark.parametrize("init", ["scaled", "baseline"])
def test_recognizer_logits(oracle, init):
    # The recogniser with its CTC head as a plain 1x1 layer: the 80 x 18385
    # logits of every line within 1e-5 relative plus 1e-5 absolute.
    plan = nets.recognizer_plan(init=init, logits=True)
    lines = nets.line_images(16)
    got = gpu_run(plan, list(lines))
    m = oracle.OracleModel(plan)
    worst = 0.0
    for i in range(16):
        want = m.run(lines[i])[0].astype(np.float64)
        assert got[i].shape == want.shape == (80 * 18385,)
        err = np.abs(got[i] - want)
        lim = 1e-5 * np.abs(want) + 1e-5
        assert (err <= lim).all(), f"line {i}: {(err > lim).sum()} logits outside, worst excess {(err - lim).max():.3g}"
        worst = max(worst, float((err / lim).max()))
    print(f"rec logits {init}: worst |d| / (1e-5 |y| + 1e-5) = {worst:.3f}")


def test_recognizer_lanes_of_different_widths(oracle):
    plan = nets.recognizer_plan(init="scaled", vocab=6625)
    rng = np.random.default_rng(3)
    widths = [640, 96, 1280]
    lines = [rng.uniform(-1, 1, (48, w, 3)).astype(np.float32) for w in widths]
    together = gpu_run(plan, lines)
    m = oracle.OracleModel(plan)
    for line, got in zip(lines, together):
        m.set_size(48, line.shape[1])
        check_rec(got, m.run(line)[0])
    # A lane alone gives the bits it gives beside others.
    alone = gpu_run(plan, [lines[1]])[0]
    assert np.array_equal(alone.view(np.uint32), together[1].view(np.uint32))


def test_same_width_lane_alone_matches_batch():
    plan = nets.recognizer_plan(init="scaled")
    lines = nets.line_images(5, seed=21)
    batch = gpu_run(plan, list(lines))
    for i in [0, 3]:
        alone = gpu_run(plan, [lines[i]])[0]
        assert np.array_equal(alone.view(np.uint32), batch[i].view(np.uint32))


def test_graph_replays_match_eager_run(oracle):
    # The first run launches eagerly; later runs replay the captured graph.
    # Every replay, with host work and synchronisation between them, must
    # give the eager run's bits; a resize records the graph again.
    plan = nets.recognizer_plan(init="scaled", vocab=6625)
    lines = nets.line_images(4, seed=31)
    g = GpuModel.load(plan)
    g.set_sizes([(48, 320)] * 4)
    for i in range(4):
        g.lane_input_mut(i)[:] = lines[i].reshape(-1)
    g.run()
    eager = [g.lane_output(i) for i in range(4)]
    m = oracle.OracleModel(plan)
    for i in range(4):
        check_rec(eager[i], m.run(lines[i])[0])
    for _ in range(4):
        g.lane_input_mut(0)[:] = lines[0].reshape(-1)  # host work between replays
        g.run()
        for i in range(4):
            assert np.array_equal(g.lane_output(i).view(np.uint32), eager[i].view(np.uint32))
    g.set_sizes([(48, 160)] * 2)
    for i in range(2):
        g.lane_input_mut(i)[:] = lines[i][:, :160].reshape(-1)
    outs = []
    for _ in range(3):
        g.run()
        outs.append([g.lane_output(i) for i in range(2)])
    m.set_size(48, 160)
    for i in range(2):
        check_rec(outs[0][i], m.run(np.ascontiguousarray(lines[i][:, :160]))[0])
        assert np.array_equal(outs[1][i], outs[0][i]) and np.array_equal(outs[2][i], outs[0][i])
    g.close()


def test_resize_between_runs(oracle):
    # set_sizes up, down and back on one model (src/engine/mod.rs:1496-1507).
    plan = nets.detector_plan(h=64, w=64, init="scaled")
    g = GpuModel.load(plan)
    m = oracle.OracleModel(plan)
    for h, w in [(128, 96), (32, 64), (64, 64), (96, 160)]:
        g.set_input_size(h, w)
        m.set_size(h, w)
        img = nets.page_image(h, w, seed=h + w)
        g.input_mut()[:] = img.reshape(-1)
        g.run()
        assert np.abs(g.output().astype(np.float64) - m.run(img)[0]).max() <= 4e-5
    with pytest.raises(Exception):
        g.set_input_size(48, 40)  # not a multiple of 32: the neck's sums disagree
    g.close()


def test_max_lanes_bounded_by_memory():
    # The lane bound follows the plan's size: a 960 x 960 detector lane holds
    # far more than a 48 x 320 line, so fewer of them fit; both leave room for
    # the worker's batches of 16, and asking for more than the bound is
    # refused with a message instead of failing in an allocation.
    det = GpuModel.load(nets.detector_plan(h=960, w=960))
    rec = GpuModel.load(nets.recognizer_plan())
    try:
        nd, nr = det.max_lanes(), rec.max_lanes()
        assert 16 <= nd < nr, (nd, nr)
        with pytest.raises(RuntimeError, match="more than the"):
            det.set_sizes([(960, 960)] * (nd + 1))
        rec.set_sizes([(48, 320)] * 16)
    finally:
        det.close()
        rec.close()
