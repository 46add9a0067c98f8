"""The layer kernels on device memory (ppocr_hip_*) against the oracle at
the benchmark's microkernel sizes: add, mul and hard swish over
1x256x240x240; channel mean over 1x480x60x60; channel-broadcast multiply of
1x480x60x60; LayerNorm over [16x80, 120]; row argmax over [16x80, 18385]."""
import numpy as np
import pytest

import ppocr_native_amd as P
from ppocr_native_amd.devmem import DeviceArray, synchronize

pytestmark = pytest.mark.gpu


def test_add_mul_hardswish(oracle):
    rng = np.random.default_rng(0)
    n = 240 * 240 * 256
    a = rng.uniform(-1, 1, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    da, db, dy = DeviceArray.of(a), DeviceArray.of(b), DeviceArray(4 * n)
    P.hip_add(da.addr, db.addr, dy.addr, n)
    synchronize()
    assert np.array_equal(dy.download(n), oracle.add(a, b))
    P.hip_mul(da.addr, db.addr, dy.addr, n)
    synchronize()
    assert np.array_equal(dy.download(n), oracle.mul(a, b))
    P.hip_activation(da.addr, dy.addr, n, 7)
    synchronize()
    assert np.array_equal(dy.download(n), oracle.act(a, "hardswish"))
    P.hip_add(da.addr, db.addr, dy.addr, n, 4)  # with swish folded
    synchronize()
    assert np.array_equal(dy.download(n), oracle.add(a, b, "swish"))


def test_odd_length_add(oracle):
    rng = np.random.default_rng(9)
    n = 1001
    a = rng.uniform(-1, 1, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    da, db, dy = DeviceArray.of(a), DeviceArray.of(b), DeviceArray(4 * n)
    P.hip_add(da.addr, db.addr, dy.addr, n, 1)
    synchronize()
    assert np.array_equal(dy.download(n), oracle.add(a, b, "relu"))


@pytest.mark.parametrize("pixels,c", [(3600, 480), (25600, 96), (7, 3)])
def test_channel_mean(oracle, pixels, c):
    x = np.random.default_rng(1).uniform(-1, 1, pixels * c).astype(np.float32)
    dx, dy = DeviceArray.of(x), DeviceArray(4 * c)
    P.hip_channel_mean(dx.addr, dy.addr, pixels, c)
    synchronize()
    want = oracle.channel_mean(x, pixels, c)
    # f64 sums in another order: equal after rounding to f32 but for a tie.
    np.testing.assert_allclose(dy.download(c), want, rtol=1e-7, atol=1e-9)


def test_channel_mul(oracle):
    rng = np.random.default_rng(2)
    x = rng.uniform(-1, 1, 3600 * 480).astype(np.float32)
    g = rng.uniform(-1, 1, 480).astype(np.float32)
    dx, dg, dy = DeviceArray.of(x), DeviceArray.of(g), DeviceArray(x.nbytes)
    P.hip_channel_mul(dx.addr, dg.addr, dy.addr, 3600, 480)
    synchronize()
    assert np.array_equal(dy.download(x.size), oracle.channel_mul(x, g, 3600, 480))


def test_layer_norm(oracle):
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, 1280 * 120).astype(np.float32)
    w = np.concatenate([rng.normal(1, 0.1, 120), rng.normal(0, 0.1, 120), [1e-6]]).astype(np.float32)
    dx, dw, dy = DeviceArray.of(x), DeviceArray.of(w), DeviceArray(x.nbytes)
    P.hip_layer_norm(dx.addr, dw.addr, dy.addr, 1280, 120)
    synchronize()
    assert np.array_equal(dy.download(x.size), oracle.layer_norm(x, w, 1280, 120))


def test_row_argmax(oracle):
    rng = np.random.default_rng(4)
    rows, cols = 1280, 18385
    x = rng.normal(0, 3, rows * cols).astype(np.float32)
    x[5 * cols + 17] = x[5 * cols + 18000] = 40.0  # a tie: the first column wins
    dx, dy = DeviceArray.of(x), DeviceArray(8 * rows)
    P.hip_row_argmax(dx.addr, dy.addr, rows, cols)
    synchronize()
    got = dy.download(2 * rows).reshape(rows, 2)
    want = oracle.row_argmax(x, rows, cols).reshape(rows, 2)
    assert np.array_equal(got[:, 0], want[:, 0])
    assert got[5, 0] == 17
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rows,cols", [(7, 1), (5, 3), (9, 6), (11, 101), (6, 8199), (3, 20000)])
def test_row_argmax_ragged(oracle, rows, cols):
    # Rows whose starts fall on every 4-byte phase of a 16-byte boundary, so
    # the aligned middle, the head and the tail each take every length; a tie
    # in the head, the middle and the tail of three rows.
    rng = np.random.default_rng(cols)
    x = rng.normal(0, 3, rows * cols).astype(np.float32)
    for r, c in ((0, 0), (1, cols // 2), (2, cols - 1)):
        x[r * cols + c] = x[r * cols + max(0, c - 1)] = 40.0
    dx, dy = DeviceArray.of(x), DeviceArray(8 * rows)
    P.hip_row_argmax(dx.addr, dy.addr, rows, cols)
    synchronize()
    got = dy.download(2 * rows).reshape(rows, 2)
    want = oracle.row_argmax(x, rows, cols).reshape(rows, 2)
    assert np.array_equal(got[:, 0], want[:, 0])
    for r, c in ((0, 0), (1, cols // 2), (2, cols - 1)):
        assert got[r, 0] == max(0, c - 1)
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n", [320 * 320, 1001])
def test_db_mask_gives_the_boxes(n):
    # The DB threshold on the GPU, bytes out; on the reference's own map it
    # gives the mask boxes_from_prob thresholds on the host, and so the same
    # 11 boxes (tests/golden/prob.npy).
    from pathlib import Path
    from ppocr_native_amd import post
    gold = Path(__file__).resolve().parent / "golden"
    prob = np.load(gold / "prob.npy", allow_pickle=False).reshape(-1)[:n].copy()
    prob[:8] = np.float32(0.3)  # on the threshold: not text
    dp, dm = DeviceArray.of(prob), DeviceArray(n)
    P.lib().ppocr_hip_db_mask(dp.addr, dm.addr, n, 0.3, None)
    synchronize()
    mask = dm.download(n, np.uint8)
    assert np.array_equal(mask, (prob > np.float32(0.3)).astype(np.uint8))
    if n == 320 * 320:
        full = np.load(gold / "prob.npy", allow_pickle=False)
        dp2 = DeviceArray.of(full.reshape(-1).copy())
        P.lib().ppocr_hip_db_mask(dp2.addr, dm.addr, n, 0.3, None)
        synchronize()
        got = post.boxes_from_prob(full, 320, 320, 325, 323, mask=dm.download(n, np.uint8))
        assert np.array_equal(post.boxes_from_prob(full, 320, 320, 325, 323), got)
        assert got.shape == (11, 4, 2)


@pytest.mark.parametrize("n", [240 * 240 * 256, 4 * 1000 + 4 * 513])
def test_copy_through_lds(n):
    # The counters' calibration copy by direct-to-LDS loads: every float in
    # place, a partial last block included.
    x = np.random.default_rng(3).uniform(-1, 1, n).astype(np.float32)
    dx, dy = DeviceArray.of(x), DeviceArray(4 * n)
    P.hip_copy_lds(dx.addr, dy.addr, n)
    synchronize()
    assert np.array_equal(dy.download(n).view(np.uint32), x.view(np.uint32))
