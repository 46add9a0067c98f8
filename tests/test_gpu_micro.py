"""The layer kernels on device memory (ppocr_hip_*) against the oracle at
the benchmark's microkernel sizes: add, mul and hard swish over
1x256x240x240; channel mean over 1x480x60x60; channel-broadcast multiply of
1x480x60x60; LayerNorm over [16x80, 120]; row argmax over [16x80, 18385].
torch provides the device memory only."""
import numpy as np
import pytest

import ppocr_native_amd as P

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available()
    return t


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def test_add_mul_hardswish(oracle, torch):
    rng = np.random.default_rng(0)
    n = 240 * 240 * 256
    a = rng.uniform(-1, 1, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    da, db, dy = dev(torch, a), dev(torch, b), torch.empty(n, device="cuda")
    P.hip_add(da.data_ptr(), db.data_ptr(), dy.data_ptr(), n)
    torch.cuda.synchronize()
    assert np.array_equal(host(dy), oracle.add(a, b))
    P.hip_mul(da.data_ptr(), db.data_ptr(), dy.data_ptr(), n)
    torch.cuda.synchronize()
    assert np.array_equal(host(dy), oracle.mul(a, b))
    P.hip_activation(da.data_ptr(), dy.data_ptr(), n, 7)
    torch.cuda.synchronize()
    assert np.array_equal(host(dy), oracle.act(a, "hardswish"))
    P.hip_add(da.data_ptr(), db.data_ptr(), dy.data_ptr(), n, 4)  # with swish folded
    torch.cuda.synchronize()
    assert np.array_equal(host(dy), oracle.add(a, b, "swish"))


@pytest.mark.parametrize("pixels,c", [(3600, 480), (25600, 96), (7, 3)])
def test_channel_mean(oracle, torch, pixels, c):
    x = np.random.default_rng(1).uniform(-1, 1, pixels * c).astype(np.float32)
    dx, dy = dev(torch, x), torch.empty(c, device="cuda")
    P.hip_channel_mean(dx.data_ptr(), dy.data_ptr(), pixels, c)
    torch.cuda.synchronize()
    want = oracle.channel_mean(x, pixels, c)
    # f64 sums in another order: equal after rounding to f32 but for a tie.
    np.testing.assert_allclose(host(dy), want, rtol=1e-7, atol=1e-9)


def test_channel_mul(oracle, torch):
    rng = np.random.default_rng(2)
    x = rng.uniform(-1, 1, 3600 * 480).astype(np.float32)
    g = rng.uniform(-1, 1, 480).astype(np.float32)
    dx, dg, dy = dev(torch, x), dev(torch, g), torch.empty(x.size, device="cuda")
    P.hip_channel_mul(dx.data_ptr(), dg.data_ptr(), dy.data_ptr(), 3600, 480)
    torch.cuda.synchronize()
    assert np.array_equal(host(dy), oracle.channel_mul(x, g, 3600, 480))


def test_layer_norm(oracle, torch):
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, 1280 * 120).astype(np.float32)
    w = np.concatenate([rng.normal(1, 0.1, 120), rng.normal(0, 0.1, 120), [1e-6]]).astype(np.float32)
    dx, dw, dy = dev(torch, x), dev(torch, w), torch.empty(x.size, device="cuda")
    P.hip_layer_norm(dx.data_ptr(), dw.data_ptr(), dy.data_ptr(), 1280, 120)
    torch.cuda.synchronize()
    assert np.array_equal(host(dy), oracle.layer_norm(x, w, 1280, 120))


def test_row_argmax(oracle, torch):
    rng = np.random.default_rng(4)
    rows, cols = 1280, 18385
    x = rng.normal(0, 3, rows * cols).astype(np.float32)
    x[5 * cols + 17] = x[5 * cols + 18000] = 40.0  # a tie: the first column wins
    dx, dy = dev(torch, x), torch.empty(2 * rows, device="cuda")
    P.hip_row_argmax(dx.data_ptr(), dy.data_ptr(), rows, cols)
    torch.cuda.synchronize()
    got = host(dy).reshape(rows, 2)
    want = oracle.row_argmax(x, rows, cols).reshape(rows, 2)
    assert np.array_equal(got[:, 0], want[:, 0])
    assert got[5, 0] == 17
    np.testing.assert_allclose(got[:, 1], want[:, 1], rtol=1e-5, atol=1e-5)
