"""The allocation-free channel mean (ppocr_hip_channel_mean_noalloc) against
the channel mean that allocates its workspace (ppocr_hip_channel_mean): the
same kernel, so the same bits, on two calls in a row (the second smaller),
and the size limit of its device scratch reported as an error."""
import numpy as np
import pytest

import ppocr_native_amd as P
from ppocr_native_amd.devmem import DeviceArray, synchronize

pytestmark = pytest.mark.gpu


def _both(x, pixels, c):
    dx, dy, dz = DeviceArray.of(x), DeviceArray(4 * c), DeviceArray(4 * c)
    print(f"channel mean without allocation: pixels {pixels}, channels {c}", flush=True)
    P.hip_channel_mean_noalloc(dx.addr, dz.addr, pixels, c)
    synchronize()
    P.hip_channel_mean(dx.addr, dy.addr, pixels, c)
    synchronize()
    return dz.download(c), dy.download(c)


def test_channel_mean_noalloc_matches(oracle):
    rng = np.random.default_rng(5)
    for pixels, c in [(3600, 480), (900, 96)]:
        x = rng.uniform(-1, 1, pixels * c).astype(np.float32)
        got, want = _both(x, pixels, c)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        np.testing.assert_allclose(got, oracle.channel_mean(x, pixels, c), rtol=1e-7, atol=1e-9)


def test_channel_mean_noalloc_limit():
    x = DeviceArray(4 * 8 * 4097)
    y = DeviceArray(4 * 4097)
    with pytest.raises(RuntimeError, match="4096"):
        P.hip_channel_mean_noalloc(x.addr, y.addr, 8, 4097)
