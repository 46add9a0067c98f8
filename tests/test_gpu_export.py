"""Plans written by the exporter (ppocr_native_amd.export) from ONNX graphs
built in tests/test_export.py, run on the GPU through the C ABI against the
CPU oracle: what an exported model would do once loaded. Detector outputs
within the benchmark's 4e-5; the recogniser's CTC argmax indices bit-exact
and its probabilities within 1e-5 * |cpu| + 1e-5.
"""
import numpy as np
import pytest

from ppocr_native_amd import GpuModel, export

import test_export as T

pytestmark = pytest.mark.gpu


def test_exported_detector(oracle):
    plan = export.export(T.detector_graph())
    x = T.hwc(np.random.default_rng(1).uniform(-1, 1, (1, 3, 64, 64))).astype(np.float32)
    want = oracle.OracleModel(plan).run(x)
    g = GpuModel.load(plan)
    g.input_mut()[:] = x.reshape(-1)
    g.run()
    got = [g.output(i) for i in range(len(want))]
    g.close()
    for a, b in zip(got, want):
        assert np.abs(a - b).max() <= 4e-5


def test_exported_recogniser(oracle):
    plan = export.export(T.recogniser_graph(), argmax=True)
    x = T.hwc(np.random.default_rng(2).uniform(-1, 1, (1, 3, 48, 320))).astype(np.float32)
    want = oracle.OracleModel(plan).run(x)[0].reshape(-1, 2)
    g = GpuModel.load(plan)
    g.input_mut()[:] = x.reshape(-1)
    g.run()
    got = g.output(0).reshape(-1, 2)
    g.close()
    assert np.array_equal(got[:, 0], want[:, 0])
    assert np.all(np.abs(got[:, 1] - want[:, 1]) <= 1e-5 * np.abs(want[:, 1]) + 1e-5)
