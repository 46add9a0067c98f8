"""The synthetic networks on the oracle: their shapes follow the benchmark's
configurations, and the scaled initialisation is well conditioned, so that a
fixed tolerance between two summation orders is meaningful.

A one-ulp relative change of every input value moves the scaled detector's
probabilities by far less than the 4e-5 the GPU must meet; a network that
amplified it past 4e-5 would make that bound test the network rather than
the kernels.
"""
import numpy as np

from ppocr_native_amd import nets


def one_ulp(img, seed=0):
    rng = np.random.default_rng(seed)
    return (img * (1 + rng.choice([-1, 1], img.shape) * 2.0 ** -24)).astype(np.float32)


def test_detector_shapes_and_conditioning(oracle):
    m = oracle.OracleModel(nets.detector_plan(h=256, w=256, init="scaled"))
    img = nets.page_image(256, 256)
    a = m.run(img)[0]
    assert a.shape == (256 * 256,)
    assert 0.05 < a.std() < 0.45 and 0.0 <= a.min() and a.max() <= 1.0
    b = m.run(one_ulp(img))[0]
    assert np.abs(a.astype(np.float64) - b).max() < 4e-6
    kinds = {o["kind"] for o in m.ops()}
    assert kinds >= {"conv", "dwconv", "maxpool", "mean", "channelmul", "add", "upsample",
                     "upsampleadd", "concatc", "convtranspose"}
    last = m.ops()[-1]
    assert (last["oh"], last["ow"], last["oc"], last["fused"]) == (256, 256, 1, "sigmoid")


def test_recognizer_shapes(oracle):
    m = oracle.OracleModel(nets.recognizer_plan(init="scaled"))
    head = m.ops()[-1]
    assert head["kind"] == "ctcargmax" and head["iw"] == 80 and head["n2"] == 18385
    attn = [o for o in m.ops() if o["kind"] == "attention"]
    assert len(attn) == 2 and attn[0]["oc"] == 120 and attn[0]["n2"] == 8
    out = m.run(nets.line_images(1)[0])[0].reshape(80, 2)
    assert np.all((out[:, 0] >= 0) & (out[:, 0] < 18385))
    assert len(set(out[:, 0].astype(int).tolist())) > 5  # not one class everywhere
    assert np.all((out[:, 1] > 0) & (out[:, 1] <= 1))


def test_block_shape(oracle):
    m = oracle.OracleModel(nets.fused_block_plan())
    kinds = [o["kind"] for o in m.ops()]
    assert kinds == ["dwconv", "mean", "conv", "conv", "channelmul", "conv", "add"]
    assert m.ops()[0]["fused"] == "hardswish" and m.input_shape() == (160, 160, 96)
