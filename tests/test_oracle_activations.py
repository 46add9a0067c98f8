"""The oracle's activations against libm / f64 closed forms.

Mirrors the reference's own known-answer tests:
sigmoid vs libm (src/engine/kernels/activation.rs:270-304), GELU vs the f64
error function and swish vs the exact product (src/engine/layers.rs:1098-1130),
and the hard sigmoid slopes (layers.rs:41-44, 212-226).
"""
import math

import numpy as np
import pytest


def inputs():
    v = [0.0, -0.0, 1e-40, -1e-40, 1e-30, -1e-30, 87.0, -87.0, 88.5, -88.5, 100.0, -100.0,
         float(np.finfo(np.float32).max), float(np.finfo(np.float32).min)]
    v += [(i - 2000.0) * 0.0517 for i in range(4000)]
    return np.array(v, np.float32)


def test_exp_neg_matches_libm(oracle):
    z = np.linspace(-87.0, 0.0, 20001, dtype=np.float32)
    got = np.array([oracle.exp_neg(float(v)) for v in z], np.float64)
    want = np.exp(z.astype(np.float64))
    rel = np.abs(got - want) / want
    assert rel.max() < 4 * np.finfo(np.float32).eps, rel.max()
    # Below the cutoff the result is exactly zero.
    assert oracle.exp_neg(-88.0) == 0.0 and oracle.exp_neg(-1000.0) == 0.0


def test_sigmoid_within_libm_bounds(oracle):
    x = inputs()
    got = oracle.act(x, "sigmoid").astype(np.float64)
    with np.errstate(over="ignore"):
        exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    gap = np.abs(got - exact)
    assert gap.max() <= 1e-7
    normal = exact >= np.finfo(np.float32).tiny
    assert np.all(gap[normal] <= 4 * np.finfo(np.float32).eps * exact[normal])
    ends = np.array([-np.inf, -100.0, 0.0, -0.0, 100.0, np.inf], np.float32)
    assert oracle.act(ends, "sigmoid").tolist() == [0.0, 0.0, 0.5, 0.5, 1.0, 1.0]


def test_gelu_against_erf(oracle):
    x = inputs()
    x = x[np.abs(x) < 1e6]
    got = oracle.act(x, "gelu").astype(np.float64)
    xd = x.astype(np.float64)
    want = xd * 0.5 * (1.0 + np.array([math.erf(v / math.sqrt(2.0)) for v in xd]))
    assert np.all(np.abs(got - want) <= 5e-7 * np.maximum(1.0, np.abs(xd)))


def test_swish_against_exact(oracle):
    x = inputs()
    x = x[np.abs(x) < 1e6]
    got = oracle.act(x, "swish").astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / (1.0 + np.exp(-xd))
    assert np.all(np.abs(got - want) <= 2e-6 * np.maximum(1.0, np.abs(xd)))


@pytest.mark.parametrize("name,slope", [("hardsigmoid", np.float32(0.16666670143604279)),
                                        ("hardsigmoidfifth", np.float32(0.2))])
def test_hard_sigmoids(oracle, name, slope):
    x = inputs()
    want = np.clip(x * slope + np.float32(0.5), 0.0, 1.0).astype(np.float32)
    assert np.array_equal(oracle.act(x, name), want)
    # Past the knees the clamp holds exactly; at zero it is one half.
    knee = np.float32(0.5) / slope * np.float32(1.001)
    got = oracle.act(np.array([-knee, knee, 0.0], np.float32), name).tolist()
    assert got == [0.0, 1.0, 0.5]


def test_hardswish_closed_form(oracle):
    x = inputs()
    sixth = np.float32(1.0 / 6.0)
    want = x * np.clip(x * sixth + np.float32(0.5), 0.0, 1.0)
    assert np.array_equal(oracle.act(x, "hardswish"), want.astype(np.float32))
    # x * relu6(x + 3) / 6 in f64 agrees to f32 rounding.
    xd = x.astype(np.float64)
    ref = xd * np.clip(xd + 3.0, 0.0, 6.0) / 6.0
    assert np.all(np.abs(oracle.act(x, "hardswish") - ref) <= 4e-7 * np.maximum(1.0, np.abs(xd)))


def test_relu_keeps_negative_zero(oracle):
    x = np.array([-1.0, -0.0, 0.0, 2.5, -np.inf, np.inf], np.float32)
    got = oracle.act(x, "relu")
    assert got.tolist() == [0.0, 0.0, 0.0, 2.5, 0.0, np.inf]
    assert np.signbit(got[1])


def test_softmax_rows(oracle):
    rng = np.random.default_rng(0)
    for n in [1, 7, 8, 9, 80, 497]:
        v = rng.normal(0, 3, n).astype(np.float32)
        got = oracle.softmax_row(v).astype(np.float64)
        e = np.exp(v.astype(np.float64) - v.max())
        assert np.allclose(got, e / e.sum(), rtol=2e-6, atol=1e-9)
