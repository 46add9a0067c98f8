"""The near-tie bound of the CTC merge (ctc_merge in csrc/gemm.hip).

A column's logit is its bias plus ci products (src/engine/layers.rs:770-776:
the bias, then one fused multiply-add per input in order). Any order that
rounds once per addition lies within n u T of the exact sum, n = ci + 1,
u = 2^-24, T = |bias| + sum |w_i x_i|; so two orders lie within 2 n u T of
each other, and the merge, which needs two columns' differences (4 n u T),
tests against 8 n u T with T bounded by bias_max + wsum_max * max |x_i|.
These checks hold the error of several orders (the CPU's chain, its
reverse, random orders, and blocks of four products added together as an
MFMA step does) to n u T on inputs with heavy cancellation, against exact
sums, so a bound written too tight fails here."""
import math

import numpy as np
import pytest

U = 2.0 ** -24


def chain(bias, w, x, order):
    """One rounding per step: v = round(v + w_i x_i), the product exact."""
    v = np.float32(bias)
    for i in order:
        v = np.float32(float(v) + float(w[i]) * float(x[i]))
    return float(v)


def blocks_of_four(bias, w, x):
    """Each step adds four exact products at once (one rounding), the bias last."""
    v = 0.0
    for i in range(0, len(w), 4):
        v = float(np.float32(v + math.fsum(float(w[j]) * float(x[j]) for j in range(i, min(i + 4, len(w))))))
    return float(np.float32(v + float(bias)))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_orders_within_bound(seed):
    rng = np.random.default_rng(seed)
    ci = 120
    n = ci + 1
    worst = 0.0
    for trial in range(60):
        x = rng.normal(0, rng.choice([0.5, 3.0]), ci).astype(np.float32)
        w = rng.normal(0, 0.05, ci).astype(np.float32)
        if trial % 3 == 0:  # heavy cancellation: the products sum to about zero
            p = w.astype(np.float64) * x.astype(np.float64)
            w[-1] = np.float32(-(p[:-1].sum()) / float(x[-1])) if x[-1] != 0 else w[-1]
        bias = np.float32(rng.normal(0, 0.5))
        exact = math.fsum([float(bias)] + [float(a) * float(b) for a, b in zip(w, x)])
        T = abs(float(bias)) + sum(abs(float(a) * float(b)) for a, b in zip(w, x))
        orders = [range(ci), range(ci - 1, -1, -1)] + [rng.permutation(ci) for _ in range(3)]
        got = [chain(bias, w, x, o) for o in orders] + [blocks_of_four(bias, w, x)]
        for g in got:
            err = abs(g - exact)
            assert err <= n * U * T * (1 + 1e-6), (trial, err, n * U * T)
            worst = max(worst, err / (n * U * T))
        # Two orders: within 2 n u T of each other, a quarter of the merge's test.
        assert max(got) - min(got) <= 2 * n * U * T * (1 + 1e-6)
    assert worst > 0.0


def test_merge_bound_covers_column_bounds():
    # T of a row's column is at most bias_max + wsum_max * max |x_i|, the
    # per-model bounds the merge is given.
    rng = np.random.default_rng(7)
    ci, vocab = 120, 300
    w = rng.normal(0, 0.05, (ci, vocab)).astype(np.float32)
    bias = rng.normal(0, 0.5, vocab).astype(np.float32)
    bias_max = float(np.abs(bias).max())
    wsum_max = float(np.abs(w.astype(np.float64)).sum(axis=0).max())
    for _ in range(20):
        x = rng.normal(0, 2.0, ci).astype(np.float32)
        T = np.abs(bias.astype(np.float64)) + np.abs(w.astype(np.float64) * x[:, None]).sum(axis=0)
        assert T.max() <= bias_max + wsum_max * float(np.abs(x).max())
