"""The recogniser's transformer encoder on the GPU, through the C ABI,
against the CPU oracle: pre-norm blocks (LayerNorm, q|k|v 1x1, attention,
output 1x1 + residual, LayerNorm, MLP + residual) and the final LayerNorm,
as the fused steps run them: ln_linear, then attention_block (attention,
projection, residual, the MLP and the next LayerNorm folded in); with the
attention's sum read elsewhere too, attention_proj and ln_mlp apart; for
lines too long for the fused attention's LDS, the attention rows, the
projection and the MLP as three launches.

The 1x1 layers' sums run on the MFMA units and the fused LayerNorm's
statistics are 32-lane butterfly sums, both in another order than the
CPU's: every output within 1e-5 * |cpu| + 1e-5, the benchmark's tolerance
for the recogniser's logits.
"""
import numpy as np
import pytest

from ppocr_native_amd import GpuModel
from ppocr_native_amd.planfile import PlanBuilder

pytestmark = pytest.mark.gpu


def near(got, want, rtol=1e-5, atol=1e-5):
    """|gpu - cpu| <= rtol * |cpu| + atol, element by element."""
    for a, b in zip(got, want):
        assert a.shape == b.shape
        err = np.abs(a.astype(np.float64) - b)
        lim = rtol * np.abs(b) + atol
        bad = np.flatnonzero(err > lim)
        assert bad.size == 0, (f"{bad.size} of {err.size} outside, worst excess "
                               f"{float((err - lim).max()):.3g}, max |cpu| {float(np.abs(b).max()):.3g}")


def encoder_plan(t, c, heads, hidden, depth, act, seed, expose=False):
    """`depth` pre-norm blocks over 1 x t x c rows and a final LayerNorm;
    `expose`: each attention sum is a plan output too."""
    rng = np.random.default_rng(seed)
    b = PlanBuilder(1, t, c)

    def ln(x):
        return b.layernorm(x, rng.normal(1.0, 0.1, c).astype(np.float32),
                           rng.normal(0.0, 0.1, c).astype(np.float32), 1e-6)

    def w(ci, co):
        return rng.normal(0, 1 / np.sqrt(ci), (1, 1, ci, co)).astype(np.float32)

    def bias(co):
        return rng.normal(0, 0.1, co).astype(np.float32)

    z = b.input
    scale = float(np.float32((c // heads) ** -0.5))
    sums = []
    for _ in range(depth):
        qkv = b.conv(ln(z), w(c, 3 * c), bias(3 * c))
        a = b.attention(qkv, heads, scale)
        z = b.add(z, b.conv(a, w(c, c), bias(c)))
        sums.append(z)
        f = b.conv(ln(z), w(c, hidden), bias(hidden), fused=act)
        z = b.add(z, b.conv(f, w(hidden, c), bias(c)))
    return b.to_bytes([ln(z)] + (sums if expose else []))


def run_both(plan, t, c, lanes, oracle, seed=3, outs=1):
    """Every output of every lane, GPU and oracle, flattened in that order."""
    rng = np.random.default_rng(seed)
    xs = [rng.uniform(-1, 1, (1, t, c)).astype(np.float32) for _ in range(lanes)]
    g = GpuModel.load(plan)
    g.set_sizes([(1, t)] * lanes)
    for i, x in enumerate(xs):
        g.lane_input_mut(i)[:] = x.reshape(-1)
    g.run()
    got = [g.lane_output(i, k) for i in range(lanes) for k in range(outs)]
    names = [n for n, _ in g.launches()]
    g.close()
    m = oracle.OracleModel(plan)
    return got, [o for x in xs for o in m.run(x)[:outs]], names


@pytest.mark.parametrize("t,lanes", [(80, 16), (41, 3), (9, 2), (100, 2)])
def test_encoder_fused(oracle, t, lanes):
    # The recogniser's encoder: width 120, 8 heads of 15, MLP 240 with swish.
    plan = encoder_plan(t, 120, 8, 240, 2, "swish", seed=t)
    got, want, names = run_both(plan, t, 120, lanes, oracle)
    assert names == ["ln_linear", "attention_block"] * 2, names
    near(got, want)


def test_encoder_sum_read_elsewhere(oracle):
    # The attention's sum is an output too: attention_proj stores it and
    # ln_mlp reads it back.
    plan = encoder_plan(80, 120, 8, 240, 2, "swish", seed=2, expose=True)
    got, want, names = run_both(plan, 80, 120, 4, oracle, outs=3)
    assert names == ["ln_linear", "attention_proj", "ln_mlp"] * 2, names
    near(got, want)


def test_encoder_long_line(oracle):
    # 130 steps: K and V of the line overflow LDS; attention rows to the
    # workspace, the projection with the residual, then the MLP.
    plan = encoder_plan(130, 120, 8, 240, 2, "swish", seed=5)
    got, want, names = run_both(plan, 130, 120, 2, oracle)
    assert names == ["ln_linear", "attention", "ln_linear", "ln_mlp"] * 2, names
    near(got, want)


def test_encoder_long_line_sum_read_elsewhere(oracle):
    # 130 steps with each attention sum an output: the attention rows go to
    # the workspace and the score spill sits right after them (the workspace
    # holds no second sum here), then the projection, then the MLP.
    plan = encoder_plan(130, 120, 8, 240, 2, "swish", seed=6, expose=True)
    got, want, names = run_both(plan, 130, 120, 2, oracle, outs=3)
    assert names == ["ln_linear", "attention", "ln_linear", "ln_mlp"] * 2, names
    near(got, want)


@pytest.mark.parametrize("c,heads,hidden,act", [(64, 4, 128, "gelu"), (32, 2, 96, "hardswish"),
                                                (96, 8, 200, "relu")])
def test_encoder_widths(oracle, c, heads, hidden, act):
    # Other widths: 64 (heads of 16), 32 and 96 (12 per head, 200 hidden).
    plan = encoder_plan(37, c, heads, hidden, 2, act, seed=c)
    got, want, names = run_both(plan, 37, c, 3, oracle)
    assert names == ["ln_linear", "attention_block"] * 2, names
    near(got, want)
