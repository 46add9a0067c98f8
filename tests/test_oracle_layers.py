"""Every layer of the oracle against an independent f64 restatement in numpy,
on small seeded shapes (the method of the reference's layer tests,
src/engine/layers.rs:1143-1319 and kernels/*: each layer against its f64
definition). Each reference below indexes the data its own way (padded
arrays, einsum, explicit windows) so that a dropped term, a wrong sign,
a transposed operand or an off-by-one window fails the comparison;
`test_checks_have_teeth` plants such mistakes and checks they are caught.
"""
import numpy as np
import pytest

from ppocr_native_amd.planfile import PlanBuilder

RNG = np.random.default_rng(1234)


def run1(build, x, oracle):
    """Build a plan of `build(b, input)` over HWC input x; run on the oracle."""
    h, w, c = x.shape
    b = PlanBuilder(h, w, c)
    out = build(b, b.input)
    outs = out if isinstance(out, list) else [out]
    m = oracle.OracleModel(b.to_bytes(outs))
    got = m.run(x)
    return got, outs


def ref_conv(x, w, bias, s, pad, x2=None):
    """Dense conv in f64: x [H][W][C], w [kh][kw][C(+C2)][oc]."""
    if x2 is not None:
        x = np.concatenate([x, x2], axis=2)
    x = x.astype(np.float64)
    kh, kw, ci, oc = w.shape
    pt, pb, pl, pr = pad
    xp = np.zeros((x.shape[0] + pt + pb, x.shape[1] + pl + pr, ci))
    xp[pt:pt + x.shape[0], pl:pl + x.shape[1]] = x
    oh = (xp.shape[0] - kh) // s[0] + 1
    ow = (xp.shape[1] - kw) // s[1] + 1
    y = np.zeros((oh, ow, oc))
    for ky in range(kh):
        for kx in range(kw):
            patch = xp[ky:ky + s[0] * (oh - 1) + 1:s[0], kx:kx + s[1] * (ow - 1) + 1:s[1]]
            y += np.einsum("hwc,co->hwo", patch, w[ky, kx].astype(np.float64))
    if bias is not None:
        y += bias
    return y


def ref_dw(x, w, bias, s, pad):
    x = x.astype(np.float64)
    kh, kw, c = w.shape
    pt, pb, pl, pr = pad
    xp = np.zeros((x.shape[0] + pt + pb, x.shape[1] + pl + pr, c))
    xp[pt:pt + x.shape[0], pl:pl + x.shape[1]] = x
    oh = (xp.shape[0] - kh) // s[0] + 1
    ow = (xp.shape[1] - kw) // s[1] + 1
    y = np.zeros((oh, ow, c)) + (bias if bias is not None else 0)
    for ky in range(kh):
        for kx in range(kw):
            y += xp[ky:ky + s[0] * (oh - 1) + 1:s[0], kx:kx + s[1] * (ow - 1) + 1:s[1]] * w[ky, kx]
    return y


def close(got, want, rtol=2e-5, atol=2e-5):
    want = np.asarray(want, np.float64).reshape(-1)
    got = np.asarray(got, np.float64).reshape(-1)
    scale = max(1.0, np.abs(want).max())
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol * scale)


@pytest.mark.parametrize("k,s,pad", [((3, 3), (1, 1), (1, 1, 1, 1)), ((3, 3), (2, 2), (1, 1, 1, 1)),
                                     ((2, 2), (1, 1), (0, 1, 0, 1)), ((1, 3), (1, 1), (0, 0, 1, 1)),
                                     ((5, 5), (2, 1), (2, 2, 2, 2))])
def test_conv_windowed(oracle, k, s, pad):
    x = RNG.uniform(-1, 1, (9, 11, 5)).astype(np.float32)
    w = RNG.normal(0, 0.3, (k[0], k[1], 5, 7)).astype(np.float32)
    bias = RNG.normal(0, 0.3, 7).astype(np.float32)
    got, _ = run1(lambda b, t: b.conv(t, w, bias, k=k, s=s, pad=pad), x, oracle)
    close(got[0], ref_conv(x, w, bias, s, pad))


def test_conv_two_inputs(oracle):
    x = RNG.uniform(-1, 1, (6, 7, 4)).astype(np.float32)
    x2v = RNG.uniform(-1, 1, (6, 7, 3)).astype(np.float32)
    w = RNG.normal(0, 0.3, (3, 3, 7, 8)).astype(np.float32)
    bias = RNG.normal(0, 0.3, 8).astype(np.float32)

    def build(b, t):
        other = b.conv(t, np.eye(4, 3, dtype=np.float32).reshape(1, 1, 4, 3), None)
        return b.conv(t, w, bias, k=(3, 3), pad=(1, 1, 1, 1), x2=other)

    got, _ = run1(build, x, oracle)
    # The second input is a 1x1 projection of x: channels 0..2 of x.
    close(got[0], ref_conv(x, w, bias, (1, 1), (1, 1, 1, 1), x2=x[:, :, :3]))


@pytest.mark.parametrize("co", [16, 12, 48])
def test_pointwise_bias_rules(oracle, co):
    # Row groups of ceil(48 / ow) rows; bias first except the last count % 4
    # pixels when co % 16 == 0, bias last otherwise.
    x = RNG.uniform(-1, 1, (7, 5, 9)).astype(np.float32)
    w = RNG.normal(0, 0.3, (1, 1, 9, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    got, _ = run1(lambda b, t: b.conv(t, w, bias), x, oracle)
    close(got[0], ref_conv(x, w, bias, (1, 1), (0, 0, 0, 0)))
    # Exact f32 restatement of the order: per pixel, fma chain then bias.
    xf = x.reshape(-1, 9)
    rows = min(-(-48 // 5), 7)
    y = got[0].reshape(-1, co)
    for p in range(xf.shape[0]):
        group_start = (p // (rows * 5)) * rows * 5
        count = min(rows * 5, xf.shape[0] - group_start)
        first = co % 16 == 0 and (p - group_start) < count // 4 * 4
        for j in range(0, co, 5):
            acc = np.float32(bias[j]) if first else np.float32(0)
            for i in range(9):
                if j < co // 8 * 8:  # fused multiply-add
                    acc = np.float32(np.float64(w[0, 0, i, j]) * np.float64(xf[p, i]) + np.float64(acc))
                else:                # the tail columns: product, then sum
                    acc = np.float32(acc + np.float32(xf[p, i] * w[0, 0, i, j]))
            if not first:
                acc = np.float32(acc + bias[j])
            assert y[p, j] == acc, (p, j)


@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (5, 1), (5, 2), (7, 1)])
def test_depthwise(oracle, k, s):
    x = RNG.uniform(-1, 1, (10, 13, 8)).astype(np.float32)
    w = RNG.normal(0, 0.3, (k, k, 8)).astype(np.float32)
    bias = RNG.normal(0, 0.3, 8).astype(np.float32)
    p = (k - 1) // 2
    got, _ = run1(lambda b, t: b.dwconv(t, w, bias, k=(k, k), s=(s, s)), x, oracle)
    close(got[0], ref_dw(x, w, bias, (s, s), (p, p, p, p)))


@pytest.mark.parametrize("fused", ["relu", "sigmoid", "gelu", "swish", "hardsigmoid",
                                   "hardsigmoidfifth", "hardswish"])
def test_folded_activation_equals_applied_after(oracle, fused):
    # The folded tail gives the bits of the activation applied on its own
    # (src/engine/schedule.rs:1123-1195).
    x = RNG.uniform(-1, 1, (5, 6, 8)).astype(np.float32)
    w = RNG.normal(0, 0.5, (3, 3, 8)).astype(np.float32)
    plain, _ = run1(lambda b, t: b.dwconv(t, w, None, k=(3, 3)), x, oracle)
    folded, _ = run1(lambda b, t: b.dwconv(t, w, None, k=(3, 3), fused=fused), x, oracle)
    assert np.array_equal(folded[0], oracle.act(plain[0], fused))


def test_maxpool_cut_window(oracle):
    x = RNG.uniform(-1, 1, (5, 6, 3)).astype(np.float32)
    got, _ = run1(lambda b, t: b.maxpool(t), x, oracle)
    xp = np.full((6, 7, 3), -np.inf, np.float32)
    xp[:5, :6] = x
    want = np.maximum(np.maximum(xp[:5, :6], xp[1:, :6]), np.maximum(xp[:5, 1:], xp[1:, 1:]))
    assert np.array_equal(got[0], want.reshape(-1))


def test_avgpool(oracle):
    x = RNG.uniform(-1, 1, (3, 8, 4)).astype(np.float32)
    got, _ = run1(lambda b, t: b.avgpool(t, (3, 2), (3, 2)), x, oracle)
    want = x.astype(np.float64).reshape(1, 3, 4, 2, 4).mean(axis=(1, 3))
    close(got[0], want, rtol=1e-6, atol=1e-6)


def test_upsample_concat_add(oracle):
    x = RNG.uniform(-1, 1, (3, 4, 4)).astype(np.float32)

    def build(b, t):
        up = b.upsample(t, 2)
        big = b.conv(up, np.eye(4, dtype=np.float32).reshape(1, 1, 4, 4), None)
        ua = b.upsampleadd(t, big, 2)
        cat = b.concat(ua, up)
        return [up, ua, cat]

    got, _ = run1(build, x, oracle)
    up = x.repeat(2, 0).repeat(2, 1)
    assert np.array_equal(got[0], up.reshape(-1))
    assert np.array_equal(got[1], (up + up).reshape(-1))
    assert np.array_equal(got[2], np.concatenate([up + up, up], axis=2).reshape(-1))


def test_mean_gate_and_residual(oracle):
    x = RNG.uniform(-1, 1, (30, 40, 6)).astype(np.float32)

    def build(b, t):
        m = b.mean(t)
        g = b.conv(m, np.eye(6, dtype=np.float32).reshape(1, 1, 6, 6), None)
        cm = b.channelmul(t, g)
        return [m, b.add(t, cm, fused="relu")]

    got, _ = run1(build, x, oracle)
    mean = x.astype(np.float64).mean(axis=(0, 1))
    assert np.array_equal(got[0], mean.astype(np.float32))
    want = np.maximum(x + x * mean.astype(np.float32), 0)
    assert np.array_equal(got[1], want.reshape(-1).astype(np.float32))


def test_layernorm(oracle):
    x = RNG.normal(0, 2, (1, 10, 120)).astype(np.float32)
    gamma = RNG.normal(1, 0.1, 120).astype(np.float32)
    beta = RNG.normal(0, 0.1, 120).astype(np.float32)
    got, _ = run1(lambda b, t: b.layernorm(t, gamma, beta, 1e-6), x, oracle)
    xd = x.astype(np.float64)
    mu = xd.mean(-1, keepdims=True)
    var = ((xd - mu) ** 2).mean(-1, keepdims=True)
    close(got[0], (xd - mu) / np.sqrt(var + 1e-6) * gamma + beta, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("t,heads,hd", [(9, 2, 3), (80, 8, 15), (17, 4, 8)])
def test_attention(oracle, t, heads, hd):
    c = heads * hd
    x = RNG.normal(0, 1, (1, t, 3 * c)).astype(np.float32)
    scale = float(np.float32(hd ** -0.5))
    got, _ = run1(lambda b, tt: b.attention(tt, heads, scale), x, oracle)
    xd = x[0].astype(np.float64)
    out = np.zeros((t, c))
    for h in range(heads):
        q = xd[:, h * hd:(h + 1) * hd] * scale
        k = xd[:, c + h * hd:c + (h + 1) * hd]
        v = xd[:, 2 * c + h * hd:2 * c + (h + 1) * hd]
        s = q @ k.T
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[:, h * hd:(h + 1) * hd] = p @ v
    close(got[0], out, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("vocab", [37, 48, 18385])
def test_ctc_argmax(oracle, vocab):
    t, ci = 12, 24
    x = RNG.normal(0, 1, (1, t, ci)).astype(np.float32)
    w = RNG.normal(0, 0.5, (ci, vocab)).astype(np.float32)
    bias = RNG.normal(0, 0.5, vocab).astype(np.float32)
    got, _ = run1(lambda b, tt: b.ctcargmax(tt, w, bias), x, oracle)
    logits = x[0].astype(np.float64) @ w.astype(np.float64) + bias
    best = got[0].reshape(t, 2)
    assert np.array_equal(best[:, 0].astype(int), logits.argmax(1))
    e = np.exp(logits - logits.max(1, keepdims=True))
    np.testing.assert_allclose(best[:, 1], 1.0 / e.sum(1), rtol=2e-5)


def test_row_argmax_ties_take_first(oracle):
    x = RNG.normal(0, 3, (6, 100)).astype(np.float32)
    x[0, 10] = x[0, 90] = 50.0
    x[1, 3] = x[1, 19] = x[1, 35] = 50.0  # tie across lanes and panels
    x[2, :] = 1.0                          # all equal: the first column
    y = oracle.row_argmax(x, 6, 100).reshape(6, 2)
    assert y[:, 0].astype(int).tolist()[:3] == [10, 3, 0]
    assert np.array_equal(y[3:, 0].astype(int), x[3:].argmax(1))
    assert abs(y[2, 1] - 0.01) < 1e-8


def test_convtranspose(oracle):
    x = RNG.uniform(-1, 1, (4, 5, 6)).astype(np.float32)
    w = RNG.normal(0, 0.3, (6, 2, 2, 3)).astype(np.float32)
    bias = RNG.normal(0, 0.3, 3).astype(np.float32)
    got, _ = run1(lambda b, t: b.convtranspose(t, w, bias, k=(2, 2), fused="relu"), x, oracle)
    want = np.einsum("hwc,cyxo->hywxo", x.astype(np.float64), w.astype(np.float64)) + bias
    want = np.maximum(want.reshape(8, 10, 3), 0)
    close(got[0], want)


def test_checks_have_teeth(oracle):
    # A transposed kernel, a dropped bias and a one-pixel shift each fail the
    # comparison the conv test above makes.
    x = RNG.uniform(-1, 1, (9, 11, 5)).astype(np.float32)
    w = RNG.normal(0, 0.3, (3, 3, 5, 7)).astype(np.float32)
    bias = RNG.normal(0, 0.3, 7).astype(np.float32)
    got, _ = run1(lambda b, t: b.conv(t, w, bias, k=(3, 3), pad=(1, 1, 1, 1)), x, oracle)
    good = ref_conv(x, w, bias, (1, 1), (1, 1, 1, 1))
    close(got[0], good)
    for bad in [ref_conv(x, w.transpose(1, 0, 2, 3).copy(), bias, (1, 1), (1, 1, 1, 1)),
                ref_conv(x, w, None, (1, 1), (1, 1, 1, 1)),
                ref_conv(x, w, bias, (1, 1), (0, 2, 1, 1))]:
        with pytest.raises(AssertionError):
            close(got[0], bad)
