"""Each layer on the GPU (through the C ABI) against the CPU oracle, as
single-operation plans on seeded inputs, several lanes at once.

Bit-exact where the kernel keeps the engine's order (depthwise, pooling,
elementwise modes, upsampling, concatenation, layer norm, attention, the
narrow transposed convolution, the squeeze-and-excite layers given the same
mean); within the benchmark's tolerance for the recogniser's logits for the
MFMA products, whose sums run in another order: |gpu - cpu| <= 1e-5 * |cpu|
+ 1e-5.
"""
import numpy as np
import pytest

from ppocr_native_amd import GpuModel
from ppocr_native_amd.planfile import PlanBuilder

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(99)


def both(build, shape, oracle, lanes=3, seed=0):
    """Run `build` as a plan over `lanes` seeded images on the GPU and on the
    oracle; returns (gpu outputs, oracle outputs) per lane."""
    h, w, c = shape
    b = PlanBuilder(h, w, c)
    outs = build(b, b.input)
    outs = outs if isinstance(outs, list) else [outs]
    plan = b.to_bytes(outs)
    rng = np.random.default_rng(seed)
    xs = [rng.uniform(-1, 1, shape).astype(np.float32) for _ in range(lanes)]
    g = GpuModel.load(plan)
    g.set_sizes([(h, w)] * lanes)
    for i, x in enumerate(xs):
        g.lane_input_mut(i)[:] = x.reshape(-1)
    g.run()
    got = [[g.lane_output(i, k) for k in range(len(outs))] for i in range(lanes)]
    m = oracle.OracleModel(plan)
    want = [m.run(x) for x in xs]
    g.close()
    return got, want


def exact(got, want):
    for gl, wl in zip(got, want):
        for a, b in zip(gl, wl):
            assert a.shape == b.shape
            bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
            assert bad.size == 0, f"{bad.size} of {a.size} differ, first {bad[:5]}: {a[bad[:5]]} vs {b[bad[:5]]}"


def near(got, want, rtol=1e-5, atol=1e-5):
    """|gpu - cpu| <= rtol * |cpu| + atol, element by element."""
    for gl, wl in zip(got, want):
        for a, b in zip(gl, wl):
            assert a.shape == b.shape
            err = np.abs(a.astype(np.float64) - b)
            lim = rtol * np.abs(b) + atol
            bad = np.flatnonzero(err > lim)
            assert bad.size == 0, (f"{bad.size} of {err.size} outside, worst excess "
                                   f"{float((err - lim).max()):.3g}, max |cpu| {float(np.abs(b).max()):.3g}")


@pytest.mark.parametrize("k,s,c", [(3, 1, 16), (3, 2, 24), (5, 1, 48), (5, 2, 12), (7, 1, 32),
                                   (3, 1, 6), (7, 1, 5)])
def test_depthwise_exact(oracle, k, s, c):
    w = RNG.normal(0, 0.3, (k, k, c)).astype(np.float32)
    bias = RNG.normal(0, 0.3, c).astype(np.float32)
    got, want = both(lambda b, t: b.dwconv(t, w, bias, k=(k, k), s=(s, s), fused="hardswish"),
                     (19, 23, c), oracle)
    exact(got, want)


@pytest.mark.parametrize("ci,co", [(16, 16), (24, 48), (96, 96), (12, 20), (480, 120), (8, 64),
                                   (20, 10), (36, 6), (64, 200), (120, 18385)])
def test_pointwise_gemm(oracle, ci, co):
    w = RNG.normal(0, 1 / np.sqrt(ci), (1, 1, ci, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    got, want = both(lambda b, t: b.conv(t, w, bias, fused="relu"), (13, 17, ci), oracle)
    near(got, want)


@pytest.mark.parametrize("k,s,pad,ci,co", [((3, 3), (2, 2), (1, 1, 1, 1), 3, 24),
                                           ((3, 3), (1, 1), (1, 1, 1, 1), 96, 24),
                                           ((2, 2), (1, 1), (0, 1, 0, 1), 24, 12),
                                           ((1, 3), (1, 1), (0, 0, 1, 1), 40, 60),
                                           ((3, 3), (2, 1), (1, 1, 1, 1), 7, 33),
                                           ((3, 3), (1, 1), (1, 1, 1, 1), 10, 20)])
def test_windowed_gemm(oracle, k, s, pad, ci, co):
    w = RNG.normal(0, 1 / np.sqrt(ci * k[0] * k[1]), (k[0], k[1], ci, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    got, want = both(lambda b, t: b.conv(t, w, bias, k=k, s=s, pad=pad, fused="swish"),
                     (15, 18, ci), oracle)
    near(got, want)


@pytest.mark.parametrize("k,s,pad,ci,co,hw,lanes,two", [
    ((2, 2), (1, 1), (0, 1, 0, 1), 24, 12, (130, 131), 1, False),   # the stem's 2 x 2 on a large map
    ((3, 3), (2, 2), (1, 1, 1, 1), 24, 32, (262, 258), 1, True),    # stride 2 over two sources
    ((5, 5), (1, 1), (2, 2, 2, 2), 8, 20, (17, 23), 2, False),      # wider than the halo tiles take
    ((3, 3), (2, 1), (1, 1, 1, 1), 12, 40, (21, 18), 3, False),     # unequal strides
    ((1, 1), (2, 2), (0, 0, 0, 0), 16, 24, (19, 26), 2, False),     # a strided 1 x 1
    ((5, 5), (1, 1), (2, 2, 2, 2), 8, 12, (15, 14), 2, True),       # two sources, wide window
])
def test_ring_windowed(oracle, k, s, pad, ci, co, hw, lanes, two):
    # Windowed convolutions: the wide window, unequal strides and the strided
    # 1 x 1 run on the LDS ring, each lane's direct loads gathering its row's
    # window (zeros outside the image and past the channels); the stem's
    # shapes on large maps run on the register-staged implicit GEMM.
    cin = 2 * ci if two else ci
    w = RNG.normal(0, 1 / np.sqrt(cin * k[0] * k[1]), (k[0], k[1], cin, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    wx = RNG.normal(0, 0.3, (1, 1, ci, ci)).astype(np.float32)

    def build(b, t):
        x2 = b.conv(t, wx, None, fused="relu") if two else None
        return b.conv(t, w, bias, k=k, s=s, pad=pad, fused="hardswish", x2=x2)

    got, want = both(build, (*hw, ci), oracle, lanes=lanes)
    near(got, want)


@pytest.mark.parametrize("ci,co,co2,hw,lanes", [
    (16, 24, 20, (260, 262), 1),   # the detector stem's shape: a 3 x 3 stride-2 conv, then its 1 x 1
    (16, 32, 32, (258, 256), 2),
    (16, 12, 7, (262, 258), 1),    # columns past the tile's and the 1 x 1's last
])
def test_conv_then_pointwise_folded(oracle, ci, co, co2, hw, lanes):
    # A 1 x 1 convolution whose input only the implicit-GEMM convolution
    # before it writes: one launch, the 1 x 1 in its epilogue on the tile's
    # activated outputs, only the 1 x 1's map stored.
    w = RNG.normal(0, 1 / np.sqrt(9 * ci), (3, 3, ci, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    w2 = RNG.normal(0, 1 / np.sqrt(co), (1, 1, co, co2)).astype(np.float32)
    b2 = RNG.normal(0, 0.3, co2).astype(np.float32)

    def build(b, t):
        y = b.conv(t, w, bias, k=(3, 3), s=(2, 2), pad=(1, 1, 1, 1), fused="hardswish")
        return b.conv(y, w2, b2, fused="hardswish")

    b = PlanBuilder(*hw, ci)
    g = GpuModel.load(b.to_bytes([build(b, b.input)]))
    launches, ops = g.launches(), g.launch_ops()
    g.close()
    assert [n for n, _ in launches] == ["conv_gemm"] and ops == [[0, 1]], (launches, ops)
    got, want = both(build, (*hw, ci), oracle, lanes=lanes)
    near(got, want)


@pytest.mark.parametrize("k,s,c,n,hw,lanes,residual", [
    (3, (1, 1), 32, 48, (62, 70), 1, False),    # the detector's first block, on a smaller map
    (3, (2, 2), 48, 96, (61, 66), 1, False),    # stride 2
    (3, (1, 1), 96, 96, (33, 40), 1, True),     # 96 channels with the block's residual
    (5, (2, 2), 96, 192, (30, 31), 1, False),   # 5 x 5 stride 2, twelve column blocks
    (3, (1, 1), 48, 64, (24, 40), 3, False),    # the recogniser's first block, three lanes
    (3, (2, 1), 64, 128, (12, 20), 2, False),   # unequal strides
    (5, (1, 1), 128, 128, (9, 13), 2, True),    # 128 channels, tiles past the map
    (3, (1, 1), 16, 20, (5, 7), 1, False),      # columns past the last block's, one tile
])
def test_depthwise_then_pointwise_folded(oracle, k, s, c, n, hw, lanes, residual):
    # A 1 x 1 convolution (and its residual Add) that alone reads a
    # depthwise layer: one launch, the depthwise rows made in LDS and
    # multiplied there, the depthwise map never stored.
    p = (k - 1) // 2
    wd = RNG.normal(0, 1 / k, (k, k, c)).astype(np.float32)
    bd = RNG.normal(0, 0.3, c).astype(np.float32)
    w2 = RNG.normal(0, 1 / np.sqrt(c), (1, 1, c, n)).astype(np.float32)
    b2 = RNG.normal(0, 0.3, n).astype(np.float32)

    def build(b, t):
        d = b.dwconv(t, wd, bd, k=(k, k), s=s, pad=(p, p, p, p), fused="hardswish")
        y = b.conv(d, w2, b2, fused="none" if residual else "hardswish")
        return b.add(y, t) if residual else y

    b = PlanBuilder(*hw, c)
    g = GpuModel.load(b.to_bytes([build(b, b.input)]))
    launches, ops = g.launches(), g.launch_ops()
    g.close()
    assert [nm for nm, _ in launches] == ["dwconv_pw"] and ops == [[0, 1]], (launches, ops)
    got, want = both(build, (*hw, c), oracle, lanes=lanes)
    near(got, want)


def test_ring_upsampled_sources(oracle):
    # A 5 x 5 convolution (on the LDS ring) over a map upsampled by 2 stacked
    # with a full-size one: the direct loads read the small map at (y/2, x/2).
    c = 8
    wq = RNG.normal(0, 0.3, (1, 1, 4, c)).astype(np.float32)
    w5 = RNG.normal(0, 0.1, (5, 5, 2 * c, 12)).astype(np.float32)

    def build(b, t):
        full = b.conv(t, wq, None)
        half = b.avgpool(full, (2, 2), (2, 2))
        return b.conv(b.upsample(half, 2), w5, None, k=(5, 5), pad=(2, 2, 2, 2), fused="relu", x2=full)

    got, want = both(build, (14, 18, 4), oracle)
    near(got, want)


@pytest.mark.parametrize("k,s,ci,co,hw,lanes", [
    (3, 1, 96, 24, (30, 40), 3),     # the neck's 3 x 3: 8-row tiles? no, 4-row
    (3, 1, 96, 24, (256, 256), 1),   # 512 tiles of 8 rows: columns 16-23 on the 4 x 4 MFMA
    (3, 1, 32, 20, (256, 256), 1),   # the same with 4 padded columns in the remainder
    (3, 2, 24, 17, (512, 512), 1),   # stride 2, one real column in the remainder
    (3, 2, 48, 32, (33, 50), 2),     # stride 2, two sources below
    (2, 1, 24, 12, (37, 29), 2),     # the stem's 2 x 2
    (3, 1, 20, 96, (17, 35), 2),     # two column tiles of 64, channel block 16 + 4 padding
    (1, 3, 40, 60, (9, 70), 2),
    (3, 1, 32, 32, (20, 24), 2),     # residual add folded into the epilogue
])
def test_patch_conv(oracle, k, s, ci, co, hw, lanes):
    # Windowed convolutions on halo tiles: two sources (the second input of
    # a two-input conv), a residual add folded into the epilogue, and a
    # channel gate folded into the first source.
    kh, kw = (k, k) if k != 1 else (1, 3)
    half = ci // 2 if ci % 8 == 0 else 0
    w = RNG.normal(0, 1 / np.sqrt(ci * kh * kw), (kh, kw, ci, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    g = RNG.uniform(0.5, 1.5, (1, 1, ci - half if half else ci)).astype(np.float32)
    pad = (kh // 2, (kh - 1) // 2, kw // 2, (kw - 1) // 2) if kh != 2 else (0, 1, 0, 1)
    wg1 = RNG.normal(0, 0.3, (1, 1, ci - half if half else ci, 4)).astype(np.float32)
    wg2 = RNG.normal(0, 0.3, (1, 1, 4, ci - half if half else ci)).astype(np.float32)

    def build(b, t):
        if half:
            x1 = b.conv(t, RNG.normal(0, 0.3, (1, 1, ci, ci - half)).astype(np.float32), None)
            x2 = b.conv(t, RNG.normal(0, 0.3, (1, 1, ci, half)).astype(np.float32), None)
        else:
            x1, x2 = t, None
        m = b.mean(x1)
        gate = b.conv(b.conv(m, wg1, None, fused="relu"), wg2, None, fused="hardsigmoid")
        y = b.conv(b.channelmul(x1, gate), w, bias, k=(kh, kw), s=(s, s), pad=pad, fused="hardswish", x2=x2)
        if s == 1 and co == ci and kh != 2:
            y = b.add(y, t)
        return y

    got, want = both(build, (*hw, ci), oracle, lanes=lanes)
    near(got, want)


@pytest.mark.parametrize("k,c,hw", [(3, 32, (21, 19)), (5, 96, (40, 52)), (3, 200, (9, 9)),
                                     (5, 384, (14, 11)), (3, 480, (12, 13))])
def test_gemm_gate_and_residual(oracle, k, c, hw):
    # dw -> SE (mean, 1x1 ReLU, 1x1 hard sigmoid) -> gated pointwise + input.
    # The depthwise kernel also sums its outputs per channel for the mean.
    # The SE weights reach LDS together (c <= 200), one layer after the
    # other (384 x 96 each) or not at all (480 x 120, read from memory).
    mid = c // 4
    wd = RNG.normal(0, 0.3, (k, k, c)).astype(np.float32)
    w1 = RNG.normal(0, 0.3, (1, 1, c, mid)).astype(np.float32)
    w2 = RNG.normal(0, 0.3, (1, 1, mid, c)).astype(np.float32)
    wp = RNG.normal(0, 0.2, (1, 1, c, c)).astype(np.float32)
    bv = RNG.normal(0, 0.3, c).astype(np.float32)

    def build(b, t):
        d = b.dwconv(t, wd, bv, k=(k, k), fused="hardswish")
        m = b.mean(d)
        h = b.conv(m, w1, bv[:mid], fused="relu")
        g = b.conv(h, w2, bv, fused="hardsigmoid")
        y = b.conv(b.channelmul(d, g), wp, bv)
        return [b.add(y, t), g]

    got, want = both(build, (*hw, c), oracle)
    near([[gl[0]] for gl in got], [[wl[0]] for wl in want])
    # The gate: the same mean to f64 rounding, then the same 1x1 sums.
    near([[gl[1]] for gl in got], [[wl[1]] for wl in want], rtol=1e-6, atol=1e-6)


def test_gated_pointwise_many_lanes(oracle):
    # 15-pixel lanes: a 32-row tile of the 1x1 GEMM spans up to four lanes,
    # each with its own gate row; the residual rides along.
    c = 64
    w1 = RNG.normal(0, 0.3, (1, 1, c, 16)).astype(np.float32)
    w2 = RNG.normal(0, 0.3, (1, 1, 16, c)).astype(np.float32)
    wp = RNG.normal(0, 0.2, (1, 1, c, c)).astype(np.float32)
    bv = RNG.normal(0, 0.3, c).astype(np.float32)

    def build(b, t):
        g = b.conv(b.conv(b.mean(t), w1, None, fused="relu"), w2, None, fused="hardsigmoid")
        return b.add(b.conv(b.channelmul(t, g), wp, bv), t)

    got, want = both(build, (3, 5, c), oracle, lanes=7)
    near(got, want)


def test_upsampled_concat_sources(oracle):
    # The DB head's input: maps at 1/8, 1/4, 1/2 upsampled and stacked with a
    # full-size one under a 3x3 convolution (four shifted sources).
    c = 8
    wq = RNG.normal(0, 0.3, (1, 1, 4, c)).astype(np.float32)
    wh = RNG.normal(0, 0.2, (3, 3, 4 * c, 12)).astype(np.float32)

    def build(b, t):
        full = b.conv(t, wq, None)
        half = b.avgpool(full, (2, 2), (2, 2))
        quarter = b.avgpool(half, (2, 2), (2, 2))
        eighth = b.avgpool(quarter, (2, 2), (2, 2))
        cat = b.concat(b.upsample(eighth, 8), b.upsample(quarter, 4))
        cat = b.concat(cat, b.upsample(half, 2))
        return b.conv(cat, wh, None, k=(3, 3), pad=(1, 1, 1, 1), fused="relu", x2=full)

    got, want = both(build, (16, 24, 4), oracle)
    near(got, want)


@pytest.mark.parametrize("co,hw,lanes", [(24, (40, 48), 2), (16, (13, 21), 3), (32, (30, 17), 1),
                                         (20, (8, 8), 5)])
def test_halo_conv_head_sources(oracle, co, hw, lanes):
    # Halo tiles over 96 channels from four sources of 24, three of them
    # upsampled by 8, 4 and 2 as in the DB head, maps whose sides are not
    # multiples of the 16 x 4 tile, several lanes, and 16-column tiles when
    # co <= 16.
    c = 24
    wq = RNG.normal(0, 0.3, (1, 1, 4, c)).astype(np.float32)
    wh = RNG.normal(0, 0.2, (3, 3, 4 * c, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    h, w = hw
    up = 8 if h % 8 == 0 and w % 8 == 0 else 1

    def build(b, t):
        full = b.conv(t, wq, None)
        if up == 8:
            half = b.avgpool(full, (2, 2), (2, 2))
            quarter = b.avgpool(half, (2, 2), (2, 2))
            eighth = b.avgpool(quarter, (2, 2), (2, 2))
            cat = b.concat(b.upsample(eighth, 8), b.upsample(quarter, 4))
            cat = b.concat(cat, b.upsample(half, 2))
        else:
            cat = b.concat(b.concat(full, b.conv(t, wq, None)), b.conv(t, wq, None))
        return b.conv(cat, wh, bias, k=(3, 3), pad=(1, 1, 1, 1), fused="relu", x2=full)

    got, want = both(build, (h, w, 4), oracle, lanes=lanes)
    near(got, want)


@pytest.mark.parametrize("c", [480, 1024])
def test_large_se_gate_exact(oracle, c):
    # Squeeze-and-excite layers too large to stage in LDS (c -> c/4 -> c):
    # each row's weights read from memory, every output in the CPU's order.
    w1 = RNG.normal(0, 1 / np.sqrt(c), (1, 1, c, c // 4)).astype(np.float32)
    b1 = RNG.normal(0, 0.3, c // 4).astype(np.float32)
    w2 = RNG.normal(0, 2 / np.sqrt(c), (1, 1, c // 4, c)).astype(np.float32)
    b2 = RNG.normal(0, 0.3, c).astype(np.float32)

    def build(b, t):
        h = b.conv(b.mean(t), w1, b1, fused="relu")
        return b.channelmul(t, b.conv(h, w2, b2, fused="hardsigmoid"))

    got, want = both(build, (5, 7, c), oracle)
    exact(got, want)


@pytest.mark.parametrize("hw,c,lanes,dw", [((60, 61), 96, 3, False), ((33, 17), 30, 2, False),
                                          ((160, 160), 96, 1, True), ((8, 9), 1024, 2, True),
                                          ((30, 30), 384, 1, True), ((3, 80), 480, 16, True),
                                          ((240, 240), 24, 1, False)])
def test_mean_se_launch_shapes(oracle, hw, c, lanes, dw):
    # The one-launch channel mean and squeeze-and-excite on the shapes that
    # take each of its paths: an input summed in several pixel chunks and
    # channel slices (the last chunk of a slice joins, the last slice of a
    # lane runs the SE layers), channels not a multiple of four (scalar
    # loads), a depthwise convolution's partial rows joined in slices of 4 to
    # 32 channels, and SE layers of one, two and four outputs a thread, fused
    # and separate products, inputs a multiple of four or not. The gate is
    # the CPU's to the bit.
    mid = max(1, c // 4)
    w1 = RNG.normal(0, 1 / np.sqrt(c), (1, 1, c, mid)).astype(np.float32)
    b1 = RNG.normal(0, 0.3, mid).astype(np.float32)
    w2 = RNG.normal(0, 2 / np.sqrt(mid), (1, 1, mid, c)).astype(np.float32)
    b2 = RNG.normal(0, 0.3, c).astype(np.float32)
    wd = RNG.normal(0, 0.3, (3, 3, c)).astype(np.float32)

    def build(b, t):
        x = b.dwconv(t, wd, b2, k=(3, 3), fused="hardswish") if dw else t
        m = b.mean(x)
        g = b.conv(b.conv(m, w1, b1, fused="relu"), w2, b2, fused="hardsigmoid")
        return [g, b.mean(x)]

    got, want = both(build, (*hw, c), oracle, lanes=lanes)
    exact(got, want)


@pytest.mark.parametrize("mode", ["add", "resgate", "upsampleadd_resgate", "concat", "upsample"])
def test_elementwise_exact(oracle, mode):
    c = 12
    w1 = RNG.normal(0, 0.5, (1, 1, c, 4)).astype(np.float32)
    w2 = RNG.normal(0, 0.5, (1, 1, 4, c)).astype(np.float32)

    def build(b, t):
        if mode == "add":
            return b.add(t, b.dwconv(t, np.ones((1, 1, c), np.float32), None, k=(1, 1)),
                         fused="gelu")
        # A gate from the squeeze-and-excite step: the CPU's bits.
        h = b.conv(b.mean(t), w1, None, fused="relu")
        g = b.conv(h, w2, None, fused="hardsigmoidfifth")
        if mode == "resgate":
            return b.add(t, b.channelmul(t, g))
        if mode == "concat":
            return b.concat(t, b.channelmul(t, g))
        small = b.avgpool(t, (2, 2), (2, 2))
        if mode == "upsample":
            return b.upsample(small, 2)
        r = b.add(t, b.channelmul(t, g))
        return b.upsampleadd(small, r, 2)

    got, want = both(build, (10, 14, c), oracle)
    exact(got, want)


@pytest.mark.parametrize("hw,c,levels,lanes", [((48, 64), 8, 3, 3), ((40, 24), 24, 3, 2), ((16, 8), 12, 2, 3),
                                                 ((24, 40), 6, 3, 2)])
def test_upsample_add_chain_exact(oracle, hw, c, levels, lanes):
    # A feature pyramid's top-down sums: each level the gated addend plus the
    # coarser level upsampled 2x, the finest addend ungated. With channels a
    # multiple of 4 the levels run as one chain launch that writes each.
    def build(b, t):
        pyr = [t]
        for _ in range(levels):
            pyr.append(b.maxpool(pyr[-1], k=(2, 2), s=(2, 2), pad_after=(0, 0)))

        def gated(x):
            return b.add(x, b.channelmul(x, b.mean(x)))

        outs, up = [], pyr[levels]
        for k in range(levels - 1, -1, -1):
            up = b.upsampleadd(up, gated(pyr[k]) if k else pyr[k], 2)
            outs.append(up)
        return outs

    h, w = hw
    b = PlanBuilder(h, w, c)
    g = GpuModel.load(b.to_bytes(build(b, b.input)))
    names = [name for name, _ in g.launches()]
    g.close()
    assert ("upsample_add_chain" in names) == (c % 4 == 0)
    got, want = both(build, (h, w, c), oracle, lanes=lanes)
    exact(got, want)


@pytest.mark.parametrize("c", [20, 6])
def test_pools_exact(oracle, c):
    # Four channels at a time when c % 4 == 0, else one.
    def build(b, t):
        return [b.maxpool(t), b.avgpool(t, (3, 1), (3, 1))]

    got, want = both(build, (6, 11, c), oracle)
    exact(got, want)


@pytest.mark.parametrize("ci,co,k,s,pad,hw", [
    (3, 24, 3, 2, 1, (19, 30)),   # RGB stem: every output from its bias
    (3, 24, 3, 2, 1, (64, 70)),   # blocks of 256 pixels inside one lane and across two
    (3, 48, 3, 2, 1, (16, 22)),
    (3, 16, 3, 2, 1, (21, 37)),   # small maps: a quarter of the outputs a wave
    (3, 32, 3, 2, 1, (33, 60)),
    (3, 48, 3, 2, 1, (740, 720)),  # 133,200 pixels: one pixel and all outputs a thread
    (3, 16, 3, 1, 1, (370, 360)),
    (3, 24, 2, 2, 0, (12, 14)),
    (6, 16, 3, 1, 1, (7, 14)),    # bias first except the row's last ow % 4 pixels
    (5, 12, 3, 1, 1, (8, 13)),    # bias last; columns 8..11 multiply and add apart
    (12, 24, 2, 1, (0, 1, 0, 1), (17, 40)),  # the stem's 12 -> 24 2 x 2: one thread per pixel
    (12, 24, 2, 1, (0, 1, 0, 1), (400, 380)),  # the same over 152,000 pixels
])
def test_direct_conv_exact(oracle, ci, co, k, s, pad, hw):
    w = RNG.normal(0, 0.3, (k, k, ci, co)).astype(np.float32)
    bias = RNG.normal(0, 0.3, co).astype(np.float32)
    pad = pad if isinstance(pad, tuple) else (pad,) * 4
    got, want = both(lambda b, t: b.conv(t, w, bias, k=(k, k), s=(s, s), pad=pad,
                                         fused="hardswish"), (*hw, ci), oracle)
    exact(got, want)


@pytest.mark.parametrize("hw,biased,lanes", [
    ((19, 30), True, 3),     # one 14 x 14 tile of the 10 x 15 maps, cut at both edges
    ((64, 70), True, 3),     # 32 x 35: whole and partial tiles
    ((61, 97), False, 2),    # odd input sides; no biases (every sum from zero)
    ((480, 452), True, 1),   # 240 x 226: many tiles, the last row and column partial
])
def test_stem_block(oracle, hw, biased, lanes):
    # The RGB stem, its 2x2 max pool and two 2x2 layers padded right and
    # bottom: one fused step whose s1 and first 2x2 maps stay on chip. The
    # pool (of s1, which keeps the engine's order) bit-exact; the 2x2 layers
    # run on MFMA: within the MFMA tolerance.
    rng = np.random.default_rng(7)
    w1 = rng.normal(0, 0.3, (3, 3, 3, 24)).astype(np.float32)
    w2 = rng.normal(0, 0.3, (2, 2, 24, 12)).astype(np.float32)
    w3 = rng.normal(0, 0.3, (2, 2, 12, 24)).astype(np.float32)
    bs = [rng.normal(0, 0.3, c).astype(np.float32) if biased else None for c in (24, 12, 24)]

    def build(b, t):
        s1 = b.conv(t, w1, bs[0], k=(3, 3), s=(2, 2), pad=(1, 1, 1, 1), fused="hardswish")
        s2 = b.conv(s1, w2, bs[1], k=(2, 2), pad=(0, 1, 0, 1), fused="hardswish")
        s3 = b.conv(s2, w3, bs[2], k=(2, 2), pad=(0, 1, 0, 1), fused="hardswish")
        return [b.maxpool(s1), s3]

    h, w = hw
    b = PlanBuilder(h, w, 3)
    g = GpuModel.load(b.to_bytes(build(b, b.input)))
    assert "stem_block" in [name for name, _ in g.launches()]
    g.close()
    got, want = both(build, (h, w, 3), oracle, lanes=lanes)
    exact([[g[0]] for g in got], [[w_[0]] for w_ in want])
    near([[g[1]] for g in got], [[w_[1]] for w_ in want])


@pytest.mark.parametrize("hw,lanes", [((64, 70), 2), ((480, 452), 1)])
def test_stem_block_joint_map(oracle, hw, lanes):
    # The stem block whose pool and second 2x2 only the next 3x3 stride-2
    # convolution reads (its two sources): one map of both, that
    # convolution's single source. Within the MFMA tolerance.
    rng = np.random.default_rng(8)
    w1 = rng.normal(0, 0.3, (3, 3, 3, 24)).astype(np.float32)
    w2 = rng.normal(0, 0.3, (2, 2, 24, 12)).astype(np.float32)
    w3 = rng.normal(0, 0.3, (2, 2, 12, 24)).astype(np.float32)
    w4 = rng.normal(0, 0.1, (3, 3, 48, 32)).astype(np.float32)
    bs = [rng.normal(0, 0.3, c).astype(np.float32) for c in (24, 12, 24, 32)]

    def build(b, t):
        s1 = b.conv(t, w1, bs[0], k=(3, 3), s=(2, 2), pad=(1, 1, 1, 1), fused="hardswish")
        s2 = b.conv(s1, w2, bs[1], k=(2, 2), pad=(0, 1, 0, 1), fused="hardswish")
        s3 = b.conv(s2, w3, bs[2], k=(2, 2), pad=(0, 1, 0, 1), fused="hardswish")
        return b.conv(b.maxpool(s1), w4, bs[3], k=(3, 3), s=(2, 2), pad=(1, 1, 1, 1), fused="hardswish", x2=s3)

    h, w = hw
    b = PlanBuilder(h, w, 3)
    g = GpuModel.load(b.to_bytes([build(b, b.input)]))
    names = [name for name, _ in g.launches()]
    assert len(names) == 2 and names[0] == "stem_block", names
    g.close()
    got, want = both(build, (h, w, 3), oracle, lanes=lanes)
    near(got, want)


@pytest.mark.parametrize("oc1,hw", [(24, (9, 13)), (16, (6, 8))])
def test_db_head_exact(oracle, oc1, hw):
    # A wide 2x2 transposed conv read only by a narrow one: one fused step.
    w1 = RNG.normal(0, 0.3, (24, 2, 2, oc1)).astype(np.float32)
    b1 = RNG.normal(0, 0.3, oc1).astype(np.float32)
    w2 = RNG.normal(0, 0.3, (oc1, 2, 2, 1)).astype(np.float32)
    b2 = RNG.normal(0, 0.3, 1).astype(np.float32)

    def build(b, t):
        m = b.convtranspose(t, w1, b1, k=(2, 2), fused="relu")
        return b.convtranspose(m, w2, b2, k=(2, 2), fused="sigmoid")

    got, want = both(build, (*hw, 24), oracle)
    exact(got, want)


def test_layernorm_attention_exact(oracle):
    c, heads = 120, 8
    g = RNG.normal(1, 0.1, c).astype(np.float32)
    be = RNG.normal(0, 0.1, c).astype(np.float32)
    wq = RNG.normal(0, 1 / np.sqrt(c), (1, 1, c, 3 * c)).astype(np.float32)

    def build(b, t):
        n = b.layernorm(t, g, be, 1e-6)
        qkv = b.conv(n, wq, None)
        return [n, qkv, b.attention(qkv, heads, float(np.float32(15 ** -0.5)))]

    got, want = both(build, (1, 80, c), oracle)
    exact([[gl[0]] for gl in got], [[wl[0]] for wl in want])
    # Attention's own arithmetic is the CPU's: fed the GPU's qkv, it is exact.
    near([[gl[1]] for gl in got], [[wl[1]] for wl in want])
    qkv = [gl[1] for gl in got]
    b = PlanBuilder(1, 80, 3 * c)
    plan = b.to_bytes([b.attention(b.input, heads, float(np.float32(15 ** -0.5)))])
    m = oracle.OracleModel(plan)
    for gl, q in zip(got, qkv):
        assert np.array_equal(gl[2], m.run(q)[0])


@pytest.mark.parametrize("t,heads,hd", [(80, 8, 15), (41, 8, 15), (9, 2, 3), (160, 4, 32),
                                        (320, 8, 15)])
def test_attention_exact(oracle, t, heads, hd):
    # Keys past t // 8 * 8 use separate products and sums; 320 steps keep
    # the scores in global scratch instead of LDS.
    c = heads * hd
    got, want = both(lambda b, x: b.attention(x, heads, float(np.float32(hd ** -0.5))),
                     (1, t, 3 * c), oracle, lanes=2)
    exact(got, want)


@pytest.mark.parametrize("oc", [1, 4])
def test_narrow_convtranspose_exact(oracle, oc):
    w = RNG.normal(0, 0.3, (24, 2, 2, oc)).astype(np.float32)
    bias = RNG.normal(0, 0.3, oc).astype(np.float32)
    got, want = both(lambda b, t: b.convtranspose(t, w, bias, k=(2, 2), fused="sigmoid"),
                     (9, 13, 24), oracle)
    exact(got, want)


def test_wide_convtranspose(oracle):
    w = RNG.normal(0, 0.3, (24, 2, 2, 24)).astype(np.float32)
    bias = RNG.normal(0, 0.3, 24).astype(np.float32)
    got, want = both(lambda b, t: b.convtranspose(t, w, bias, k=(2, 2), fused="relu"),
                     (9, 13, 24), oracle)
    near(got, want)


@pytest.mark.parametrize("vocab", [37, 6625, 18385])
def test_ctc_argmax(oracle, vocab):
    c = 120
    w = RNG.normal(0, 1 / np.sqrt(c), (c, vocab)).astype(np.float32)
    bias = RNG.normal(0, 0.5, vocab).astype(np.float32)
    got, want = both(lambda b, t: b.ctcargmax(t, w, bias), (1, 80, c), oracle, lanes=4)
    for gl, wl in zip(got, want):
        a, b = gl[0].reshape(-1, 2), wl[0].reshape(-1, 2)
        assert np.array_equal(a[:, 0], b[:, 0])
        np.testing.assert_allclose(a[:, 1], b[:, 1], rtol=1e-5, atol=1e-5)


def test_ctc_argmax_near_ties(oracle):
    # Groups of ten columns that differ by one ulp in a few weights: within a
    # group the logits differ by less than the rounding of a 120-term sum, so
    # the summation order decides the argmax among them, the CPU's one way,
    # the GPU's (MFMA) another. The near-tie check recomputes such rows in
    # the CPU's order, so the indices match the oracle's exactly. Also two
    # identical columns (an exact tie: the first one wins).
    c, vocab, group = 120, 700, 10
    w = np.empty((c, vocab), np.float32)
    for g in range(vocab // group):
        base = RNG.normal(0, 1 / np.sqrt(c), c).astype(np.float32)
        for k in range(group):
            col = base.copy()
            for i in RNG.choice(c, 3, replace=False):
                col[i] = np.nextafter(col[i], np.float32(np.inf) if RNG.random() < 0.5 else np.float32(-np.inf))
            w[:, g * group + k] = col
    bias = np.repeat(RNG.normal(0, 0.5, vocab // group).astype(np.float32), group)
    w[:, 401], bias[401] = w[:, 77], bias[77]

    def build(b, t):
        return b.ctcargmax(t, w, bias)

    got, want = both(build, (1, 40, c), oracle, lanes=3, seed=5)
    for gl, wl in zip(got, want):
        a, b = gl[0].reshape(-1, 2), wl[0].reshape(-1, 2)
        assert np.array_equal(a[:, 0], b[:, 0]), np.flatnonzero(a[:, 0] != b[:, 0])
        np.testing.assert_allclose(a[:, 1], b[:, 1], rtol=1e-5, atol=1e-5)
    assert 401 not in {int(v) for gl in got for v in gl[0].reshape(-1, 2)[:, 0]}
