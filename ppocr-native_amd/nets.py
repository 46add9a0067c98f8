"""Synthetic PP-OCR plans with seeded weights, at the shapes the benchmark names.

The shipped PP-OCRv6-small plans are not available here, so these
generators write plans of the same op vocabulary and graph idioms
(tools/export_ocr.py): depthwise + pointwise blocks with squeeze-and-excite
gates, an RGB stem with a 2x2 max pool feeding a two-input convolution,
a residual-SE FPN neck with upsampled sums and an upsampled concatenation
feeding a 3x3 convolution, a DB head of two 2x2 transposed convolutions,
and an SVTR-style recogniser (avg-pool to one row, LayerNorm, attention,
swish MLP) ending in the CTC argmax head.

``init="baseline"`` draws every weight and bias from N(0, sigma) with the
sigma the benchmark states (0.05 detector, 0.02 recogniser).
``init="scaled"`` draws weights from N(0, gain / sqrt(fan_in)) so that the
signal keeps its scale through the depth, which makes parity checks see
non-trivial outputs. The default gain, 1.3, keeps the detector well
conditioned: a one-ulp change of every input pixel moves its probabilities
by about 1e-6, while at 1.6 the same change moves them by 4e-4, beyond any
fixed tolerance between two summation orders. The recogniser uses 1.6:
its LayerNorms renormalise the signal, and with less its argmax settles on
one class.
"""

from __future__ import annotations

import numpy as np

from .planfile import PlanBuilder, Tensor


class Init:
    """Seeded weights. `role` names what a layer does in the graph; these
    draws ignore it (the ink detector below uses it)."""

    def __init__(self, seed: int, init: str, sigma: float, gain: float = 1.3):
        self.rng = np.random.default_rng(seed)
        self.init = init
        self.sigma = sigma
        self.gain = gain

    def w(self, shape, fan_in: int, gain: float | None = None, role: str = "") -> np.ndarray:
        if self.init == "baseline":
            std = self.sigma
        else:
            std = (self.gain if gain is None else gain) / np.sqrt(fan_in)
        return self.rng.normal(0.0, std, size=shape).astype(np.float32)

    def b(self, n: int, role: str = "") -> np.ndarray:
        std = self.sigma if self.init == "baseline" else 0.05
        return self.rng.normal(0.0, std, size=n).astype(np.float32)


class InkInit(Init):
    """The detector's weights for the page pipeline: every weight seeded
    N(0, sigma) as in the baseline, except what feeds output channel 0 of
    each layer on the path from the input to the map, which carries an ink
    signal: the stem's channel 0 is 5.5 minus the mean of the normalised
    RGB over its 3 x 3 window (about 3.06 on white paper, up to 7.5 on
    black ink, so that hard swish passes it unchanged), later layers copy it
    (centre tap 1) or average it (3 x 3 box, `box` roles), the 1/4-scale
    branch of the neck carries it to the head while the coarser branches
    give channel 0 nothing, squeeze-and-excite gates on channel 0 are held
    open (1, 'se') or shut (0, 'rse'), and the last transposed convolution
    maps it to gain * (v - level) before the sigmoid. The map is then high
    over ink and low over paper, so the DB boxes fall on the page's lines.
    Layers off that path keep their seeded weights in every channel."""

    GAIN = 6.0
    LEVEL = 3.6

    def w(self, shape, fan_in: int, gain: float | None = None, role: str = "") -> np.ndarray:
        a = super().w(shape, fan_in, gain, role)
        if not role:
            return a
        if role.startswith("convt"):  # [ic][kh][kw][oc]
            a[..., 0] = 0.0
            a[0, :, :, 0] = self.GAIN if role == "convt_out" else 1.0
            return a
        if len(shape) == 3:  # depthwise [kh][kw][c]
            kh, kw, _ = shape
            a[:, :, 0] = 0.0
            if role == "box":
                a[:, :, 0] = 1.0 / (kh * kw)
            elif role == "hbox":
                a[kh // 2, :, 0] = 1.0 / kw
            else:
                a[kh // 2, kw // 2, 0] = 1.0
            return a
        kh, kw, ci, _ = shape  # dense [kh][kw][ci][oc]
        a[..., 0] = 0.0
        src = 0  # "carry@72": from input channel 72
        if "@" in role:
            role, at = role.split("@")
            src = int(at)
        if role == "stem":
            a[..., 0] = -1.0 / (kh * kw * ci)
        elif role == "box":
            a[:, :, src, 0] = 1.0 / (kh * kw)
        elif role == "hbox":
            a[kh // 2, :, src, 0] = 1.0 / kw
        elif role == "carry":
            a[kh // 2, kw // 2, src, 0] = 1.0
        # "zero", "se", "rse": nothing reaches channel 0
        return a

    def b(self, n: int, role: str = "") -> np.ndarray:
        a = super().b(n, role)
        if role:
            a[0] = {"stem": 5.5, "se": 10.0, "rse": -10.0,
                    "convt_out": -self.GAIN * self.LEVEL}.get(role, 0.0)
        return a


def se_gate(b: PlanBuilder, x: Tensor, r: Init, *, reduce: int = 4,
            gate: str = "hardsigmoid") -> Tensor:
    """mean -> 1x1 c->c/reduce + ReLU -> 1x1 c/reduce->c + hard sigmoid."""
    mid = max(1, x.c // reduce)
    m = b.mean(x)
    h = b.conv(m, r.w((1, 1, x.c, mid), x.c), r.b(mid), fused="relu")
    role = "se" if gate == "hardsigmoid" else "rse"
    return b.conv(h, r.w((1, 1, mid, x.c), mid, role=role), r.b(x.c, role=role), fused=gate)


def dw_block(b: PlanBuilder, x: Tensor, r: Init, *, k: int, s=(1, 1), cout: int,
             se: bool = False, act: str = "hardswish", dw_role: str = "carry") -> Tensor:
    """Depthwise k x k (+bias, act) [-> SE gate] -> pointwise 1x1 (+bias);
    with stride 1 and equal channels the pointwise output is added to the
    block input (no activation after), else it takes the activation."""
    p = (k - 1) // 2
    d = b.dwconv(x, r.w((k, k, x.c), k * k, role=dw_role), r.b(x.c, role=dw_role), k=(k, k), s=s,
                 pad=(p, p, p, p), fused=act)
    if se:
        d = b.channelmul(d, se_gate(b, d, r))
    residual = s == (1, 1) and cout == x.c
    y = b.conv(d, r.w((1, 1, x.c, cout), x.c, role="carry"), r.b(cout, role="carry"),
               fused="none" if residual else act)
    return b.add(y, x) if residual else y


def fused_block_plan(*, h: int = 160, w: int = 160, c: int = 96, seed: int = 1,
                     init: str = "baseline", sigma: float = 0.05) -> bytes:
    """The single depthwise-separable block: dw 3x3 + bias + hard swish, SE
    (mean, FC c->c/4 ReLU, FC c/4->c hard sigmoid, channel scale), pointwise
    c->c + bias, plus the block input."""
    r = Init(seed, init, sigma)
    b = PlanBuilder(h, w, c)
    y = dw_block(b, b.input, r, k=3, cout=c, se=True)
    return b.to_bytes([y])


def rse(b: PlanBuilder, x: Tensor, r: Init, *, cout: int, k: int, role: str = "zero") -> Tensor:
    """Residual SE layer of the neck: conv, then y + y * gate with the 0.2
    hard sigmoid (plan.rs:160-163)."""
    p = (k - 1) // 2
    y = b.conv(x, r.w((k, k, x.c, cout), k * k * x.c, role=role), r.b(cout, role=role), k=(k, k),
               pad=(p, p, p, p))
    g = se_gate(b, y, r, gate="hardsigmoidfifth")
    return b.add(y, b.channelmul(y, g))


def detector_plan(*, h: int = 960, w: int = 960, seed: int = 3, init: str = "baseline",
                  sigma: float = 0.05) -> bytes:
    """A PP-OCR mobile-style DB detector: LCNet-style backbone, RSE-FPN neck
    of 96 channels, DB head to a 1-channel sigmoid map at the input size.
    Input sides must be multiples of 32. ``init="ink"`` draws the baseline
    weights and then sets those feeding channel 0 on the path to the map so
    that the map finds dark ink on light paper (`InkInit`)."""
    r = InkInit(seed, "baseline", sigma) if init == "ink" else Init(seed, init, sigma)
    b = PlanBuilder(h, w, 3)
    x = b.input
    act = "hardswish"
    s1 = b.conv(x, r.w((3, 3, 3, 24), 27, role="stem"), r.b(24, role="stem"), k=(3, 3), s=(2, 2),
                pad=(1, 1, 1, 1), fused=act)
    s2a = b.conv(s1, r.w((2, 2, 24, 12), 96, role="carry"), r.b(12, role="carry"), k=(2, 2),
                 pad=(0, 1, 0, 1), fused=act)
    s2b = b.conv(s2a, r.w((2, 2, 12, 24), 48, role="carry"), r.b(24, role="carry"), k=(2, 2),
                 pad=(0, 1, 0, 1), fused=act)
    pool = b.maxpool(s1)
    s3 = b.conv(pool, r.w((3, 3, 48, 32), 9 * 48, role="box"), r.b(32, role="box"), k=(3, 3),
                s=(2, 2), pad=(1, 1, 1, 1), fused=act, x2=s2b)
    z = b.conv(s3, r.w((1, 1, 32, 32), 32, role="carry"), r.b(32, role="carry"), fused=act)
    c2 = dw_block(b, z, r, k=3, cout=48, dw_role="hbox")
    z = dw_block(b, c2, r, k=3, s=(2, 2), cout=96)
    c3 = dw_block(b, z, r, k=3, cout=96)
    z = dw_block(b, c3, r, k=5, s=(2, 2), cout=192)
    z = dw_block(b, z, r, k=5, cout=192)
    c4 = dw_block(b, z, r, k=7, cout=192, se=True)
    z = dw_block(b, c4, r, k=5, s=(2, 2), cout=384, se=True)
    c5 = dw_block(b, z, r, k=7, cout=384, se=True)
    # Neck: 1x1 residual-SE inputs, top-down upsampled sums, 3x3 residual-SE
    # outputs, upsampled to 1/4 and stacked under the head's 3x3 conv.
    in5 = rse(b, c5, r, cout=96, k=1)
    in4 = rse(b, c4, r, cout=96, k=1)
    out4 = b.upsampleadd(in5, in4, 2)
    in3 = rse(b, c3, r, cout=96, k=1)
    out3 = b.upsampleadd(out4, in3, 2)
    in2 = rse(b, c2, r, cout=96, k=1, role="carry")
    out2 = b.upsampleadd(out3, in2, 2)
    p5 = rse(b, in5, r, cout=24, k=3)
    p4 = rse(b, out4, r, cout=24, k=3)
    p3 = rse(b, out3, r, cout=24, k=3)
    p2 = rse(b, out2, r, cout=24, k=3, role="hbox")
    up5 = b.upsample(p5, 8)
    up4 = b.upsample(p4, 4)
    cat = b.concat(up5, up4)
    up3 = b.upsample(p3, 2)
    cat = b.concat(cat, up3)
    # DB head: 3x3 conv over [p5 x8 | p4 x4 | p3 x2] and p2, ReLU; two 2x2
    # transposed convolutions, ReLU then the sigmoid.
    hd = b.conv(cat, r.w((3, 3, 96, 24), 9 * 96, role="hbox@72"), r.b(24, role="carry"), k=(3, 3),
                pad=(1, 1, 1, 1), fused="relu", x2=p2)
    hd = b.convtranspose(hd, r.w((24, 2, 2, 24), 24, role="convt"), r.b(24, role="convt"), k=(2, 2),
                         fused="relu")
    prob = b.convtranspose(hd, r.w((24, 2, 2, 1), 24, role="convt_out"), r.b(1, role="convt_out"),
                           k=(2, 2), fused="sigmoid")
    return b.to_bytes([prob])


def recognizer_plan(*, h: int = 48, w: int = 320, vocab: int = 18385, dim: int = 120,
                    heads: int = 8, depth: int = 2, seed: int = 4, init: str = "baseline",
                    sigma: float = 0.02, logits: bool = False) -> bytes:
    """An SVTR-style CTC recogniser: LCNet-style backbone with stride-(2,1)
    stages, average pool of the 3 remaining rows to W/4 time steps, a 1x1
    projection to `dim`, `depth` pre-norm transformer blocks (LayerNorm eps
    1e-6, `heads`-head attention, MLP ratio 2 with swish), a final
    LayerNorm and the CTC argmax head over `vocab` classes. With `logits`
    the same weights end in a plain 1x1 layer whose output is the logits
    (time steps x vocab), for checking them directly."""
    r = Init(seed, init, sigma, gain=1.6)
    b = PlanBuilder(h, w, 3)
    act = "hardswish"
    z = b.conv(b.input, r.w((3, 3, 3, 48), 27), r.b(48), k=(3, 3), s=(2, 2),
               pad=(1, 1, 1, 1), fused=act)
    z = dw_block(b, z, r, k=3, cout=64)
    z = dw_block(b, z, r, k=3, s=(2, 2), cout=128)
    z = dw_block(b, z, r, k=3, cout=128)
    z = dw_block(b, z, r, k=3, s=(2, 1), cout=256)
    z = dw_block(b, z, r, k=5, cout=256)
    z = dw_block(b, z, r, k=5, cout=256)
    z = dw_block(b, z, r, k=5, s=(2, 1), cout=480, se=True)
    z = dw_block(b, z, r, k=5, cout=480, se=True)
    z = b.avgpool(z, (z.h, 1), (z.h, 1))
    z = b.conv(z, r.w((1, 1, 480, dim), 480), r.b(dim), fused="swish")

    def ln(x):
        return b.layernorm(x, r.rng.normal(1.0, 0.1, dim), r.rng.normal(0.0, 0.1, dim), 1e-6)

    hd = dim // heads
    for _ in range(depth):
        n = ln(z)
        qkv = b.conv(n, r.w((1, 1, dim, 3 * dim), dim, 1.0), r.b(3 * dim))
        a = b.attention(qkv, heads, float(np.float32(hd ** -0.5)))
        p = b.conv(a, r.w((1, 1, dim, dim), dim, 1.0), r.b(dim))
        z = b.add(z, p)
        n = ln(z)
        f = b.conv(n, r.w((1, 1, dim, 2 * dim), dim), r.b(2 * dim), fused="swish")
        f = b.conv(f, r.w((1, 1, 2 * dim, dim), 2 * dim, 1.0), r.b(dim))
        z = b.add(z, f)
    n = ln(z)
    wv, bv = r.w((dim, vocab), dim, 1.0), r.b(vocab)
    out = b.conv(n, wv.reshape(1, 1, dim, vocab), bv) if logits else b.ctcargmax(n, wv, bv)
    return b.to_bytes([out])


def page_image(h: int = 960, w: int = 960, seed: int = 7) -> np.ndarray:
    """A synthetic page, HWC f32: white background with seeded dark
    horizontal stroke bands 20-40 px tall, normalised (v/255 - 0.5) / 0.5."""
    rng = np.random.default_rng(seed)
    img = np.full((h, w, 3), 255.0, np.float32)
    y = int(rng.integers(10, 40))
    while y < h - 20:
        band = min(int(rng.integers(20, 41)), h - y)
        x0 = int(rng.integers(0, w // 8))
        x1 = int(rng.integers(w // 2, w))
        strokes = rng.random((band, x1 - x0)) < 0.45
        shade = rng.integers(0, 90, size=(band, x1 - x0)).astype(np.float32)
        region = img[y:y + band, x0:x1]
        region[strokes] = shade[strokes][:, None]
        y += band + int(rng.integers(12, 40))
    return ((img / 255.0 - 0.5) / 0.5).astype(np.float32)


def letter_page(lines: int = 44, seed: int = 5, width: int = 2550, height: int = 3300) -> np.ndarray:
    """A letter page at 300 dpi, HWC uint8 RGB: white paper with `lines`
    seeded text-like lines of dark glyph blocks (24-30 px tall, word gaps),
    one every (height - 300) / lines pixels between 150 px margins."""
    rng = np.random.default_rng(seed)
    img = np.full((height, width, 3), 255, np.uint8)
    top, bottom = 150, height - 150
    pitch = (bottom - top) / lines
    for i in range(lines):
        y0 = int(top + i * pitch + rng.integers(0, 8))
        lh = int(rng.integers(24, 31))
        x = int(rng.integers(150, 260))
        end = int(rng.integers(width // 3, width - 150))
        while x < end:
            cw = int(rng.integers(14, 34))
            glyph = rng.random((lh, cw)) < 0.4
            img[y0:y0 + lh, x:x + cw][glyph] = int(rng.integers(0, 80))
            x += cw + int(rng.integers(4, 12))
            if rng.random() < 0.12:
                x += int(rng.integers(20, 40))
    return img


def line_images(n: int = 16, h: int = 48, w: int = 320, seed: int = 11) -> np.ndarray:
    """`n` text-line crops, HWC f32 in [-1, 1], of seeded stroke patterns."""
    rng = np.random.default_rng(seed)
    out = np.ones((n, h, w, 3), np.float32)
    for i in range(n):
        x = int(rng.integers(2, 12))
        end = int(rng.integers(w // 3, w - 2))
        while x < end:
            cw = int(rng.integers(8, 24))
            glyph = rng.random((h - 12, cw)) < 0.35
            val = rng.uniform(-1.0, -0.2)
            out[i, 6:h - 6, x:x + cw][glyph[:, :min(cw, w - x)]] = val
            x += cw + int(rng.integers(2, 8))
    return out
