"""PPOCRPL1 plan files: the op vocabulary and a writer.

The layout is the engine's own (src/engine/plan.rs:9-20, written by
tools/export_ocr.py:839-870): the magic ``PPOCRPL1``; seven little-endian
u32 (input buffer, input height, width, channels, buffer count, output
count, operation count); one u32 per output buffer; 20 u32 per operation
(kind, folded activation, x, x2, y, ic, oc, kh, kw, sh, sw, pt, pb, pl, pr,
n2, weights start and length, bias start and length, counted in floats);
zero padding to a 64-byte boundary; then the weights as f32 to the end.

Kind and activation codes keep the reference's order (plan.rs:130-175).
Activation code 7, hard swish, is this backend's extension: the reference
reads codes 0-6 only, so a plan using it is not readable there.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"PPOCRPL1"
OP_FIELDS = 20

KINDS = [
    "conv", "dwconv", "add", "maxpool", "avgpool", "channelmul", "concatc",
    "layernorm", "attention", "mean", "ctchead", "ctcargmax", "upsample",
    "upsampleadd", "convtranspose",
]
FUSED = [
    "none", "relu", "sigmoid", "gelu", "swish", "hardsigmoid",
    "hardsigmoidfifth", "hardswish",
]


@dataclass
class Op:
    """One operation record; spatial sizes are derived on load."""

    kind: str
    x: int
    y: int
    ic: int
    oc: int
    fused: str = "none"
    x2: int = 0
    kh: int = 0
    kw: int = 0
    sh: int = 0
    sw: int = 0
    pt: int = 0
    pb: int = 0
    pl: int = 0
    pr: int = 0
    n2: int = 0
    w: tuple[int, int] = (0, 0)
    b: tuple[int, int] = (0, 0)

    def words(self) -> list[int]:
        return [
            KINDS.index(self.kind), FUSED.index(self.fused), self.x, self.x2, self.y,
            self.ic, self.oc, self.kh, self.kw, self.sh, self.sw, self.pt, self.pb,
            self.pl, self.pr, self.n2, self.w[0], self.w[1], self.b[0], self.b[1],
        ]


def encode(input_: tuple[int, int, int, int], buffers: int, outputs: list[int],
           ops: list[Op], weights: np.ndarray) -> bytes:
    """A plan file laid out as plan.rs:848-898 writes one."""
    slot, h, w, c = input_
    words = [slot, h, w, c, buffers, len(outputs), len(ops), *outputs]
    for op in ops:
        words += op.words()
    head = MAGIC + struct.pack(f"<{len(words)}I", *words)
    head += b"\0" * (-len(head) % 64)
    return head + np.ascontiguousarray(weights, dtype="<f4").tobytes()


def flush_subnormals(a: np.ndarray) -> np.ndarray:
    """Subnormal values to signed zero, as plan.rs:819-842 loads them."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = a.view(np.uint32)
    sub = (bits & 0x7F800000) == 0
    out = bits.copy()
    out[sub] &= 0x80000000
    return out.view(np.float32)


@dataclass
class Tensor:
    slot: int
    h: int
    w: int
    c: int


@dataclass
class PlanBuilder:
    """Emits operations in run order, one buffer per tensor, weights on
    64-byte boundaries (tools/export_ocr.py:143-153, 830-836)."""

    h: int
    w: int
    c: int
    ops: list[Op] = field(default_factory=list)
    blob: list[np.ndarray] = field(default_factory=list)
    floats: int = 0
    slots: int = 1

    def __post_init__(self) -> None:
        self.input = Tensor(0, self.h, self.w, self.c)

    # -- storage
    def put(self, array: np.ndarray) -> tuple[int, int]:
        pad = (-self.floats) % 16
        if pad:
            self.blob.append(np.zeros(pad, np.float32))
            self.floats += pad
        data = flush_subnormals(np.asarray(array, np.float32).reshape(-1))
        if not np.isfinite(data).all():
            raise ValueError("refusing a weight that is not a finite number")
        start = self.floats
        self.blob.append(data)
        self.floats += data.size
        return (start, int(data.size))

    def new(self, h: int, w: int, c: int) -> Tensor:
        t = Tensor(self.slots, h, w, c)
        self.slots += 1
        return t

    def emit(self, op: Op, h: int, w: int, c: int) -> Tensor:
        y = self.new(h, w, c)
        op.y = y.slot
        self.ops.append(op)
        return y

    # -- operations
    def conv(self, x: Tensor, weight: np.ndarray, bias: np.ndarray | None, *, k=(1, 1),
             s=(1, 1), pad=(0, 0, 0, 0), fused="none", x2: Tensor | None = None) -> Tensor:
        """Dense convolution; weight is [kh][kw][ic + n2][oc]."""
        kh, kw = k
        n2 = x2.c if x2 is not None else 0
        oc = weight.shape[-1]
        assert weight.shape == (kh, kw, x.c + n2, oc), weight.shape
        pt, pb, pl, pr = pad
        oh = (x.h + pt + pb - kh) // s[0] + 1
        ow = (x.w + pl + pr - kw) // s[1] + 1
        op = Op("conv", x.slot, 0, x.c, oc, fused, x2.slot if x2 else 0, kh, kw, s[0], s[1],
                pt, pb, pl, pr, n2, self.put(weight),
                self.put(bias) if bias is not None else (0, 0))
        return self.emit(op, oh, ow, oc)

    def dwconv(self, x: Tensor, weight: np.ndarray, bias: np.ndarray | None, *, k, s=(1, 1),
               pad=None, fused="none") -> Tensor:
        """Depthwise convolution; weight is [kh][kw][c]."""
        kh, kw = k
        if pad is None:
            pad = ((kh - 1) // 2, (kh - 1) // 2, (kw - 1) // 2, (kw - 1) // 2)
        assert weight.shape == (kh, kw, x.c)
        pt, pb, pl, pr = pad
        oh = (x.h + pt + pb - kh) // s[0] + 1
        ow = (x.w + pl + pr - kw) // s[1] + 1
        op = Op("dwconv", x.slot, 0, x.c, x.c, fused, 0, kh, kw, s[0], s[1], pt, pb, pl, pr, 0,
                self.put(weight), self.put(bias) if bias is not None else (0, 0))
        return self.emit(op, oh, ow, x.c)

    def add(self, a: Tensor, b: Tensor, fused="none") -> Tensor:
        assert (a.h, a.w, a.c) == (b.h, b.w, b.c)
        return self.emit(Op("add", a.slot, 0, a.c, a.c, fused, b.slot), a.h, a.w, a.c)

    def channelmul(self, x: Tensor, gate: Tensor) -> Tensor:
        assert (gate.h, gate.w, gate.c) == (1, 1, x.c)
        return self.emit(Op("channelmul", x.slot, 0, x.c, x.c, x2=gate.slot), x.h, x.w, x.c)

    def mean(self, x: Tensor) -> Tensor:
        return self.emit(Op("mean", x.slot, 0, x.c, x.c), 1, 1, x.c)

    def maxpool(self, x: Tensor, k=(2, 2), s=(1, 1), pad_after=(1, 1)) -> Tensor:
        oh = (x.h + pad_after[0] - k[0]) // s[0] + 1
        ow = (x.w + pad_after[1] - k[1]) // s[1] + 1
        op = Op("maxpool", x.slot, 0, x.c, x.c, kh=k[0], kw=k[1], sh=s[0], sw=s[1],
                pb=pad_after[0], pr=pad_after[1])
        return self.emit(op, oh, ow, x.c)

    def avgpool(self, x: Tensor, k, s) -> Tensor:
        oh = (x.h - k[0]) // s[0] + 1
        ow = (x.w - k[1]) // s[1] + 1
        op = Op("avgpool", x.slot, 0, x.c, x.c, kh=k[0], kw=k[1], sh=s[0], sw=s[1])
        return self.emit(op, oh, ow, x.c)

    def concat(self, a: Tensor, b: Tensor) -> Tensor:
        assert (a.h, a.w) == (b.h, b.w)
        op = Op("concatc", a.slot, 0, a.c, a.c + b.c, x2=b.slot, n2=b.c)
        return self.emit(op, a.h, a.w, a.c + b.c)

    def upsample(self, x: Tensor, f) -> Tensor:
        """Nearest upsampling by a whole factor, or (height, width) factors."""
        fh, fw = (f, f) if isinstance(f, int) else f
        return self.emit(Op("upsample", x.slot, 0, x.c, x.c, sh=fh, sw=fw), x.h * fh, x.w * fw, x.c)

    def upsampleadd(self, x: Tensor, addend: Tensor, f) -> Tensor:
        fh, fw = (f, f) if isinstance(f, int) else f
        assert (addend.h, addend.w, addend.c) == (x.h * fh, x.w * fw, x.c)
        op = Op("upsampleadd", x.slot, 0, x.c, x.c, x2=addend.slot, sh=fh, sw=fw)
        return self.emit(op, x.h * fh, x.w * fw, x.c)

    def layernorm(self, x: Tensor, gamma, beta, eps: float) -> Tensor:
        wts = np.concatenate([gamma, beta, [eps]]).astype(np.float32)
        return self.emit(Op("layernorm", x.slot, 0, x.c, x.c, w=self.put(wts)), x.h, x.w, x.c)

    def attention(self, qkv: Tensor, heads: int, scale: float) -> Tensor:
        c = qkv.c // 3
        op = Op("attention", qkv.slot, 0, qkv.c, c, n2=heads,
                w=self.put(np.array([scale], np.float32)))
        return self.emit(op, qkv.h, qkv.w, c)

    def convtranspose(self, x: Tensor, weight: np.ndarray, bias: np.ndarray | None, *, k,
                      fused="none") -> Tensor:
        """Non-overlapping transposed conv; weight is [ic][kh][kw][oc], bias [oc]."""
        kh, kw = k
        oc = weight.shape[-1]
        assert weight.shape == (x.c, kh, kw, oc)
        b = self.put(np.tile(bias, kh * kw)) if bias is not None else (0, 0)
        op = Op("convtranspose", x.slot, 0, x.c, oc, fused, kh=kh, kw=kw, sh=kh, sw=kw,
                w=self.put(weight), b=b)
        return self.emit(op, x.h * kh, x.w * kw, oc)

    def ctc(self, x: Tensor, weight: np.ndarray, bias: np.ndarray, argmax: bool = True) -> Tensor:
        """CTC head over [ic][vocab] weights: each step's best class and its
        probability (`ctcargmax`), or every class's probability (`ctchead`).
        The engine reads the weights in panels of 16 columns, zero weights and
        -1e30 bias past the vocabulary (tools/export_ocr.py:716-724)."""
        ci, vocab = weight.shape
        columns = -(-vocab // 16) * 16
        padded = np.zeros((ci, columns), np.float32)
        padded[:, :vocab] = weight
        panels = padded.reshape(ci, columns // 16, 16).transpose(1, 0, 2)
        b = np.full(columns, -1e30, np.float32)
        b[:vocab] = np.asarray(bias, np.float32).reshape(-1)
        if argmax:
            op = Op("ctcargmax", x.slot, 0, ci, 2, n2=vocab, w=self.put(panels), b=self.put(b))
            return self.emit(op, x.h, x.w, 2)
        op = Op("ctchead", x.slot, 0, ci, vocab, w=self.put(panels), b=self.put(b))
        return self.emit(op, x.h, x.w, vocab)

    def ctcargmax(self, x: Tensor, weight: np.ndarray, bias: np.ndarray) -> Tensor:
        return self.ctc(x, weight, bias, argmax=True)

    def to_bytes(self, outputs: list[Tensor]) -> bytes:
        weights = np.concatenate(self.blob) if self.blob else np.zeros(0, np.float32)
        return encode((0, self.h, self.w, self.c), self.slots, [t.slot for t in outputs],
                      self.ops, weights)
