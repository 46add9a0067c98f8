"""ONNX PP-OCR graphs to PPOCRPL1 plans: the graph-to-plan rules of the
engine's exporter (tools/export_ocr.py:96-870), over this package's plan
writer (`planfile.encode`) and ONNX reader (`onnxproto`).

The graph is traced at one size: a recogniser (input height 48) at width
320, a detector at a 64 x 64 page (export_ocr.py:97-103); every shape
below is worked out at that size, so the Shape / Slice / Concat nodes on
shapes fold to constants and the Reshape / Transpose / Squeeze / Identity
nodes of the recogniser's sequence part become aliases of one storage
(NHWC storage makes [1, C, 1, T] and [1, T, C] the same bytes). The rules:

- Conv, then an Add of a constant or a BatchNormalization folded in (the
  BN's scale and shift in float64 from the float32 epsilon,
  export_ocr.py:264-342), then the activation that alone reads it: Relu,
  HardSigmoid (alpha 0x3e2aaaad or 0.2, beta 0.5), Sigmoid, erf GELU
  (x/sqrt2 -> Erf -> +1 -> x*() -> *0.5), x*sigmoid(x) (:200-242); a
  depthwise conv (group = channels) becomes `dwconv`; weights to HWIO
  (HW-C for depthwise);
- ReduceMean over [2, 3] and GlobalAveragePool -> `mean`; ReduceMean over
  [-1] starts the written-out LayerNorm (Sub, Pow 2, ReduceMean, Add eps,
  Sqrt, Div, Mul gamma, Add beta) -> `layernorm` (:420-553);
- nearest, asymmetric, floor Resize by whole factors -> `upsample`, or
  `upsampleadd` when one Add of a map of the upsampled size reads it
  (:445-480); ConvTranspose whose windows tile -> `convtranspose` with the
  bias tiled over the window (:482-520);
- channel Concat -> a chain of `concatc`, its last input read in place by a
  windowed dense Conv that alone reads the concatenation (:378-418);
- Mul by a 1 x 1 x C map -> `channelmul`; Add of equal maps -> `add`;
  AveragePool without padding -> `avgpool`; the stem's SAME_UPPER stride-1
  2 x 2 MaxPool -> `maxpool` padded after (:344-376, 554-618);
- MatMul by a constant -> a 1 x 1 conv over the T steps (with the Add of a
  constant bias and the activation folded); MatMul + Add + Softmax over more
  than 4096 columns -> the CTC head, columns padded to a multiple of 16 in
  panels of 16 with bias -1e30 (`ctcargmax` with `argmax`, else `ctchead`)
  (:674-758);
- Reshape to [0, -1, 3, heads, dim] opens the attention block (Transpose,
  three Slice + Squeeze, the scale Mul, a zero Add, Transpose, MatMul,
  Softmax, MatMul, Transpose, Reshape) -> one `attention` (:760-822);
- every tensor its own buffer, aliases their root's; input buffer 0
  (:824-837).

Anything else is refused with the node that has no rule, as the reference
does. No `onnx` package and no PP-OCR model are in this image: the rules
are checked on graphs built in the tests, against a numpy evaluation of the
ONNX operators, through the CPU oracle.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import onnxproto
from .onnxproto import Graph, Node
from .planfile import Op, encode

WIDTH = 320  # the recogniser's traced width
PAGE = 64    # the detector's traced page
# HardSigmoid's (alpha, beta) as the exports carry them (export_ocr.py:91-94):
# alpha 0x3e2aaaad, the constant of the engine's hard sigmoid, or 0.2.
HARDSIGMOID = {
    (np.float32(0.16666670143604279), np.float32(0.5)): "hardsigmoid",
    (np.float32(0.2), np.float32(0.5)): "hardsigmoidfifth",
}


class ExportError(ValueError):
    """A graph the rules do not cover."""


@dataclass
class _Emit:
    kind: str
    x: str
    y: str
    x2: str | None = None
    fused: str = "none"
    f: dict = field(default_factory=dict)  # integer fields of the record
    w: tuple[int, int] = (0, 0)
    b: tuple[int, int] = (0, 0)


class Exporter:
    def __init__(self, graph: Graph, argmax: bool = False) -> None:
        self.g = graph
        self.argmax = argmax
        self.const: dict[str, np.ndarray] = {k: np.asarray(v) for k, v in graph.initializers.items()}
        if not graph.inputs:
            raise ExportError("the graph has no input")
        dims = list(graph.inputs[0].dims)
        if len(dims) != 4:
            raise ExportError("the input is not N x C x H x W")
        c = dims[1]
        h = dims[2] if isinstance(dims[2], int) and dims[2] > 0 else PAGE
        w = WIDTH if h == 48 else PAGE
        if not isinstance(c, int) or c <= 0:
            raise ExportError("the input's channel count is not fixed")
        self.hwc: dict[str, tuple[int, int, int]] = {graph.inputs[0].name: (h, w, c)}
        self.alias: dict[str, str] = {}
        self.pairs: dict[str, tuple[str, str]] = {}
        self.done: set[int] = set()
        self.emitted: list[_Emit] = []
        self.blob: list[np.ndarray] = []
        self.floats = 0
        # Identity nodes vanish: their readers read the Identity's input.
        same: dict[str, str] = {}
        self.nodes: list[Node] = []
        for n in graph.nodes:
            if n.op_type == "Identity":
                same[n.outputs[0]] = same.get(n.inputs[0], n.inputs[0])
            else:
                self.nodes.append(n)
        for n in self.nodes:
            n.inputs = [same.get(x, x) for x in n.inputs]
        self.outputs = [same.get(v.name, v.name) for v in graph.outputs]
        self.readers: dict[str, list[Node]] = {}
        for n in self.nodes:
            for x in n.inputs:
                self.readers.setdefault(x, []).append(n)

    # -------------------------------------------------------------- helpers

    def put(self, array) -> tuple[int, int]:
        """Weights on a 64-byte boundary; (start, length) in floats."""
        pad = (-self.floats) % 16
        if pad:
            self.blob.append(np.zeros(pad, np.float32))
            self.floats += pad
        data = np.ascontiguousarray(array, dtype=np.float32).reshape(-1)
        if not np.isfinite(data).all():
            raise ExportError("a weight that is not a finite number")
        start = self.floats
        self.blob.append(data)
        self.floats += data.size
        return start, int(data.size)

    def dims(self, name: str) -> tuple[int, int, int]:
        if name not in self.hwc:
            raise ExportError(f"no shape for tensor {name}")
        return self.hwc[name]

    def root(self, name: str) -> str:
        while name in self.alias:
            name = self.alias[name]
        return name

    def alias_to(self, out: str, src: str) -> None:
        self.alias[out] = src
        self.hwc[out] = self.hwc[src]

    def sole(self, name: str, op_type: str | None = None) -> Node | None:
        """The one node reading `name` (of `op_type`), if exactly one does."""
        r = self.readers.get(name, [])
        if len(r) != 1 or (op_type is not None and r[0].op_type != op_type):
            return None
        return r[0]

    def scalar(self, name: str) -> float | None:
        v = self.const.get(name)
        if v is None or v.size != 1:
            return None
        return float(v.reshape(-1)[0])

    def take(self, *nodes: Node) -> None:
        for n in nodes:
            self.done.add(id(n))

    @staticmethod
    def ints(node: Node, key: str, default=None):
        v = node.attrs.get(key, default)
        return [int(x) for x in v] if isinstance(v, (list, tuple, np.ndarray)) else v

    @staticmethod
    def text(node: Node, key: str, default: str = "") -> str:
        v = node.attrs.get(key)
        return v.decode() if isinstance(v, bytes) else default

    def emit(self, kind: str, x: str, y: str, hwc: tuple[int, int, int], x2: str | None = None,
             fused: str = "none", w=(0, 0), b=(0, 0), **f) -> None:
        self.hwc[y] = hwc
        self.emitted.append(_Emit(kind, x, y, x2, fused, f, w, b))

    # ------------------------------------------------------------ activation

    def activation(self, out: str) -> tuple[str, str]:
        """The activation that alone follows `out`: (fused kind, its output)."""
        r = self.readers.get(out, [])
        if len(r) == 1:
            n = r[0]
            if n.op_type == "Relu":
                self.take(n)
                return "relu", n.outputs[0]
            if n.op_type == "Sigmoid":
                self.take(n)
                return "sigmoid", n.outputs[0]
            if n.op_type == "HardSigmoid":
                key = (np.float32(n.attrs.get("alpha", 0.2)), np.float32(n.attrs.get("beta", 0.5)))
                if key not in HARDSIGMOID:
                    raise ExportError(f"HardSigmoid with alpha, beta {key}")
                self.take(n)
                return HARDSIGMOID[key], n.outputs[0]
        if len(r) == 2:
            kinds = sorted(n.op_type for n in r)
            if kinds == ["Div", "Mul"]:
                div = next(n for n in r if n.op_type == "Div")
                mul = next(n for n in r if n.op_type == "Mul")
                erf = self.sole(div.outputs[0], "Erf")
                one = self.sole(erf.outputs[0], "Add") if erf else None
                half = self.sole(mul.outputs[0], "Mul")
                root2 = self.scalar(div.inputs[1])
                if (root2 is not None and abs(root2 - np.sqrt(2.0)) < 1e-6 and one is not None
                        and self.scalar(one.inputs[1]) == 1.0 and one.outputs[0] in mul.inputs
                        and half is not None and self.scalar(half.inputs[1]) == 0.5):
                    self.take(div, erf, one, mul, half)
                    return "gelu", half.outputs[0]
            if kinds == ["Mul", "Sigmoid"]:
                sig = next(n for n in r if n.op_type == "Sigmoid")
                mul = next(n for n in r if n.op_type == "Mul")
                if sig.outputs[0] in mul.inputs and out in mul.inputs:
                    self.take(sig, mul)
                    return "swish", mul.outputs[0]
        return "none", out

    # ----------------------------------------------------------------- rules

    def run(self) -> None:
        for n in self.nodes:
            if id(n) in self.done:
                continue
            rule = getattr(self, "r_" + n.op_type.lower(), None)
            if rule is None:
                raise ExportError(f"no rule for {n.op_type} {n.name}")
            rule(n)

    def r_conv(self, n: Node) -> None:
        weight = self.const[n.inputs[1]].astype(np.float64)
        oc, per_group, kh, kw = weight.shape
        group = self.ints(n, "group", 1)
        sh, sw = self.ints(n, "strides", [1, 1])
        pads = self.ints(n, "pads", [0, 0, 0, 0])
        if self.ints(n, "dilations", [1, 1]) != [1, 1]:
            raise ExportError(f"dilated convolution {n.name}")
        auto = self.text(n, "auto_pad", "NOTSET")
        if auto == "SAME_UPPER":
            if (sh, sw) != (1, 1):
                raise ExportError("SAME_UPPER only at stride 1")
            pads = [(kh - 1) // 2, (kw - 1) // 2, kh // 2, kw // 2]
        elif auto not in ("NOTSET", "VALID"):
            raise ExportError(f"auto_pad {auto}")
        x, second = self.pairs.get(n.inputs[0], (n.inputs[0], None))
        ih, iw, ic = self.dims(x)
        n2 = self.dims(second)[2] if second else 0
        bias = self.const[n.inputs[2]].astype(np.float64) if len(n.inputs) > 2 else np.zeros(oc)
        out = n.outputs[0]
        nxt = self.sole(out)
        if nxt is not None and nxt.op_type == "Add" and nxt.inputs[1] in self.const:
            bias = bias + self.const[nxt.inputs[1]].reshape(-1).astype(np.float64)
            self.take(nxt)
            out = nxt.outputs[0]
        elif nxt is not None and nxt.op_type == "BatchNormalization":
            gamma, beta, mean, var = (self.const[t].astype(np.float64) for t in nxt.inputs[1:5])
            eps = np.float64(np.float32(nxt.attrs.get("epsilon", 1e-5)))
            scale = gamma / np.sqrt(var + eps)
            weight = weight * scale[:, None, None, None]
            bias = (bias - mean) * scale + beta
            self.take(nxt)
            out = nxt.outputs[0]
        fused, out = self.activation(out)
        oh = (ih + pads[0] + pads[2] - kh) // sh + 1
        ow = (iw + pads[1] + pads[3] - kw) // sw + 1
        depthwise = group > 1 and per_group == 1
        if depthwise:
            if not group == ic == oc:
                raise ExportError("grouped convolution that is not depthwise")
            packed = weight.reshape(oc, kh, kw).transpose(1, 2, 0)
        else:
            if group != 1:
                raise ExportError("grouped convolution")
            if per_group != ic + n2:
                raise ExportError(f"convolution {n.name} reads {ic + n2} channels, weights take {per_group}")
            packed = weight.transpose(2, 3, 1, 0)
        self.emit("dwconv" if depthwise else "conv", x, out, (oh, ow, oc), x2=second, fused=fused,
                  w=self.put(packed), b=self.put(bias), ic=ic, oc=oc, kh=kh, kw=kw, sh=sh, sw=sw,
                  pt=pads[0], pl=pads[1], pb=pads[2], pr=pads[3], n2=n2)

    def r_maxpool(self, n: Node) -> None:
        kh, kw = self.ints(n, "kernel_shape")
        sh, sw = self.ints(n, "strides", [1, 1])
        if (self.text(n, "auto_pad") != "SAME_UPPER" or (sh, sw) != (1, 1)
                or self.ints(n, "dilations", [1, 1]) != [1, 1] or max(kh, kw) > 2):
            raise ExportError("only the stem's SAME_UPPER stride-1 2x2 max pool")
        ih, iw, ic = self.dims(n.inputs[0])
        self.emit("maxpool", n.inputs[0], n.outputs[0], (ih, iw, ic), ic=ic, oc=ic, kh=kh, kw=kw, sh=1,
                  sw=1, pb=kh - 1, pr=kw - 1)

    def r_concat(self, n: Node) -> None:
        if all(x in self.const for x in n.inputs):
            self.const[n.outputs[0]] = np.concatenate([self.const[x].reshape(-1) for x in n.inputs])
            return
        if self.ints(n, "axis") != 1:
            raise ExportError("only channel concatenation")
        conv = self.sole(n.outputs[0], "Conv")
        inplace = (conv is not None and self.ints(conv, "group", 1) == 1
                   and self.const[conv.inputs[1]].shape[2:] != (1, 1))
        head, last = n.inputs[0], len(n.inputs) - int(inplace)
        for k in range(1, last):
            name = n.inputs[k]
            (h, w, c), (h2, w2, c2) = self.dims(head), self.dims(name)
            if (h2, w2) != (h, w):
                raise ExportError("concatenated maps differ in size")
            out = n.outputs[0] if k == len(n.inputs) - 1 else f"{n.outputs[0]}/{k + 1}"
            self.emit("concatc", head, out, (h, w, c + c2), x2=name, ic=c, oc=c + c2, n2=c2)
            head = out
        if inplace:
            (h, w, c), (h2, w2, c2) = self.dims(head), self.dims(n.inputs[-1])
            if (h2, w2) != (h, w):
                raise ExportError("concatenated maps differ in size")
            self.hwc[n.outputs[0]] = (h, w, c + c2)
            self.pairs[n.outputs[0]] = (head, n.inputs[-1])

    def r_reducemean(self, n: Node) -> None:
        axes = self.ints(n, "axes")
        if axes == [2, 3]:
            self.r_globalaveragepool(n)
        elif axes == [-1]:
            self.layernorm(n)
        else:
            raise ExportError(f"ReduceMean over {axes}")

    def r_globalaveragepool(self, n: Node) -> None:
        ih, iw, ic = self.dims(n.inputs[0])
        self.emit("mean", n.inputs[0], n.outputs[0], (1, 1, ic), ic=ic, oc=ic)

    def r_resize(self, n: Node) -> None:
        modes = {k: v.decode() for k, v in n.attrs.items() if isinstance(v, bytes) and v}
        want = {"mode": "nearest", "coordinate_transformation_mode": "asymmetric", "nearest_mode": "floor"}
        scales = self.const.get(n.inputs[2]) if len(n.inputs) > 2 else None
        if modes != want or scales is None or scales.size != 4:
            raise ExportError(f"unsupported Resize {n.name}")
        scales = scales.reshape(-1)
        fh, fw = int(scales[2]), int(scales[3])
        if list(scales) != [1, 1, fh, fw]:
            raise ExportError("Resize by a fractional factor")
        ih, iw, ic = self.dims(n.inputs[0])
        out, kind, second = n.outputs[0], "upsample", None
        add = self.sole(out, "Add")
        if add is not None:
            other = add.inputs[1] if add.inputs[0] == out else add.inputs[0]
            if other in self.hwc and self.dims(other) == (ih * fh, iw * fw, ic):
                self.take(add)
                out, kind, second = add.outputs[0], "upsampleadd", other
        self.emit(kind, n.inputs[0], out, (ih * fh, iw * fw, ic), x2=second, ic=ic, oc=ic, sh=fh, sw=fw)

    def r_convtranspose(self, n: Node) -> None:
        weight = self.const[n.inputs[1]]
        ic, oc, kh, kw = weight.shape
        if (self.ints(n, "strides") != [kh, kw] or any(self.ints(n, "pads", [0, 0, 0, 0]))
                or self.ints(n, "group", 1) != 1 or self.ints(n, "dilations", [1, 1]) != [1, 1]):
            raise ExportError("only transposed convolutions whose windows tile")
        # The bias: the node's own third input (which export_ocr.py:493
        # leaves out; the PP-OCR exports carry theirs in an Add) plus an Add
        # of a constant that alone follows.
        bias = self.const[n.inputs[2]].reshape(-1).astype(np.float64) if len(n.inputs) > 2 else np.zeros(oc)
        out = n.outputs[0]
        nxt = self.sole(out, "Add")
        if nxt is not None and nxt.inputs[1] in self.const:
            bias = bias + self.const[nxt.inputs[1]].reshape(-1)
            self.take(nxt)
            out = nxt.outputs[0]
        fused, out = self.activation(out)
        ih, iw, _ = self.dims(n.inputs[0])
        self.emit("convtranspose", n.inputs[0], out, (ih * kh, iw * kw, oc), fused=fused,
                  w=self.put(weight.transpose(0, 2, 3, 1)), b=self.put(np.tile(bias, kh * kw)),
                  ic=ic, oc=oc, kh=kh, kw=kw, sh=kh, sw=kw)

    def layernorm(self, mean: Node) -> None:
        x = mean.inputs[0]
        sub = next((u for u in self.readers[x] if u.op_type == "Sub"), None)
        if sub is None:
            raise ExportError("not a layer normalization")
        after = self.readers.get(sub.outputs[0], [])
        pw = next((u for u in after if u.op_type == "Pow"), None)
        div = next((u for u in after if u.op_type == "Div"), None)
        var = self.sole(pw.outputs[0], "ReduceMean") if pw else None
        add = self.sole(var.outputs[0], "Add") if var else None
        sqrt = self.sole(add.outputs[0], "Sqrt") if add else None
        mul = self.sole(div.outputs[0], "Mul") if div else None
        beta = self.sole(mul.outputs[0], "Add") if mul else None
        if (beta is None or sqrt is None or self.scalar(pw.inputs[1]) != 2.0
                or div.inputs[1] != sqrt.outputs[0]):
            raise ExportError("not a layer normalization")
        eps = self.const[add.inputs[1]].reshape(-1)
        gamma = self.const[mul.inputs[1]].reshape(-1)
        shift = self.const[beta.inputs[1]].reshape(-1)
        self.take(mean, sub, pw, var, add, sqrt, div, mul, beta)
        h, w, c = self.dims(x)
        self.emit("layernorm", x, beta.outputs[0], (h, w, c), ic=c, oc=c,
                  w=self.put(np.concatenate([gamma, shift, eps])))

    def r_mul(self, n: Node) -> None:
        a, b = n.inputs
        if b in self.const or a in self.const:
            raise ExportError(f"unexpected constant Mul {n.name}")
        (ha, wa, ca), (hb, wb, cb) = self.dims(a), self.dims(b)
        if (hb, wb) == (1, 1) and cb == ca and (ha, wa) != (1, 1):
            self.emit("channelmul", a, n.outputs[0], (ha, wa, ca), x2=b, ic=ca, oc=ca)
            return
        raise ExportError(f"unsupported Mul {n.name}")

    def r_add(self, n: Node) -> None:
        a, b = n.inputs
        if a in self.const or b in self.const:
            raise ExportError(f"constant Add {n.name} not folded")
        if self.dims(a) != self.dims(b):
            raise ExportError(f"Add of different shapes {n.name}")
        h, w, c = self.dims(a)
        self.emit("add", a, n.outputs[0], (h, w, c), x2=b, ic=c, oc=c)

    def r_averagepool(self, n: Node) -> None:
        if any(self.ints(n, "pads", [0, 0, 0, 0])) or self.text(n, "auto_pad", "NOTSET") not in ("NOTSET", "VALID"):
            raise ExportError("padded average pool")
        if self.ints(n, "ceil_mode", 0):
            raise ExportError("average pool rounding its output up")
        kh, kw = self.ints(n, "kernel_shape")
        sh, sw = self.ints(n, "strides", [1, 1])
        ih, iw, ic = self.dims(n.inputs[0])
        oh, ow = (ih - kh) // sh + 1, (iw - kw) // sw + 1
        self.emit("avgpool", n.inputs[0], n.outputs[0], (oh, ow, ic), ic=ic, oc=ic, kh=kh, kw=kw, sh=sh, sw=sw)

    # Shapes are constants at the traced size.
    def r_shape(self, n: Node) -> None:
        h, w, c = self.dims(n.inputs[0])
        self.const[n.outputs[0]] = np.array([1, c, h, w], np.int64)

    def r_slice(self, n: Node) -> None:
        if n.inputs[0] not in self.const:
            raise ExportError("Slice of a runtime tensor outside attention")
        data = self.const[n.inputs[0]]
        starts, ends = self.const[n.inputs[1]].reshape(-1), self.const[n.inputs[2]].reshape(-1)
        axes = self.const[n.inputs[3]].reshape(-1) if len(n.inputs) > 3 else np.array([0])
        if list(axes) != [0]:
            raise ExportError("Slice of a shape on another axis")
        self.const[n.outputs[0]] = data[int(starts[0]):int(ends[0])]

    def r_squeeze(self, n: Node) -> None:
        if n.inputs[0] in self.const:
            self.const[n.outputs[0]] = self.const[n.inputs[0]].reshape(())
            return
        h, _, _ = self.dims(n.inputs[0])
        if self.ints(n, "axes") != [2] or h != 1:
            raise ExportError("unsupported Squeeze")
        self.alias_to(n.outputs[0], n.inputs[0])

    def r_unsqueeze(self, n: Node) -> None:
        if n.inputs[0] not in self.const:
            raise ExportError("Unsqueeze of a runtime tensor")
        self.const[n.outputs[0]] = self.const[n.inputs[0]].reshape(1)

    def r_reshape(self, n: Node) -> None:
        if n.inputs[0] in self.const:
            self.const[n.outputs[0]] = self.const[n.inputs[0]].reshape(self.const[n.inputs[1]])
            return
        target = [int(v) for v in self.const[n.inputs[1]].reshape(-1)]
        if len(target) == 5 and target[:3] == [0, -1, 3]:
            self.attention(n, target[3], target[4])
            return
        h, w, c = self.dims(n.inputs[0])
        if h == 1 and target in ([1, c, -1], [1, c, w], [0, 1, -1, c], [0, 1, w, c]):
            self.alias_to(n.outputs[0], n.inputs[0])
            return
        raise ExportError(f"unsupported Reshape to {target}")

    def r_transpose(self, n: Node) -> None:
        perm = self.ints(n, "perm")
        h, _, _ = self.dims(n.inputs[0])
        if h == 1 and perm in ([0, 2, 1], [0, 3, 1, 2]):
            self.alias_to(n.outputs[0], n.inputs[0])
            return
        raise ExportError(f"unsupported Transpose {perm}")

    def r_matmul(self, n: Node) -> None:
        x, wname = n.inputs
        if wname not in self.const:
            raise ExportError("MatMul of two runtime tensors outside attention")
        weight = self.const[wname]
        ci, co = weight.shape
        h, t, c = self.dims(x)
        if (h, c) != (1, ci):
            raise ExportError("MatMul input is not [T][C]")
        out = n.outputs[0]
        add = self.sole(out, "Add")
        soft = self.sole(add.outputs[0], "Softmax") if add is not None else None
        if co > 4096 and soft is not None:
            self.ctc_head(x, weight, self.const[add.inputs[1]].reshape(-1), add, soft)
            return
        bias = np.zeros(co, np.float32)
        if add is not None and add.inputs[1] in self.const:
            bias = self.const[add.inputs[1]].reshape(-1)
            self.take(add)
            out = add.outputs[0]
        fused, out = self.activation(out)
        self.emit("conv", x, out, (1, t, co), fused=fused, w=self.put(weight), b=self.put(bias), ic=ci, oc=co,
                  kh=1, kw=1, sh=1, sw=1)

    def ctc_head(self, x: str, weight: np.ndarray, bias: np.ndarray, add: Node, soft: Node) -> None:
        ci, vocab = weight.shape
        cols = -(-vocab // 16) * 16
        padded = np.zeros((ci, cols), np.float32)
        padded[:, :vocab] = weight
        panels = padded.reshape(ci, cols // 16, 16).transpose(1, 0, 2)  # [panel][ci][16]
        b = np.full(cols, -1e30, np.float32)
        b[:vocab] = bias
        _, t, _ = self.dims(x)
        self.take(add, soft)
        out = soft.outputs[0]
        if self.argmax:
            self.emit("ctcargmax", x, out, (1, t, 2), w=self.put(panels), b=self.put(b), ic=ci, oc=2, n2=vocab)
        else:
            self.emit("ctchead", x, out, (1, t, vocab), w=self.put(panels), b=self.put(b), ic=ci, oc=vocab)

    def attention(self, start: Node, heads: int, dim: int) -> None:
        qkv = start.inputs[0]
        _, t, c3 = self.dims(qkv)
        if heads * dim * 3 != c3:
            raise ExportError("attention heads do not split the q|k|v width")
        seen, todo, end, scale = [start], [start], None, None
        while todo:
            node = todo.pop()
            for user in self.readers.get(node.outputs[0], []):
                if any(user is s for s in seen):
                    continue
                seen.append(user)
                if user.op_type == "Reshape":
                    end = user
                    continue
                if user.op_type == "Mul":
                    scale = self.scalar(user.inputs[1])
                if user.op_type == "Add" and self.scalar(user.inputs[1]) not in (0.0, None):
                    raise ExportError("attention bias is not zero")
                todo.append(user)
        expect = sorted(["Reshape", "Transpose", "Slice", "Squeeze", "Slice", "Squeeze", "Slice", "Squeeze", "Mul",
                         "Add", "Transpose", "MatMul", "Softmax", "MatMul", "Transpose", "Reshape"])
        if sorted(s.op_type for s in seen) != expect or end is None or scale is None:
            raise ExportError(f"not the expected attention block: {sorted(s.op_type for s in seen)}")
        self.take(*seen)
        c = c3 // 3
        self.emit("attention", qkv, end.outputs[0], (1, t, c), w=self.put(np.array([scale], np.float32)), ic=c3,
                  oc=c, n2=heads)

    # ---------------------------------------------------------------- output

    def plan(self) -> bytes:
        """Convert and write the plan bytes."""
        self.run()
        name = self.g.inputs[0].name
        slot = {self.root(name): 0}
        for e in self.emitted:
            e.x, e.y = self.root(e.x), self.root(e.y)
            if e.x2 is not None:
                e.x2 = self.root(e.x2)
            slot.setdefault(e.y, len(slot))
        ops = []
        for e in self.emitted:
            f = dict(e.f)
            if e.x not in slot or (e.x2 is not None and e.x2 not in slot):
                raise ExportError(f"{e.kind} reads a tensor nothing writes")
            ops.append(Op(e.kind, slot[e.x], slot[e.y], f.pop("ic", 0), f.pop("oc", 0), fused=e.fused,
                          x2=slot[e.x2] if e.x2 is not None else 0, w=e.w, b=e.b, **f))
        outs = []
        for o in self.outputs:
            if self.root(o) not in slot:
                raise ExportError(f"output {o} is not computed")
            outs.append(slot[self.root(o)])
        h, w, c = self.dims(name)
        for op in ops:
            if min(op.words()) < 0 or max(op.words()) >= 1 << 32:
                raise ExportError("a field does not fit the plan's 32-bit words")
        weights = np.concatenate(self.blob) if self.blob else np.zeros(0, np.float32)
        return encode((0, h, w, c), len(slot), outs, ops, weights)


def export(model, argmax: bool = False) -> bytes:
    """Plan bytes for an ONNX model: a path, ModelProto bytes or a Graph."""
    if isinstance(model, Graph):
        graph = model
    elif isinstance(model, (bytes, bytearray)):
        graph = onnxproto.decode_model(bytes(model))
    else:
        graph = onnxproto.load(model)
    return Exporter(graph, argmax).plan()


def main(argv=None) -> int:
    import argparse
    from pathlib import Path
    p = argparse.ArgumentParser(description="ONNX PP-OCR model to a PPOCRPL1 plan")
    p.add_argument("model", type=Path)
    p.add_argument("plan", type=Path)
    p.add_argument("--argmax", action="store_true",
                   help="each step's best class and probability instead of all probabilities")
    a = p.parse_args(argv)
    data = export(a.model, a.argmax)
    a.plan.parent.mkdir(parents=True, exist_ok=True)
    a.plan.write_bytes(data)
    print(f"{a.plan}: {len(data)} bytes")
    return 0
