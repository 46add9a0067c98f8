"""Test infrastructure for the exporter: an ONNX graph builder and a numpy
evaluation of the ONNX operators PP-OCR graphs use (float64, NCHW, the
operator definitions of the ONNX specification, opset 11 attributes).

The evaluation is the check: a graph exported to a plan and run on the CPU
oracle must give what the graph itself computes.
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from ppocr_native_amd.onnxproto import Graph, Node, Value


class GraphMaker:
    """Nodes in order, constants as initializers, one output name each."""

    def __init__(self, name: str, dims: list) -> None:
        self.nodes: list[Node] = []
        self.inits: dict[str, np.ndarray] = {}
        self.input = Value(name, list(dims))
        self.outs: list[str] = []
        self.k = 0

    def const(self, value, dtype=np.float32) -> str:
        self.k += 1
        name = f"c{self.k}"
        self.inits[name] = np.asarray(value, dtype=dtype)
        return name

    def op(self, op_type: str, *inputs: str, n_out: int = 1, **attrs):
        self.k += 1
        outs = [f"{op_type.lower()}{self.k}_{i}" for i in range(n_out)]
        self.nodes.append(Node(op_type, list(inputs), outs, name=f"{op_type}_{self.k}", attrs=attrs))
        return outs[0] if n_out == 1 else outs

    def output(self, name: str) -> None:
        self.outs.append(name)

    def graph(self) -> Graph:
        return Graph(self.nodes, dict(self.inits), [self.input], [Value(o, []) for o in self.outs])


def _pad_hw(x, pads, value=0.0):
    t, l, b, r = pads
    return np.pad(x, ((0, 0), (0, 0), (t, b), (l, r)), constant_values=value)


def _conv(x, w, b, a):
    group = a.get("group", 1)
    sh, sw = a.get("strides", [1, 1])
    oc, cpg, kh, kw = w.shape
    pads = a.get("pads", [0, 0, 0, 0])
    if a.get("auto_pad", b"NOTSET") in (b"SAME_UPPER", "SAME_UPPER"):
        pads = [(kh - 1) // 2, (kw - 1) // 2, kh // 2, kw // 2]
    xp = _pad_hw(x, (pads[0], pads[1], pads[2], pads[3]))
    n, c, hp, wp = xp.shape
    oh, ow = (hp - kh) // sh + 1, (wp - kw) // sw + 1
    y = np.zeros((n, oc, oh, ow))
    opg = oc // group
    for g in range(group):
        xs = xp[:, g * cpg:(g + 1) * cpg]
        ws = w[g * opg:(g + 1) * opg]
        for ky in range(kh):
            for kx in range(kw):
                patch = xs[:, :, ky:ky + sh * (oh - 1) + 1:sh, kx:kx + sw * (ow - 1) + 1:sw]
                y[:, g * opg:(g + 1) * opg] += np.einsum("nchw,oc->nohw", patch, ws[:, :, ky, kx])
    if b is not None:
        y += b.reshape(1, -1, 1, 1)
    return y


def _softmax(x, axis):
    e = np.exp(x - x.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


def evaluate(g: Graph, x: np.ndarray) -> list[np.ndarray]:
    """The graph's outputs for input x (float64)."""
    v = {k: np.asarray(a) for k, a in g.initializers.items()}
    v[g.inputs[0].name] = np.asarray(x, np.float64)
    for n in g.nodes:
        a, i = n.attrs, [v[name] if name else None for name in n.inputs]
        t = n.op_type
        if t == "Conv":
            r = _conv(i[0], i[1].astype(np.float64), i[2] if len(i) > 2 else None, a)
        elif t == "BatchNormalization":
            xx, gam, bet, mu, var = i
            sh = (1, -1, 1, 1)
            r = (xx - mu.reshape(sh)) / np.sqrt(var.reshape(sh) + a.get("epsilon", 1e-5)) * gam.reshape(sh) + bet.reshape(sh)
        elif t == "Relu":
            r = np.maximum(i[0], 0)
        elif t == "Sigmoid":
            r = 1 / (1 + np.exp(-i[0]))
        elif t == "HardSigmoid":
            r = np.clip(a.get("alpha", 0.2) * i[0] + a.get("beta", 0.5), 0, 1)
        elif t == "HardSwish":
            r = i[0] * np.clip(i[0] / 6 + 0.5, 0, 1)
        elif t == "Erf":
            r = erf(i[0])
        elif t in ("Add", "Sub", "Mul", "Div", "Pow"):
            f = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide, "Pow": np.power}[t]
            r = f(i[0].astype(np.float64), i[1].astype(np.float64))
        elif t == "Sqrt":
            r = np.sqrt(i[0])
        elif t == "ReduceMean":
            axes = a["axes"] if "axes" in a else [int(k) for k in i[1]]
            r = i[0].mean(axis=tuple(axes), keepdims=bool(a.get("keepdims", 1)))
        elif t == "GlobalAveragePool":
            r = i[0].mean(axis=(2, 3), keepdims=True)
        elif t == "Resize":
            if len(i) > 3 and i[3] is not None:
                fh, fw = (int(s) // d for s, d in zip(i[3][2:], i[0].shape[2:]))
            else:
                fh, fw = (int(s) for s in i[2][2:])
            r = np.repeat(np.repeat(i[0], fh, axis=2), fw, axis=3)
        elif t == "ConvTranspose":
            w = i[1]
            ic, oc, kh, kw = w.shape
            nb, _, h, ww = i[0].shape
            r = np.einsum("nchw,coyx->nohywx", i[0], w).reshape(nb, oc, h * kh, ww * kw)
            if len(i) > 2:
                r = r + i[2].reshape(1, -1, 1, 1)
        elif t == "Concat":
            r = np.concatenate(i, axis=a["axis"])
        elif t == "MaxPool":
            kh, kw = a["kernel_shape"]
            xp = _pad_hw(i[0], ((kh - 1) // 2, (kw - 1) // 2, kh // 2, kw // 2), -np.inf)
            h, w = i[0].shape[2:]
            r = np.max([xp[:, :, y:y + h, z:z + w] for y in range(kh) for z in range(kw)], axis=0)
        elif t == "AveragePool":
            kh, kw = a["kernel_shape"]
            sh, sw = a.get("strides", [1, 1])
            h, w = i[0].shape[2:]
            oh, ow = (h - kh) // sh + 1, (w - kw) // sw + 1
            r = np.mean([i[0][:, :, y:y + sh * (oh - 1) + 1:sh, z:z + sw * (ow - 1) + 1:sw]
                         for y in range(kh) for z in range(kw)], axis=0)
        elif t == "Shape":
            r = np.array(i[0].shape, np.int64)
        elif t == "Slice":
            data = i[0]
            axes = list(i[3]) if len(i) > 3 else list(range(len(i[1])))
            sl = [slice(None)] * data.ndim
            for ax, s0, s1 in zip(axes, i[1], i[2]):
                sl[int(ax)] = slice(int(s0), int(min(s1, 2 ** 62)))
            r = data[tuple(sl)]
        elif t == "Squeeze":
            r = np.squeeze(i[0], axis=tuple(a["axes"] if "axes" in a else [int(k) for k in i[1]]))
        elif t == "Gather":
            r = np.take(i[0], i[1], axis=a.get("axis", 0))
        elif t == "Flatten":
            ax = a.get("axis", 1)
            r = i[0].reshape(int(np.prod(i[0].shape[:ax])), -1)
        elif t == "Unsqueeze":
            r = np.expand_dims(i[0], axis=tuple(a["axes"]))
        elif t == "Reshape":
            shape = [int(s) for s in i[1]]
            shape = [i[0].shape[k] if s == 0 else s for k, s in enumerate(shape)]
            r = i[0].reshape(shape)
        elif t == "Transpose":
            r = np.transpose(i[0], a["perm"])
        elif t == "MatMul":
            r = np.matmul(i[0].astype(np.float64), i[1].astype(np.float64))
        elif t == "Softmax":
            r = _softmax(i[0], a.get("axis", -1))
        elif t == "Identity":
            r = i[0]
        else:
            raise NotImplementedError(t)
        v[n.outputs[0]] = r
    return [v[o.name] for o in g.outputs]
