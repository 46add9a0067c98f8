"""ONNX PP-OCR graphs to PPOCRPL1 plans.

What a plan must say is fixed by the engine's exporter and reader
(tools/export_ocr.py:1-40 lists the rules, src/engine/plan.rs:9-28 the
format): the graph is traced at one size (a recogniser, input height 48, at
width 320; a detector on a 64 x 64 page) and the engine derives every other
size; Conv and ConvTranspose take their bias (an Add of a constant or a
BatchNormalization) and the activation after them as one operation; the
written-out LayerNorm, the attention block and the CTC head are one
operation each; the reshapes of the recogniser's sequence part cost nothing.

How this module gets there is its own, in three passes:

1. `Net` holds the graph as values with a producer and readers; an Identity
   node merges its output into its input.
2. `Net.infer` gives every value at the traced size either a constant
   (numpy; so the arithmetic on Shape, Slice, Concat ... folds away) or a
   runtime tensor with its ONNX dims and its *storage order*: its axes from
   outermost to innermost in memory. Plan operations write NHWC, so an NCHW
   map lies as (0, 2, 3, 1) and a [1, T, C] sequence as (0, 1, 2). A
   Reshape, Transpose, Squeeze, Unsqueeze or Flatten gets the storage order
   that leaves every element where it was, found by pushing an index tensor
   through the node; where there is none the node moves data, which no plan
   operation does, and only a template that swallows it (the attention
   block) can take it.
3. Rules claim nodes in graph order. Most are written as `Template`s:
   small DAGs of `Step`s (op type, operand specs, an attribute test) that a
   generic backtracking matcher binds by walking the readers of values
   already bound, trying both operand orders of Add and Mul, and requiring
   every value made inside a match to be read only inside it. A rule is a
   head plus optional *stages* (a bias, an activation, an upsample's
   addend), each matched on the value the one before leaves. Each claim is
   then lowered through `planfile.PlanBuilder` in the order of its last
   node, so every operand is written before it is read.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from typing import Callable

import numpy as np

from . import onnxproto
from .onnxproto import Graph, Node
from .planfile import PlanBuilder, Tensor

REC_HEIGHT = 48      # an input of this fixed height is a text-line recogniser
TRACE_WIDTH = 320    # ... traced at this width (RapidOCR's narrowest)
TRACE_PAGE = 64      # a detector is traced on a page of this many pixels a side
CTC_MIN_CLASSES = 4097  # MatMul + Add + Softmax wider than 4096 columns: the CTC head


def _f32(bits: int) -> np.float32:
    return np.array([bits], np.uint32).view(np.float32)[0]


# HardSigmoid(alpha, beta) pairs the engine folds, by the fused kind they
# become (plan.rs:148-175): alpha 0x3e2aaaad is the engine's 1/6.
HARD_SIGMOID_KINDS = {
    (_f32(0x3E2AAAAD), np.float32(0.5)): "hardsigmoid",
    (np.float32(0.2), np.float32(0.5)): "hardsigmoidfifth",
}


class ExportError(ValueError):
    """The graph holds something no plan operation expresses."""


# =================================================================== the net

@dataclass
class Info:
    """A value at the traced size: a constant, or a runtime tensor."""

    const: np.ndarray | None = None
    dims: tuple[int, ...] | None = None


@dataclass(frozen=True)
class Layout:
    """Where a runtime tensor's elements lie: its axes outermost-first in
    memory (None: no order keeps them in place), and the value whose
    storage it shares when it is a view."""

    order: tuple[int, ...] | None
    base: str | None = None


def _natural_order(rank: int) -> tuple[int, ...]:
    """How a plan operation lays out a result of this rank: NCHW maps as
    NHWC, everything else row-major."""
    return (0, 2, 3, 1) if rank == 4 else tuple(range(rank))


def _placed(dims, order) -> np.ndarray:
    """Each element's position in memory, as an array of the logical dims."""
    size = int(np.prod(dims, dtype=np.int64))
    stored = np.arange(size, dtype=np.int64).reshape([dims[a] for a in order])
    return stored.transpose(np.argsort(order))


def _order_of(placed: np.ndarray) -> tuple[int, ...] | None:
    """An axis order under which `placed` reads 0, 1, 2, ... in memory
    (unit axes put outermost); None when the elements are not in place."""
    dims = placed.shape
    unit = [a for a in range(placed.ndim) if dims[a] == 1]
    live = [a for a in range(placed.ndim) if dims[a] != 1]
    want = np.arange(placed.size, dtype=np.int64)
    for perm in itertools.permutations(live):
        if np.array_equal(placed.transpose(unit + list(perm)).reshape(-1), want):
            return tuple(unit) + perm
    return None


def _live(dims, order) -> tuple[int, ...]:
    """The storage order of the axes longer than one."""
    return tuple(a for a in order if dims[a] != 1)


def _attr_ints(node: Node, key: str, default=None):
    v = node.attrs.get(key, default)
    if isinstance(v, np.ndarray):
        v = v.tolist()
    return [int(x) for x in v] if isinstance(v, (list, tuple)) else v


def _attr_text(node: Node, key: str, default: str) -> str:
    v = node.attrs.get(key)
    return v.decode() if isinstance(v, (bytes, bytearray)) else default


class Net:
    """Nodes (Identity merged away), producers, readers and inferred values."""

    def __init__(self, graph: Graph) -> None:
        if not graph.inputs:
            raise ExportError("the model declares no input tensor")
        merged: dict[str, str] = {}

        def canon(name: str) -> str:
            while name in merged:
                name = merged[name]
            return name

        self.nodes: list[Node] = []
        for n in graph.nodes:
            if n.op_type == "Identity":
                merged[n.outputs[0]] = canon(n.inputs[0])
                continue
            self.nodes.append(Node(n.op_type, [canon(x) if x else "" for x in n.inputs],
                                   list(n.outputs), n.name or f"{n.op_type}#{len(self.nodes)}",
                                   dict(n.attrs)))
        self.input = graph.inputs[0].name
        self.outputs = [canon(v.name) for v in graph.outputs]
        self.producer: dict[str, int] = {}
        self.readers: dict[str, list[int]] = {}
        for i, n in enumerate(self.nodes):
            for y in n.outputs:
                self.producer[y] = i
            for x in n.inputs:
                if x and i not in self.readers.setdefault(x, []):
                    self.readers[x].append(i)
        self.info: dict[str, Info] = {k: Info(const=np.asarray(v)) for k, v in graph.initializers.items()}
        self.folded: set[int] = set()
        self.written: set[str] = set()  # values a plan operation writes whatever op made them
        self._layouts: dict[str, Layout] = {}
        self._trace_input(graph.inputs[0].dims)
        self.infer()

    # -- the traced size
    def _trace_input(self, dims) -> None:
        if len(dims) != 4:
            raise ExportError(f"input '{self.input}' has {len(dims)} axes; an image is N x C x H x W")
        c = dims[1]
        if not isinstance(c, int) or c <= 0:
            raise ExportError(f"input '{self.input}' has no fixed channel count")
        h = dims[2] if isinstance(dims[2], int) and dims[2] > 0 else TRACE_PAGE
        w = TRACE_WIDTH if h == REC_HEIGHT else TRACE_PAGE
        self.info[self.input] = Info(dims=(1, c, h, w))

    # -- queries
    def const(self, name: str) -> np.ndarray | None:
        i = self.info.get(name)
        return None if i is None else i.const

    def dims(self, name: str) -> tuple[int, ...]:
        i = self.info.get(name)
        if i is None or i.dims is None:
            raise ExportError(f"'{name}' is not a runtime tensor of known shape")
        return i.dims

    def layout(self, name: str) -> Layout:
        """A value's layout. What an operation writes lies as a plan
        operation lays it down; a view node's result lies where its input's
        elements already are, if some axis order says so."""
        got = self._layouts.get(name)
        if got is not None:
            return got
        dims = self.dims(name)
        ni = self.producer.get(name)
        node = self.nodes[ni] if ni is not None else None
        got = Layout(_natural_order(len(dims)))
        if node is not None and node.op_type in _VIEWS and name not in self.written:
            src = self.layout(node.inputs[0])
            got = Layout(None)
            if src.order is not None:
                ins = [self.info.get(v) if v else None for v in node.inputs]
                moved = _VIEWS[node.op_type](node, _placed(self.dims(node.inputs[0]), src.order), ins)
                order = _order_of(moved)
                got = Layout(order, node.inputs[0] if order is not None else None)
        self._layouts[name] = got
        return got

    def root(self, name: str) -> str:
        """The value that owns the storage `name` reads."""
        while self.layout(name).base is not None:
            name = self.layout(name).base
        return name

    # -- inference
    def infer(self) -> None:
        for i, n in enumerate(self.nodes):
            ins = [self.info.get(x) if x else None for x in n.inputs]
            for x, got in zip(n.inputs, ins):
                if x and got is None:
                    raise ExportError(f"{n.op_type} node '{n.name}' reads '{x}', which nothing makes")
            if n.op_type == "Constant":
                value = n.attrs.get("value")
                if not isinstance(value, np.ndarray):
                    raise ExportError(f"Constant node '{n.name}' holds no tensor")
                self.info[n.outputs[0]] = Info(const=value)
                self.folded.add(i)
                continue
            if n.op_type == "Shape":
                src = ins[0]
                shape = src.const.shape if src.const is not None else src.dims
                self.info[n.outputs[0]] = Info(const=np.array(shape, np.int64))
                self.folded.add(i)
                continue
            live = [x for x in ins if x is not None]
            if live and all(x.const is not None for x in live) and n.op_type in _FOLD:
                arrays = [x.const if x is not None else None for x in ins]
                self.info[n.outputs[0]] = Info(const=np.asarray(_FOLD[n.op_type](n, arrays)))
                self.folded.add(i)
                continue
            rule = _SHAPE.get(n.op_type)
            if rule is None:
                raise ExportError(f"unsupported operator {n.op_type} (node '{n.name}')")
            dims = tuple(int(d) for d in rule(n, ins))
            if any(d <= 0 for d in dims):
                raise ExportError(f"{n.op_type} node '{n.name}' makes an empty tensor {dims} at the traced size")
            self.info[n.outputs[0]] = Info(dims=dims)


# -- shape rules (runtime tensors)

def _window(node: Node, size: int, k: int, s: int, axis: int, rank_pads) -> tuple[int, int]:
    """(begin, end) padding of one spatial axis, auto_pad honoured."""
    auto = _attr_text(node, "auto_pad", "NOTSET")
    if auto in ("SAME_UPPER", "SAME_LOWER"):
        total = max((-(-size // s) - 1) * s + k - size, 0)
        small = total // 2
        return (small, total - small) if auto == "SAME_UPPER" else (total - small, small)
    if auto == "VALID":
        return 0, 0
    return rank_pads[axis], rank_pads[axis + 2]


def _pads(node: Node, hw, kernel, strides) -> list[int]:
    """ONNX order [top, left, bottom, right]."""
    given = _attr_ints(node, "pads", [0, 0, 0, 0])
    (t, b), (l, r) = (_window(node, hw[a], kernel[a], strides[a], a, given) for a in (0, 1))
    return [t, l, b, r]


def _pooled(size: int, k: int, s: int, lo: int, hi: int, ceil: bool) -> int:
    span = size + lo + hi - k
    return (-(-span // s) if ceil else span // s) + 1


def _shape_conv(n, ins):
    _, _, h, w = ins[0].dims
    oc, _, kh, kw = ins[1].const.shape
    sh, sw = _attr_ints(n, "strides", [1, 1])
    t, l, b, r = _pads(n, (h, w), (kh, kw), (sh, sw))
    return 1, oc, _pooled(h, kh, sh, t, b, False), _pooled(w, kw, sw, l, r, False)


def _shape_convt(n, ins):
    _, _, h, w = ins[0].dims
    ic, ocg, kh, kw = ins[1].const.shape
    sh, sw = _attr_ints(n, "strides", [1, 1])
    t, l, b, r = _attr_ints(n, "pads", [0, 0, 0, 0])
    eh, ew = _attr_ints(n, "output_padding", [0, 0])
    return 1, ocg * _attr_ints(n, "group", 1), (h - 1) * sh + kh - t - b + eh, (w - 1) * sw + kw - l - r + ew


def _shape_pool(n, ins):
    _, c, h, w = ins[0].dims
    kh, kw = _attr_ints(n, "kernel_shape")
    sh, sw = _attr_ints(n, "strides", [1, 1])
    t, l, b, r = _pads(n, (h, w), (kh, kw), (sh, sw))
    ceil = bool(_attr_ints(n, "ceil_mode", 0))
    return 1, c, _pooled(h, kh, sh, t, b, ceil), _pooled(w, kw, sw, l, r, ceil)


def _axes(n: Node, ins, rank: int, slot: int = 1):
    """Axes from the attribute (older opsets) or a constant input (newer)."""
    axes = _attr_ints(n, "axes")
    if axes is None and len(ins) > slot and ins[slot] is not None:
        if ins[slot].const is None:
            raise ExportError(f"{n.op_type} node '{n.name}' takes its axes from a runtime tensor")
        axes = [int(a) for a in ins[slot].const.reshape(-1)]
    return None if axes is None else sorted(a % rank for a in axes)


def _shape_reduce(n, ins):
    dims = list(ins[0].dims)
    axes = _axes(n, ins, len(dims)) or list(range(len(dims)))
    if _attr_ints(n, "keepdims", 1):
        return [1 if a in axes else d for a, d in enumerate(dims)]
    return [d for a, d in enumerate(dims) if a not in axes]


def _resize_factors(n: Node, ins) -> list[float]:
    dims = ins[0].dims
    scales = ins[2].const if len(ins) > 2 and ins[2] is not None else None
    sizes = ins[3].const if len(ins) > 3 and ins[3] is not None else None
    if scales is not None and scales.size == len(dims):
        return [float(s) for s in scales.reshape(-1)]
    if sizes is not None and sizes.size == len(dims):
        return [int(s) / d for s, d in zip(sizes.reshape(-1), dims)]
    raise ExportError(f"Resize node '{n.name}' has neither constant scales nor constant sizes")


def _shape_resize(n, ins):
    return [int(np.floor(d * f)) for d, f in zip(ins[0].dims, _resize_factors(n, ins))]


def _operand_dims(x: Info) -> tuple[int, ...]:
    return x.const.shape if x.const is not None else x.dims


def _shape_broadcast(n, ins):
    return np.broadcast_shapes(*(_operand_dims(x) for x in ins if x is not None))


def _shape_matmul(n, ins):
    a, b = (_operand_dims(x) for x in ins)
    if len(a) < 2 or len(b) < 2 or a[-1] != b[-2]:
        raise ExportError(f"MatMul node '{n.name}' multiplies {a} by {b}")
    return (*np.broadcast_shapes(a[:-2], b[:-2]), a[-2], b[-1])


def _shape_concat(n, ins):
    shapes = [_operand_dims(x) for x in ins]
    axis = _attr_ints(n, "axis", 0) % len(shapes[0])
    out = list(shapes[0])
    out[axis] = sum(s[axis] for s in shapes)
    return out


def _reshape_target(n: Node, ins, dims) -> list[int]:
    if ins[1] is None or ins[1].const is None:
        raise ExportError(f"Reshape node '{n.name}' takes its shape from a runtime tensor")
    target = [int(v) for v in ins[1].const.reshape(-1)]
    out = [dims[k] if v == 0 and not _attr_ints(n, "allowzero", 0) else v for k, v in enumerate(target)]
    if -1 in out:
        known = int(np.prod([v for v in out if v != -1]))
        out[out.index(-1)] = int(np.prod(dims)) // known
    return out


def _slice_window(n: Node, ins, dims):
    consts = [x.const.reshape(-1).astype(np.int64) if x is not None and x.const is not None else None
              for x in ins[1:]]
    if consts[0] is None or consts[1] is None:
        raise ExportError(f"Slice node '{n.name}' takes its bounds from a runtime tensor")
    starts, ends = consts[0], consts[1]
    axes = consts[2] if len(consts) > 2 and consts[2] is not None else np.arange(starts.size)
    steps = consts[3] if len(consts) > 3 and consts[3] is not None else np.ones(starts.size, np.int64)
    window = [slice(None)] * len(dims)
    for a, s0, s1, st in zip(axes, starts, ends, steps):
        window[int(a) % len(dims)] = slice(int(s0), int(max(min(s1, 2 ** 62), -2 ** 62)), int(st))
    return tuple(window)


def _shape_slice(n, ins):
    dims = ins[0].dims
    return np.empty(dims, np.int8)[_slice_window(n, ins, dims)].shape


def _shape_gather(n, ins):
    dims = ins[0].dims
    idx = ins[1].const
    if idx is None:
        raise ExportError(f"Gather node '{n.name}' takes its indices from a runtime tensor")
    axis = _attr_ints(n, "axis", 0) % len(dims)
    return (*dims[:axis], *idx.shape, *dims[axis + 1:])


def _same(n, ins):
    return ins[0].dims


_SHAPE: dict[str, Callable] = {
    "Conv": _shape_conv,
    "ConvTranspose": _shape_convt,
    "MaxPool": _shape_pool,
    "AveragePool": _shape_pool,
    "GlobalAveragePool": lambda n, ins: (*ins[0].dims[:2], 1, 1),
    "ReduceMean": _shape_reduce,
    "Resize": _shape_resize,
    "MatMul": _shape_matmul,
    "Concat": _shape_concat,
    "Slice": _shape_slice,
    "Gather": _shape_gather,
    **{op: _shape_broadcast for op in ("Add", "Sub", "Mul", "Div", "Pow")},
    **{op: _same for op in ("Relu", "Sigmoid", "HardSigmoid", "HardSwish", "Erf", "Sqrt", "Softmax",
                            "BatchNormalization", "Tanh", "Exp", "Neg", "LeakyRelu", "Clip")},
}


# -- views: the logical rearrangement, applied to an index tensor

def _view_reshape(n, placed, ins):
    return placed.reshape(_reshape_target(n, ins, placed.shape))


def _view_transpose(n, placed, ins):
    return placed.transpose(_attr_ints(n, "perm") or list(range(placed.ndim))[::-1])


def _view_squeeze(n, placed, ins):
    axes = _axes(n, ins, placed.ndim)
    return placed.squeeze(axis=tuple(axes) if axes is not None else None)


def _view_unsqueeze(n, placed, ins):
    raw = _attr_ints(n, "axes")
    if raw is None:
        if len(ins) < 2 or ins[1] is None or ins[1].const is None:
            raise ExportError(f"Unsqueeze node '{n.name}' takes its axes from a runtime tensor")
        raw = [int(v) for v in ins[1].const.reshape(-1)]
    out = placed
    for a in sorted(x % (placed.ndim + len(raw)) for x in raw):
        out = np.expand_dims(out, a)
    return out


def _view_flatten(n, placed, ins):
    axis = _attr_ints(n, "axis", 1) % (placed.ndim + 1)
    return placed.reshape(int(np.prod(placed.shape[:axis])), -1)


_VIEWS: dict[str, Callable] = {
    "Reshape": _view_reshape,
    "Transpose": _view_transpose,
    "Squeeze": _view_squeeze,
    "Unsqueeze": _view_unsqueeze,
    "Flatten": _view_flatten,
}
for _op, _fn in _VIEWS.items():
    _SHAPE[_op] = (lambda fn: lambda n, ins: fn(n, np.empty(ins[0].dims, np.int8), ins).shape)(_fn)


# -- constant folding (shape arithmetic and constant subgraphs)

def _fold_unsqueeze(n, a):
    axes = _attr_ints(n, "axes")
    if axes is None:
        axes = [int(v) for v in a[1].reshape(-1)]
    out = a[0]
    for ax in sorted(x % (out.ndim + len(axes)) for x in axes):
        out = np.expand_dims(out, ax)
    return out


def _fold_squeeze(n, a):
    axes = _attr_ints(n, "axes")
    if axes is None and len(a) > 1 and a[1] is not None:
        axes = [int(v) for v in a[1].reshape(-1)]
    return np.squeeze(a[0], axis=tuple(axes) if axes is not None else None)


def _fold_slice(n, a):
    ins = [Info(const=x) if x is not None else None for x in a]
    return a[0][_slice_window(n, ins, a[0].shape)]


_FOLD: dict[str, Callable] = {
    "Add": lambda n, a: a[0] + a[1],
    "Sub": lambda n, a: a[0] - a[1],
    "Mul": lambda n, a: a[0] * a[1],
    "Div": lambda n, a: a[0] // a[1] if a[0].dtype.kind in "iu" else a[0] / a[1],
    "Pow": lambda n, a: np.power(a[0], a[1]),
    "Sqrt": lambda n, a: np.sqrt(a[0]),
    "Neg": lambda n, a: -a[0],
    "Cast": lambda n, a: a[0].astype(onnxproto.DTYPES[_attr_ints(n, "to")]),
    "Concat": lambda n, a: np.concatenate([np.atleast_1d(x) for x in a], axis=_attr_ints(n, "axis", 0)),
    "Slice": _fold_slice,
    "Gather": lambda n, a: np.take(a[0], a[1], axis=_attr_ints(n, "axis", 0)),
    "Squeeze": _fold_squeeze,
    "Unsqueeze": _fold_unsqueeze,
    "Reshape": lambda n, a: a[0].reshape(_reshape_target(n, [None, Info(const=a[1])], a[0].shape)),
    "Transpose": lambda n, a: a[0].transpose(_attr_ints(n, "perm") or list(range(a[0].ndim))[::-1]),
    "ConstantOfShape": lambda n, a: np.full([int(v) for v in a[0].reshape(-1)],
                                            n.attrs.get("value", np.zeros(1, np.float32)).reshape(-1)[0]),
}


# ============================================================== the templates

@dataclass(frozen=True)
class K:
    """A constant operand, bound under `name` when it passes `test`."""

    name: str | None = None
    test: Callable[[np.ndarray], bool] | None = None
    optional: bool = False


@dataclass(frozen=True)
class R:
    """A runtime operand made outside the template, bound under `name`."""

    name: str


@dataclass(frozen=True)
class Step:
    """One node: its op type, one spec per input (the name of a value bound
    earlier, a `K` or an `R`) and a test on (net, node, bindings)."""

    name: str
    op: str
    args: tuple
    test: Callable | None = None


@dataclass(frozen=True)
class Template:
    name: str
    steps: tuple[Step, ...]
    out: str


@dataclass
class Bound:
    nodes: dict[str, int] = field(default_factory=dict)
    vals: dict[str, str] = field(default_factory=dict)
    consts: dict[str, np.ndarray | None] = field(default_factory=dict)

    def copy(self) -> "Bound":
        return Bound(dict(self.nodes), dict(self.vals), dict(self.consts))


_SYMMETRIC = {"Add", "Mul"}


def _operands(net: Net, step: Step, specs: tuple, ni: int, b: Bound) -> Bound | None:
    node = net.nodes[ni]
    names = list(node.inputs) + [""] * max(0, len(specs) - len(node.inputs))
    if len(node.inputs) > len(specs) and any(node.inputs[len(specs):]):
        return None
    out = b.copy()
    for spec, name in zip(specs, names):
        if isinstance(spec, str):
            if out.vals.get(spec) != name:
                return None
        elif isinstance(spec, K):
            if not name:
                if not spec.optional:
                    return None
                if spec.name:
                    out.consts[spec.name] = None
                continue
            c = net.const(name)
            if c is None or (spec.test is not None and not spec.test(c)):
                return None
            if spec.name:
                out.consts[spec.name] = c
        elif isinstance(spec, R):
            if not name or net.const(name) is not None:
                return None
            out.vals[spec.name] = name
    out.nodes[step.name] = ni
    out.vals[step.name] = node.outputs[0]
    if step.test is not None and not step.test(net, node, out):
        return None
    return out


def _bind(net: Net, tpl: Template, k: int, b: Bound, taken: set[int], first: int | None) -> Bound | None:
    if k == len(tpl.steps):
        return b if _sealed(net, tpl, b) else None
    step = tpl.steps[k]
    if first is not None:
        candidates = [first]
    else:
        hook = next(a for a in step.args if isinstance(a, str))
        candidates = net.readers.get(b.vals[hook], [])
    for ni in candidates:
        if net.nodes[ni].op_type != step.op or ni in taken or ni in b.nodes.values():
            continue
        orders = [step.args]
        if step.op in _SYMMETRIC and len(step.args) == 2:
            orders.append(step.args[::-1])
        for specs in orders:
            got = _operands(net, step, specs, ni, b)
            if got is not None:
                done = _bind(net, tpl, k + 1, got, taken, None)
                if done is not None:
                    return done
    return None


def _sealed(net: Net, tpl: Template, b: Bound) -> bool:
    """Every value made inside the match, but its result, is read only inside."""
    inside = set(b.nodes.values())
    for st in tpl.steps:
        if st.name == tpl.out:
            continue
        v = b.vals[st.name]
        if v in net.outputs or any(r not in inside for r in net.readers.get(v, [])):
            return False
    return True


def match_at(net: Net, tpl: Template, ni: int, taken: set[int]) -> Bound | None:
    """`tpl` with its first step on node `ni`; its first input is the entry."""
    b = Bound()
    entry = next(a for a in tpl.steps[0].args if isinstance(a, str))
    b.vals[entry] = net.nodes[ni].inputs[0]
    return _bind(net, tpl, 0, b, taken, ni)


def match_after(net: Net, tpl: Template, value: str, entry: str, taken: set[int]) -> Bound | None:
    """`tpl` hung from `value`, which must end up read only by the match."""
    if value in net.outputs:
        return None
    b = Bound(vals={entry: value})
    got = _bind(net, tpl, 0, b, taken, None)
    if got is None or any(r not in got.nodes.values() for r in net.readers.get(value, [])):
        return None
    return got


# -- tests used by the templates

def _scalar(test=None):
    return lambda c: c.size == 1 and (test is None or test(float(c.reshape(-1)[0])))


def _near(v: float, tol: float = 1e-6):
    return _scalar(lambda x: abs(x - v) <= tol)


def _is(v: float):
    return _scalar(lambda x: x == v)


def _ints_are(*want):
    return lambda c: c.size == len(want) and [int(x) for x in c.reshape(-1)] == list(want)


def _perm(*perm):
    return lambda net, node, b: _attr_ints(node, "perm") == list(perm)


def _reduces_last(net, node, b):
    """ReduceMean over the last axis alone, keeping it."""
    rank = len(net.dims(node.inputs[0]))
    ins = [net.info.get(v) if v else None for v in node.inputs]
    return _axes(node, ins, rank) == [rank - 1] and _attr_ints(node, "keepdims", 1) == 1


def _softmax_last(net, node, b):
    """Softmax over the last axis, said explicitly (the default axis differs
    between opsets, and opset 11's flattens the axes after it)."""
    axis = _attr_ints(node, "axis")
    rank = len(net.dims(node.inputs[0]))
    return axis is not None and axis % rank == rank - 1


def _squeezes_front(net, node, b):
    axes = _attr_ints(node, "axes")
    if axes is None and len(node.inputs) > 1 and node.inputs[1]:
        axes = [int(v) for v in net.const(node.inputs[1]).reshape(-1)]
    return axes == [0]


def _whole_factor(net, node, b):
    return (_attr_text(node, "mode", "nearest") == "nearest"
            and _attr_text(node, "coordinate_transformation_mode", "half_pixel") == "asymmetric"
            and _attr_text(node, "nearest_mode", "round_prefer_floor") == "floor")


def _same_dims_as(entry: str, other: str):
    return lambda net, node, b: net.dims(b.vals[entry]) == net.dims(b.vals[other])


def _gathers_front(net, node, b):
    return _attr_ints(node, "axis", 0) == 0


# -- activations folded into the operation that makes their input

def _one(name: str, op: str, test=None) -> Template:
    return Template(name, (Step("act", op, ("y",), test),), "act")


ACTIVATIONS: tuple[Template, ...] = (
    _one("relu", "Relu"),
    Template("swish", (Step("s", "Sigmoid", ("y",)), Step("act", "Mul", ("y", "s"))), "act"),
    _one("sigmoid", "Sigmoid"),
    _one("hardsigmoid", "HardSigmoid"),
    _one("hardswish", "HardSwish"),
    Template("gelu", (
        Step("scaled", "Div", ("y", K(test=_near(np.sqrt(2.0))))),
        Step("erf", "Erf", ("scaled",)),
        Step("plus1", "Add", ("erf", K(test=_is(1.0)))),
        Step("prod", "Mul", ("y", "plus1")),
        Step("act", "Mul", ("prod", K(test=_is(0.5)))),
    ), "act"),
)

# -- the bias a convolution or a linear layer takes after it
BIAS_ADD = Template("add", (Step("b", "Add", ("y", K("bias"))),), "b")
BATCH_NORM = Template("bn", (Step("b", "BatchNormalization",
                                  ("y", K("gamma"), K("beta"), K("mean"), K("var"))),), "b")

LAYER_NORM = Template("layernorm", (
    Step("mu", "ReduceMean", ("x", K(optional=True)), _reduces_last),
    Step("dev", "Sub", ("x", "mu")),
    Step("sq", "Pow", ("dev", K(test=_is(2.0)))),
    Step("var", "ReduceMean", ("sq", K(optional=True)), _reduces_last),
    Step("vare", "Add", ("var", K("eps", test=_scalar()))),
    Step("sd", "Sqrt", ("vare",)),
    Step("norm", "Div", ("dev", "sd")),
    Step("scaled", "Mul", ("norm", K("gamma"))),
    Step("y", "Add", ("scaled", K("beta"))),
), "y")

CTC_HEAD = Template("ctc", (
    Step("mm", "MatMul", ("x", K("w", test=lambda c: c.ndim == 2 and c.shape[1] >= CTC_MIN_CLASSES))),
    Step("logits", "Add", ("mm", K("b"))),
    Step("y", "Softmax", ("logits",), _softmax_last),
), "y")


def _attention(select: str, zero_add: bool) -> Template:
    """The multi-head attention block of the recogniser's encoder."""
    steps = [
        Step("split", "Reshape", ("qkv", K("shape", test=lambda c: c.size == 5 and list(c[:3]) == [0, -1, 3]))),
        Step("heads", "Transpose", ("split",), _perm(2, 0, 3, 1, 4)),
    ]
    for i, part in enumerate("qkv"):
        if select == "slice":
            steps += [Step(f"pick_{part}", "Slice", ("heads", K(test=_ints_are(i)), K(test=_ints_are(i + 1)),
                                                     K(test=_ints_are(0), optional=True),
                                                     K(test=_ints_are(1), optional=True))),
                      Step(part, "Squeeze", (f"pick_{part}", K(optional=True)), _squeezes_front)]
        else:
            steps.append(Step(part, "Gather", ("heads", K(test=_ints_are(i))), _gathers_front))
    steps += [
        Step("q_scaled", "Mul", ("q", K("scale", test=_scalar()))),
        Step("k_t", "Transpose", ("k",), _perm(0, 1, 3, 2)),
        Step("scores", "MatMul", ("q_scaled", "k_t")),
    ]
    last = "scores"
    if zero_add:
        steps.append(Step("scores_b", "Add", ("scores", K("score_bias", test=_scalar()))))
        last = "scores_b"
    steps += [
        Step("probs", "Softmax", (last,), _softmax_last),
        Step("mixed", "MatMul", ("probs", "v")),
        Step("merged", "Transpose", ("mixed",), _perm(0, 2, 1, 3)),
        Step("y", "Reshape", ("merged", K())),
    ]
    return Template("attention", tuple(steps), "y")


ATTENTIONS = tuple(_attention(s, z) for s in ("slice", "gather") for z in (True, False))

UPSAMPLE = Template("upsample", (Step("up", "Resize", ("x", K(optional=True), K(optional=True),
                                                       K(optional=True)), _whole_factor),), "up")
UPSAMPLE_ADD = Template("addend", (Step("sum", "Add", ("y", R("addend")), _same_dims_as("y", "addend")),), "sum")


# ================================================================== claims

@dataclass
class Claim:
    rule: "Rule"
    nodes: set[int]
    b: Bound
    out: str
    stages: dict[str, Template] = field(default_factory=dict)
    extra: dict = field(default_factory=dict)


class Rule:
    anchors: tuple[str, ...] = ()

    def claim(self, net: Net, ni: int, taken: set[int]) -> Claim | None:
        raise NotImplementedError

    def lower(self, low: "Lowering", c: Claim) -> None:
        raise NotImplementedError


class Chain(Rule):
    """A head template, then optional stages on the value each leaves."""

    def __init__(self, head: Template, stages: tuple[tuple[str, tuple[Template, ...]], ...],
                 lower: Callable, anchors: tuple[str, ...] | None = None) -> None:
        self.head, self.stage_list, self.lower_fn = head, stages, lower
        self.anchors = anchors or (head.steps[0].op,)

    def claim(self, net, ni, taken):
        b = match_at(net, self.head, ni, taken)
        if b is None:
            return None
        out = b.vals[self.head.out]
        c = Claim(self, set(b.nodes.values()), b, out)
        for stage, options in self.stage_list:
            for tpl in options:
                entry = next(a for a in tpl.steps[0].args if isinstance(a, str))
                got = match_after(net, tpl, out, entry, taken | c.nodes)
                if got is None:
                    continue
                c.stages[stage] = tpl
                c.nodes |= set(got.nodes.values())
                for k, v in got.consts.items():
                    c.b.consts[f"{stage}.{k}"] = v
                for k, v in got.vals.items():
                    c.b.vals[f"{stage}.{k}"] = v
                for k, v in got.nodes.items():
                    c.b.nodes[f"{stage}.{k}"] = v
                out = got.vals[tpl.out]
                break
        c.out = out
        net.written.add(out)
        return c

    def lower(self, low, c):
        self.lower_fn(low, c)


class Single(Rule):
    """One node, checked and lowered by one function."""

    def __init__(self, anchors: tuple[str, ...], lower: Callable, test: Callable | None = None) -> None:
        self.anchors, self.lower_fn, self.test = anchors, lower, test

    def claim(self, net, ni, taken):
        if self.test is not None and not self.test(net, net.nodes[ni]):
            return None
        node = net.nodes[ni]
        if node.op_type not in _VIEWS:
            net.written.add(node.outputs[0])
        return Claim(self, {ni}, Bound(nodes={"node": ni}), node.outputs[0])

    def lower(self, low, c):
        self.lower_fn(low, low.net.nodes[c.b.nodes["node"]], c)


# ================================================================ lowering

class Lowering:
    """Plan tensors for the net's values, emitted through a PlanBuilder."""

    def __init__(self, net: Net, argmax: bool) -> None:
        self.net, self.argmax = net, argmax
        _, c, h, w = net.dims(net.input)
        self.plan = PlanBuilder(h, w, c)
        self.tensors: dict[str, Tensor] = {net.input: self.plan.input}
        self.pairs: dict[str, tuple[Tensor, Tensor]] = {}  # a Concat a windowed conv reads as two maps
        self.loose: set[str] = set()  # plan tensors shaped other than the graph's value (CTC argmax)

    def hwc(self, value: str) -> tuple[int, int, int]:
        """The plan's (h, w, c) of a channels-last value: an NCHW map stored
        NHWC, or a [1, T, C] sequence with C innermost."""
        dims = self.net.dims(value)
        order = self.net.layout(value).order
        if dims[0] != 1:
            raise ExportError(f"'{value}' is not a batch-1 tensor")
        if order is None:
            raise ExportError(f"'{value}' is a rearrangement of its input that no plan buffer holds")
        if len(dims) == 4 and _live(dims, order) == _live(dims, (0, 2, 3, 1)):
            return dims[2], dims[3], dims[1]
        if len(dims) == 3 and _live(dims, order) == _live(dims, (0, 1, 2)):
            return 1, dims[1], dims[2]
        raise ExportError(f"'{value}' of shape {list(dims)} does not lie channels-last in memory")

    def read(self, value: str) -> Tensor:
        if value in self.pairs:
            raise ExportError(f"concatenation '{value}' is only readable by the windowed convolution it feeds")
        root = self.net.root(value)
        t = self.tensors.get(root)
        if t is None:
            raise ExportError(f"'{value}' is read before any operation writes it")
        if root not in self.loose and (t.h, t.w, t.c) != self.hwc(value):
            raise ExportError(f"'{value}' is read as {self.hwc(value)} but was written as {(t.h, t.w, t.c)}")
        return t

    def write(self, value: str, t: Tensor) -> None:
        if (t.h, t.w, t.c) != self.hwc(value):
            raise ExportError(f"the plan would make '{value}' {(t.h, t.w, t.c)}; the graph says "
                              f"{self.hwc(value)}")
        self.tensors[value] = t

    def finish(self) -> bytes:
        outs = []
        for o in self.net.outputs:
            if self.net.const(o) is not None:
                raise ExportError(f"output '{o}' is a constant")
            outs.append(self.read(o))
        for op in self.plan.ops:
            if min(op.words()) < 0 or max(op.words()) >= 1 << 32:
                raise ExportError(f"a field of the {op.kind} record does not fit a 32-bit word")
        return self.plan.to_bytes(outs)


def _per_channel(c: np.ndarray, rank: int, axis: int, n: int, what: str) -> np.ndarray:
    """A constant that broadcasts along `axis` only, as n values."""
    shape = (1,) * (rank - c.ndim) + c.shape
    if c.size != n or any(d != 1 for a, d in enumerate(shape) if a != axis):
        raise ExportError(f"{what} of shape {list(c.shape)} is not one value per channel")
    return c.reshape(-1).astype(np.float64)


def _fused(low: Lowering, c: Claim) -> str:
    tpl = c.stages.get("act")
    if tpl is None:
        return "none"
    if tpl.name == "hardsigmoid":
        node = low.net.nodes[c.b.nodes["act.act"]]
        pair = (np.float32(node.attrs.get("alpha", 0.2)), np.float32(node.attrs.get("beta", 0.5)))
        kind = HARD_SIGMOID_KINDS.get(pair)
        if kind is None:
            raise ExportError(f"HardSigmoid node '{node.name}' (alpha {pair[0]}, beta {pair[1]}) is neither "
                              "of the engine's hard sigmoids")
        return kind
    return tpl.name


def _plan_pads(node: Node, hw, kernel, strides) -> tuple[int, int, int, int]:
    """(top, bottom, left, right) for the plan; SAME padding only where it
    does not depend on the input size."""
    auto = _attr_text(node, "auto_pad", "NOTSET")
    if auto not in ("NOTSET", "VALID", "SAME_UPPER"):
        raise ExportError(f"{node.op_type} node '{node.name}': auto_pad {auto}")
    if auto == "SAME_UPPER" and tuple(strides) != (1, 1):
        raise ExportError(f"{node.op_type} node '{node.name}': SAME_UPPER padding at stride {list(strides)} "
                          "depends on the input size, which a plan cannot follow")
    t, l, b, r = _pads(node, hw, kernel, strides)
    return t, b, l, r


def _lower_conv(low: Lowering, c: Claim) -> None:
    net = low.net
    node = net.nodes[c.b.nodes["conv"]]
    w = c.b.consts["w"].astype(np.float64)
    if w.ndim != 4:
        raise ExportError(f"Conv node '{node.name}' is not two-dimensional")
    oc, per_group, kh, kw = w.shape
    if _attr_ints(node, "dilations", [1, 1]) != [1, 1]:
        raise ExportError(f"Conv node '{node.name}' is dilated; the engine's windows are dense")
    strides = _attr_ints(node, "strides", [1, 1])
    x = c.b.vals["x"]
    _, _, ih, iw = net.dims(x)
    pt, pb, pl, pr = _plan_pads(node, (ih, iw), (kh, kw), strides)
    bias = np.zeros(oc) if c.b.consts.get("b") is None else c.b.consts["b"].reshape(-1).astype(np.float64)
    bias_stage = c.stages.get("bias")
    if bias_stage is BIAS_ADD:
        bias = bias + _per_channel(c.b.consts["bias.bias"], 4, 1, oc, f"the bias added after '{node.name}'")
    elif bias_stage is BATCH_NORM:
        bn = net.nodes[c.b.nodes["bias.b"]]
        gamma, beta, mean, var = (c.b.consts[f"bias.{k}"].reshape(-1).astype(np.float64)
                                  for k in ("gamma", "beta", "mean", "var"))
        eps = np.float64(np.float32(bn.attrs.get("epsilon", 1e-5)))
        scale = gamma / np.sqrt(var + eps)
        w = w * scale[:, None, None, None]
        bias = (bias - mean) * scale + beta
    group = _attr_ints(node, "group", 1)
    fused = _fused(low, c)
    pair = low.pairs.pop(x, None)
    first, second = pair if pair is not None else (low.read(x), None)
    if group > 1 and per_group == 1:
        if not group == first.c == oc or second is not None:
            raise ExportError(f"Conv node '{node.name}' groups {group} of {first.c} channels into {oc}: only "
                              "depthwise grouping is supported")
        y = low.plan.dwconv(first, w.reshape(oc, kh, kw).transpose(1, 2, 0), bias, k=(kh, kw),
                            s=tuple(strides), pad=(pt, pb, pl, pr), fused=fused)
    else:
        if group != 1:
            raise ExportError(f"Conv node '{node.name}' has {group} groups; only depthwise grouping is supported")
        n2 = second.c if second is not None else 0
        if per_group != first.c + n2:
            raise ExportError(f"Conv node '{node.name}' takes {per_group} channels from a {first.c + n2}-channel map")
        y = low.plan.conv(first, w.transpose(2, 3, 1, 0), bias, k=(kh, kw), s=tuple(strides),
                          pad=(pt, pb, pl, pr), fused=fused, x2=second)
    low.write(c.out, y)


def _lower_convt(low: Lowering, c: Claim) -> None:
    node = low.net.nodes[c.b.nodes["convt"]]
    w = c.b.consts["w"]
    if w.ndim != 4:
        raise ExportError(f"ConvTranspose node '{node.name}' is not two-dimensional")
    ic, oc, kh, kw = w.shape
    if (_attr_ints(node, "strides", [1, 1]) != [kh, kw] or any(_attr_ints(node, "pads", [0, 0, 0, 0]))
            or _attr_ints(node, "group", 1) != 1 or _attr_ints(node, "dilations", [1, 1]) != [1, 1]
            or any(_attr_ints(node, "output_padding", [0, 0]))):
        raise ExportError(f"ConvTranspose node '{node.name}': only ungrouped, unpadded windows that tile the "
                          "output (stride = kernel) are supported")
    # The node's own bias input and a constant Add after it both count.
    bias = np.zeros(oc) if c.b.consts.get("b") is None else c.b.consts["b"].reshape(-1).astype(np.float64)
    if c.stages.get("bias") is BIAS_ADD:
        bias = bias + _per_channel(c.b.consts["bias.bias"], 4, 1, oc, f"the bias added after '{node.name}'")
    y = low.plan.convtranspose(low.read(c.b.vals["x"]), w.transpose(0, 2, 3, 1), bias, k=(kh, kw),
                               fused=_fused(low, c))
    low.write(c.out, y)


def _lower_linear(low: Lowering, c: Claim) -> None:
    x = c.b.vals["x"]
    w = c.b.consts["w"]
    if w.ndim != 2 or len(low.net.dims(x)) != 3:
        raise ExportError(f"MatMul '{c.out}' is not a [1, T, C] sequence times a constant matrix")
    ci, co = w.shape
    t = low.read(x)
    if t.c != ci:
        raise ExportError(f"linear layer '{c.out}' takes {ci} channels from a {t.c}-channel sequence")
    bias = np.zeros(co)
    if c.stages.get("bias") is BIAS_ADD:
        bias = _per_channel(c.b.consts["bias.bias"], 3, 2, co, f"the bias of linear layer '{c.out}'")
    y = low.plan.conv(t, w.reshape(1, 1, ci, co), bias, fused=_fused(low, c))
    low.write(c.out, y)


def _lower_ctc(low: Lowering, c: Claim) -> None:
    x = c.b.vals["x"]
    w = c.b.consts["w"]
    vocab = w.shape[1]
    bias = _per_channel(c.b.consts["b"], 3, 2, vocab, "the CTC head's bias")
    t = low.read(x)
    if t.c != w.shape[0]:
        raise ExportError(f"the CTC head takes {w.shape[0]} channels from a {t.c}-channel sequence")
    y = low.plan.ctc(t, w, bias, argmax=low.argmax)
    low.tensors[c.out] = y
    if low.argmax:
        low.loose.add(c.out)  # [1, T, 2]: each step's class and probability, not the graph's [1, T, V]


def _lower_layernorm(low: Lowering, c: Claim) -> None:
    x = low.read(c.b.vals["x"])
    rank = len(low.net.dims(c.out))
    eps = float(c.b.consts["eps"].reshape(-1)[0])
    gamma = _per_channel(c.b.consts["gamma"], rank, rank - 1, x.c, "the layer norm's scale")
    beta = _per_channel(c.b.consts["beta"], rank, rank - 1, x.c, "the layer norm's shift")
    low.write(c.out, low.plan.layernorm(x, gamma, beta, eps))


def _lower_attention(low: Lowering, c: Claim) -> None:
    qkv = low.read(c.b.vals["qkv"])
    heads, width = (int(v) for v in c.b.consts["shape"].reshape(-1)[3:])
    if 3 * heads * width != qkv.c:
        raise ExportError(f"attention splits {qkv.c} channels into 3 x {heads} heads x {width}")
    bias = c.b.consts.get("score_bias")
    if bias is not None and float(bias.reshape(-1)[0]) != 0.0:
        raise ExportError("the attention scores get a nonzero constant added; the engine's attention has none")
    scale = float(c.b.consts["scale"].reshape(-1)[0])
    low.write(c.out, low.plan.attention(qkv, heads, scale))


def _lower_upsample(low: Lowering, c: Claim) -> None:
    net = low.net
    node = net.nodes[c.b.nodes["up"]]
    x = c.b.vals["x"]
    ins = [net.info.get(v) if v else None for v in node.inputs]
    factors = _resize_factors(node, ins)
    fh, fw = factors[2], factors[3]
    if factors[:2] != [1.0, 1.0] or fh != int(fh) or fw != int(fw) or fh < 1 or fw < 1:
        raise ExportError(f"Resize node '{node.name}' scales by {factors}: only whole factors over height and width")
    t = low.read(x)
    if "addend" in c.stages:
        y = low.plan.upsampleadd(t, low.read(c.b.vals["addend.addend"]), (int(fh), int(fw)))
    else:
        y = low.plan.upsample(t, (int(fh), int(fw)))
    low.write(c.out, y)


class ConcatRule(Rule):
    """A channel Concat: a chain of `concatc`, the last map left for a
    windowed dense conv that alone reads the result to take in place."""

    anchors = ("Concat",)

    def claim(self, net, ni, taken):
        node = net.nodes[ni]
        if any(net.const(x) is not None for x in node.inputs):
            return None
        c = Claim(self, {ni}, Bound(nodes={"node": ni}), node.outputs[0])
        net.written.add(node.outputs[0])
        readers = net.readers.get(node.outputs[0], [])
        reader = net.nodes[readers[0]] if len(readers) == 1 else None
        c.extra["in_place"] = bool(
            reader is not None and node.outputs[0] not in net.outputs and reader.op_type == "Conv"
            and reader.inputs[0] == node.outputs[0] and _attr_ints(reader, "group", 1) == 1
            and net.const(reader.inputs[1]) is not None and net.const(reader.inputs[1]).shape[2:] != (1, 1))
        return c

    def lower(self, low, c):
        node = low.net.nodes[c.b.nodes["node"]]
        dims = low.net.dims(node.outputs[0])
        if len(dims) != 4 or _attr_ints(node, "axis", 0) % 4 != 1:
            raise ExportError(f"Concat node '{node.name}' joins along another axis than channels")
        parts = [low.read(x) for x in node.inputs]
        for p in parts[1:]:
            if (p.h, p.w) != (parts[0].h, parts[0].w):
                raise ExportError(f"Concat node '{node.name}' joins maps of different sizes")
        keep = c.extra["in_place"]
        head = parts[0]
        for p in parts[1:len(parts) - keep]:
            head = low.plan.concat(head, p)
        if keep:
            low.pairs[node.outputs[0]] = (head, parts[-1])
        else:
            low.write(node.outputs[0], head)


def _lower_mean(low, node, c):
    low.write(node.outputs[0], low.plan.mean(low.read(node.inputs[0])))


def _is_spatial_mean(net, node):
    if node.op_type == "GlobalAveragePool":
        return len(net.dims(node.inputs[0])) == 4
    dims = net.dims(node.inputs[0])
    ins = [net.info.get(v) if v else None for v in node.inputs]
    return len(dims) == 4 and _axes(node, ins, 4) == [2, 3] and _attr_ints(node, "keepdims", 1) == 1


def _lower_gate(low, node, c):
    net = low.net
    a, b = node.inputs
    if net.const(a) is not None or net.const(b) is not None:
        raise ExportError(f"Mul node '{node.name}' by a constant folds into nothing the plan has")
    da, db = net.dims(a), net.dims(b)
    if len(da) == 4 and da[2:] == (1, 1) and db[2:] != (1, 1):
        a, b, da, db = b, a, db, da
    if len(da) != 4 or db[2:] != (1, 1) or da[1] != db[1] or da[2:] == (1, 1):
        raise ExportError(f"Mul node '{node.name}' is not a map times one gate per channel")
    low.write(node.outputs[0], low.plan.channelmul(low.read(a), low.read(b)))


def _lower_add(low: Lowering, c: Claim) -> None:
    net = low.net
    node = net.nodes[c.b.nodes["sum"]]
    a, b = node.inputs
    if net.const(a) is not None or net.const(b) is not None:
        raise ExportError(f"Add node '{node.name}' of a constant follows nothing that takes a bias")
    if net.dims(a) != net.dims(b):
        raise ExportError(f"Add node '{node.name}' broadcasts {list(net.dims(a))} against {list(net.dims(b))}")
    low.write(c.out, low.plan.add(low.read(a), low.read(b), fused=_fused(low, c)))


def _lower_maxpool(low, node, c):
    kh, kw = _attr_ints(node, "kernel_shape")
    strides = _attr_ints(node, "strides", [1, 1])
    if (_attr_text(node, "auto_pad", "NOTSET") != "SAME_UPPER" or strides != [1, 1]
            or _attr_ints(node, "dilations", [1, 1]) != [1, 1] or max(kh, kw) > 2):
        raise ExportError(f"MaxPool node '{node.name}': the engine's max pool is the stem's stride-1 window of "
                          "at most 2 x 2 with SAME_UPPER padding")
    y = low.plan.maxpool(low.read(node.inputs[0]), k=(kh, kw), s=(1, 1), pad_after=(kh - 1, kw - 1))
    low.write(node.outputs[0], y)


def _lower_avgpool(low, node, c):
    kh, kw = _attr_ints(node, "kernel_shape")
    if (any(_attr_ints(node, "pads", [0, 0, 0, 0]))
            or _attr_text(node, "auto_pad", "NOTSET") not in ("NOTSET", "VALID") or _attr_ints(node, "ceil_mode", 0)):
        raise ExportError(f"AveragePool node '{node.name}': the engine averages whole windows only (no padding, "
                          "no ceil mode)")
    strides = _attr_ints(node, "strides", [1, 1])
    low.write(node.outputs[0], low.plan.avgpool(low.read(node.inputs[0]), (kh, kw), tuple(strides)))


def _is_view(net, node):
    return net.layout(node.outputs[0]).base is not None


def _lower_view(low, node, c):
    """Nothing to run: the result is its input's storage, read in another
    order; whoever reads it as a plan tensor checks that order."""
    if low.net.root(node.outputs[0]) not in low.tensors:
        raise ExportError(f"{node.op_type} node '{node.name}' views '{node.inputs[0]}' before anything writes it")


_ACT = ("act", ACTIVATIONS)
RULES: tuple[Rule, ...] = (
    *(Chain(t, (), _lower_attention) for t in ATTENTIONS),
    Chain(LAYER_NORM, (), _lower_layernorm),
    Chain(CTC_HEAD, (), _lower_ctc),
    Chain(Template("conv", (Step("conv", "Conv", ("x", K("w"), K("b", optional=True))),), "conv"),
          (("bias", (BIAS_ADD, BATCH_NORM)), _ACT), _lower_conv),
    Chain(Template("convt", (Step("convt", "ConvTranspose", ("x", K("w"), K("b", optional=True))),), "convt"),
          (("bias", (BIAS_ADD,)), _ACT), _lower_convt),
    Chain(Template("linear", (Step("mm", "MatMul", ("x", K("w"))),), "mm"),
          (("bias", (BIAS_ADD,)), _ACT), _lower_linear),
    Chain(UPSAMPLE, (("addend", (UPSAMPLE_ADD,)),), _lower_upsample),
    Chain(Template("add", (Step("sum", "Add", ("x", R("other"))),), "sum"), (_ACT,), _lower_add),
    ConcatRule(),
    Single(("GlobalAveragePool", "ReduceMean"), _lower_mean, _is_spatial_mean),
    Single(("Mul",), _lower_gate),
    Single(("MaxPool",), _lower_maxpool),
    Single(("AveragePool",), _lower_avgpool),
    Single(tuple(_VIEWS), _lower_view, _is_view),
)
_BY_OP: dict[str, list[Rule]] = {}
for _rule in RULES:
    for _op in _rule.anchors:
        _BY_OP.setdefault(_op, []).append(_rule)


# ==================================================================== driver

def plan_bytes(graph: Graph, argmax: bool = False) -> bytes:
    net = Net(graph)
    claims: list[Claim] = []
    taken: set[int] = set(net.folded)
    for ni, node in enumerate(net.nodes):
        if ni in taken:
            continue
        for rule in _BY_OP.get(node.op_type, ()):
            c = rule.claim(net, ni, taken)
            if c is not None:
                break
        else:
            if node.op_type in _VIEWS and net.const(node.inputs[0]) is None:
                raise ExportError(f"{node.op_type} node '{node.name}' is a rearrangement of its input that moves "
                                  "data; no plan operation does that")
            raise ExportError(f"unsupported {node.op_type} node '{node.name}': it fits none of the plan's "
                              "operations here")
        taken |= c.nodes
        claims.append(c)
    low = Lowering(net, argmax)
    try:
        for c in sorted(claims, key=lambda c: max(c.nodes)):
            c.rule.lower(low, c)
    except ExportError:
        raise
    except ValueError as e:  # a weight the plan refuses (not finite)
        raise ExportError(str(e)) from e
    return low.finish()


def export(model, argmax: bool = False) -> bytes:
    """Plan bytes for an ONNX model: a path, ModelProto bytes or a Graph."""
    if isinstance(model, Graph):
        graph = model
    elif isinstance(model, (bytes, bytearray)):
        graph = onnxproto.decode_model(bytes(model))
    else:
        graph = onnxproto.load(model)
    return plan_bytes(graph, argmax)


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


if __name__ == "__main__":
    raise SystemExit(main())
