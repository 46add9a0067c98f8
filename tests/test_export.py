"""The exporter (ppocr_native_amd.export: the graph-to-plan behaviour of
tools/export_ocr.py:1-40, by templates over a use-def graph) on ONNX graphs
built here: each graph goes
through the ONNX wire format and back, is exported to a plan, and the plan
run on the CPU oracle must give what a numpy evaluation of the graph's ONNX
operators gives (tests/onnx_eval.py), within 2e-4 * |ref| + 1e-4 (the
oracle runs in float32, the evaluation in float64).

This pins the layouts (NCHW weights to HWIO, depthwise to HW-C, transposed
convs, the CTC panels), the folds (bias Add, BatchNormalization, the
activations, concatenations read in place, upsample + add, the LayerNorm and
attention patterns, aliased reshapes) and the buffer assignment. What stays
unpinned: the PP-OCRv6 exports themselves (no `onnx` package and no model in
this image), so that a shipped graph matches these patterns node for node.
"""
import numpy as np
import pytest

from ppocr_native_amd import export, onnxproto
from ppocr_native_amd.export import ExportError
from ppocr_native_amd.planfile import KINDS, FUSED

from onnx_eval import GraphMaker, evaluate

RNG = np.random.default_rng(41)
HS = 0.16666670143604279


def weights(seed):
    """Seeded weight maker: the same graph each time a builder runs."""
    rng = np.random.default_rng(seed)

    def w(*shape, s=0.3):
        return rng.normal(0, s, shape).astype(np.float32)

    w.rng = rng
    return w


def roundtrip(g):
    """The graph through ModelProto bytes and back."""
    return onnxproto.decode_model(onnxproto.encode_model(g))


def plan_ops(plan: bytes):
    """(kind, fused) of each operation record of a plan."""
    import struct
    words = struct.unpack_from("<7I", plan, 8)
    n_out, n_ops = words[5], words[6]
    base = 8 + 4 * (7 + n_out)
    out = []
    for k in range(n_ops):
        kind, fused = struct.unpack_from("<2I", plan, base + 80 * k)
        out.append((KINDS[kind], FUSED[fused]))
    return out


def near(got, want, rtol=2e-4, atol=1e-4):
    got, want = np.asarray(got, np.float64).reshape(-1), np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    bad = np.flatnonzero(err > rtol * np.abs(want) + atol)
    assert bad.size == 0, f"{bad.size} of {got.size} differ, worst {err.max():.3g} at {bad[:5]}"


def hwc(t):
    """An NCHW batch-1 tensor in the plan's HWC storage."""
    return np.transpose(t[0], (1, 2, 0))


def detector_graph(seed=3):
    w = weights(seed)
    m = GraphMaker("x", [1, 3, "h", "w"])
    x = m.input.name
    # Stem: 3x3 stride 2 + BatchNorm + Relu, the SAME_UPPER 2x2 max pool.
    c = m.op("Conv", x, m.const(w(8, 3, 3, 3)), m.const(w(8)), strides=[2, 2], pads=[1, 1, 1, 1])
    bn = m.op("BatchNormalization", c, m.const(w.rng.uniform(0.5, 1.5, 8)), m.const(w(8)),
              m.const(w(8, s=0.1)), m.const(w.rng.uniform(0.5, 2.0, 8)), epsilon=1e-5)
    s = m.op("Relu", bn)
    s = m.op("MaxPool", s, kernel_shape=[2, 2], strides=[1, 1], auto_pad=b"SAME_UPPER")
    # Depthwise 3x3, bias by an Add, hard sigmoid (the exports' 1/6).
    d = m.op("Conv", s, m.const(w(8, 1, 3, 3)), group=8, pads=[1, 1, 1, 1])
    d = m.op("Add", d, m.const(w(1, 8, 1, 1)))
    d = m.op("HardSigmoid", d, alpha=HS, beta=0.5)
    # Squeeze-and-excite: mean, 1x1 + Relu, 1x1 + hard sigmoid 0.2, gate.
    g = m.op("GlobalAveragePool", d)
    g = m.op("Relu", m.op("Conv", g, m.const(w(4, 8, 1, 1)), m.const(w(4))))
    g = m.op("HardSigmoid", m.op("Conv", g, m.const(w(8, 4, 1, 1)), m.const(w(8))), alpha=0.2, beta=0.5)
    d = m.op("Mul", d, g)
    # 1x1 + Sigmoid, residual Add; 1x1 + x*sigmoid(x); 1x1 + erf GELU.
    e = m.op("Sigmoid", m.op("Conv", d, m.const(w(8, 8, 1, 1)), m.const(w(8))))
    e = m.op("Add", e, s)
    f = m.op("Conv", e, m.const(w(8, 8, 1, 1)), m.const(w(8)))
    f = m.op("Mul", f, m.op("Sigmoid", f))
    gl = m.op("Conv", f, m.const(w(8, 8, 1, 1)), m.const(w(8)))
    half = m.op("Mul", m.op("Mul", gl, m.op("Add", m.op("Erf", m.op("Div", gl, m.const(np.sqrt(2.0)))),
                                             m.const(1.0))), m.const(0.5))
    # A second SE by ReduceMean over H, W.
    r = m.op("ReduceMean", half, axes=[2, 3], keepdims=1)
    r = m.op("Sigmoid", m.op("Conv", r, m.const(w(8, 8, 1, 1)), m.const(w(8))))
    half = m.op("Mul", half, r)
    # Down by 2, then up again: upsample + add of the skip, plain upsample.
    lo = m.op("Relu", m.op("Conv", half, m.const(w(8, 8, 3, 3)), m.const(w(8)), strides=[2, 2], pads=[1, 1, 1, 1]))
    up = m.op("Resize", lo, "", m.const([1, 1, 2, 2]), mode=b"nearest",
              coordinate_transformation_mode=b"asymmetric", nearest_mode=b"floor")
    up = m.op("Add", up, half)
    lo2 = m.op("Resize", lo, "", m.const([1, 1, 2, 2]), mode=b"nearest",
               coordinate_transformation_mode=b"asymmetric", nearest_mode=b"floor")
    # Three-way concat read in place by a 3x3 conv; two-way by a 1x1 (chained).
    cat = m.op("Concat", up, lo2, half, axis=1)
    k3 = m.op("Relu", m.op("Conv", cat, m.const(w(8, 24, 3, 3, s=0.1)), m.const(w(8)), pads=[1, 1, 1, 1]))
    cat2 = m.op("Concat", k3, up, axis=1)
    k1 = m.op("Conv", cat2, m.const(w(6, 16, 1, 1)), m.const(w(6)))
    # The DB head: two 2x2 transposed convs (Add bias + Relu, then Sigmoid).
    t1 = m.op("Relu", m.op("Add", m.op("ConvTranspose", k1, m.const(w(6, 4, 2, 2)), strides=[2, 2]),
                           m.const(w(1, 4, 1, 1))))
    t2 = m.op("Sigmoid", m.op("ConvTranspose", t1, m.const(w(4, 1, 2, 2)), m.const(w(1)), strides=[2, 2]))
    m.output(t2)
    # And an average-pooled side output through an Identity.
    m.output(m.op("Identity", m.op("AveragePool", k1, kernel_shape=[2, 2], strides=[2, 2])))
    return m.graph()


def test_onnx_wire_format_roundtrip():
    g = detector_graph()
    back = roundtrip(g)
    assert [n.op_type for n in back.nodes] == [n.op_type for n in g.nodes]
    assert [n.inputs for n in back.nodes] == [n.inputs for n in g.nodes]
    for a, b in zip(g.nodes, back.nodes):
        assert set(a.attrs) == set(b.attrs)
        for k in a.attrs:
            va, vb = a.attrs[k], b.attrs[k]
            if isinstance(va, float):
                assert np.float32(va) == np.float32(vb)
            else:
                assert va == vb or list(va) == list(vb)
    assert set(back.initializers) == set(g.initializers)
    for k, v in g.initializers.items():
        assert np.array_equal(back.initializers[k], v) and back.initializers[k].dtype == v.dtype
    assert back.inputs[0].dims == [1, 3, "h", "w"]


def test_detector_rules(oracle):
    g = roundtrip(detector_graph())
    plan = export.export(g)
    kinds = plan_ops(plan)
    # The folds the rules promise, in run order.
    assert kinds[0] == ("conv", "relu")
    assert ("maxpool", "none") in kinds and ("dwconv", "hardsigmoid") in kinds
    assert ("conv", "hardsigmoidfifth") in kinds and ("conv", "swish") in kinds and ("conv", "gelu") in kinds
    assert [k for k, _ in kinds].count("mean") == 2 and [k for k, _ in kinds].count("channelmul") == 2
    assert ("upsampleadd", "none") in kinds and ("upsample", "none") in kinds
    assert [k for k, _ in kinds].count("concatc") == 2  # one for the 3-way (last in place), one 2-way
    assert ("convtranspose", "relu") in kinds and ("convtranspose", "sigmoid") in kinds
    assert ("avgpool", "none") in kinds
    x = RNG.uniform(-1, 1, (1, 3, 64, 64))
    want = evaluate(roundtrip(detector_graph()), x)
    got = oracle.OracleModel(plan).run(hwc(x).astype(np.float32))
    assert len(got) == 2
    near(got[0], hwc(want[0]))
    near(got[1], hwc(want[1]))


def recogniser_graph(heads=4, dim=8, vocab=4100, seed=5, select="slice", zero_add=True, axes_inputs=False,
                     swapped=False):
    """An SVTR-like recogniser. The options write the same network other
    ways: q, k, v picked by Gather instead of Slice + Squeeze, no zero Add on
    the scores, axes given as inputs (opset 13+) instead of attributes, and
    the commutative operands of the bias Adds and the swish Mul swapped."""
    w = weights(seed)
    c = heads * dim
    m = GraphMaker("x", [1, 3, 48, "w"])
    x = m.input.name
    s = m.op("Relu", m.op("Conv", x, m.const(w(16, 3, 3, 3)), m.const(w(16)), strides=[2, 2], pads=[1, 1, 1, 1]))
    s = m.op("Conv", s, m.const(w(c, 16, 3, 3, s=0.2)), m.const(w(c)), strides=[2, 1], pads=[1, 1, 1, 1])
    s = m.op("AveragePool", s, kernel_shape=[12, 2], strides=[12, 2])   # [1, c, 1, 80]
    # [1, c, 1, T] -> [1, c, T] by a Reshape whose target is worked out from
    # the Shape, then -> [1, T, c]: storage aliases.
    shp = m.op("Shape", s)
    head = m.op("Slice", shp, m.const([0], np.int64), m.const([2], np.int64), m.const([0], np.int64))
    tgt = m.op("Concat", head, m.const([-1], np.int64), axis=0)
    z = m.op("Transpose", m.op("Reshape", s, tgt), perm=[0, 2, 1])

    def mean_last(t):
        if axes_inputs:
            return m.op("ReduceMean", t, m.const([-1], np.int64), keepdims=1)
        return m.op("ReduceMean", t, axes=[-1], keepdims=1)

    def ln(t):
        mu = mean_last(t)
        d = m.op("Sub", t, mu)
        var = mean_last(m.op("Pow", d, m.const(2.0)))
        y = m.op("Div", d, m.op("Sqrt", m.op("Add", var, m.const([1e-6]))))
        return m.op("Add", m.op("Mul", y, m.const(w.rng.normal(1, 0.1, c))), m.const(w(c, s=0.1)))

    def linear(t, ci, co, s=None):
        mm = m.op("MatMul", t, m.const(w(ci, co, s=s or 1 / np.sqrt(ci))))
        b = m.const(w(co, s=0.1))
        return m.op("Add", b, mm) if swapped else m.op("Add", mm, b)

    def pick(r, i):
        if select == "gather":
            return m.op("Gather", r, m.const(i, np.int64), axis=0)
        part = m.op("Slice", r, m.const([i], np.int64), m.const([i + 1], np.int64), m.const([0], np.int64))
        if axes_inputs:
            return m.op("Squeeze", part, m.const([0], np.int64))
        return m.op("Squeeze", part, axes=[0])

    qkv = linear(ln(z), c, 3 * c)
    r = m.op("Transpose", m.op("Reshape", qkv, m.const([0, -1, 3, heads, dim], np.int64)), perm=[2, 0, 3, 1, 4])
    q, k, v = (pick(r, i) for i in range(3))
    q = m.op("Mul", m.const(dim ** -0.5), q) if swapped else m.op("Mul", q, m.const(dim ** -0.5))
    a = m.op("MatMul", q, m.op("Transpose", k, perm=[0, 1, 3, 2]))
    if zero_add:
        a = m.op("Add", a, m.const(0.0))
    a = m.op("Softmax", a, axis=-1)
    o = m.op("Reshape", m.op("Transpose", m.op("MatMul", a, v), perm=[0, 2, 1, 3]), m.const([0, -1, c], np.int64))
    z = m.op("Add", z, linear(o, c, c))
    f = linear(ln(z), c, 2 * c)
    f = m.op("Mul", m.op("Sigmoid", f), f) if swapped else m.op("Mul", f, m.op("Sigmoid", f))
    z = m.op("Add", z, linear(f, 2 * c, c))
    logits = m.op("Softmax", linear(m.op("Identity", ln(z)), c, vocab, s=1.0), axis=-1)
    m.output(logits)
    return m.graph()


@pytest.mark.parametrize("argmax", [False, True])
def test_recogniser_rules(oracle, argmax):
    plan = export.export(onnxproto.encode_model(recogniser_graph()), argmax=argmax)
    kinds = [k for k, _ in plan_ops(plan)]
    assert kinds.count("layernorm") == 3 and kinds.count("attention") == 1
    assert kinds[-1] == ("ctcargmax" if argmax else "ctchead")
    assert ("conv", "swish") in plan_ops(plan)
    x = RNG.uniform(-1, 1, (1, 3, 48, 320))
    probs = evaluate(recogniser_graph(), x)[0][0]  # [T, V]
    got = oracle.OracleModel(plan).run(hwc(x).astype(np.float32))[0]
    if argmax:
        got = got.reshape(-1, 2)
        assert np.array_equal(got[:, 0].astype(np.int64), probs.argmax(axis=1))
        near(got[:, 1], probs.max(axis=1))
    else:
        near(got, probs, rtol=2e-3, atol=1e-7)


def test_refusals():
    w = weights(9)
    m = GraphMaker("x", [1, 4, 8, 8])
    m.output(m.op("Conv", m.input.name, m.const(w(4, 4, 3, 3)), dilations=[2, 2]))
    with pytest.raises(ExportError, match="dilated"):
        export.export(m.graph())
    m = GraphMaker("x", [1, 4, 8, 8])
    m.output(m.op("Tanh", m.input.name))
    with pytest.raises(ExportError, match="unsupported Tanh node"):
        export.export(m.graph())
    m = GraphMaker("x", [1, 4, 8, 8])
    m.output(m.op("HardSigmoid", m.op("Conv", m.input.name, m.const(w(4, 4, 1, 1))), alpha=0.3, beta=0.5))
    with pytest.raises(ExportError, match="HardSigmoid"):
        export.export(m.graph())


@pytest.mark.parametrize("select,zero_add,axes_inputs,swapped", [
    ("gather", False, False, False), ("slice", True, True, False), ("slice", False, False, True),
    ("gather", True, True, True)])
def test_recogniser_written_other_ways(oracle, select, zero_add, axes_inputs, swapped):
    """The same network written with other operators and operand orders
    gives the same operations and the same results."""
    kw = dict(select=select, zero_add=zero_add, axes_inputs=axes_inputs, swapped=swapped)
    plan = export.export(onnxproto.encode_model(recogniser_graph(**kw)), argmax=True)
    assert [k for k, _ in plan_ops(plan)] == [k for k, _ in plan_ops(export.export(recogniser_graph(), argmax=True))]
    assert ("conv", "swish") in plan_ops(plan)
    x = RNG.uniform(-1, 1, (1, 3, 48, 320))
    probs = evaluate(recogniser_graph(**kw), x)[0][0]
    got = oracle.OracleModel(plan).run(hwc(x).astype(np.float32))[0].reshape(-1, 2)
    assert np.array_equal(got[:, 0].astype(np.int64), probs.argmax(axis=1))
    near(got[:, 1], probs.max(axis=1))


def extension_graph(seed=11):
    """Forms the plan holds that the engine's own exporter does not write:
    a HardSwish folded into its conv (activation code 7), an Add of two maps
    with its ReLU folded, Resize by output sizes, a residual Add whose
    operands come in the other order."""
    w = weights(seed)
    m = GraphMaker("x", [1, 3, "h", "w"])
    x = m.input.name
    a = m.op("HardSwish", m.op("Conv", x, m.const(w(8, 3, 3, 3)), m.const(w(8)), pads=[1, 1, 1, 1]))
    b = m.op("Conv", a, m.const(w(8, 8, 1, 1)), m.const(w(8)))
    s = m.op("Relu", m.op("Add", b, a))
    lo = m.op("Conv", s, m.const(w(8, 8, 3, 3, s=0.1)), m.const(w(8)), strides=[2, 2], pads=[1, 1, 1, 1])
    up = m.op("Resize", lo, "", "", m.const([1, 8, 64, 64], np.int64), mode=b"nearest",
              coordinate_transformation_mode=b"asymmetric", nearest_mode=b"floor")
    m.output(m.op("Add", s, up))
    return m.graph()


def test_extensions(oracle):
    plan = export.export(roundtrip(extension_graph()))
    kinds = plan_ops(plan)
    assert kinds[0] == ("conv", "hardswish") and ("add", "relu") in kinds
    assert ("upsampleadd", "none") in kinds
    x = RNG.uniform(-1, 1, (1, 3, 64, 64))
    want = evaluate(extension_graph(), x)[0]
    got = oracle.OracleModel(plan).run(hwc(x).astype(np.float32))[0]
    near(got, hwc(want))


def _refused(build, match):
    m = GraphMaker("x", [1, 4, 8, 8])
    m.output(build(m, weights(13)))
    with pytest.raises(ExportError, match=match):
        export.export(m.graph())


def test_more_refusals():
    x = "x"
    # A transpose that swaps height and width keeps every byte in place but
    # is no longer channels-last; a reshape across the channel axis moves data.
    _refused(lambda m, w: m.op("Conv", m.op("Transpose", x, perm=[0, 1, 3, 2]), m.const(w(4, 4, 1, 1))),
             "channels-last")
    _refused(lambda m, w: m.op("Conv", m.op("Reshape", x, m.const([1, 8, 4, 64], np.int64)), m.const(w(4, 8, 1, 1))),
             "rearrangement")
    # SAME padding at stride 2 depends on the input size.
    _refused(lambda m, w: m.op("Conv", x, m.const(w(4, 4, 3, 3)), strides=[2, 2], auto_pad=b"SAME_UPPER"),
             "SAME_UPPER")
    # Groups that are not depthwise.
    _refused(lambda m, w: m.op("Conv", x, m.const(w(4, 2, 3, 3)), group=2, pads=[1, 1, 1, 1]), "groups")
    # Concatenation along the height.
    _refused(lambda m, w: m.op("Conv", m.op("Concat", x, x, axis=2), m.const(w(4, 4, 1, 1))), "another axis")
    # An activation whose input another node also reads cannot fold into
    # its conv, and no plan operation is a ReLU alone.
    def shared(m, w):
        c = m.op("Conv", x, m.const(w(4, 4, 1, 1)))
        return m.op("Add", m.op("Relu", c), c)
    _refused(shared, "unsupported Relu node")
    # A Softmax without an explicit axis is not the CTC head (the default axis differs between opsets).
    m = GraphMaker("x", [1, 3, 48, "w"])
    t = m.op("Transpose", m.op("Reshape", m.op("AveragePool", m.input.name, kernel_shape=[48, 4], strides=[48, 4]),
                                m.const([1, 3, -1], np.int64)), perm=[0, 2, 1])
    m.output(m.op("Softmax", m.op("Add", m.op("MatMul", t, m.const(np.ones((3, 4100), np.float32))),
                                  m.const(np.zeros(4100, np.float32)))))
    with pytest.raises(ExportError, match="unsupported Softmax node"):
        export.export(m.graph())


def test_reader_dimension_fields_and_external_data():
    """A dimension's denotation (field 3) leaves its extent alone; a tensor
    stored in an external file is refused by name."""
    from ppocr_native_amd.onnxproto import _bytes, _int
    dim = lambda *fields: _bytes(1, b"".join(fields))
    shape = dim(_int(1, 1)) + dim(_int(1, 3), _bytes(3, b"DATA_CHANNEL")) + dim(_bytes(2, b"h")) + dim()
    value = _bytes(1, b"x") + _bytes(2, _bytes(1, _int(1, 1) + _bytes(2, shape)))
    assert onnxproto._read_value(value).dims == [1, 3, "h", None]
    external = _int(1, 4) + _int(2, 1) + _bytes(8, b"w0") + _bytes(13, _bytes(1, b"location") + _bytes(2, b"w.bin"))
    with pytest.raises(ValueError, match="w0 keeps its data in an external file"):
        onnxproto.read_tensor(external)
