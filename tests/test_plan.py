"""Plan reading and checking: the reference's own plan tests
(src/engine/plan.rs:947-1059, src/engine/mod.rs:1509-1554), run against both
readers: the oracle's (CPU) and the HIP library's (whose parser runs before
it looks for a GPU, so a refusal is visible without one).
"""
import struct

import numpy as np
import pytest

from ppocr_native_amd import GpuError, GpuModel
from ppocr_native_amd.planfile import MAGIC, Op, encode


def pointwise():
    # A 1x1 convolution, 4 channels to 4, over a 2x2 image (plan.rs:934-940).
    return Op("conv", 0, 1, 4, 4, kh=1, kw=1, sh=1, sw=1, w=(0, 16), b=(16, 4))


def file(ops, weights):
    return encode((0, 2, 2, 4), 2, [1], ops, np.arange(weights, dtype=np.float32))


def product_refuses(data: bytes) -> str | None:
    """The HIP library's refusal, or None when it got past the plan."""
    try:
        GpuModel.load(data).close()
        return None
    except GpuError as e:
        msg = str(e)
        if msg.startswith("no GPU") or "GPU" in msg.split(":")[0]:
            return None
        return msg


def test_round_trip(oracle):
    m = oracle.OracleModel(file([pointwise()], 20))
    op = m.ops()[0]
    assert (op["ih"], op["iw"], op["oh"], op["ow"]) == (2, 2, 2, 2)
    assert (m.pool(0), m.pool(1)) == (16, 16)
    assert product_refuses(file([pointwise()], 20)) is None


def malformed_files():
    good = file([pointwise()], 20)
    header = len(MAGIC) + 4 * 8
    cases = [
        ("not a plan", b"not a plan at all, really"),
        ("truncated description", good[:header + 10]),
        ("no weights", good[:128]),
        ("truncated weights", good[:-2]),
    ]

    def edit(what, at, v):
        b = bytearray(good)
        b[at:at + 4] = struct.pack("<I", v)
        cases.append((what, bytes(b)))

    def field(k):
        return header + 4 * k

    edit("unknown kind", field(0), 99)
    edit("unknown activation", field(1), 99)
    edit("missing buffer", field(4), 7)
    edit("weights past the end", field(16), 8)
    edit("weights the shape contradicts", field(17), 12)
    edit("a zero-sized image", len(MAGIC) + 4, 0)
    edit("no buffers", len(MAGIC) + 16, 0)
    edit("an operation count past the file", len(MAGIC) + 24, 0xFFFFFFFF)
    nan = bytearray(good)
    nan[-4:] = struct.pack("<f", float("nan"))
    cases.append(("a weight that is not a number", bytes(nan)))
    inf = bytearray(good)
    inf[-4:] = struct.pack("<f", float("inf"))
    cases.append(("an infinite weight", bytes(inf)))
    return cases


@pytest.mark.parametrize("what,data", malformed_files(), ids=[c[0] for c in malformed_files()])
def test_malformed_files_refused(oracle, what, data):
    with pytest.raises(oracle.OracleError):
        oracle.OracleModel(data)
    assert product_refuses(data) is not None, what


def test_subnormal_weights_load_as_zero(oracle):
    vals = np.arange(20, dtype=np.float32)
    vals[-1] = -np.float32(np.finfo(np.float32).smallest_subnormal)
    data = encode((0, 2, 2, 4), 2, [1], [pointwise()], vals)
    m = oracle.OracleModel(data)
    # Bias 3 is the last weight: -0 now, so output channel 3 is the plain sum.
    x = np.ones((2, 2, 4), np.float32)
    y = m.run(x)[0].reshape(4, 4)
    w = np.arange(16, dtype=np.float32).reshape(4, 4)
    assert np.array_equal(y[:, 3], np.full(4, w[:, 3].sum(), np.float32))


def bad_ops():
    def mut(**kw):
        op = pointwise()
        for k, v in kw.items():
            setattr(op, k, v)
        return op

    return [
        ("zero input channels", mut(ic=0)),
        ("zero stride", mut(sw=0)),
        ("padding past the window limit", mut(pl=1 << 20)),
        ("bias of the wrong length", mut(b=(16, 3))),
        ("output over its input", mut(y=0)),
        ("folded activation on a mean", mut(kind="mean", fused="relu", w=(0, 0), b=(0, 0))),
        ("unused weights on an addition", mut(kind="add")),
        ("second input on a pointwise layer", mut(n2=4)),
        ("overlapping transposed windows",
         mut(kind="convtranspose", kh=2, kw=2, sh=1, sw=1, w=(0, 64), b=(0, 0))),
    ]


@pytest.mark.parametrize("what,op", bad_ops(), ids=[c[0] for c in bad_ops()])
def test_malformed_operations_refused(oracle, what, op):
    data = file([op], 80)
    with pytest.raises(oracle.OracleError):
        oracle.OracleModel(data)
    assert product_refuses(data) is not None, what


def test_sizes_follow_the_input(oracle):
    # A padded stride-2 3x3 convolution, then a 2x upsampling (plan.rs:1038-1059).
    stem = Op("conv", 0, 1, 3, 4, kh=3, kw=3, sh=2, sw=2, pt=1, pb=1, pl=1, pr=1,
              w=(0, 108), b=(108, 4))
    up = Op("upsample", 1, 0, 4, 4, sh=2, sw=2)
    data = encode((0, 8, 8, 3), 2, [0], [stem, up], np.full(112, 0.5, np.float32))
    m = oracle.OracleModel(data)
    m.set_size(6, 10)
    assert [(o["oh"], o["ow"]) for o in m.ops()] == [(3, 5), (6, 10)]
    assert (m.pool(0), m.pool(1)) == (240, 60)
    with pytest.raises(oracle.OracleError):
        m.set_size(1 << 20, 1 << 20)
    assert m.input_shape() == (6, 10, 3) and m.ops()[1]["ow"] == 10
    # The upsampling writes the input's buffer, its only writer: accepted
    # (src/engine/gpu/mod.rs:622-630 counts operations, not the image).
    assert product_refuses(data) is None


def test_rewritten_buffer_is_refused():
    # src/engine/gpu/mod.rs:1071-1088: a chain of adds writing buffer 1 twice.
    def plan(last_y):
        ops = [Op("add", 0, 1, 3, 3, x2=0), Op("add", 1, 2, 3, 3, x2=1),
               Op("add", 2, last_y, 3, 3, x2=2)]
        return encode((0, 2, 2, 3), 4, [last_y], ops, np.zeros(0, np.float32))

    assert product_refuses(plan(3)) is None
    assert "again" in product_refuses(plan(1))


def test_ctchead_with_probabilities_refused():
    # The GPU runs only the argmax head (src/engine/gpu/mod.rs:642).
    ci, vocab = 4, 20
    cols = 32
    head = Op("ctchead", 0, 1, ci, vocab, w=(0, cols * ci), b=(cols * ci, cols))
    data = encode((0, 1, 5, ci), 2, [1], [head], np.zeros(cols * ci + cols, np.float32))
    assert "probabilities" in product_refuses(data)


def test_bad_sizes_keep_model_size(oracle, pkg):
    from ppocr_native_amd import nets
    m = oracle.OracleModel(nets.detector_plan(h=64, w=64, init="scaled"))
    for h, w in [(48, 40), (0, 64), (64, 0), (1 << 20, 1 << 20)]:
        with pytest.raises(oracle.OracleError):
            m.set_size(h, w)
        assert m.input_shape() == (64, 64, 3)
    m.set_size(96, 32)
    assert m.input_shape() == (96, 32, 3)
