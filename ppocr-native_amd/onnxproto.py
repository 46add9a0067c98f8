"""A reader and writer for the part of the ONNX file format the exporter
uses, straight on the protobuf wire format (no `onnx` package: this image
has none).

Messages and field numbers follow the published `onnx.proto` (ONNX IR):
ModelProto.graph = 7; GraphProto node = 1, name = 2, initializer = 5,
input = 11, output = 12, value_info = 13; NodeProto input = 1, output = 2,
name = 3, op_type = 4, attribute = 5; AttributeProto name = 1, f = 2,
i = 3, s = 4, t = 5, floats = 7, ints = 8, type = 20; TensorProto dims = 1,
data_type = 2, float_data = 4, int32_data = 5, int64_data = 7, name = 8,
raw_data = 9, double_data = 10; ValueInfoProto name = 1, type = 2;
TypeProto tensor_type = 1; Tensor elem_type = 1, shape = 2;
TensorShapeProto dim = 1; Dimension dim_value = 1, dim_param = 2,
denotation = 3 (ignored); TensorProto external_data = 13 and
data_location = 14 are refused with the tensor's name.

The graph comes back as plain Python objects (`Graph`, `Node`, `Value`)
with initializers as numpy arrays; `encode_model` writes such a graph back
as ModelProto bytes (used to build test models).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

# TensorProto.DataType codes and the numpy types they hold.
DTYPES = {1: np.float32, 2: np.uint8, 3: np.int8, 6: np.int32, 7: np.int64, 9: np.bool_,
          10: np.float16, 11: np.float64}
CODES = {np.dtype(v): k for k, v in DTYPES.items()}


@dataclass
class Node:
    op_type: str
    inputs: list[str]
    outputs: list[str]
    name: str = ""
    attrs: dict = field(default_factory=dict)  # name -> int, float, bytes, list or ndarray


@dataclass
class Value:
    name: str
    dims: list  # int, or a str for a symbolic dimension, or None when unknown
    elem_type: int = 1


@dataclass
class Graph:
    nodes: list[Node]
    initializers: dict[str, np.ndarray]
    inputs: list[Value]
    outputs: list[Value]
    name: str = ""


# ----------------------------------------------------------------- reading

def _varint(buf: bytes, i: int) -> tuple[int, int]:
    v = shift = 0
    while True:
        b = buf[i]
        i += 1
        v |= (b & 0x7F) << shift
        if b < 0x80:
            return v, i
        shift += 7


def _fields(buf: bytes):
    """(field number, wire type, value) of each field of a message: an int
    for varints, bytes for length-delimited and fixed-width fields."""
    i, n = 0, len(buf)
    while i < n:
        key, i = _varint(buf, i)
        num, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
        elif wt == 1:
            v, i = buf[i:i + 8], i + 8
        elif wt == 2:
            ln, i = _varint(buf, i)
            v, i = buf[i:i + ln], i + ln
        elif wt == 5:
            v, i = buf[i:i + 4], i + 4
        else:
            raise ValueError(f"unsupported protobuf wire type {wt}")
        if i > n:
            raise ValueError("truncated protobuf message")
        yield num, wt, v


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _packed_ints(wt: int, v) -> list[int]:
    if wt == 0:
        return [_signed(v)]
    out, i = [], 0
    while i < len(v):
        x, i = _varint(v, i)
        out.append(_signed(x))
    return out


def _packed_floats(wt: int, v) -> list[float]:
    if wt == 5:
        return [struct.unpack("<f", v)[0]]
    return list(struct.unpack(f"<{len(v) // 4}f", v))


def read_tensor(buf: bytes) -> tuple[str, np.ndarray]:
    dims, dtype, name, raw, external = [], 1, "", None, False
    floats, ints32, ints64, doubles = [], [], [], []
    for num, wt, v in _fields(buf):
        if num == 1:
            dims += _packed_ints(wt, v)
        elif num == 2:
            dtype = v
        elif num == 4:
            floats += _packed_floats(wt, v)
        elif num == 5:
            ints32 += _packed_ints(wt, v)
        elif num == 7:
            ints64 += _packed_ints(wt, v)
        elif num == 8:
            name = v.decode()
        elif num == 9:
            raw = v
        elif num == 10:
            doubles += list(struct.unpack(f"<{len(v) // 8}d", v)) if wt == 2 else [struct.unpack("<d", v)[0]]
        elif num == 13 or (num == 14 and v == 1):  # external_data, data_location = EXTERNAL
            external = True
    if external:
        raise ValueError(f"tensor {name or '(unnamed)'} keeps its data in an external file, which this "
                         "reader does not follow; save the model with its weights inside")
    if dtype not in DTYPES:
        raise ValueError(f"tensor {name}: unsupported data type {dtype}")
    np_type = np.dtype(DTYPES[dtype]).newbyteorder("<")
    if raw is not None:
        arr = np.frombuffer(raw, dtype=np_type).astype(DTYPES[dtype])
    elif dtype == 1:
        arr = np.asarray(floats, np.float32)
    elif dtype == 11:
        arr = np.asarray(doubles, np.float64)
    elif dtype == 7:
        arr = np.asarray(ints64, np.int64)
    else:
        arr = np.asarray(ints32, DTYPES[dtype])
    return name, arr.reshape([int(d) for d in dims]) if dims else arr.reshape(())


def _read_attr(buf: bytes):
    name, kind = "", None
    f = i = s = t = None
    floats, ints = [], []
    for num, wt, v in _fields(buf):
        if num == 1:
            name = v.decode()
        elif num == 2:
            f = struct.unpack("<f", v)[0]
        elif num == 3:
            i = _signed(v)
        elif num == 4:
            s = bytes(v)
        elif num == 5:
            t = read_tensor(v)[1]
        elif num == 7:
            floats += _packed_floats(wt, v)
        elif num == 8:
            ints += _packed_ints(wt, v)
        elif num == 20:
            kind = v
    # AttributeType: FLOAT 1, INT 2, STRING 3, TENSOR 4, FLOATS 6, INTS 7.
    value = {1: f, 2: i, 3: s, 4: t, 6: floats, 7: ints}.get(kind)
    if value is None:  # no type field: the one that is set
        value = next((x for x in (f, i, s, t) if x is not None), floats or ints)
    return name, value


def _read_node(buf: bytes) -> Node:
    node = Node("", [], [])
    for num, _, v in _fields(buf):
        if num == 1:
            node.inputs.append(v.decode())
        elif num == 2:
            node.outputs.append(v.decode())
        elif num == 3:
            node.name = v.decode()
        elif num == 4:
            node.op_type = v.decode()
        elif num == 5:
            k, val = _read_attr(v)
            node.attrs[k] = val
    return node


def _read_value(buf: bytes) -> Value:
    val = Value("", [])
    for num, _, v in _fields(buf):
        if num == 1:
            val.name = v.decode()
        elif num == 2:
            for n2, _, tt in _fields(v):
                if n2 != 1:
                    continue
                for n3, _, tv in _fields(tt):
                    if n3 == 1:
                        val.elem_type = tv
                    elif n3 == 2:
                        for n4, _, dim in _fields(tv):
                            if n4 != 1:
                                continue
                            d = None  # neither set: an unknown extent
                            for n5, _, dv in _fields(dim):
                                if n5 == 1:
                                    d = _signed(dv)
                                elif n5 == 2:
                                    d = dv.decode()
                                # field 3, the denotation, names the axis and changes nothing
                            val.dims.append(d)
    return val


def decode_model(data: bytes) -> Graph:
    """The graph of a serialized ModelProto."""
    graph = None
    for num, _, v in _fields(data):
        if num == 7:
            graph = v
    if graph is None:
        raise ValueError("not an ONNX model: no graph")
    g = Graph([], {}, [], [])
    for num, _, v in _fields(graph):
        if num == 1:
            g.nodes.append(_read_node(v))
        elif num == 2:
            g.name = v.decode()
        elif num == 5:
            name, arr = read_tensor(v)
            g.initializers[name] = arr
        elif num == 11:
            g.inputs.append(_read_value(v))
        elif num == 12:
            g.outputs.append(_read_value(v))
    # Initializers listed among the inputs are weights, not inputs.
    g.inputs = [x for x in g.inputs if x.name not in g.initializers]
    return g


def load(path) -> Graph:
    with open(path, "rb") as f:
        return decode_model(f.read())


# ----------------------------------------------------------------- writing

def _enc_varint(v: int) -> bytes:
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(num: int, wt: int) -> bytes:
    return _enc_varint(num << 3 | wt)


def _bytes(num: int, b: bytes) -> bytes:
    return _key(num, 2) + _enc_varint(len(b)) + b


def _int(num: int, v: int) -> bytes:
    return _key(num, 0) + _enc_varint(v)


def encode_tensor(name: str, arr: np.ndarray) -> bytes:
    arr = np.asarray(arr)
    code = CODES.get(arr.dtype)
    if code is None:
        raise ValueError(f"tensor {name}: unsupported dtype {arr.dtype}")
    out = b"".join(_int(1, int(d)) for d in arr.shape)
    out += _int(2, code) + _bytes(8, name.encode())
    return out + _bytes(9, np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<")).tobytes())


def _encode_attr(name: str, value) -> bytes:
    out = _bytes(1, name.encode())
    if isinstance(value, (bool, int, np.integer)):
        return out + _int(3, int(value)) + _int(20, 2)
    if isinstance(value, (float, np.floating)):
        return out + _key(2, 5) + struct.pack("<f", float(value)) + _int(20, 1)
    if isinstance(value, (bytes, str)):
        return out + _bytes(4, value.encode() if isinstance(value, str) else value) + _int(20, 3)
    if isinstance(value, np.ndarray):
        return out + _bytes(5, encode_tensor("", value)) + _int(20, 4)
    value = list(value)
    if value and all(isinstance(x, (int, np.integer)) for x in value):
        return out + _bytes(8, b"".join(_enc_varint(int(x)) for x in value)) + _int(20, 7)
    return out + _bytes(7, struct.pack(f"<{len(value)}f", *value)) + _int(20, 6)


def _encode_value(v: Value) -> bytes:
    dims = b""
    for d in v.dims:
        dims += _bytes(1, _int(1, d) if isinstance(d, int) else _bytes(2, str(d).encode()))
    tensor = _int(1, v.elem_type) + _bytes(2, dims)
    return _bytes(1, v.name.encode()) + _bytes(2, _bytes(1, tensor))


def encode_model(g: Graph) -> bytes:
    """ModelProto bytes (IR version 6, default domain opset 11) for graph g."""
    body = b""
    for n in g.nodes:
        nb = b"".join(_bytes(1, x.encode()) for x in n.inputs)
        nb += b"".join(_bytes(2, x.encode()) for x in n.outputs)
        nb += _bytes(3, n.name.encode()) + _bytes(4, n.op_type.encode())
        nb += b"".join(_bytes(5, _encode_attr(k, v)) for k, v in n.attrs.items())
        body += _bytes(1, nb)
    body += _bytes(2, g.name.encode())
    body += b"".join(_bytes(5, encode_tensor(k, v)) for k, v in g.initializers.items())
    body += b"".join(_bytes(11, _encode_value(v)) for v in g.inputs)
    body += b"".join(_bytes(12, _encode_value(v)) for v in g.outputs)
    opset = _bytes(1, b"") + _int(2, 11)
    return _int(1, 6) + _bytes(8, opset) + _bytes(7, body)
