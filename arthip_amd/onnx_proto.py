"""Minimal ONNX protobuf codec (writer and reader), no ``onnx`` dependency.

The ``onnx`` package is not available here, so models are encoded and decoded
directly in the protobuf wire format, using the field numbers of the public
``onnx.proto`` (ModelProto, GraphProto, NodeProto, AttributeProto, TensorProto,
ValueInfoProto, TypeProto, TensorShapeProto). Only what conv-chain models use
is covered. The native engine has its own independent C++ decoder
(``arthip_amd/csrc/onnx.cc``); tests run models through both.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Iterable

import numpy as np

# TensorProto.DataType
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64 = 1, 2, 3, 4, 5, 6, 7
STRING, BOOL, FLOAT16, DOUBLE, UINT32, UINT64, BFLOAT16 = 8, 9, 10, 11, 12, 13, 16

# AttributeProto.AttributeType
A_FLOAT, A_INT, A_STRING, A_TENSOR, A_GRAPH = 1, 2, 3, 4, 5
A_FLOATS, A_INTS, A_STRINGS = 6, 7, 8

_NP_OF = {FLOAT: np.float32, FLOAT16: np.float16, DOUBLE: np.float64, INT64: np.int64,
          INT32: np.int32, INT8: np.int8, UINT8: np.uint8, INT16: np.int16, UINT16: np.uint16,
          BOOL: np.bool_}
_ONNX_OF = {np.dtype(v): k for k, v in _NP_OF.items()}


# ---------------------------------------------------------------------------
# Message model
# ---------------------------------------------------------------------------

@dataclass
class Tensor:
    name: str = ""
    dims: list[int] = field(default_factory=list)
    data_type: int = 0
    raw_data: bytes = b""
    float_data: list[float] = field(default_factory=list)
    int32_data: list[int] = field(default_factory=list)
    int64_data: list[int] = field(default_factory=list)
    double_data: list[float] = field(default_factory=list)
    data_location: int = 0
    external_data: list[tuple[str, str]] = field(default_factory=list)

    def to_numpy(self) -> np.ndarray:
        """Values in the declared dtype. FLOAT16 in int32_data are bit patterns."""
        if self.data_location == 1 or self.external_data:
            raise ValueError(f"tensor {self.name!r} uses external data")
        dt = _NP_OF.get(self.data_type)
        if dt is None:
            raise ValueError(f"tensor {self.name!r}: unsupported dtype {self.data_type}")
        shape = tuple(self.dims)
        if self.raw_data:
            return np.frombuffer(self.raw_data, dtype=dt).reshape(shape).copy()
        if self.float_data:
            return np.asarray(self.float_data, dtype=dt).reshape(shape)
        if self.double_data:
            return np.asarray(self.double_data, dtype=dt).reshape(shape)
        if self.int64_data:
            return np.asarray(self.int64_data, dtype=dt).reshape(shape)
        if self.int32_data:
            if self.data_type in (FLOAT16, BFLOAT16):
                bits = np.asarray(self.int32_data, dtype=np.int64).astype(np.uint16)
                return bits.view(np.float16).reshape(shape)
            return np.asarray(self.int32_data, dtype=dt).reshape(shape)
        return np.zeros(shape, dtype=dt)


@dataclass
class Attribute:
    name: str
    type: int = 0
    f: float = 0.0
    i: int = 0
    s: bytes = b""
    t: Tensor | None = None
    floats: list[float] = field(default_factory=list)
    ints: list[int] = field(default_factory=list)
    strings: list[bytes] = field(default_factory=list)

    @property
    def value(self):
        return {A_FLOAT: self.f, A_INT: self.i, A_STRING: self.s.decode(), A_TENSOR: self.t,
                A_FLOATS: list(self.floats), A_INTS: list(self.ints),
                A_STRINGS: [x.decode() for x in self.strings]}.get(self.type)


@dataclass
class Node:
    op_type: str
    inputs: list[str]
    outputs: list[str]
    name: str = ""
    domain: str = ""
    attributes: list[Attribute] = field(default_factory=list)

    def attr(self, name: str, default=None):
        for a in self.attributes:
            if a.name == name:
                return a.value
        return default


@dataclass
class ValueInfo:
    name: str
    elem_type: int = FLOAT16
    shape: list | None = None  # ints, strings (symbolic) or None (unknown)


@dataclass
class Graph:
    nodes: list[Node] = field(default_factory=list)
    name: str = "graph"
    initializers: list[Tensor] = field(default_factory=list)
    inputs: list[ValueInfo] = field(default_factory=list)
    outputs: list[ValueInfo] = field(default_factory=list)


@dataclass
class Model:
    graph: Graph
    ir_version: int = 8
    opset_imports: list[tuple[str, int]] = field(default_factory=lambda: [("", 17)])
    producer_name: str = "arthip_amd"


# ---------------------------------------------------------------------------
# Encoding
# ---------------------------------------------------------------------------

def _varint(v: int) -> bytes:
    if v < 0:
        v += 1 << 64
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(f: int, wire: int) -> bytes:
    return _varint((f << 3) | wire)


def _len(f: int, payload: bytes) -> bytes:
    return _key(f, 2) + _varint(len(payload)) + payload


def _str(f: int, s: str | bytes) -> bytes:
    return _len(f, s.encode() if isinstance(s, str) else s)


def _int(f: int, v: int) -> bytes:
    return _key(f, 0) + _varint(int(v))


def _packed_varints(f: int, vals: Iterable[int]) -> bytes:
    vals = list(vals)
    return _len(f, b"".join(_varint(int(v)) for v in vals)) if vals else b""


def encode_tensor(t: Tensor) -> bytes:
    out = _packed_varints(1, t.dims)
    out += _int(2, t.data_type)
    if t.float_data:
        out += _len(4, struct.pack(f"<{len(t.float_data)}f", *t.float_data))
    if t.int32_data:
        out += _packed_varints(5, t.int32_data)
    if t.int64_data:
        out += _packed_varints(7, t.int64_data)
    if t.name:
        out += _str(8, t.name)
    if t.raw_data:
        out += _len(9, t.raw_data)
    if t.double_data:
        out += _len(10, struct.pack(f"<{len(t.double_data)}d", *t.double_data))
    for k, v in t.external_data:
        out += _len(13, _str(1, k) + _str(2, v))
    if t.data_location:
        out += _int(14, t.data_location)
    return out


def encode_attribute(a: Attribute) -> bytes:
    out = _str(1, a.name) + _int(20, a.type)
    if a.type == A_FLOAT:
        out += _key(2, 5) + struct.pack("<f", a.f)
    elif a.type == A_INT:
        out += _int(3, a.i)
    elif a.type == A_STRING:
        out += _str(4, a.s)
    elif a.type == A_TENSOR:
        out += _len(5, encode_tensor(a.t))
    elif a.type == A_FLOATS:
        out += _len(7, struct.pack(f"<{len(a.floats)}f", *a.floats))
    elif a.type == A_INTS:
        out += _packed_varints(8, a.ints)
    elif a.type == A_STRINGS:
        for s in a.strings:
            out += _str(9, s)
    return out


def encode_node(n: Node) -> bytes:
    out = b"".join(_str(1, i) for i in n.inputs)
    out += b"".join(_str(2, o) for o in n.outputs)
    if n.name:
        out += _str(3, n.name)
    out += _str(4, n.op_type)
    for a in n.attributes:
        out += _len(5, encode_attribute(a))
    if n.domain:
        out += _str(7, n.domain)
    return out


def encode_value_info(v: ValueInfo) -> bytes:
    tt = _int(1, v.elem_type)
    if v.shape is not None:
        dims = b""
        for d in v.shape:
            dims += _len(1, _int(1, d) if isinstance(d, int) else _str(2, str(d)))
        tt += _len(2, dims)
    return _str(1, v.name) + _len(2, _len(1, tt))


def encode_graph(g: Graph) -> bytes:
    out = b"".join(_len(1, encode_node(n)) for n in g.nodes)
    out += _str(2, g.name)
    out += b"".join(_len(5, encode_tensor(t)) for t in g.initializers)
    out += b"".join(_len(11, encode_value_info(v)) for v in g.inputs)
    out += b"".join(_len(12, encode_value_info(v)) for v in g.outputs)
    return out


def encode_model(m: Model) -> bytes:
    out = _int(1, m.ir_version) + _str(2, m.producer_name)
    out += _len(7, encode_graph(m.graph))
    for dom, ver in m.opset_imports:
        out += _len(8, _str(1, dom) + _int(2, ver))
    return out


# ---------------------------------------------------------------------------
# Decoding
# ---------------------------------------------------------------------------

class _Reader:
    def __init__(self, buf: bytes, pos: int = 0, end: int | None = None):
        self.buf = buf
        self.pos = pos
        self.end = len(buf) if end is None else end

    def done(self) -> bool:
        return self.pos >= self.end

    def varint(self) -> int:
        v = shift = 0
        while True:
            if self.pos >= self.end:
                raise ValueError("truncated varint")
            b = self.buf[self.pos]
            self.pos += 1
            v |= (b & 0x7F) << shift
            if not b & 0x80:
                return v
            shift += 7
            if shift > 63:
                raise ValueError("varint too long")

    def key(self) -> tuple[int, int]:
        k = self.varint()
        return k >> 3, k & 7

    def bytes_(self) -> bytes:
        n = self.varint()
        if self.pos + n > self.end:
            raise ValueError("truncated length-delimited field")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def sub(self) -> "_Reader":
        n = self.varint()
        if self.pos + n > self.end:
            raise ValueError("truncated submessage")
        r = _Reader(self.buf, self.pos, self.pos + n)
        self.pos += n
        return r

    def skip(self, wire: int) -> None:
        if wire == 0:
            self.varint()
        elif wire == 1:
            self.pos += 8
        elif wire == 2:
            self.bytes_()
        elif wire == 5:
            self.pos += 4
        else:
            raise ValueError(f"unsupported wire type {wire}")


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _rep_varint(r: _Reader, wire: int, out: list) -> None:
    if wire == 0:
        out.append(_signed(r.varint()))
    else:
        s = r.sub()
        while not s.done():
            out.append(_signed(s.varint()))


def _rep_fixed(r: _Reader, wire: int, out: list, fmt: str, size: int) -> None:
    if wire == 2:
        b = r.bytes_()
        out.extend(struct.unpack(f"<{len(b) // size}{fmt}", b))
    else:
        out.append(struct.unpack(f"<{fmt}", r.buf[r.pos:r.pos + size])[0])
        r.pos += size


def _int32(v: int) -> int:
    v &= 0xFFFFFFFF
    return v - (1 << 32) if v >= 1 << 31 else v


def _dec_tensor(r: _Reader) -> Tensor:
    t = Tensor()
    while not r.done():
        f, w = r.key()
        if f == 1:
            _rep_varint(r, w, t.dims)
        elif f == 2:
            t.data_type = r.varint()
        elif f == 4:
            _rep_fixed(r, w, t.float_data, "f", 4)
        elif f == 5:
            vals: list[int] = []
            _rep_varint(r, w, vals)
            t.int32_data.extend(_int32(v) for v in vals)
        elif f == 7:
            _rep_varint(r, w, t.int64_data)
        elif f == 8:
            t.name = r.bytes_().decode()
        elif f == 9:
            t.raw_data = r.bytes_()
        elif f == 10:
            _rep_fixed(r, w, t.double_data, "d", 8)
        elif f == 13:
            s = r.sub()
            k = v = ""
            while not s.done():
                ff, ww = s.key()
                if ff == 1:
                    k = s.bytes_().decode()
                elif ff == 2:
                    v = s.bytes_().decode()
                else:
                    s.skip(ww)
            t.external_data.append((k, v))
        elif f == 14:
            t.data_location = r.varint()
        else:
            r.skip(w)
    return t


def _dec_attribute(r: _Reader) -> Attribute:
    a = Attribute(name="")
    while not r.done():
        f, w = r.key()
        if f == 1:
            a.name = r.bytes_().decode()
        elif f == 20:
            a.type = r.varint()
        elif f == 2:
            a.f = struct.unpack("<f", r.buf[r.pos:r.pos + 4])[0]
            r.pos += 4
        elif f == 3:
            a.i = _signed(r.varint())
        elif f == 4:
            a.s = r.bytes_()
        elif f == 5:
            a.t = _dec_tensor(r.sub())
        elif f == 7:
            _rep_fixed(r, w, a.floats, "f", 4)
        elif f == 8:
            _rep_varint(r, w, a.ints)
        elif f == 9:
            a.strings.append(r.bytes_())
        else:
            r.skip(w)
    return a


def _dec_node(r: _Reader) -> Node:
    n = Node(op_type="", inputs=[], outputs=[])
    while not r.done():
        f, w = r.key()
        if f == 1:
            n.inputs.append(r.bytes_().decode())
        elif f == 2:
            n.outputs.append(r.bytes_().decode())
        elif f == 3:
            n.name = r.bytes_().decode()
        elif f == 4:
            n.op_type = r.bytes_().decode()
        elif f == 5:
            n.attributes.append(_dec_attribute(r.sub()))
        elif f == 7:
            n.domain = r.bytes_().decode()
        else:
            r.skip(w)
    return n


def _dec_value_info(r: _Reader) -> ValueInfo:
    v = ValueInfo(name="", elem_type=0, shape=None)
    while not r.done():
        f, w = r.key()
        if f == 1:
            v.name = r.bytes_().decode()
        elif f == 2:
            tp = r.sub()
            while not tp.done():
                ff, ww = tp.key()
                if ff != 1:
                    tp.skip(ww)
                    continue
                tt = tp.sub()
                while not tt.done():
                    f3, w3 = tt.key()
                    if f3 == 1:
                        v.elem_type = tt.varint()
                    elif f3 == 2:
                        v.shape = []
                        sh = tt.sub()
                        while not sh.done():
                            f4, w4 = sh.key()
                            if f4 != 1:
                                sh.skip(w4)
                                continue
                            dm = sh.sub()
                            d: int | str | None = None
                            while not dm.done():
                                f5, w5 = dm.key()
                                if f5 == 1:
                                    d = _signed(dm.varint())
                                elif f5 == 2:
                                    d = dm.bytes_().decode()
                                else:
                                    dm.skip(w5)
                            v.shape.append(d)
                    else:
                        tt.skip(w3)
        else:
            r.skip(w)
    return v


def decode_model(buf: bytes) -> Model:
    r = _Reader(bytes(buf))
    m = Model(graph=Graph(), opset_imports=[])
    while not r.done():
        f, w = r.key()
        if f == 1:
            m.ir_version = r.varint()
        elif f == 2:
            m.producer_name = r.bytes_().decode()
        elif f == 7:
            g = r.sub()
            gr = m.graph
            while not g.done():
                ff, ww = g.key()
                if ff == 1:
                    gr.nodes.append(_dec_node(g.sub()))
                elif ff == 2:
                    gr.name = g.bytes_().decode()
                elif ff == 5:
                    gr.initializers.append(_dec_tensor(g.sub()))
                elif ff == 11:
                    gr.inputs.append(_dec_value_info(g.sub()))
                elif ff == 12:
                    gr.outputs.append(_dec_value_info(g.sub()))
                else:
                    g.skip(ww)
        elif f == 8:
            s = r.sub()
            dom, ver = "", 0
            while not s.done():
                ff, ww = s.key()
                if ff == 1:
                    dom = s.bytes_().decode()
                elif ff == 2:
                    ver = s.varint()
                else:
                    s.skip(ww)
            m.opset_imports.append((dom, ver))
        else:
            r.skip(w)
    return m


def load(path) -> Model:
    with open(path, "rb") as f:
        return decode_model(f.read())


def save(model: Model, path) -> None:
    with open(path, "wb") as f:
        f.write(encode_model(model))


# ---------------------------------------------------------------------------
# Builders (the subset of onnx.helper that the model generators use)
# ---------------------------------------------------------------------------

def tensor(name: str, array, *, typed_half: bool = False) -> Tensor:
    """Initializer from a numpy array (raw_data), or FLOAT16 values stored as
    16-bit patterns in int32_data when ``typed_half``."""
    a = np.ascontiguousarray(array)
    if typed_half:
        h = a.astype(np.float16)
        return Tensor(name=name, dims=list(h.shape), data_type=FLOAT16,
                      int32_data=[int(b) for b in h.view(np.uint16).ravel()])
    dt = _ONNX_OF.get(a.dtype)
    if dt is None:
        raise ValueError(f"unsupported numpy dtype {a.dtype}")
    return Tensor(name=name, dims=list(a.shape), data_type=dt, raw_data=a.tobytes())


def attr(name: str, value) -> Attribute:
    if isinstance(value, float):
        return Attribute(name, A_FLOAT, f=value)
    if isinstance(value, bool) or isinstance(value, int):
        return Attribute(name, A_INT, i=int(value))
    if isinstance(value, str):
        return Attribute(name, A_STRING, s=value.encode())
    if isinstance(value, Tensor):
        return Attribute(name, A_TENSOR, t=value)
    if isinstance(value, (list, tuple)):
        if all(isinstance(v, int) for v in value):
            return Attribute(name, A_INTS, ints=list(value))
        return Attribute(name, A_FLOATS, floats=[float(v) for v in value])
    raise TypeError(f"unsupported attribute value {value!r}")


def node(op_type: str, inputs, outputs, **attrs) -> Node:
    return Node(op_type=op_type, inputs=list(inputs), outputs=list(outputs),
                attributes=[attr(k, v) for k, v in attrs.items()])


def value_info(name: str, elem_type: int, shape) -> ValueInfo:
    return ValueInfo(name=name, elem_type=elem_type, shape=list(shape) if shape is not None else None)
