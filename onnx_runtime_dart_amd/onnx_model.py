"""Load path for big int4 models: MatMulNBits initializers go from the ONNX
file (or its external-data companion files) straight into HBM.

Reference: OnnxModel.fromFile / readOnnxSource (lib/src/model_source.dart:58),
the external-data resolver (lib/src/onnx_proto_loader.dart:80-125: an
initializer with data_location EXTERNAL names location / offset / length;
length 0 means "implied by the shape") and the packed NBits operands, which
the reference keeps as a Uint8List view of the raw bytes
(lib/src/onnx_proto_loader.dart:252-266).

Here the model file is parsed with a small protobuf wire reader (only the
fields the load path needs), and every MatMulNBits node's B / scales /
zero_points are handed to mg_weight_nbits_create_streamed as file ranges
(external data) or zero-copy views of the model bytes (inline raw_data).
The library streams them through pinned staging and repacks on the GPU, so
the host never holds a second copy of a multi-GB weight set.  fp16 scales
and float zero points are widened to f32 on the host first (small tensors),
as the reference's loader does (lib/src/onnx_proto_loader.dart:241-251).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from .errors import ArgumentError, StateError, UnsupportedError
from .ops import (MG_ZP_FLOAT, MG_ZP_NONE, MG_ZP_UINT4, Context, NBitsWeight, TensorSource,
                  default_context)

# TensorProto.DataType
FLOAT, UINT8, INT8, FLOAT16 = 1, 2, 3, 10
_ITEM = {FLOAT: 4, UINT8: 1, INT8: 1, FLOAT16: 2, 6: 4, 7: 8, 11: 8}


def _varint(buf, pos: int):
    out = shift = 0
    while True:
        b = buf[pos]
        pos += 1
        out |= (b & 0x7F) << shift
        if b < 0x80:
            return out, pos
        shift += 7


def _fields(buf, start: int = 0, end: int | None = None):
    """(field number, wire type, value, value start) of one message; length-
    delimited values come as (start, end) offsets into buf (no copies)."""
    pos = start
    end = len(buf) if end is None else end
    while pos < end:
        key, pos = _varint(buf, pos)
        fno, wt = key >> 3, key & 7
        if wt == 0:
            v, pos = _varint(buf, pos)
        elif wt == 1:
            v, pos = (pos, pos + 8), pos + 8
        elif wt == 2:
            ln, pos = _varint(buf, pos)
            v, pos = (pos, pos + ln), pos + ln
        elif wt == 5:
            v, pos = (pos, pos + 4), pos + 4
        else:
            raise ArgumentError(f"Malformed ONNX model: wire type {wt}")
        yield fno, wt, v


def _ints(buf, wt, v):
    if wt == 0:
        return [v]
    out, pos = [], v[0]
    while pos < v[1]:
        x, pos = _varint(buf, pos)
        out.append(x - (1 << 64) if x >= 1 << 63 else x)
    return out


def _str(buf, v) -> str:
    return bytes(buf[v[0]:v[1]]).decode()


@dataclass
class Initializer:
    """One TensorProto: its dims, type and where its bytes are."""
    name: str
    dims: list
    data_type: int
    raw: tuple | None = None          # (start, end) of raw_data in the model bytes
    external: dict = field(default_factory=dict)  # location / offset / length
    float_data: list = field(default_factory=list)
    int32_data: list = field(default_factory=list)

    @property
    def count(self) -> int:
        return int(np.prod(self.dims)) if self.dims else 1


@dataclass
class Node:
    op_type: str
    inputs: list
    outputs: list
    name: str
    attrs: dict


def _parse_tensor(buf, v) -> Initializer:
    t = Initializer("", [], FLOAT)
    location_external = False
    for fno, wt, x in _fields(buf, *v):
        if fno == 1:
            t.dims += _ints(buf, wt, x)
        elif fno == 2:
            t.data_type = x
        elif fno == 4:
            t.float_data += ([struct.unpack("<f", bytes(buf[x[0]:x[1]]))[0]] if wt == 5 else
                             list(np.frombuffer(buf, "<f4", (x[1] - x[0]) // 4, x[0])))
        elif fno == 5:
            t.int32_data += _ints(buf, wt, x)
        elif fno == 8:
            t.name = _str(buf, x)
        elif fno == 9:
            t.raw = x
        elif fno == 13:  # external_data: StringStringEntryProto {key 1, value 2}
            k = val = ""
            for f2, _, x2 in _fields(buf, *x):
                if f2 == 1:
                    k = _str(buf, x2)
                elif f2 == 2:
                    val = _str(buf, x2)
            t.external[k] = val
        elif fno == 14:
            location_external = x == 1
    if not location_external:
        t.external = {}
    return t


def _parse_attr(buf, v):
    name, val, ints = "", None, []
    for fno, wt, x in _fields(buf, *v):
        if fno == 1:
            name = _str(buf, x)
        elif fno == 3:
            val = x - (1 << 64) if x >= 1 << 63 else x
        elif fno == 8:
            ints += _ints(buf, wt, x)
        elif fno == 4:
            val = _str(buf, x)
    return name, (val if val is not None else ints)


class OnnxModel:
    """The nodes and initializers of an ONNX model file (the fields the
    matmul load path reads)."""

    def __init__(self, path):
        self.path = Path(path)
        self.data = memoryview(np.fromfile(self.path, dtype=np.uint8))
        buf = self.data
        graph = None
        for fno, _, v in _fields(buf):
            if fno == 7:
                graph = v
        if graph is None:
            raise ArgumentError(f"Malformed ONNX model (no graph): {self.path}")
        self.nodes: list[Node] = []
        self.initializers: dict[str, Initializer] = {}
        for fno, _, v in _fields(buf, *graph):
            if fno == 1:
                node = Node("", [], [], "", {})
                for f2, _, x in _fields(buf, *v):
                    if f2 == 1:
                        node.inputs.append(_str(buf, x))
                    elif f2 == 2:
                        node.outputs.append(_str(buf, x))
                    elif f2 == 3:
                        node.name = _str(buf, x)
                    elif f2 == 4:
                        node.op_type = _str(buf, x)
                    elif f2 == 5:
                        k, a = _parse_attr(buf, x)
                        node.attrs[k] = a
                self.nodes.append(node)
            elif fno == 5:
                t = _parse_tensor(buf, v)
                self.initializers[t.name] = t

    def source(self, t: Initializer, expected_bytes: int) -> TensorSource:
        """The tensor's bytes as a TensorSource: a file range for external
        data, else a zero-copy view of raw_data."""
        if t.external:
            loc = t.external.get("location", "")
            if not loc:
                raise StateError(f'"{t.name}" stores its weights externally without a location')
            length = int(t.external.get("length", "0") or 0)
            return TensorSource.from_file(self.path.parent / loc,
                                          int(t.external.get("offset", "0") or 0),
                                          length if length > 0 else expected_bytes)
        if t.raw is not None:
            if t.raw[1] - t.raw[0] < expected_bytes:
                raise ArgumentError(f'"{t.name}": raw_data holds {t.raw[1] - t.raw[0]} bytes, '
                                    f"needs {expected_bytes}")
            view = np.frombuffer(self.data, np.uint8, t.raw[1] - t.raw[0], t.raw[0])
            return TensorSource.from_array(view)
        if t.int32_data:  # inline carrier of uint8 / int8
            return TensorSource.from_array(np.array(t.int32_data, np.int64).astype(np.uint8))
        if t.float_data:
            return TensorSource.from_array(np.array(t.float_data, np.float32))
        raise ArgumentError(f'"{t.name}" has no data')

    def read_array(self, t: Initializer, dtype) -> np.ndarray:
        """A small tensor read into host memory (widening fp16 to f32)."""
        n = t.count
        item = _ITEM.get(t.data_type)
        if item is None:
            raise UnsupportedError(f'"{t.name}": data type {t.data_type}')
        src = self.source(t, n * item)
        if src.host:
            raw = np.asarray(src._keep).view(np.uint8)[: n * item]
        else:
            with open(src.path.decode(), "rb") as f:
                f.seek(src.offset)
                raw = np.frombuffer(f.read(n * item), np.uint8)
            if raw.size < n * item:
                raise ArgumentError(f'"{t.name}": external data is short')
        if t.data_type == FLOAT16:
            return raw.view("<f2").astype(np.float32).astype(dtype)
        npdt = {FLOAT: "<f4", UINT8: np.uint8, INT8: np.int8, 6: "<i4", 7: "<i8", 11: "<f8"}
        return raw.view(npdt[t.data_type]).astype(dtype)


def load_matmul_nbits(path, ctx: Context | None = None, chunk_bytes: int = 0
                      ) -> dict[str, NBitsWeight]:
    """Uploads the weights of every MatMulNBits node whose B and scales are
    initializers; returns them by the node's first output name.  Attribute
    and input checks follow opMatMulNBits (lib/src/onnx_qlinear_ops.dart:
    115-166) and the dispatcher (lib/src/onnx_graph.dart:2918-2934)."""
    ctx = ctx or default_context()
    model = OnnxModel(path)
    out: dict[str, NBitsWeight] = {}
    for node in model.nodes:
        if node.op_type != "MatMulNBits":
            continue
        ins = node.inputs + [""] * (6 - len(node.inputs))
        if ins[1] not in model.initializers or ins[2] not in model.initializers:
            continue  # runtime weights take the per-call path
        if ins[4]:
            raise UnsupportedError("MatMulNBits: g_idx input not supported")
        at = node.attrs
        k, n = int(at["K"]), int(at["N"])
        bits, bs = int(at.get("bits", 4)), int(at["block_size"])
        nb = -(-k // bs)
        tb = model.initializers[ins[1]]
        if tb.data_type != UINT8:
            raise ArgumentError("MatMulNBits: invalid packed weights or scales")
        b_src = model.source(tb, n * nb * (bs // 2))
        ts = model.initializers[ins[2]]
        if ts.data_type == FLOAT:
            s_src = model.source(ts, n * nb * 4)
        else:  # fp16 scales widen to f32
            s_src = TensorSource.from_array(np.ascontiguousarray(model.read_array(ts, np.float32)))
        zp_kind, z_src = MG_ZP_NONE, None
        if ins[3]:
            tz = model.initializers.get(ins[3])
            if tz is None:
                raise ArgumentError("MatMulNBits: zero_points must be an initializer here")
            if tz.data_type == UINT8:
                zp_kind, z_src = MG_ZP_UINT4, model.source(tz, n * ((nb + 1) // 2))
            else:
                zp_kind = MG_ZP_FLOAT
                z_src = TensorSource.from_array(
                    np.ascontiguousarray(model.read_array(tz, np.float32)))
        bias = None
        if ins[5]:
            tbias = model.initializers.get(ins[5])
            if tbias is None:
                raise ArgumentError("MatMulNBits: bias must be an initializer here")
            bias = model.read_array(tbias, np.float32)
        out[node.outputs[0]] = NBitsWeight.streamed(
            b_src, s_src, z_src, zp_kind=zp_kind, k=k, n=n, bits=bits, block_size=bs,
            bias=bias, chunk_bytes=chunk_bytes, ctx=ctx)
    return out
