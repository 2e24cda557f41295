"""Writes small ONNX models (protobuf wire format) for the load-path tests:
ModelProto.graph (7) -> GraphProto.node (1) / initializer (5); TensorProto
dims (1), data_type (2), name (8), raw_data (9), external_data (13, key 1 /
value 2), data_location (14: 1 = EXTERNAL); NodeProto input (1), output (2),
name (3), op_type (4), attribute (5), domain (7); AttributeProto name (1),
i (3), type (20: 2 = INT)."""
from __future__ import annotations


def varint(x: int) -> bytes:
    x &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = x & 0x7F
        x >>= 7
        if x:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(fno: int, wt: int) -> bytes:
    return varint((fno << 3) | wt)


def ld(fno: int, payload: bytes) -> bytes:
    return key(fno, 2) + varint(len(payload)) + payload


def vi(fno: int, x: int) -> bytes:
    return key(fno, 0) + varint(x)


def tensor(name: str, dims, data_type: int, raw: bytes | None = None,
           external: dict | None = None) -> bytes:
    out = b"".join(vi(1, d) for d in dims) + vi(2, data_type) + ld(8, name.encode())
    if raw is not None:
        out += ld(9, raw)
    if external is not None:
        for k, v in external.items():
            out += ld(13, ld(1, k.encode()) + ld(2, str(v).encode()))
        out += vi(14, 1)
    return out


def attr_int(name: str, v: int) -> bytes:
    return ld(1, name.encode()) + vi(3, v) + vi(20, 2)


def node(op_type: str, inputs, outputs, attrs: dict, name: str = "", domain: str = "") -> bytes:
    out = b"".join(ld(1, i.encode()) for i in inputs)
    out += b"".join(ld(2, o.encode()) for o in outputs)
    if name:
        out += ld(3, name.encode())
    out += ld(4, op_type.encode())
    out += b"".join(ld(5, attr_int(k, v)) for k, v in attrs.items())
    if domain:
        out += ld(7, domain.encode())
    return out


def model(nodes, initializers) -> bytes:
    graph = b"".join(ld(1, n) for n in nodes) + b"".join(ld(5, t) for t in initializers)
    return vi(1, 8) + ld(7, graph)
