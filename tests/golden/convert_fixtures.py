"""Re-encode the reference's ORT-oracle fixtures for the matmul family as JSON.

Provenance: the inputs are `test/fixtures/<name>/{model.onnx,case.json}` of
PieroSoria/onnx_runtime_dart (MIT; expected outputs were produced there by
ONNX Runtime, see tool/gen_fixtures.py:891-925, :713-760, :789-799, the
conv recipes and tool/gen_transformer_fixtures.py:55-63).  Each fixture becomes one JSON file
holding the node's op type, its attributes, every operand in node-input order
(initializers merged with the case's feeds) and the expected outputs.  The
result files are data only; they are what the tests read.

Run (only where the reference checkout exists):
    python tests/golden/convert_fixtures.py /root/reference/test/fixtures

The ONNX files are decoded with a minimal protobuf wire reader written here
(ModelProto.graph -> GraphProto.{node, initializer}; NodeProto.{input, output,
op_type, attribute, domain}; TensorProto.{dims, data_type, raw_data,
float_data, int32_data, int64_data, name}; AttributeProto.{name, f, i, ints,
floats}) so neither `onnx` nor `onnxruntime` is needed.
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

HOT_PATH = [
    "matmulnbits_basic",
    "matmulnbits_zeropoints",
    "matmulnbits_partial_block",
    "matmulnbits_bias_1_False",
    "matmulnbits_bias_1_True",
    "matmulnbits_bias_3_False",
    "matmulnbits_bias_3_True",
    "matmulinteger_u8i8",
    "matmulinteger_nozp",
    "matmulinteger_batched",
    "matmulinteger_percol_bzp",
    "qlinearmatmul",
    "dynamicquantizelinear",
    "matmul_batched",
    "gemm_transB_bias",
    "einsum_matmul",
    "mha_with_bias",
    "mha_no_bias",
    "gqa_causal",
    "gqa_kvcache",
    "gqa_kvcache_bias",
    "gqa_kvcache_rotary",
    "conv1d",
    "conv2d_basic",
    "conv2d_bias",
    "conv2d_depthwise",
    "conv2d_dilation",
    "conv2d_groups",
    "conv2d_pads",
    "conv2d_pads_asym",
    "conv2d_same_lower",
    "conv2d_same_upper",
    "conv2d_strides",
    "conv3d",
    "convinteger",
    "convinteger_1d",
    "convtranspose_1d",
    "convtranspose_basic",
    "convtranspose_bias",
    "convtranspose_groups",
    "convtranspose_outpad",
    "convtranspose_output_shape",
    "convtranspose_pads",
    "convtranspose_stride2",
    "qlinearconv_perchannel_bias",
    "qlinearconv_pertensor",
    # elementwise ops between the products of a decoder layer
    "add_bias_broadcast_lastdim",
    "add_broadcast_middle",
    "skipsimplifiedlayernorm",
]

# Multi-node patterns the reference's graph rewrite fuses into one op
# (lib/src/onnx_graph.dart:466-500, :500-560): stored as the fused op with
# the pattern's feeds, constants and attributes.
FUSED = {
    # Pow(2) -> ReduceMean(ax) -> Add(eps) -> Sqrt -> Reciprocal -> Mul(x) ->
    # Mul(gamma)  =>  _FusedRMSNorm(x, gamma; axis, epsilon)
    "rmsnorm_pattern": "_FusedRMSNorm",
    # Split(axis, 2) -> Sigmoid(b) -> Mul(a, .)  =>  _FusedGlu(x; axis)
    "glu_gate": "_FusedGlu",
}

# ONNX TensorProto.DataType -> (numpy dtype, json dtype name)
_DT = {
    1: (np.float32, "float32"),
    2: (np.uint8, "uint8"),
    3: (np.int8, "int8"),
    6: (np.int32, "int32"),
    7: (np.int64, "int64"),
    10: (np.float16, "float16"),
    11: (np.float64, "float64"),
}


def _varint(buf: bytes, pos: int) -> tuple[int, int]:
    shift = 0
    out = 0
    while True:
        b = buf[pos]
        pos += 1
        out |= (b & 0x7F) << shift
        if b < 0x80:
            return out, pos
        shift += 7


def _fields(buf: bytes):
    """Yield (field_number, wire_type, value) for one protobuf message."""
    pos = 0
    while pos < len(buf):
        key, pos = _varint(buf, pos)
        fno, wt = key >> 3, key & 7
        if wt == 0:
            v, pos = _varint(buf, pos)
        elif wt == 1:
            v = buf[pos:pos + 8]
            pos += 8
        elif wt == 2:
            ln, pos = _varint(buf, pos)
            v = buf[pos:pos + ln]
            pos += ln
        elif wt == 5:
            v = buf[pos:pos + 4]
            pos += 4
        else:
            raise ValueError(f"unsupported wire type {wt}")
        yield fno, wt, v


def _packed_varints(v, wt):
    if wt == 0:
        return [v]
    out, pos = [], 0
    while pos < len(v):
        x, pos = _varint(v, pos)
        out.append(x)
    return out


def _s64(x: int) -> int:
    return x - (1 << 64) if x >= 1 << 63 else x


def parse_tensor(buf: bytes) -> tuple[str, np.ndarray]:
    dims, dt, raw, name = [], 1, None, ""
    floats, i32, i64 = [], [], []
    for fno, wt, v in _fields(buf):
        if fno == 1:
            dims += [_s64(x) for x in _packed_varints(v, wt)]
        elif fno == 2:
            dt = v
        elif fno == 4:
            if wt == 5:
                floats.append(struct.unpack("<f", v)[0])
            else:
                floats += list(struct.unpack(f"<{len(v) // 4}f", v))
        elif fno == 5:
            i32 += [_s64(x) for x in _packed_varints(v, wt)]
        elif fno == 7:
            i64 += [_s64(x) for x in _packed_varints(v, wt)]
        elif fno == 8:
            name = v.decode()
        elif fno == 9:
            raw = v
    npdt = _DT[dt][0]
    if raw is not None:
        arr = np.frombuffer(raw, dtype=np.dtype(npdt).newbyteorder("<")).astype(npdt)
    elif floats:
        arr = np.array(floats, dtype=npdt)
    elif i64:
        arr = np.array(i64, dtype=npdt)
    else:  # int32_data also carries uint8/int8/float16 payloads
        arr = np.array(i32, dtype=np.int64).astype(npdt)
    return name, arr.reshape(dims) if dims else arr.reshape(())


def parse_attribute(buf: bytes):
    name, val = "", None
    ints, floats = [], []
    for fno, wt, v in _fields(buf):
        if fno == 1:
            name = v.decode()
        elif fno == 2:
            val = struct.unpack("<f", v)[0]
        elif fno == 3:
            val = _s64(v)
        elif fno == 7:
            floats += [struct.unpack("<f", v)[0]] if wt == 5 else list(
                struct.unpack(f"<{len(v) // 4}f", v))
        elif fno == 8:
            ints += [_s64(x) for x in _packed_varints(v, wt)]
        elif fno == 4:
            val = v.decode()
    if val is None:
        val = ints if ints else floats
    return name, val


def parse_model(buf: bytes):
    graph = None
    for fno, _, v in _fields(buf):
        if fno == 7:
            graph = v
    nodes, inits = [], {}
    for fno, _, v in _fields(graph):
        if fno == 1:
            node = {"input": [], "output": [], "attrs": {}, "domain": ""}
            for f2, _, v2 in _fields(v):
                if f2 == 1:
                    node["input"].append(v2.decode())
                elif f2 == 2:
                    node["output"].append(v2.decode())
                elif f2 == 4:
                    node["op_type"] = v2.decode()
                elif f2 == 5:
                    k, a = parse_attribute(v2)
                    node["attrs"][k] = a
                elif f2 == 7:
                    node["domain"] = v2.decode()
            nodes.append(node)
        elif fno == 5:
            name, arr = parse_tensor(v)
            inits[name] = arr
    return nodes, inits


def tensor_json(arr: np.ndarray, dtype: str) -> dict:
    flat = arr.ravel()
    if dtype.startswith("float"):
        data = [float(x) if np.isfinite(x) else str(float(x)) for x in flat]
    else:
        data = [int(x) for x in flat]
    return {"dtype": dtype, "shape": list(arr.shape), "data": data}


def convert(src: Path, dst: Path) -> None:
    dst.mkdir(parents=True, exist_ok=True)
    for name in HOT_PATH:
        d = src / name
        nodes, inits = parse_model((d / "model.onnx").read_bytes())
        case = json.loads((d / "case.json").read_text())
        assert len(nodes) == 1, (name, len(nodes))
        node = nodes[0]
        operands = []
        for inp in node["input"]:
            if inp == "":
                operands.append(None)
            elif inp in inits:
                arr = inits[inp]
                dtname = {np.dtype(t): n for t, n in _DT.values()}[arr.dtype]
                operands.append({"name": inp, "initializer": True,
                                 **tensor_json(arr, dtname)})
            else:
                feed = case["inputs"][inp]
                operands.append({"name": inp, "initializer": False, **feed})
        out = {
            "name": name,
            "source": f"test/fixtures/{name}",
            "op_type": node["op_type"],
            "domain": node["domain"],
            "attrs": node["attrs"],
            "inputs": operands,
            "outputs": node["output"],
            "expected": case["expected"],
        }
        (dst / f"{name}.json").write_text(json.dumps(out, separators=(",", ":")))
        print(name, node["op_type"], node["attrs"],
              [(o["name"], o["dtype"], o["shape"]) if o else None for o in operands])


def convert_fused(src: Path, dst: Path) -> None:
    for name, fused in FUSED.items():
        d = src / name
        nodes, inits = parse_model((d / "model.onnx").read_bytes())
        case = json.loads((d / "case.json").read_text())
        by_op = {n["op_type"]: n for n in nodes}

        def feed(nm):
            return {"name": nm, "initializer": False, **case["inputs"][nm]}

        def init(nm):
            arr = inits[nm]
            dtname = {np.dtype(t): n for t, n in _DT.values()}[arr.dtype]
            return {"name": nm, "initializer": True, **tensor_json(arr, dtname)}

        if fused == "_FusedRMSNorm":
            x = by_op["Pow"]["input"][0]
            gamma = [i for i in nodes[-1]["input"] if i in inits][0]
            eps = [i for i in by_op["Add"]["input"] if i in inits][0]
            axis = int(inits[by_op["ReduceMean"]["input"][1]].ravel()[0])
            operands = [feed(x), init(gamma)]
            attrs = {"axis": axis, "epsilon": float(inits[eps].ravel()[0])}
        else:
            split = by_op["Split"]
            operands = [feed(split["input"][0])]
            attrs = {"axis": int(split["attrs"]["axis"])}
        out = {
            "name": name,
            "source": f"test/fixtures/{name}",
            "op_type": fused,
            "domain": "",
            "attrs": attrs,
            "inputs": operands,
            "outputs": [nodes[-1]["output"][0]],
            "expected": case["expected"],
        }
        (dst / f"{name}.json").write_text(json.dumps(out, separators=(",", ":")))
        print(name, fused, attrs, [(o["name"], o["dtype"], o["shape"]) for o in operands])


if __name__ == "__main__":
    src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/test/fixtures")
    convert(src, Path(__file__).resolve().parent / "fixtures")
    convert_fused(src, Path(__file__).resolve().parent / "fixtures")
