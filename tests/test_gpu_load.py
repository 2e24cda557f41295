"""The int4 load path on the GPU: MatMulNBits weights streamed from host
arrays or file ranges (ONNX external data) and repacked on the device give
the oracle's results, the same results for any chunking, and the ONNX loader
builds them from a model file with external data."""
import numpy as np
import pytest

import golden_io as G
import onnx_writer as W
import oracle

pytestmark = pytest.mark.gpu
# The MatMulNBits bar: max|gpu - ref| <= 1e-3 * rms(ref).  A repacking mistake
# gives errors of order one; the 64-row launches run the fp6 prefill GEMM
# (three e2m3 activation digits, ~1.5e-4 at these shapes).
TOL = 1e-3


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


def _weight(rng, k, n, bs, zp_mode):
    nb = -(-k // bs)
    b = rng.integers(0, 256, (n, nb, bs // 2)).astype(np.uint8)
    s = rng.uniform(0.005, 0.02, (n, nb)).astype(np.float32)
    if zp_mode == "u4":
        zp = rng.integers(0, 256, (n, (nb + 1) // 2)).astype(np.uint8)
    elif zp_mode == "f32":
        zp = rng.uniform(0, 15, (n, nb)).astype(np.float32)
    else:
        zp = None
    return b, s, zp


def _kind(ops, zp):
    return ops.MG_ZP_NONE if zp is None else (ops.MG_ZP_UINT4 if zp.dtype == np.uint8
                                              else ops.MG_ZP_FLOAT)


CASES = [
    # k, n, bs, zp mode
    (1024, 3072, 32, "u4"),     # the single-op config
    (1000, 777, 128, "u4"),     # ragged k and n, odd block count
    (2048, 512, 64, "f32"),
    (256, 130, 16, None),
]


@pytest.mark.parametrize("k,n,bs,zpm", CASES)
def test_streamed_from_file_matches_oracle_for_any_chunking(ops, tmp_path, k, n, bs, zpm):
    rng = np.random.default_rng(k + n + bs)
    b, s, zp = _weight(rng, k, n, bs, zpm)
    bias = rng.standard_normal(n).astype(np.float32)
    # the three tensors back to back in one file, at unaligned offsets
    blob = bytearray(b"\x07" * 13)
    offs = []
    for t in (b, s, zp):
        offs.append(len(blob))
        if t is not None:
            blob += t.tobytes()
            blob += b"\x00" * 3
    path = tmp_path / "w.bin"
    path.write_bytes(bytes(blob))
    src = [ops.TensorSource.from_file(path, o, 0) for o in offs]
    a1 = rng.standard_normal((1, k)).astype(np.float32)
    a64 = rng.standard_normal((64, k)).astype(np.float32)
    ref1 = oracle.matmul_nbits(a1, b, s, zp, k=k, n=n, block_size=bs, bias=bias)
    ref64 = oracle.matmul_nbits(a64, b, s, zp, k=k, n=n, block_size=bs, bias=bias)
    outs = []
    # chunks of one column group, of three, and the default (one chunk)
    for chunk in (1, 3 * 64 * (b[0].nbytes + s[0].nbytes), 0):
        w = ops.NBitsWeight.streamed(src[0], src[1], src[2] if zp is not None else None,
                                     zp_kind=_kind(ops, zp), k=k, n=n, block_size=bs,
                                     bias=bias, chunk_bytes=chunk)
        y1, y64 = w(a1), w(a64)
        w.release()
        assert G.rms_error(y1, ref1) <= TOL and G.rms_error(y64, ref64) <= TOL
        outs.append((y1, y64))
    for y1, y64 in outs[1:]:
        np.testing.assert_array_equal(y1, outs[0][0])
        np.testing.assert_array_equal(y64, outs[0][1])
    # host-array sources and the shape-checked create give the same bits
    hw = ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=bs, bias=bias)
    np.testing.assert_array_equal(hw(a64), outs[0][1])
    hs = ops.NBitsWeight.streamed(ops.TensorSource.from_array(b), ops.TensorSource.from_array(s),
                                  ops.TensorSource.from_array(zp) if zp is not None else None,
                                  zp_kind=_kind(ops, zp), k=k, n=n, block_size=bs, bias=bias,
                                  chunk_bytes=1)
    np.testing.assert_array_equal(hs(a1), outs[0][0])
    hw.release()
    hs.release()


def test_onnx_loader_end_to_end(ops, tmp_path):
    from onnx_runtime_dart_amd import onnx_model
    rng = np.random.default_rng(12)
    specs = [("q", 1024, 2048, 128), ("lm_head", 1024, 3000, 32)]
    blob, inits, nodes, want = bytearray(), [], [], {}
    for name, k, n, bs in specs:
        b, s, zp = _weight(rng, k, n, bs, "u4")
        s16 = s.astype(np.float16)  # fp16 scales, widened on load
        for tname, t, dt in ((f"{name}.B", b, 2), (f"{name}.S", s16, 10), (f"{name}.Z", zp, 2)):
            off = len(blob)
            blob += t.tobytes()
            inits.append(W.tensor(tname, t.shape, dt,
                                  external={"location": "model.data", "offset": off,
                                            "length": t.nbytes}))
        nodes.append(W.node("MatMulNBits", ["x", f"{name}.B", f"{name}.S", f"{name}.Z"],
                            [f"{name}.out"], {"K": k, "N": n, "bits": 4, "block_size": bs},
                            domain="com.microsoft"))
        want[f"{name}.out"] = (b, s16.astype(np.float32), zp, k, n, bs)
    (tmp_path / "model.data").write_bytes(bytes(blob))
    (tmp_path / "model.onnx").write_bytes(W.model(nodes, inits))
    weights = onnx_model.load_matmul_nbits(tmp_path / "model.onnx", chunk_bytes=1 << 20)
    assert set(weights) == set(want)
    for out, (b, s, zp, k, n, bs) in want.items():
        a = rng.standard_normal((3, k)).astype(np.float32)
        ref = oracle.matmul_nbits(a, b, s, zp, k=k, n=n, block_size=bs)
        assert G.rms_error(weights[out](a), ref) <= TOL
        weights[out].release()


def test_streamed_errors(ops, tmp_path):
    from onnx_runtime_dart_amd.errors import ArgumentError, UnsupportedError
    b = np.zeros((8, 2, 16), np.uint8)
    s = np.ones((8, 2), np.float32)
    with pytest.raises(ArgumentError):  # missing file
        ops.NBitsWeight.streamed(ops.TensorSource.from_file(tmp_path / "nope.bin"),
                                 ops.TensorSource.from_array(s), k=64, n=8, block_size=32)
    (tmp_path / "short.bin").write_bytes(b.tobytes()[:100])
    with pytest.raises(ArgumentError):  # file shorter than the tensor
        ops.NBitsWeight.streamed(ops.TensorSource.from_file(tmp_path / "short.bin"),
                                 ops.TensorSource.from_array(s), k=64, n=8, block_size=32)
    with pytest.raises(ArgumentError):  # stated length below the shape's bytes
        ops.NBitsWeight.streamed(ops.TensorSource.from_file(tmp_path / "short.bin", 0, 100),
                                 ops.TensorSource.from_array(s), k=64, n=8, block_size=32)
    with pytest.raises(UnsupportedError):
        ops.NBitsWeight.streamed(ops.TensorSource.from_array(b), ops.TensorSource.from_array(s),
                                 k=64, n=8, bits=8, block_size=32)
