"""CPU checks of the load path's ONNX reader: initializer metadata, external
data ranges (location / offset / length, length 0 = implied) and zero-copy
views of inline raw_data, on models written by tests/onnx_writer.py."""
import numpy as np
import pytest

import onnx_writer as W


@pytest.fixture()
def onnx_model():
    from onnx_runtime_dart_amd import onnx_model as M
    return M


def _write(tmp_path, k=64, n=5, bs=32, ext_len_zero=False):
    rng = np.random.default_rng(3)
    nb = -(-k // bs)
    b = rng.integers(0, 256, (n, nb, bs // 2)).astype(np.uint8)
    s = rng.uniform(0.01, 0.02, (n, nb)).astype(np.float16)
    zp = rng.integers(0, 256, (n, (nb + 1) // 2)).astype(np.uint8)
    blob = bytearray(b"\x00" * 17)  # leading pad: offsets are not zero
    s_off = len(blob)
    blob += s.tobytes()
    z_off = len(blob)
    blob += zp.tobytes()
    (tmp_path / "weights.bin").write_bytes(bytes(blob))
    inits = [
        W.tensor("B", b.shape, 2, raw=b.tobytes()),
        W.tensor("S", s.shape, 10, external={"location": "weights.bin", "offset": s_off,
                                              "length": 0 if ext_len_zero else s.nbytes}),
        W.tensor("Z", zp.shape, 2, external={"location": "weights.bin", "offset": z_off,
                                              "length": zp.nbytes}),
    ]
    nodes = [W.node("MatMulNBits", ["A", "B", "S", "Z"], ["Y"],
                    {"K": k, "N": n, "bits": 4, "block_size": bs}, name="mm",
                    domain="com.microsoft")]
    path = tmp_path / "model.onnx"
    path.write_bytes(W.model(nodes, inits))
    return path, b, s, zp, s_off, z_off


@pytest.mark.parametrize("ext_len_zero", [False, True])
def test_reader_finds_nodes_and_sources(tmp_path, onnx_model, ext_len_zero):
    path, b, s, zp, s_off, z_off = _write(tmp_path, ext_len_zero=ext_len_zero)
    m = onnx_model.OnnxModel(path)
    assert [n.op_type for n in m.nodes] == ["MatMulNBits"]
    node = m.nodes[0]
    assert node.inputs == ["A", "B", "S", "Z"] and node.outputs == ["Y"]
    assert node.attrs == {"K": 64, "N": 5, "bits": 4, "block_size": 32}
    tb, ts, tz = (m.initializers[x] for x in "BSZ")
    assert tb.dims == list(b.shape) and tb.data_type == 2 and not tb.external
    src = m.source(tb, b.nbytes)
    assert src.host and src.length == b.nbytes
    np.testing.assert_array_equal(np.asarray(src._keep).reshape(b.shape), b)
    src_s = m.source(ts, s.nbytes)
    assert src_s.path.decode() == str(tmp_path / "weights.bin")
    assert src_s.offset == s_off and src_s.length == s.nbytes
    np.testing.assert_array_equal(m.read_array(ts, np.float32), s.astype(np.float32).ravel())
    np.testing.assert_array_equal(m.read_array(tz, np.uint8), zp.ravel())


def test_reader_rejects_short_inline_data(tmp_path, onnx_model):
    from onnx_runtime_dart_amd.errors import ArgumentError
    inits = [W.tensor("B", [5, 2, 16], 2, raw=b"\x01" * 10)]
    path = tmp_path / "short.onnx"
    path.write_bytes(W.model([], inits))
    m = onnx_model.OnnxModel(path)
    with pytest.raises(ArgumentError):
        m.source(m.initializers["B"], 160)
