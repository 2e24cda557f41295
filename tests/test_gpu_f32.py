"""fp32 MatMul / Gemm on the GPU against the oracle and the reference's
fixtures.  Bar: max|gpu - ref| <= 1e-3 * rms(ref); the reference's own fixture
rule (2e-5 relative to max |ref|) is also checked on its fixtures."""
import numpy as np
import pytest

import golden_io as G
import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


@pytest.mark.parametrize("name", ["matmul_batched", "gemm_transB_bias", "einsum_matmul"])
def test_fixture(ops, name):
    d = G.load(name)
    x, at = d["arrays"], d["attrs"]
    if d["op_type"] == "Gemm":
        y = ops.op_gemm(x[0], x[1], x[2] if len(x) > 2 else None, alpha=at.get("alpha", 1.0),
                        beta=at.get("beta", 1.0), trans_a=bool(at.get("transA", 0)),
                        trans_b=bool(at.get("transB", 0)))
    else:
        y = ops.op_matmul(x[0], x[1])
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], name)


def test_known_answers(ops):
    w = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    c = np.array([10, 20, 30, 40], dtype=np.float32)
    x = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    want = [24, 52, 80, 108, 42, 97, 152, 207]  # test/gemm_prepack_test.dart:48
    assert ops.op_gemm(x, w, c, trans_b=True).ravel().tolist() == want
    fw = ops.F32Weight(w, trans_b=True)  # prepacked once, stable on reuse
    assert fw.gemm(x, c).ravel().tolist() == want
    assert fw.gemm(x, c).ravel().tolist() == want
    fw.release()
    xi = np.array([[5, 6], [7, 8]], dtype=np.float32)  # onnx_runtime_dart_test.dart:48-70
    assert ops.op_matmul(xi, np.eye(2, dtype=np.float32)).ravel().tolist() == [5, 6, 7, 8]


@pytest.mark.parametrize("m,k,n", [(1, 384, 384), (33, 65, 17), (7, 128, 5), (128, 64, 128),
                                   (5, 1, 9), (64, 384, 1), (1, 40, 151), (1, 896, 512),
                                   (300, 200, 100)])
def test_kernel_shapes(ops, m, k, n):
    # Shape list of test/gemm_kernel_test.dart:62-80.
    rng = np.random.default_rng(11)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    y = ops.op_matmul(a, b)
    assert G.rms_error(y, oracle.matmul_f32(a, b)) <= TOL
    assert np.abs(y - a.astype(np.float64) @ b).max() < 1e-3


@pytest.mark.parametrize("sa,sb", [((2, 3, 5, 7), (2, 3, 7, 4)), ((3, 1, 4, 6), (2, 6, 5)),
                                   ((4, 2, 8), (8, 3)), ((2, 8), (5, 8, 3)),
                                   ((1, 3, 2), (4, 1, 2, 5))])
def test_broadcast(ops, sa, sb):
    rng = np.random.default_rng(5)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    y = ops.op_matmul(a, b)
    ref = oracle.matmul_f32(a, b)
    assert y.shape == ref.shape
    assert G.rms_error(y, ref) <= TOL


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("c_shape", [None, (7,), (1, 7), (5, 1), (5, 7), ()])
def test_gemm_attributes(ops, ta, tb, c_shape):
    rng = np.random.default_rng(6)
    a = rng.standard_normal((6, 5) if ta else (5, 6)).astype(np.float32)
    b = rng.standard_normal((7, 6) if tb else (6, 7)).astype(np.float32)
    c = None if c_shape is None else rng.standard_normal(c_shape).astype(np.float32)
    y = ops.op_gemm(a, b, c, alpha=0.5, beta=2.0, trans_a=ta, trans_b=tb)
    ref = oracle.gemm_f32(a, b, c, alpha=0.5, beta=2.0, trans_a=ta, trans_b=tb)
    assert G.rms_error(y, ref) <= TOL


# Config C3 (MiniLM-L6, batch 32 x seq 128 = 4096 token rows, hidden 384,
# 12 heads x 32, FFN 1536) at the size the bench times.  Every output row is
# checked against a float64 product; row blocks at the start, across the
# XCD band boundaries and at the end are checked against the oracle.
C3_ROWS = 4096
C3_ORACLE_ROWS = np.concatenate([np.arange(0, 256), np.arange(1984, 2240),
                                 np.arange(C3_ROWS - 256, C3_ROWS)])


@pytest.mark.parametrize("name,n,k", [("q", 384, 384), ("k", 384, 384), ("v", 384, 384),
                                      ("out", 384, 384), ("ffn1", 1536, 384),
                                      ("ffn2", 384, 1536)])
def test_c3_gemm_full_size(ops, name, n, k):
    rng = np.random.default_rng(0x5EED0002 + n + k)
    x = rng.standard_normal((C3_ROWS, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    c = (rng.standard_normal(n) * 0.02).astype(np.float32)
    fw = ops.F32Weight(w, trans_b=True)
    y = fw.gemm(x, c)
    fw.release()
    full = x.astype(np.float64) @ w.T.astype(np.float64) + c
    assert G.rms_error(y, full) <= TOL
    rows = C3_ORACLE_ROWS
    ref = oracle.gemm_f32(x[rows], w, c, trans_b=True)
    assert G.rms_error(y[rows], ref) <= TOL


def test_c3_attention_matmuls_full_size(ops):
    # The unfused attention products over all 32 x 12 heads.
    rng = np.random.default_rng(0x5EED0002)
    q = rng.standard_normal((32, 12, 128, 32)).astype(np.float32)
    kt = rng.standard_normal((32, 12, 32, 128)).astype(np.float32)
    s = ops.op_matmul(q, kt)
    assert G.rms_error(s, oracle.matmul_f32(q, kt)) <= TOL
    p = rng.random((32, 12, 128, 128)).astype(np.float32)
    v = rng.standard_normal((32, 12, 128, 32)).astype(np.float32)
    assert G.rms_error(ops.op_matmul(p, v), oracle.matmul_f32(p, v)) <= TOL


@pytest.mark.parametrize("sa,sb", [((2, 3, 5, 7), (2, 3, 7, 4)),
                                   ((2, 1, 40, 24), (3, 24, 36)),
                                   ((1, 4, 3), (6, 3, 5)),
                                   ((6, 4, 3), (3, 5)),
                                   ((2, 1, 2, 1, 2, 1, 9, 8), (1, 2, 1, 2, 1, 2, 8, 12)),
                                   ((32, 12, 128, 32), (32, 12, 32, 128))])
def test_matmul_dev_broadcast_matches_host_entry(ops, sa, sb):
    # mg_matmul_f32_dev with broadcast batch dims (offsets decoded in the
    # kernel; more than four merged dims loop over launches) gives bitwise
    # the host entry point's result, twice in a row on the same buffers.
    rng = np.random.default_rng(31)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    want = ops.op_matmul(a, b)
    ad, bd = ops.DeviceBuffer.from_array(a), ops.DeviceBuffer.from_array(b)
    yd = ops.DeviceBuffer(want.nbytes)
    for _ in range(2):
        ops.matmul_f32_dev(ad.ptr, sa, bd.ptr, sb, yd.ptr)
        got = yd.to_array(want.shape, np.float32)
        np.testing.assert_array_equal(got, want)
    assert G.rms_error(want, oracle.matmul_f32(a, b)) <= TOL
    for buf in (ad, bd, yd):
        buf.free()


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_layouts_multi_tile(ops, ta, tb):
    # Every operand layout through several tiles and k stages, with ragged
    # edges in M, N and K (partial tiles and a partial last stage).
    rng = np.random.default_rng(12)
    m, k, n = 257, 129, 383
    a = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    c = rng.standard_normal(n).astype(np.float32)
    y = ops.op_gemm(a, b, c, alpha=1.5, beta=0.5, trans_a=ta, trans_b=tb)
    ref = oracle.gemm_f32(a, b, c, alpha=1.5, beta=0.5, trans_a=ta, trans_b=tb)
    assert G.rms_error(y, ref) <= TOL


@pytest.mark.parametrize("k", [40, 256])
def test_large_tile_path(ops, k):
    # Enough 128 x 128 tiles to take the large-tile kernel; N not a multiple
    # of the tile; a weight uploaded without transB (transposed on upload).
    rng = np.random.default_rng(13)
    m, n = 2176, 4160
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((k, n)).astype(np.float32)
    fw = ops.F32Weight(w, trans_b=False)
    y = fw.gemm(a)
    fw.release()
    rows = np.concatenate([np.arange(64), np.arange(m - 64, m)])
    ref = oracle.matmul_f32(a[rows], w)
    assert G.rms_error(y[rows], ref) <= TOL


@pytest.mark.parametrize("sa,sb,kinds", [
    ((3, 7), (7, 5), ("i64", "i64")),
    ((2, 3, 40, 129), (2, 3, 129, 65), ("i64", "i64")),   # batched, ragged
    ((2, 1, 4, 300), (3, 300, 17), ("u8", "i8")),         # broadcast batch dims
    ((5, 64), (64, 33), ("f32", "i64")),                  # float x integer
    ((70000, 2), (2, 3), ("i32", "f32")),                 # many rows
])
def test_matmul_non_float_operands_bitwise(ops, sa, sb, kinds):
    # opMatMul's double fallback (lib/src/onnx_ops.dart:1753-1762): a double
    # sum of getD products in k order, one rounding to f32.  Bitwise against
    # the oracle, with operands large enough that the products and sums
    # round in double.
    rng = np.random.default_rng(0x5EED00B0 + len(sa) + sa[-1])

    def make(shape, kind):
        if kind == "i64":
            return rng.integers(-2**52, 2**52, shape, dtype=np.int64)
        if kind == "i32":
            return rng.integers(-2**31, 2**31, shape, dtype=np.int64).astype(np.int32)
        if kind == "u8":
            return rng.integers(0, 256, shape, dtype=np.uint8)
        if kind == "i8":
            return rng.integers(-128, 128, shape, dtype=np.int8)
        return (rng.standard_normal(shape) * 1e6).astype(np.float32)

    a, b = make(sa, kinds[0]), make(sb, kinds[1])
    y = ops.op_matmul(a, b)
    ref = oracle.matmul_f64acc(a, b)
    assert y.dtype == np.float32 and y.shape == ref.shape
    np.testing.assert_array_equal(y, ref)


def test_matmul_non_float_cancellations(ops):
    # The closed-form cells of the oracle's pin: no fused multiply-add
    # (y[0,0] = 0, not 1) and k order (y[1,1] = 0, not 1).
    t40, t60 = 2**40, 2**60
    a = np.array([[-t40, t40 + 1, 0], [1, t60, -t60]], np.int64)
    b = np.array([[t40 + 2, 1], [t40 + 1, 1], [1, 1]], np.int64)
    y = ops.op_matmul(a, b)
    assert y[0, 0] == 0.0 and y[1, 1] == 0.0
    np.testing.assert_array_equal(y, oracle.matmul_f64acc(a, b))


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_buffer_stage_layouts_ragged_tiles(ops, ta, tb):
    # Rows 16-byte aligned and K, M, N multiples of 4: the stages load through
    # raw buffer loads in both operand layouts (k-contiguous and transposed),
    # with quads past M, N and K read as zeros and the stores past M and N
    # dropped; checked against the oracle, with a bias row and alpha / beta.
    rng = np.random.default_rng(0x5EED0090 + 2 * ta + tb)
    m, k, n = 132, 68, 100
    a = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    c = rng.standard_normal((n,)).astype(np.float32)
    y = ops.op_gemm(a, b, c, alpha=0.75, beta=1.5, trans_a=ta, trans_b=tb)
    ref = oracle.gemm_f32(a, b, c, alpha=0.75, beta=1.5, trans_a=ta, trans_b=tb)
    assert G.rms_error(y, ref) <= TOL


@pytest.mark.parametrize("m,k,n,c_shape", [(100, 1100, 70, (70,)), (300, 1536, 384, (300, 384)),
                                           (8200, 1024, 40, None)])
def test_weight_gemm_k_split(ops, m, k, n, c_shape):
    # Weight Gemms with K >= 1024 and M <= 8192 split K over two workgroup
    # sets and add the partials in a second launch (alpha, then beta C, as
    # the one-launch epilogue); M = 8200 stays in one launch.  Ragged M, N
    # and a K that ends inside a stage, against the oracle.
    rng = np.random.default_rng(0x5EED0095 + m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    c = None if c_shape is None else rng.standard_normal(c_shape).astype(np.float32)
    fw = ops.F32Weight(w, trans_b=True)
    y = fw.gemm(a, c, alpha=0.5, beta=2.0)
    ref = oracle.gemm_f32(a, w, c, alpha=0.5, beta=2.0, trans_a=0, trans_b=1)
    assert G.rms_error(y, ref) <= TOL
    fw.release()


def test_weight_gemm_k_split_column_chunks_and_slices(ops):
    # rows = 4096, K = 1100, N = 2200: the two partials of the whole weight
    # exceed 64 MiB, so it runs in column chunks (2048 + 152), while a weight
    # of its last 152 columns alone takes another tile plan (stages of 32 k
    # instead of 16).  The split falls on the same k either way, so those
    # columns are bitwise equal; a row subset is checked against the oracle.
    rng = np.random.default_rng(0x5EED0096)
    m, k, n = 4096, 1100, 2200
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    c = rng.standard_normal((n,)).astype(np.float32)
    fw = ops.F32Weight(w, trans_b=True)
    y = fw.gemm(a, c)
    fw.release()
    fs = ops.F32Weight(np.ascontiguousarray(w[2048:]), trans_b=True)
    ys = fs.gemm(a, c[2048:])
    fs.release()
    np.testing.assert_array_equal(y[:, 2048:], ys)
    rows = np.arange(0, m, 97)
    ref = oracle.gemm_f32(a[rows], w, c, alpha=1.0, beta=1.0, trans_a=0, trans_b=1)
    assert G.rms_error(y[rows], ref) <= TOL
