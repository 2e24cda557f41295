"""MatMulInteger / QLinearMatMul / DynamicQuantizeLinear on the GPU: bit-exact
against the oracle, the reference's fixtures and its known answers."""
import numpy as np
import pytest

import golden_io as G
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


@pytest.mark.parametrize("name", G.names("matmulinteger") + ["qlinearmatmul",
                                                              "dynamicquantizelinear"])
def test_fixture(ops, name):
    d = G.load(name)
    x = d["arrays"]
    if d["op_type"] == "MatMulInteger":
        y = ops.op_matmul_integer(x[0], x[1], x[2] if len(x) > 2 else None,
                                  x[3] if len(x) > 3 else None)
        G.assert_reference_parity(y, d["want"][d["outputs"][0]], name)
    elif d["op_type"] == "QLinearMatMul":
        a, as_, az, b, bs, bz, ys, yz = x
        lo, hi = (-128, 127) if yz is not None and yz.dtype == np.int8 else (0, 255)
        y = ops.op_qlinear_matmul(a, as_, az, b, bs, bz, ys, yz, lo=lo, hi=hi)
        G.assert_reference_parity(y, d["want"][d["outputs"][0]], name)
    else:
        y, s, z = ops.op_dynamic_quantize_linear(x[0])
        o = d["outputs"]
        G.assert_reference_parity(y.astype(np.int64), d["want"][o[0]], name)
        G.assert_reference_parity(np.array(s, np.float32), d["want"][o[1]], name)
        assert z == int(d["want"][o[2]])


def test_known_answer(ops):
    # test/compact_tensor_test.dart:48-57
    a = np.array([[10, 130, 250]], dtype=np.uint8)
    b = np.array([[-1, 2], [3, -4], [5, 6]], dtype=np.int8)
    assert ops.op_matmul_integer(a, b, np.array(10), np.array(1)).ravel().tolist() == [1200, 600]


SHAPES = [(1, 1, 1), (4, 6, 5), (17, 65, 33), (64, 128, 64), (33, 200, 47), (128, 1024, 1024)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("signs", [(False, True), (False, False), (True, True), (True, False)])
@pytest.mark.parametrize("zp_mode", ["none", "scalar", "vector"])
def test_matmul_integer_exact(ops, m, k, n, signs, zp_mode):
    rng = np.random.default_rng(m * 131 + k * 7 + n)
    sa, sb = signs
    a = rng.integers(-128 if sa else 0, 128 if sa else 256, (m, k)).astype(np.int8 if sa else np.uint8)
    b = rng.integers(-128 if sb else 0, 128 if sb else 256, (k, n)).astype(np.int8 if sb else np.uint8)
    if zp_mode == "none":
        az = bz = None
    elif zp_mode == "scalar":
        az, bz = np.array(rng.integers(0, 200)), np.array(rng.integers(-20, 20))
    else:
        az = rng.integers(0, 255, m) if m > 1 else np.array(rng.integers(0, 255))
        bz = rng.integers(-100, 100, n) if n > 1 else np.array(3)
    y = ops.op_matmul_integer(a, b, az, bz)
    np.testing.assert_array_equal(y, oracle.matmul_integer(a, b, az, bz))
    w = ops.Int8Weight(b, bz)
    np.testing.assert_array_equal(w.matmul_integer(a, az), oracle.matmul_integer(a, b, az, bz))
    w.release()


@pytest.mark.parametrize("ab,bb", [(3, 3), (3, 1), (1, 2)])
def test_matmul_integer_batched(ops, ab, bb):
    rng = np.random.default_rng(ab * 10 + bb)
    a = rng.integers(0, 256, (ab, 9, 70)).astype(np.uint8)
    b = rng.integers(-128, 128, (bb, 70, 21)).astype(np.int8)
    az = rng.integers(0, 255, 9)
    y = ops.op_matmul_integer(a, b, az, np.array(-3))
    np.testing.assert_array_equal(y, oracle.matmul_integer(a, b, az, np.array(-3)))


# Plans that split K over workgroups run k_i8_gemm_kw (32-row tiles whose
# waves split K) when it has at least as many workgroups with work: M = 512
# at the Qwen projection shapes, a ragged N, k steps that do not fill the
# last ring block of a wave (K = 2304: 18 steps per wave), and batches.
KW_CASES = [(512, 1024, 2048, "scalar"), (512, 3072, 600, "vector"),
            (96, 2304, 300, "vector"), (512, 2048, 1024, "none")]


@pytest.mark.parametrize("m,k,n,zp_mode", KW_CASES)
def test_wave_split_plans_exact(ops, m, k, n, zp_mode):
    rng = np.random.default_rng(0x5EED0093 + m + k + n)
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    if zp_mode == "none":
        az = bz = None
    elif zp_mode == "scalar":
        az, bz = np.array(131), np.array(-7)
    else:
        az, bz = rng.integers(0, 255, m), rng.integers(-100, 100, n)
    ref = oracle.matmul_integer(a, b, az, bz)
    np.testing.assert_array_equal(ops.op_matmul_integer(a, b, az, bz), ref)
    w = ops.Int8Weight(b, bz)
    np.testing.assert_array_equal(w.matmul_integer(a, az), ref)
    w.release()


def test_wave_split_requant_and_batches(ops):
    rng = np.random.default_rng(0x5EED0094)
    a = rng.integers(0, 256, (512, 1024)).astype(np.uint8)
    b = rng.integers(-127, 128, (1024, 512)).astype(np.int8)
    args = (a, np.float32(0.0123), np.array(118), b, np.float32(2 ** -10), np.array(0),
            np.float32(0.05), np.array(128))
    np.testing.assert_array_equal(ops.op_qlinear_matmul(*args, lo=0, hi=255),
                                  oracle.qlinear_matmul(*args, lo=0, hi=255))
    for bb in (2, 1):
        a3 = rng.integers(0, 256, (2, 96, 1024)).astype(np.uint8)
        b3 = rng.integers(-128, 128, (bb, 1024, 200)).astype(np.int8)
        az = rng.integers(0, 255, 96)
        np.testing.assert_array_equal(ops.op_matmul_integer(a3, b3, az, np.array(5)),
                                      oracle.matmul_integer(a3, b3, az, np.array(5)))


@pytest.mark.parametrize("signed_out", [False, True])
@pytest.mark.parametrize("y_scale", [0.05, 0.5, 8.0])
def test_qlinear_exact(ops, signed_out, y_scale):
    rng = np.random.default_rng(11)
    a = rng.integers(0, 256, (37, 300)).astype(np.uint8)
    b = rng.integers(-127, 128, (300, 45)).astype(np.int8)
    lo, hi = (-128, 127) if signed_out else (0, 255)
    yz = 5 if signed_out else 128
    args = (a, np.float32(0.0123), np.array(118), b, np.float32(2 ** -10), np.array(0),
            np.float32(y_scale), np.array(yz))
    y = ops.op_qlinear_matmul(*args, lo=lo, hi=hi)
    ref = oracle.qlinear_matmul(*args, lo=lo, hi=hi)
    np.testing.assert_array_equal(y, ref)
    w = ops.Int8Weight(b, np.array(0))
    y2 = w.qlinear_matmul(a, 0.0123, np.array(118), 2 ** -10, y_scale, yz, lo=lo, hi=hi)
    np.testing.assert_array_equal(y2, ref)
    w.release()


def test_config_dql_matmulinteger_qlinear_chain(ops):
    # Config C2: fp32 [128,1024] -> DQL -> MatMulInteger / QLinearMatMul with
    # B int8 [1024,1024] U[-127,127], zp 0; requant scale 0.05, zp 128.
    rng = np.random.default_rng(0x5EED0001)
    x = rng.standard_normal((128, 1024)).astype(np.float32)
    b = rng.integers(-127, 128, (1024, 1024)).astype(np.int8)
    q, s, z = ops.op_dynamic_quantize_linear(x)
    q2, s2, z2 = oracle.dynamic_quantize_linear(x)
    assert s == s2 and z == z2
    np.testing.assert_array_equal(q, q2)
    acc = ops.op_matmul_integer(q, b, np.array(z), np.array(0))
    np.testing.assert_array_equal(acc, oracle.matmul_integer(q2, b, np.array(z2), np.array(0)))
    for b_scale in (2.0 ** -10, 2.0 ** -6):  # unsaturated and saturating
        args = (q, s, np.array(z), b, np.float32(b_scale), np.array(0), np.float32(0.05),
                np.array(128, np.uint8))
        y = ops.op_qlinear_matmul(*args, lo=0, hi=255)
        np.testing.assert_array_equal(y, oracle.qlinear_matmul(*args, lo=0, hi=255))


@pytest.mark.parametrize("shape,shift", [((7,), 0.0), ((128, 1024), 0.0), ((33, 5), -3.0),
                                         ((100000,), 2.0), ((3, 4), 0.5)])
def test_dql_exact(ops, shape, shift):
    rng = np.random.default_rng(17)
    x = (rng.standard_normal(shape) + shift).astype(np.float32)
    y, s, z = ops.op_dynamic_quantize_linear(x)
    y2, s2, z2 = oracle.dynamic_quantize_linear(x)
    assert s == s2 and z == z2
    np.testing.assert_array_equal(y, y2)


def test_dql_edge_cases(ops):
    from onnx_runtime_dart_amd.errors import UnsupportedError
    y, s, z = ops.op_dynamic_quantize_linear(np.zeros(10, np.float32))
    assert s == 0 and z == 0 and not y.any()
    with pytest.raises(UnsupportedError):
        ops.op_dynamic_quantize_linear(np.array([1.0, np.inf], np.float32))


def test_errors(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError, UnsupportedError
    a = np.zeros((4, 3), np.uint8)
    b = np.zeros((3, 2), np.int8)
    with pytest.raises(UnsupportedError):
        ops.op_matmul_integer(a, b, np.zeros(3, np.int32), None)
    with pytest.raises(ArgumentError):
        ops.op_matmul_integer(a, np.zeros((4, 2), np.int8))
    with pytest.raises(ArgumentError):
        ops.op_matmul_integer(np.zeros((2, 4, 3), np.uint8), np.zeros((3, 3, 2), np.int8))


# Rows longer than 33025 k: the reference's int64 accumulator
# (lib/src/onnx_qlinear_ops.dart:55-80) holds sums past int32.  The int64
# entry point cuts K into 32768-k segments summed in int64 on the device.
LONG_K = [
    # (a batch, b batch, M, K, N, extreme): extreme operands push every sum
    # past int32 (255 * -255 per term with these zero points).
    (1, 1, 3, 40000, 70, True),
    (1, 1, 5, 70000, 33, False),   # three segments, the last one short
    (2, 1, 4, 33026, 20, True),    # one k past the int32 bound; batched A
    (2, 2, 2, 65536, 9, False),    # two whole segments; batched B
]


@pytest.mark.parametrize("ab,bb,m,k,n,extreme", LONG_K)
def test_matmul_integer_int64_long_k(ops, ab, bb, m, k, n, extreme):
    rng = np.random.default_rng(0x5EED00A0 + k + n)
    a = rng.integers(0, 256, (ab, m, k), dtype=np.uint8)
    b = rng.integers(-128, 128, (bb, k, n), dtype=np.int8)
    az, bz = np.array(3), rng.integers(-128, 128, n).astype(np.int8)
    if extreme:
        a[...] = 255
        a[0, 0, : k // 3] = 0
        b[...] = -128
        az, bz = np.array(0), np.full(n, 127, np.int8)
    y = ops.op_matmul_integer(a, b, az, bz)
    ref = oracle.matmul_integer(a, b, az, bz)
    assert y.dtype == np.int64
    np.testing.assert_array_equal(y, ref)
    if extreme:
        assert ref.min() < -2**31
    with pytest.raises(Exception, match="int64 form"):
        ops.check(ops.lib.mg_matmul_integer(
            ops.default_context().handle, ops._ptr(a), 0, ops._ptr(ops._shape_arr(a)), a.ndim,
            ops._ptr(b), 1, ops._ptr(ops._shape_arr(b)), b.ndim, None, 0, None, 0,
            ops._ptr(np.empty(ref.shape, np.int32))))


def test_matmul_integer_int64_short_k_equals_int32_form(ops):
    # The int64 entry point at ordinary K (one segment) gives the int32
    # form's values.
    rng = np.random.default_rng(0x5EED00A1)
    a = rng.integers(-128, 128, (3, 37, 1000), dtype=np.int8)
    b = rng.integers(0, 256, (1000, 300), dtype=np.uint8)
    az, bz = rng.integers(-128, 128, 37).astype(np.int8), np.array(7)
    y32 = ops.op_matmul_integer(a, b, az, bz)
    y64 = np.empty(y32.shape, np.int64)
    ops.check(ops.lib.mg_matmul_integer_i64(
        ops.default_context().handle, ops._ptr(a), 1, ops._ptr(ops._shape_arr(a)), a.ndim,
        ops._ptr(b), 0, ops._ptr(ops._shape_arr(b)), b.ndim,
        ops._ptr(np.ascontiguousarray(az.astype(np.int32))), az.size,
        ops._ptr(np.ascontiguousarray(bz.astype(np.int32).ravel())), 1, ops._ptr(y64)))
    np.testing.assert_array_equal(y64, y32)


@pytest.mark.parametrize("signed_out", [False, True])
def test_qlinear_long_k(ops, signed_out):
    # QLinearMatMul requantises the int64 sum: (double)acc * mult rounded to
    # f32, half to even, + y_zp, clamped (:100-106); sums past int32 saturate
    # and the rest round as the reference does.
    rng = np.random.default_rng(0x5EED00A2 + signed_out)
    m, k, n = 6, 50000, 40
    a = rng.integers(0, 256, (m, k), dtype=np.uint8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    a[0] = 255
    b[:, :5] = -128
    bz = np.zeros(n, np.int8)
    bz[:5] = 127  # row 0, columns 0-4: 50000 terms of 255 * -255, below -2^31
    a_s, b_s, y_s = np.float32(0.02), np.float32(2.0**-10), np.float32(0.5)
    az = np.array(0, np.uint8)
    yz = np.array(3 if signed_out else 128, np.int8 if signed_out else np.uint8)
    lo, hi = (-128, 127) if signed_out else (0, 255)
    y = ops.op_qlinear_matmul(a, a_s, az, b, b_s, bz, y_s, yz, lo=lo, hi=hi)
    ref = oracle.qlinear_matmul(a, a_s, az, b, b_s, bz, y_s, yz, lo=lo, hi=hi)
    np.testing.assert_array_equal(y.astype(np.int64), ref)
    assert oracle.matmul_integer(a[:1], b[:, :5], az, bz[:5]).max() < -2**31
    rest = ref[1:, 5:]
    assert ((rest > lo) & (rest < hi)).any()  # not all saturated


# DQL -> MatMulInteger / QLinearMatMul with the scale and zero point left in
# device memory (mg_*_w_dq_dev).  Shapes cover the fused requant epilogue
# (one K split), the split-K reduce, ragged edges and one row.
DQ_SHAPES = [(128, 1024, 1024), (300, 256, 1024), (4, 2048, 256), (17, 65, 33), (1, 1, 1)]


@pytest.mark.parametrize("m,k,n", DQ_SHAPES)
@pytest.mark.parametrize("shift", [0.0, 1.5, -4.0])
def test_dq_dev_chain(ops, m, k, n, shift):
    rng = np.random.default_rng(m * 7 + k * 3 + n + int(shift * 10) + 100)
    x = (rng.standard_normal((m, k)) + shift).astype(np.float32)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    bz = rng.integers(-3, 4, n).astype(np.int32)
    w = ops.Int8Weight(b, bz)
    xd = ops.DeviceBuffer.from_array(x)
    qd = ops.DeviceBuffer(m * k)
    szd = ops.DeviceBuffer.from_array(np.full(4, -1, np.int32))
    y32 = ops.DeviceBuffer(m * n * 4)
    y8 = ops.DeviceBuffer(m * n)
    ops.dynamic_quantize_linear_dev(xd.ptr, m * k, qd.ptr, szd.ptr)
    w.matmul_integer_dq_dev(qd.ptr, m, szd.ptr, y32.ptr)
    q2, s2, z2 = oracle.dynamic_quantize_linear(x)
    sz = szd.to_array(4, np.int32)
    assert sz[:1].view(np.float32)[0] == s2 and sz[1] == z2 and sz[2] == 0
    np.testing.assert_array_equal(qd.to_array((m, k), np.uint8), q2)
    np.testing.assert_array_equal(y32.to_array((m, n), np.int32),
                                  oracle.matmul_integer(q2, b, np.array(z2), bz))
    for b_scale, y_scale, y_zp, lo, hi in ((2.0 ** -10, 0.05, 128, 0, 255),
                                           (2.0 ** -6, 0.05, 128, 0, 255),
                                           (0.003, 0.37, -5, -128, 127)):
        w.qlinear_matmul_dq_dev(qd.ptr, m, szd.ptr, b_scale, y_scale, y_zp, y8.ptr, lo=lo, hi=hi)
        yz = np.array(y_zp, np.int8 if lo < 0 else np.uint8)
        want = oracle.qlinear_matmul(q2, np.float32(s2), np.array(z2), b, np.float32(b_scale),
                                     bz, np.float32(y_scale), yz, lo=lo, hi=hi)
        got = y8.to_array((m, n), np.int8 if lo < 0 else np.uint8)
        np.testing.assert_array_equal(got, want, err_msg=f"b_scale={b_scale} y_zp={y_zp}")
    for buf in (xd, qd, szd, y32, y8):
        buf.free()
    w.release()


def test_dq_dev_degenerate_inputs(ops):
    # All-zero activations: scale 0, zp 0 (lib/src/onnx_ops.dart:3556-3583),
    # so every QLinearMatMul output is y_zp.  Non-finite input sets the flag.
    m, k, n = 8, 64, 40
    b = np.random.default_rng(5).integers(-127, 128, (k, n)).astype(np.int8)
    w = ops.Int8Weight(b, None)
    xd = ops.DeviceBuffer.from_array(np.zeros((m, k), np.float32))
    qd = ops.DeviceBuffer(m * k)
    szd = ops.DeviceBuffer.from_array(np.full(4, -1, np.int32))
    y32 = ops.DeviceBuffer(m * n * 4)
    y8 = ops.DeviceBuffer(m * n)
    ops.dynamic_quantize_linear_dev(xd.ptr, m * k, qd.ptr, szd.ptr)
    w.matmul_integer_dq_dev(qd.ptr, m, szd.ptr, y32.ptr)
    w.qlinear_matmul_dq_dev(qd.ptr, m, szd.ptr, 0.01, 0.05, 77, y8.ptr, lo=0, hi=255)
    assert szd.to_array(4, np.int32)[:3].tolist() == [0, 0, 0]
    assert not y32.to_array((m, n), np.int32).any()
    assert (y8.to_array((m, n), np.uint8) == 77).all()
    x = np.ones((m, k), np.float32)
    x[3, 5] = np.inf
    xi = ops.DeviceBuffer.from_array(x)
    ops.dynamic_quantize_linear_dev(xi.ptr, m * k, qd.ptr, szd.ptr)
    assert szd.to_array(4, np.int32)[2] == 1
    for buf in (xd, xi, qd, szd, y32, y8):
        buf.free()
    w.release()


def test_dq_dev_errors(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError
    w = ops.Int8Weight(np.zeros((4, 4), np.int8), None)
    buf = ops.DeviceBuffer(64)
    with pytest.raises(ArgumentError):
        w.matmul_integer_dq_dev(buf.ptr, 2, 0, buf.ptr)
    with pytest.raises(ArgumentError):
        w.qlinear_matmul_dq_dev(buf.ptr, 2, 0, 1.0, 1.0, 0, buf.ptr, lo=0, hi=255)
    with pytest.raises(ArgumentError):
        w.qlinear_matmul_dq_dev(buf.ptr, 2, buf.ptr, 1.0, 1.0, 0, buf.ptr, lo=0, hi=127)
    buf.free()
    w.release()


# The Qwen3-0.6B projections as MatMulInteger at M = 512 (the shapes the
# bench times, u8 activations with zero point 128, i8 weights with zero point
# 0).  Column subsets (first, across the middle, last) are bit-exact against
# the oracle; over the whole output, exact row and column sums pin every
# element's contribution: sum_n Y[m, n] = (A[m] - zp) . (B 1) and
# sum_m Y[m, n] = (1^T (A - zp)) . B[:, n], computed in int64.
QWEN_I8 = [("q", 1024, 2048), ("k", 1024, 1024), ("o", 2048, 1024), ("gate", 1024, 3072),
           ("down", 3072, 1024), ("lm_head", 1024, 151936)]


def _column_subsets(n):
    mid = n // 2 - 96
    return np.unique(np.concatenate([np.arange(0, min(n, 160)), np.arange(mid, mid + 192),
                                     np.arange(max(0, n - 224), n)]))


@pytest.mark.parametrize("name,k,n", QWEN_I8)
def test_qwen_int8_projection_full_size(ops, name, k, n):
    rng = np.random.default_rng(0x5EED0002 + k + n)
    m = 512
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    w = ops.Int8Weight(b, np.array(0))
    y = w.matmul_integer(a, np.array(128))
    assert y.shape == (m, n)
    cols = _column_subsets(n)
    np.testing.assert_array_equal(y[:, cols], oracle.matmul_integer(a, b[:, cols].copy(),
                                                                    np.array(128), np.array(0)))
    ac = a.astype(np.int64) - 128
    np.testing.assert_array_equal(y.astype(np.int64).sum(axis=1),
                                  ac @ b.astype(np.int64).sum(axis=1))
    np.testing.assert_array_equal(y.astype(np.int64).sum(axis=0),
                                  ac.sum(axis=0) @ b.astype(np.int64))
    # QLinearMatMul through the same packed weight, bit-exact on the subsets.
    rows = np.arange(0, m, 3)
    yq = w.qlinear_matmul(a[rows], 0.0123, np.array(128), 2 ** -10, 0.05, 128, lo=0, hi=255)
    ref = oracle.qlinear_matmul(a[rows], np.float32(0.0123), np.array(128), b[:, cols].copy(),
                                np.float32(2 ** -10), np.array(0), np.float32(0.05),
                                np.array(128), lo=0, hi=255)
    np.testing.assert_array_equal(yq[:, cols], ref)
    w.release()


def test_dev_calls_with_per_row_zero_points_back_to_back(ops):
    # Asynchronous calls whose per-row zero-point tables are host arrays that
    # go away right after each call: the tables travel through the context's
    # pinned staging (16 slots), so 40 calls queued without a wait wrap it
    # and every result still uses its own table.
    rng = np.random.default_rng(41)
    m, k, n, calls = 33, 200, 70, 40
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    w = ops.Int8Weight(b, np.array(-5))
    ad = ops.DeviceBuffer.from_array(a)
    ys = [ops.DeviceBuffer(m * n * 4) for _ in range(calls)]
    zps = [rng.integers(0, 255, m) for _ in range(calls)]
    for i in range(calls):
        w.matmul_integer_dev(ad.ptr, False, m, ys[i].ptr, zps[i].copy())
    for i in range(calls):
        got = ys[i].to_array((m, n), np.int32)
        np.testing.assert_array_equal(got, oracle.matmul_integer(a, b, zps[i], np.array(-5)))
    for buf in ys + [ad]:
        buf.free()
    w.release()
