"""Pins the CPU oracle before anything is compared against it.

Three independent anchors, per op:
  * the reference's ORT golden fixtures (test/fixtures/*, re-encoded under
    tests/golden/fixtures) with the reference's own comparison rule;
  * the reference's known-answer tests (gemm_prepack_test.dart:48,
    compact_tensor_test.dart:48-57, onnx_runtime_dart_test.dart:48-70);
  * closed forms written independently here in numpy (f64 products, integer
    brute force, the f32 rounding chains), on seeded random inputs that hit
    the edge cases the reference handles (partial blocks, odd block counts,
    float zero points, bias, per-row/per-column zero points, batching,
    saturation, m<4 scalar tails).
The convolution family is pinned by its 24 fixtures and by identities that a
wrong index, pad side or weight transpose breaks: a 1x1 conv is a matmul,
a one-hot kernel shifts the input, ConvTranspose is the adjoint of Conv,
and the integer conv equals the float conv of the centred operands.
"""
import numpy as np
import pytest

import golden_io as G
import oracle

# ----------------------------------------------------------------- fixtures


def _run_fixture(d):
    op = d["op_type"]
    x = d["arrays"]
    at = d["attrs"]
    if op == "MatMulNBits":
        a, b, s = x[0], x[1], x[2]
        zp = x[3] if len(x) > 3 else None
        bias = x[5] if len(x) > 5 else None
        return {d["outputs"][0]: oracle.matmul_nbits(
            a, b, s, zp, k=at["K"], n=at["N"], bits=at.get("bits", 4),
            block_size=at["block_size"], bias=bias)}
    if op == "MatMulInteger":
        a, b = x[0], x[1]
        az = x[2] if len(x) > 2 else None
        bz = x[3] if len(x) > 3 else None
        return {d["outputs"][0]: oracle.matmul_integer(a, b, az, bz)}
    if op == "QLinearMatMul":
        a, as_, az, b, bs, bz, ys, yz = x
        signed = yz is not None and yz.dtype == np.int8
        lo, hi = (-128, 127) if signed else (0, 255)
        return {d["outputs"][0]: oracle.qlinear_matmul(
            a, as_, az, b, bs, bz, ys, yz, lo=lo, hi=hi)}
    if op == "DynamicQuantizeLinear":
        y, s, z = oracle.dynamic_quantize_linear(x[0])
        o = d["outputs"]
        return {o[0]: y, o[1]: np.array(s, dtype=np.float32),
                o[2]: np.array(z, dtype=np.int64)}
    if op == "MatMul" or (op == "Einsum" and at["equation"] == "ij,jk->ik"):
        return {d["outputs"][0]: oracle.matmul_f32(x[0], x[1])}
    if op == "Gemm":
        return {d["outputs"][0]: oracle.gemm_f32(
            x[0], x[1], x[2] if len(x) > 2 else None,
            alpha=at.get("alpha", 1.0), beta=at.get("beta", 1.0),
            trans_a=bool(at.get("transA", 0)), trans_b=bool(at.get("transB", 0)))}
    if op == "MultiHeadAttention":
        bias = x[5] if len(x) > 5 else None
        return {d["outputs"][0]: oracle.multi_head_attention(
            x[0], x[1], x[2], bias, num_heads=at["num_heads"], scale=at.get("scale"))}
    if op == "GroupQueryAttention":
        def g(i):
            return x[i] if len(x) > i else None
        outs = oracle.group_query_attention(
            x[0], x[1], x[2], num_heads=at["num_heads"], kv_num_heads=at["kv_num_heads"],
            scale=at.get("scale"), do_rotary=bool(at.get("do_rotary", 0)),
            rotary_interleaved=bool(at.get("rotary_interleaved", 0)), past_key=g(3),
            past_value=g(4), cos_cache=g(7), sin_cache=g(8), attention_bias=g(10))
        return dict(zip(d["outputs"], outs))
    if op == "Add":
        return {d["outputs"][0]: oracle.binary_f32("add", x[0], x[1])}
    if op == "_FusedRMSNorm":
        return {d["outputs"][0]: oracle.rms_norm_f32(x[0], x[1], at["axis"], at["epsilon"])}
    if op == "SkipSimplifiedLayerNormalization":
        s = oracle.binary_f32("add", x[0], x[1])
        return {"out0": oracle.rms_norm_f32(s, x[2], -1, at.get("epsilon", 1e-5)), "out3": s}
    if op == "_FusedGlu":
        a, b = np.split(x[0], 2, axis=at["axis"])
        return {d["outputs"][0]: oracle.binary_f32("mul", a, oracle.sigmoid_f32(b))}
    geo = dict(strides=at.get("strides"), pads=at.get("pads"), dilations=at.get("dilations"),
               group=at.get("group", 1))
    if op == "Conv":
        return {d["outputs"][0]: oracle.conv(x[0], x[1], x[2] if len(x) > 2 else None,
                                             auto_pad=at.get("auto_pad", "NOTSET"), **geo)}
    if op == "ConvTranspose":
        return {d["outputs"][0]: oracle.conv_transpose(
            x[0], x[1], x[2] if len(x) > 2 else None, output_padding=at.get("output_padding"),
            output_shape=at.get("output_shape"), **geo)}
    if op == "ConvInteger":
        return {d["outputs"][0]: oracle.conv_integer(
            x[0], x[1], x[2] if len(x) > 2 else None, x[3] if len(x) > 3 else None, **geo)}
    if op == "QLinearConv":
        yz = x[7] if len(x) > 7 else None
        lo, hi = (-128, 127) if yz is not None and yz.dtype == np.int8 else (0, 255)
        return {d["outputs"][0]: oracle.qlinear_conv(
            *x[:8], x[8] if len(x) > 8 else None, lo=lo, hi=hi, **geo)}
    raise AssertionError(op)


@pytest.mark.parametrize("name", G.names())
def test_oracle_matches_reference_fixture(name):
    d = G.load(name)
    got = _run_fixture(d)
    for out, want in d["want"].items():
        G.assert_reference_parity(got[out], want, f"{name}/{out}")


# ------------------------------------------------------------ known answers


def test_gemm_transb_known_answer():
    # test/gemm_prepack_test.dart:14-57
    w = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    c = np.array([10, 20, 30, 40], dtype=np.float32)
    x = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    y = oracle.gemm_f32(x, w, c, trans_b=True)
    assert y.ravel().tolist() == [24, 52, 80, 108, 42, 97, 152, 207]


def test_matmul_integer_known_answer():
    # test/compact_tensor_test.dart:48-57
    a = np.array([[10, 130, 250]], dtype=np.uint8)
    b = np.array([[-1, 2], [3, -4], [5, 6]], dtype=np.int8)
    y = oracle.matmul_integer(a, b, np.array(10), np.array(1))
    assert y.ravel().tolist() == [1200, 600]


def test_matmul_identity_known_answer():
    # test/onnx_runtime_dart_test.dart:48-70
    x = np.array([[5, 6], [7, 8]], dtype=np.float32)
    y = oracle.matmul_f32(x, np.eye(2, dtype=np.float32))
    assert y.ravel().tolist() == [5, 6, 7, 8]


def test_round_even_ties():
    assert [oracle.round_even(v) for v in (0.5, 1.5, 2.5, -0.5, -1.5, 2.4, 2.6)] \
        == [0, 2, 2, 0, -2, 2, 3]
    with pytest.raises(oracle.OracleError):
        oracle.round_even(float("nan"))


# --------------------------------------------------------------- fp32 GEMM


def _seq_f32(a, b):
    """Sequential k-order f32 mul-then-add per element (the Float32x4 lane
    arithmetic), vectorised over outputs with numpy float32."""
    m, k = a.shape
    out = np.zeros((m, b.shape[1]), dtype=np.float32)
    for kk in range(k):
        prod = (a[:, kk:kk + 1] * b[kk:kk + 1, :]).astype(np.float32)
        out = (out + prod).astype(np.float32)
    return out


@pytest.mark.parametrize("m,k,n", [(1, 384, 384), (33, 65, 17), (7, 128, 5),
                                   (128, 64, 128), (5, 1, 9), (64, 384, 1),
                                   (1, 40, 151), (1, 128, 19), (1, 896, 512),
                                   (3, 50, 7), (2, 9, 4)])
def test_kernel_matches_naive_and_rounding_chain(m, k, n):
    # Shape list of test/gemm_kernel_test.dart:62-80 (+ m<4 tails).
    rng = np.random.default_rng(11)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    y = oracle.matmul_kernel(a, b)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(y - ref).max() < 1e-4
    # Bitwise: f32 lanes are sequential mul-then-add; m<4 tail columns are
    # double sums rounded once.
    seq = _seq_f32(a, b)
    f32_cols = n if m >= 4 else n & ~3
    np.testing.assert_array_equal(y[:, :f32_cols], seq[:, :f32_cols])
    np.testing.assert_array_equal(y[:, f32_cols:], ref[:, f32_cols:].astype(np.float32))


def test_kernel_exhaustive_small():
    # test/gemm_kernel_test.dart:45-60
    rng = np.random.default_rng(3)
    for m in range(1, 7):
        for k in range(1, 7):
            for n in range(1, 7):
                a = rng.standard_normal((m, k)).astype(np.float32)
                b = rng.standard_normal((k, n)).astype(np.float32)
                y = oracle.matmul_kernel(a, b)
                assert np.abs(y - a.astype(np.float64) @ b).max() < 1e-5


def test_matmul_broadcast_batches():
    rng = np.random.default_rng(5)
    for sa, sb in [((2, 3, 5, 7), (2, 3, 7, 4)), ((3, 1, 4, 6), (2, 6, 5)),
                   ((4, 2, 8), (8, 3)), ((2, 8), (5, 8, 3)), ((1, 3, 2), (4, 1, 2, 5))]:
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32)
        y = oracle.matmul_f32(a, b)
        ref = np.matmul(a.astype(np.float64), b.astype(np.float64))
        assert y.shape == ref.shape
        assert np.abs(y - ref).max() < 1e-4


def test_matmul_non_float_exact_integer_sums():
    # Integer operands whose every partial sum stays below 2^53: the double
    # sum is the exact integer, so the f32 output is that integer rounded
    # once (numpy's int64 -> float32 conversion).  Broadcast batches and a
    # mixed float-by-int case (float values that are integers) included.
    rng = np.random.default_rng(51)
    for sa, sb in [((3, 7), (7, 5)), ((2, 3, 4, 9), (2, 3, 9, 6)), ((2, 1, 4, 6), (3, 6, 5)),
                   ((1, 64), (64, 3))]:
        a = rng.integers(-2**20, 2**20, sa, dtype=np.int64)
        b = rng.integers(-2**20, 2**20, sb, dtype=np.int64)
        exact = np.matmul(a, b)
        assert np.abs(exact).max() < 2**53
        np.testing.assert_array_equal(oracle.matmul_f64acc(a, b), exact.astype(np.float32))
        af = a.astype(np.float32)  # |a| < 2^20: exact in f32
        np.testing.assert_array_equal(oracle.matmul_f64acc(af, b), exact.astype(np.float32))


def test_matmul_non_float_rounds_each_double_step_in_k_order():
    # Beyond 2^53 each product and sum rounds.  Two cancellations fix the
    # chain in closed form:
    #   y[0,0] = -(2^40)(2^40+2) + (2^40+1)^2 = 1 exactly, but the second
    #     product rounds to 2^80 + 2^41 in double, so the reference gets 0
    #     (a fused multiply-add would give 1);
    #   y[1,1] = 1 + 2^60 - 2^60: in k order 1 is absorbed (0); in reverse
    #     order, or exactly, it is 1.
    # Random large operands are then checked against a Python-float loop
    # (IEEE double, one rounding per operation, k in order).
    t40, t60 = 2**40, 2**60
    a = np.array([[-t40, t40 + 1, 0], [1, t60, -t60]], np.int64)
    b = np.array([[t40 + 2, 1], [t40 + 1, 1], [1, 1]], np.int64)
    y = oracle.matmul_f64acc(a, b)
    assert y[0, 0] == 0.0 and y[1, 1] == 0.0
    rng = np.random.default_rng(52)
    a = rng.integers(-2**62, 2**62, (4, 23), dtype=np.int64)
    b = rng.integers(-2**40, 2**40, (23, 6), dtype=np.int64)
    y = oracle.matmul_f64acc(a, b)
    ad, bd = a.astype(np.float64), b.astype(np.float64)
    want = np.empty((4, 6), np.float32)
    for i in range(4):
        for j in range(6):
            acc = 0.0
            for k in range(23):
                acc += float(ad[i, k]) * float(bd[k, j])
            want[i, j] = acc
    np.testing.assert_array_equal(y, want)


def test_gemm_attributes():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((6, 5)).astype(np.float32)
    b = rng.standard_normal((7, 6)).astype(np.float32)
    for c_shape in [None, (7,), (1, 7), (5, 1), (5, 7), ()]:
        c = None if c_shape is None else rng.standard_normal(c_shape).astype(np.float32)
        y = oracle.gemm_f32(a, b, c, alpha=0.5, beta=2.0, trans_a=True, trans_b=True)
        ref = 0.5 * (a.T.astype(np.float64) @ b.T.astype(np.float64))
        if c is not None:
            ref = ref + 2.0 * c.astype(np.float64)
        assert np.abs(y - ref).max() < 1e-4


# ------------------------------------------------------------- MatMulNBits


def make_nbits(rng, n, k, bs, zp_mode):
    nb = (k + bs - 1) // bs
    b = rng.integers(0, 256, (n, nb, bs // 2), dtype=np.uint8)
    s = rng.uniform(0.005, 0.05, (n, nb)).astype(np.float32)
    if zp_mode == "packed":
        zp = rng.integers(0, 256, (n, (nb + 1) // 2), dtype=np.uint8)
    elif zp_mode == "float":
        zp = (rng.standard_normal((n, nb)) + 8).astype(np.float32)
    else:
        zp = None
    return b, s, zp


def nbits_dequant_numpy(b, s, zp, n, k, bs):
    """Independent closed form of the dequantised weight [N, K]."""
    nb = (k + bs - 1) // bs
    q = np.empty((n, nb, bs), dtype=np.int64)
    q[:, :, 0::2] = b & 15
    q[:, :, 1::2] = b >> 4
    if zp is None:
        z = np.full((n, nb), 8.0)
    elif zp.dtype == np.uint8:
        zz = np.empty((n, 2 * zp.shape[1]), dtype=np.int64)
        zz[:, 0::2] = zp & 15
        zz[:, 1::2] = zp >> 4
        z = zz[:, :nb].astype(np.float64)
    else:
        z = zp.astype(np.float64).reshape(n, nb)
    w = ((q - z[:, :, None]) * s.astype(np.float64).reshape(n, nb)[:, :, None])
    return w.astype(np.float32).reshape(n, nb * bs)[:, :k]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 9])
@pytest.mark.parametrize("k,bs", [(64, 32), (35, 16), (40, 32), (300, 64), (256, 128)])
@pytest.mark.parametrize("zp_mode", ["none", "packed", "float"])
def test_nbits_closed_form(m, k, bs, zp_mode):
    rng = np.random.default_rng(1000 * m + k)
    n = 37
    b, s, zp = make_nbits(rng, n, k, bs, zp_mode)
    a = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    y = oracle.matmul_nbits(a, b, s, zp, k=k, n=n, block_size=bs, bias=bias)
    w = nbits_dequant_numpy(b, s, zp, n, k, bs)
    ref = a.astype(np.float64) @ w.T.astype(np.float64) + bias
    assert G.rms_error(y, ref) < 1e-5
    if m == 1:  # f64 accumulation, one rounding: matches to f32 rounding
        np.testing.assert_allclose(y, ref.astype(np.float32), rtol=1e-6, atol=1e-6)


def test_nbits_default_zero_point_is_eight():
    # q == 8 everywhere with no zero points dequantises to exactly zero.
    n, k, bs = 4, 64, 32
    b = np.full((n, 2, 16), 0x88, dtype=np.uint8)
    s = np.ones((n, 2), dtype=np.float32)
    a = np.ones((2, k), dtype=np.float32)
    y = oracle.matmul_nbits(a, b, s, None, k=k, n=n, block_size=bs)
    assert not y.any()


def test_nbits_rejects_bad_attributes():
    a = np.zeros((1, 64), dtype=np.float32)
    b = np.zeros((2, 2, 16), dtype=np.uint8)
    s = np.zeros(4, dtype=np.float32)
    with pytest.raises(oracle.OracleError) as e:
        oracle.matmul_nbits(a, b, s, None, k=64, n=2, bits=8, block_size=32)
    assert e.value.status == oracle.UNSUPPORTED
    with pytest.raises(oracle.OracleError) as e:
        oracle.matmul_nbits(a, b, s, None, k=64, n=2, block_size=24)
    assert e.value.status == oracle.INVALID_ARGUMENT


# ------------------------------------------------- MatMulInteger / QLinear


@pytest.mark.parametrize("a_signed,b_signed", [(False, True), (False, False),
                                               (True, True), (True, False)])
def test_matmul_integer_brute_force(a_signed, b_signed):
    rng = np.random.default_rng(7)
    ta = np.int8 if a_signed else np.uint8
    tb = np.int8 if b_signed else np.uint8
    lo_a, hi_a = (-128, 128) if a_signed else (0, 256)
    lo_b, hi_b = (-128, 128) if b_signed else (0, 256)
    for batch_a, batch_b in [(1, 1), (3, 3), (3, 1), (1, 2)]:
        m, k, n = 5, 17, 6
        a = rng.integers(lo_a, hi_a, (batch_a, m, k)).astype(ta)
        b = rng.integers(lo_b, hi_b, (batch_b, k, n)).astype(tb)
        for az, bz in [(None, None), (np.array(3), np.array(-2)),
                       (rng.integers(0, 20, m), rng.integers(-5, 5, n))]:
            y = oracle.matmul_integer(a, b, az, bz)
            A = a.astype(np.int64) - (0 if az is None else az.astype(np.int64).reshape(-1, 1))
            B = b.astype(np.int64) - (0 if bz is None else bz.astype(np.int64).reshape(1, -1))
            np.testing.assert_array_equal(y.reshape(-1, m, n), np.matmul(A, B).reshape(-1, m, n))


def test_matmul_integer_rejects_bad_zero_point():
    a = np.zeros((4, 3), dtype=np.uint8)
    b = np.zeros((3, 2), dtype=np.int8)
    with pytest.raises(oracle.OracleError) as e:
        oracle.matmul_integer(a, b, np.zeros(3, dtype=np.int32), None)
    assert e.value.status == oracle.UNSUPPORTED


def _qlinear_numpy(acc, a_s, b_s, y_s, yz, lo, hi):
    ab = np.float32(np.float64(np.float32(a_s)) * np.float64(np.float32(b_s)))
    mult = np.float32(np.float64(ab) / np.float64(np.float32(y_s)))
    p = (acc.astype(np.float64) * np.float64(mult)).astype(np.float32)
    q = np.rint(p.astype(np.float64)).astype(np.int64) + yz  # rint: ties to even
    return np.clip(q, lo, hi)


@pytest.mark.parametrize("signed_out", [False, True])
def test_qlinear_closed_form(signed_out):
    rng = np.random.default_rng(9)
    a = rng.integers(0, 256, (2, 8, 40)).astype(np.uint8)
    b = rng.integers(-127, 128, (40, 9)).astype(np.int8)
    az, bz = np.array(118), np.array(0)
    lo, hi = (-128, 127) if signed_out else (0, 255)
    yz = 3 if signed_out else 128
    for ys in (0.05, 0.5, 5.0):  # saturating and unsaturated
        y = oracle.qlinear_matmul(a, 0.0123, az, b, 2.0 ** -10, bz, ys, np.array(yz),
                                  lo=lo, hi=hi)
        acc = oracle.matmul_integer(a, b, az, bz)
        np.testing.assert_array_equal(y, _qlinear_numpy(acc, 0.0123, 2.0 ** -10, ys,
                                                        yz, lo, hi))


def test_qlinear_tie_rounds_to_even():
    # acc * mult lands exactly on .5: 3 * 0.5 = 1.5 -> 2, 5 * 0.5 = 2.5 -> 2.
    a = np.array([[3, 5]], dtype=np.uint8)
    b = np.array([[1, 0], [0, 1]], dtype=np.uint8)
    y = oracle.qlinear_matmul(a, 1.0, None, b, 0.5, None, 1.0, np.array(0),
                              lo=0, hi=255)
    assert y.ravel().tolist() == [2, 2]


# ----------------------------------------------------- DynamicQuantizeLinear


def _dql_numpy(x):
    x64 = x.astype(np.float64)
    mn = min(0.0, float(x64.min()))
    mx = max(0.0, float(x64.max()))
    scale = np.float32((mx - mn) / 255.0)
    if scale == 0:
        return np.full(x.shape, 0, np.uint8), scale, 0
    zpf = np.float32(-mn / np.float64(scale))
    zp = int(np.rint(np.clip(np.float64(zpf), 0, 255)))
    r = (x64 / np.float64(scale)).astype(np.float32)
    q = np.rint(r.astype(np.float64)).astype(np.int64) + zp
    return np.clip(q, 0, 255).astype(np.uint8), scale, zp


@pytest.mark.parametrize("shape,shift", [((128, 1024), 0.0), ((7,), 3.0),
                                         ((33, 5), -2.0), ((1000,), 0.5)])
def test_dql_closed_form(shape, shift):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal(shape) + shift).astype(np.float32)
    y, s, z = oracle.dynamic_quantize_linear(x)
    y2, s2, z2 = _dql_numpy(x)
    assert s == s2 and z == z2
    np.testing.assert_array_equal(y, y2)


def test_dql_zero_input_and_nonfinite():
    y, s, z = oracle.dynamic_quantize_linear(np.zeros(5, np.float32))
    assert s == 0 and z == 0 and not y.any()
    with pytest.raises(oracle.OracleError):
        oracle.dynamic_quantize_linear(np.array([1.0, np.nan], np.float32))


# ------------------------------------------------------------- attention


def _sdpa_closed_form(a, b, v, mask, scale):
    s = np.matmul(a.astype(np.float64), b.astype(np.float64)) * scale + mask
    mx = s.max(axis=-1, keepdims=True)
    e = np.exp(s - mx)
    p = e / e.sum(axis=-1, keepdims=True)
    return np.matmul(p, v.astype(np.float64))


@pytest.mark.parametrize("shapes", [
    # a, b, v, mask
    ((2, 3, 5, 8), (2, 3, 8, 7), (2, 3, 7, 4), (2, 1, 1, 7)),   # BERT-style padding mask
    ((4, 6, 3), (4, 3, 6), (4, 6, 5), (6, 6)),                  # causal-style [S, T] mask
    ((2, 1, 5, 8), (1, 3, 8, 9), (2, 3, 9, 4), ()),             # broadcast batches, scalar mask
    ((3, 7, 16), (16, 7), (7, 16), (7,)),                        # shared K / V, per-key mask
    ((1, 1, 4), (1, 4, 2), (3, 1, 2, 5), (1, 2)),                # v broadcasts the scores
])
def test_fused_sdpa_closed_form(shapes):
    rng = np.random.default_rng(sum(len(x) for x in shapes))
    a, b, v, m = (rng.standard_normal(sh).astype(np.float32) for sh in shapes)
    got = oracle.fused_sdpa(a, b, v, m, 0.37)
    want = _sdpa_closed_form(a, b, v, m, 0.37)
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_fused_sdpa_masked_rows_and_equivalence_to_mha():
    rng = np.random.default_rng(3)
    b_, h, s_, t, d = 2, 4, 5, 6, 8
    q = rng.standard_normal((b_, s_, h * d)).astype(np.float32)
    k = rng.standard_normal((b_, t, h * d)).astype(np.float32)
    v = rng.standard_normal((b_, t, h * d)).astype(np.float32)
    bias = rng.standard_normal((b_, h, s_, t)).astype(np.float32)
    mha = oracle.multi_head_attention(q, k, v, bias, num_heads=h, scale=0.25)
    # The same attention as _FusedSDPA over per-head views.
    qh = q.reshape(b_, s_, h, d).transpose(0, 2, 1, 3)
    kt = k.reshape(b_, t, h, d).transpose(0, 2, 3, 1)
    vh = v.reshape(b_, t, h, d).transpose(0, 2, 1, 3)
    sd = oracle.fused_sdpa(qh, kt, vh, bias, 0.25).transpose(0, 2, 1, 3).reshape(b_, s_, h * d)
    np.testing.assert_allclose(mha, sd, rtol=1e-5, atol=1e-6)
    # A fully masked row is NaN (exp(-inf - -inf)); a partly masked one ignores
    # the masked keys exactly.
    m = np.zeros((s_, t), np.float32)
    m[1, :] = -np.inf
    m[2, 3:] = -np.inf
    y = oracle.fused_sdpa(qh, kt, vh, m, 0.25)
    assert np.isnan(y[:, :, 1]).all() and np.isfinite(np.delete(y, 1, axis=2)).all()
    y2 = oracle.fused_sdpa(qh[:, :, 2:3], kt[..., :3], vh[:, :, :3], np.zeros((1, 3), np.float32),
                           0.25)
    np.testing.assert_allclose(y[:, :, 2:3], y2, rtol=1e-6, atol=1e-7)


def test_mha_default_scale_and_shared_bias_head():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 3, 12)).astype(np.float32)
    k = rng.standard_normal((1, 5, 12)).astype(np.float32)
    v = rng.standard_normal((1, 5, 12)).astype(np.float32)
    bias = rng.standard_normal((1, 1, 3, 5)).astype(np.float32)
    got = oracle.multi_head_attention(q, k, v, bias, num_heads=3)
    want = np.empty((1, 3, 12))
    for hh in range(3):
        sl = slice(4 * hh, 4 * hh + 4)
        want[0, :, sl] = _sdpa_closed_form(q[0, :, sl], k[0, :, sl].T, v[0, :, sl], bias[0, 0],
                                           1 / np.sqrt(4))
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


# ------------------------------------------------------------ convolution


def test_conv_1x1_is_a_matmul():
    rng = np.random.default_rng(41)
    x = rng.standard_normal((2, 6, 5, 7)).astype(np.float32)
    w = rng.standard_normal((4, 6, 1, 1)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    want = np.einsum("mc,nchw->nmhw", w[:, :, 0, 0].astype(np.float64), x.astype(np.float64))
    want += b.reshape(1, -1, 1, 1)
    np.testing.assert_allclose(oracle.conv(x, w, b), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("nd", [1, 2, 3])
def test_conv_one_hot_kernel_shifts_input(nd):
    rng = np.random.default_rng(42 + nd)
    sp = [6, 5, 4][:nd]
    x = rng.standard_normal([1, 1] + sp).astype(np.float32)
    ker = [3, 2, 3][:nd]
    w = np.zeros([1, 1] + ker, np.float32)
    tap = tuple(k - 1 for k in ker)  # last tap of every axis
    w[(0, 0) + tap] = 1.0
    pads = [1] * nd + [0] * nd  # pad at the beginning only
    y = oracle.conv(x, w, pads=pads)
    # begin pad 1: y[o] = x[o + tap - 1] per axis (tap >= 1), 0 past the end
    want = np.zeros_like(y)
    src = x[(0, 0) + tuple(slice(t - 1, None) for t in tap)]
    n = tuple(min(a, b) for a, b in zip(src.shape, y.shape[2:]))
    want[(0, 0) + tuple(slice(0, v) for v in n)] = src[tuple(slice(0, v) for v in n)]
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("case", [
    dict(st=[1, 1], dl=[1, 1], pads=[0, 0, 0, 0], g=1),
    dict(st=[2, 2], dl=[1, 1], pads=[1, 1, 1, 1], g=1),
    dict(st=[2, 3], dl=[2, 1], pads=[2, 0, 1, 2], g=2),
    dict(st=[1, 2], dl=[1, 1], pads=[0, 1, 0, 1], g=4),
])
def test_conv_transpose_is_the_adjoint_of_conv(case):
    """<conv(x, w), y> == <x, conv_transpose(y, w)> with the same geometry
    (output_padding chosen so the transposed output has x's shape)."""
    rng = np.random.default_rng(7)
    g = case["g"]
    x = rng.standard_normal((2, 4, 9, 8))
    w = rng.standard_normal((8, 4 // g, 3, 2))
    y_shape = oracle.conv(x.astype(np.float32), w.astype(np.float32), strides=case["st"],
                          dilations=case["dl"], pads=case["pads"], group=g).shape
    y = rng.standard_normal(y_shape)
    # output_padding that gives the transposed output x's spatial shape
    op = [x.shape[2 + a] - ((y_shape[2 + a] - 1) * case["st"][a] + case["dl"][a] *
                            (w.shape[2 + a] - 1) + 1 - case["pads"][a] - case["pads"][2 + a])
          for a in range(2)]
    assert all(0 <= v < s for v, s in zip(op, case["st"])) or case["st"] == [1, 1]
    cx = oracle.conv(x, w, strides=case["st"], dilations=case["dl"], pads=case["pads"],
                     group=g).astype(np.float64)
    ty = oracle.conv_transpose(y, w, strides=case["st"], dilations=case["dl"],
                               pads=case["pads"], output_padding=op,
                               group=g).astype(np.float64)
    assert ty.shape == x.shape
    lhs = float(np.sum(cx * y))
    rhs = float(np.sum(x * ty))
    assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(lhs)), (lhs, rhs)


def test_conv_same_pads_put_the_extra_on_the_right_side():
    # even total padding split 1/1 is symmetric; with in 6, k 4, stride 1 the
    # total is 3: SAME_UPPER pads (1 begin, 2 end), SAME_LOWER (2, 1).
    assert oracle.resolve_pads([6], [4], [1], [1], "SAME_UPPER")[0] == [1, 2]
    assert oracle.resolve_pads([6], [4], [1], [1], "SAME_LOWER")[0] == [2, 1]
    assert oracle.resolve_pads([7], [3], [2], [1], "VALID") == ([0, 0], [3])
    # Dart's ~/ truncates: (2 - 3) ~/ 2 + 1 == 1 - 0 == 1? (-1 ~/ 2 == 0)
    assert oracle.resolve_pads([2], [3], [2], [1], "NOTSET", [0, 0])[1] == [1]


@pytest.mark.parametrize("xs,ws", [(False, True), (True, True), (False, False), (True, False)])
def test_conv_integer_equals_float_conv_of_centred_operands(xs, ws):
    rng = np.random.default_rng(11)
    xt = np.int8 if xs else np.uint8
    wt = np.int8 if ws else np.uint8
    lo_x, hi_x = (-128, 128) if xs else (0, 256)
    lo_w, hi_w = (-128, 128) if ws else (0, 256)
    x = rng.integers(lo_x, hi_x, (2, 6, 7, 6)).astype(xt)
    w = rng.integers(lo_w, hi_w, (4, 3, 3, 3)).astype(wt)
    xz = int(rng.integers(lo_x, hi_x))
    wz = rng.integers(lo_w, hi_w, 4).astype(wt)
    y = oracle.conv_integer(x, w, np.array(xz, xt), wz, pads=[1, 2, 0, 1], strides=[1, 2],
                            group=2)
    # padding contributes (x_zp - x_zp) = 0: pad the centred input with zeros
    xc = x.astype(np.float64) - xz
    wc = w.astype(np.float64) - wz.astype(np.float64).reshape(-1, 1, 1, 1)
    want = oracle.conv(xc, wc, pads=[1, 2, 0, 1], strides=[1, 2], group=2)
    np.testing.assert_array_equal(y, want.astype(np.float64).round().astype(np.int64))


def test_qlinear_conv_requant_rounds_half_to_even():
    # one output channel, 1x1 kernel: acc = x - x_zp; mult = 0.5 makes halves
    x = np.array([[[[1, 2, 3, 5, 7]]]], np.uint8)
    w = np.array([[[[1]]]], np.int8)
    y = oracle.qlinear_conv(x, np.float32(0.5), np.uint8(0), w, np.float32(1.0), np.int8(0),
                            np.float32(1.0), np.uint8(10), lo=0, hi=255)
    # 0.5 -> 0, 1.0 -> 1, 1.5 -> 2, 2.5 -> 2, 3.5 -> 4
    np.testing.assert_array_equal(y.ravel(), [10, 11, 12, 12, 14])
    y = oracle.qlinear_conv(x, np.float32(0.5), np.uint8(0), w, np.float32(1.0), np.int8(0),
                            np.float32(1.0), np.int8(-127), lo=-128, hi=127)
    np.testing.assert_array_equal(y.ravel(), [-127, -126, -125, -125, -123])


# ------------------------------------------------------ GroupQueryAttention


def _gqa_inputs(rng, b, s, heads, kv, hs, past=0):
    q = rng.standard_normal((b, s, heads * hs)).astype(np.float32)
    k = rng.standard_normal((b, s, kv * hs)).astype(np.float32)
    v = rng.standard_normal((b, s, kv * hs)).astype(np.float32)
    pk = rng.standard_normal((b, kv, past, hs)).astype(np.float32) if past else None
    pv = rng.standard_normal((b, kv, past, hs)).astype(np.float32) if past else None
    return q, k, v, pk, pv


def test_gqa_without_groups_or_past_is_causal_mha():
    rng = np.random.default_rng(21)
    q, k, v, _, _ = _gqa_inputs(rng, 2, 7, 3, 3, 8)
    y = oracle.group_query_attention(q, k, v, num_heads=3, kv_num_heads=3)[0]
    causal = np.triu(np.full((7, 7), -np.inf, np.float32), 1)
    bias = np.broadcast_to(causal, (2, 1, 7, 7)).copy()
    want = oracle.multi_head_attention(q, k, v, bias, num_heads=3)
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6)


def test_gqa_groups_equal_repeated_kv_heads():
    rng = np.random.default_rng(22)
    q, k, v, pk, pv = _gqa_inputs(rng, 1, 4, 8, 2, 16, past=3)
    y, prk, prv = oracle.group_query_attention(q, k, v, num_heads=8, kv_num_heads=2,
                                               past_key=pk, past_value=pv)
    rep = lambda t: np.repeat(t.reshape(1, 4, 2, 16), 4, axis=2).reshape(1, 4, 128)  # noqa
    rep_p = lambda t: np.repeat(t, 4, axis=1)  # noqa: E731
    y2 = oracle.group_query_attention(q, rep(k), rep(v), num_heads=8, kv_num_heads=8,
                                      past_key=rep_p(pk), past_value=rep_p(pv))[0]
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(prk[:, :, :3], pk)
    np.testing.assert_array_equal(prk[:, :, 3:], k.reshape(1, 4, 2, 16).transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(prv[:, :, 3:], v.reshape(1, 4, 2, 16).transpose(0, 2, 1, 3))


@pytest.mark.parametrize("interleaved", [False, True])
def test_rotary_is_a_complex_rotation(interleaved):
    rng = np.random.default_rng(23)
    x = rng.standard_normal((2, 3, 2 * 10)).astype(np.float32)  # 2 heads of 10
    theta = rng.uniform(-3, 3, (9, 3))  # rotary dims 6 of 10
    cos, sin = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    pos = [4, 0, 8]
    y = oracle.rotary_embedding(x, pos, cos, sin, num_heads=2, interleaved=interleaved)
    xh = x.reshape(2, 3, 2, 10).astype(np.float64)
    want = xh.copy()
    c = cos[pos].astype(np.float64)[None, :, None, :]
    s_ = sin[pos].astype(np.float64)[None, :, None, :]
    if interleaved:
        x0, x1 = xh[..., 0:6:2], xh[..., 1:6:2]
        want[..., 0:6:2], want[..., 1:6:2] = x0 * c - x1 * s_, x1 * c + x0 * s_
    else:
        x0, x1 = xh[..., 0:3], xh[..., 3:6]
        want[..., 0:3], want[..., 3:6] = x0 * c - x1 * s_, x1 * c + x0 * s_
    np.testing.assert_array_equal(y, want.astype(np.float32).reshape(2, 3, 20))


def test_gqa_decode_step_continues_the_prefill():
    """Prefill of 6 tokens == prefill of 5, then one decode step with the
    present cache as the past (causal attention, RoPE at the absolute
    position)."""
    rng = np.random.default_rng(24)
    q, k, v, _, _ = _gqa_inputs(rng, 1, 6, 4, 2, 8)
    cos = rng.uniform(-1, 1, (16, 4)).astype(np.float32)
    sin = rng.uniform(-1, 1, (16, 4)).astype(np.float32)
    kw = dict(num_heads=4, kv_num_heads=2, do_rotary=True, cos_cache=cos, sin_cache=sin)
    full = oracle.group_query_attention(q, k, v, **kw)
    head = oracle.group_query_attention(q[:, :5], k[:, :5], v[:, :5], **kw)
    step = oracle.group_query_attention(q[:, 5:], k[:, 5:], v[:, 5:], past_key=head[1],
                                        past_value=head[2], **kw)
    np.testing.assert_allclose(step[0], full[0][:, 5:], rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(step[1], full[1])
    np.testing.assert_allclose(head[0], full[0][:, :5], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("m,k,n,workers", [(7, 33, 50, 3), (64, 128, 1000, 8), (5, 16, 3, 4),
                                           (4, 40, 151, 2), (300, 64, 17, 16)])
def test_pool_split_is_bitwise_the_unsplit_kernel(m, k, n, workers):
    # parallel_pool_test.dart:27-111: an N-split over workers (the first n % W
    # take one more column) gives bitwise the single-kernel result, including
    # more workers than columns.  The graph pools only calls of >= 4 rows
    # (lib/src/onnx_graph.dart:856-872), where every column takes the f32
    # lanes; below 4 rows the kernel's double tails depend on n % 4.
    rng = np.random.default_rng(23)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    pool = oracle.GemmPool(b, workers)
    np.testing.assert_array_equal(pool.matmul(a), oracle.matmul_kernel(a, b))
    pool.close()
