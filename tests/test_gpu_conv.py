"""Convolution family (Conv, ConvTranspose, ConvInteger, QLinearConv) on the
GPU against the reference's ORT fixtures and the oracle.  fp32: the task's
float bar is max|d| <= 1e-3 * rms(ref); these tests hold the kernel to 1e-4.
Integer outputs are bit-exact."""
import numpy as np
import pytest

import golden_io as G
import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


def _geo(at):
    return dict(strides=at.get("strides"), pads=at.get("pads"), dilations=at.get("dilations"),
                group=at.get("group", 1))


@pytest.mark.parametrize("name", G.names("conv") + G.names("qlinearconv"))
def test_conv_fixture(ops, name):
    d = G.load(name)
    x, at, op = d["arrays"], d["attrs"], d["op_type"]
    if op == "Conv":
        y = ops.op_conv(x[0], x[1], x[2] if len(x) > 2 else None,
                        auto_pad=at.get("auto_pad", "NOTSET"), **_geo(at))
    elif op == "ConvTranspose":
        y = ops.op_conv_transpose(x[0], x[1], x[2] if len(x) > 2 else None,
                                  output_padding=at.get("output_padding"),
                                  output_shape=at.get("output_shape"), **_geo(at))
    elif op == "ConvInteger":
        y = ops.op_conv_integer(x[0], x[1], x[2] if len(x) > 2 else None,
                                x[3] if len(x) > 3 else None, **_geo(at))
    else:
        yz = x[7] if len(x) > 7 else None
        lo, hi = (-128, 127) if yz is not None and yz.dtype == np.int8 else (0, 255)
        y = ops.op_qlinear_conv(*x[:8], x[8] if len(x) > 8 else None, lo=lo, hi=hi, **_geo(at))
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], name, tolerance=1e-4)


CONV = [
    # x shape, w shape, attrs
    ((2, 3, 17, 19), (8, 3, 3, 3), dict(pads=[1, 1, 1, 1])),
    ((1, 16, 32, 32), (32, 16, 3, 3), dict(strides=[2, 2], pads=[1, 0, 0, 1])),
    ((2, 8, 15, 13), (12, 4, 3, 2), dict(group=2, dilations=[2, 3], pads=[2, 1, 0, 2])),
    ((1, 32, 20, 20), (32, 1, 3, 3), dict(group=32, pads=[1, 1, 1, 1])),      # depthwise
    ((3, 5, 40), (7, 5, 5), dict(strides=[3], pads=[2, 1])),                     # 1-D
    ((1, 4, 6, 7, 5), (6, 4, 3, 3, 2), dict(pads=[1, 1, 0, 1, 1, 1])),           # 3-D
    ((1, 7, 9, 9), (5, 7, 4, 4), dict(auto_pad="SAME_UPPER", strides=[2, 2])),
    ((1, 7, 9, 9), (5, 7, 4, 4), dict(auto_pad="SAME_LOWER", strides=[2, 2])),
    ((1, 6, 11, 10), (4, 6, 3, 5), dict(auto_pad="VALID", strides=[1, 2])),
    ((4, 64, 28, 28), (128, 64, 3, 3), dict(pads=[1, 1, 1, 1])),                 # K = 576
    ((16, 8, 64, 64), (128, 8, 3, 3), dict(pads=[1, 1, 1, 1])),    # 512 tiles of 128 x 128
    ((1, 3, 224, 224), (64, 3, 7, 7), dict(strides=[2, 2], pads=[3, 3, 3, 3])),  # ResNet stem
    ((2, 256, 14, 14), (256, 256, 1, 1), {}),                                     # pointwise
]


@pytest.mark.parametrize("xs,ws,at", CONV)
def test_conv_against_oracle(ops, xs, ws, at):
    rng = np.random.default_rng((int(np.prod(xs)) + int(np.prod(ws))) % 10007)
    x = rng.standard_normal(xs).astype(np.float32)
    w = (rng.standard_normal(ws) / np.sqrt(np.prod(ws[1:]))).astype(np.float32)
    b = rng.standard_normal(ws[0]).astype(np.float32)
    y = ops.op_conv(x, w, b, **at)
    ref = oracle.conv(x, w, b, **at)
    assert y.shape == ref.shape
    assert G.rms_error(y, ref) <= TOL, G.rms_error(y, ref)
    np.testing.assert_array_equal(ops.op_conv(x, w, b, **at), y)  # deterministic


CONVT = [
    ((1, 4, 7, 6), (4, 3, 3, 3), dict(strides=[2, 2])),
    ((2, 4, 5, 5), (4, 2, 3, 4), dict(strides=[2, 3], pads=[1, 0, 1, 2], output_padding=[1, 2],
                                      group=2, dilations=[1, 2])),
    ((1, 6, 8, 8), (6, 4, 4, 4), dict(strides=[2, 2], output_shape=[17, 16])),
    ((3, 5, 21), (5, 4, 6), dict(strides=[4], pads=[1, 2])),                    # 1-D
    ((1, 3, 4, 5, 3), (3, 2, 2, 3, 3), dict(strides=[2, 1, 2], pads=[0, 1, 0, 1, 0, 1])),
    ((2, 64, 16, 16), (64, 32, 4, 4), dict(strides=[2, 2], pads=[1, 1, 1, 1])),  # VAE-like upsample
    ((16, 16, 32, 32), (16, 128, 2, 2), dict(strides=[2, 2])),     # 512 tiles of 128 x 128
    # Sub-pixel phases (unit dilation, stride > 1): kernels smaller than the
    # stride leave phases with no taps (bias only); 8 phases in 3-D; 16 in
    # 2-D at stride 4; groups; pads past the kernel; the bench's upsampler.
    ((1, 3, 5, 5), (3, 2, 1, 1), dict(strides=[2, 2])),
    ((2, 4, 6, 7), (4, 3, 5, 5), dict(strides=[3, 3], pads=[2, 1, 2, 1])),
    ((1, 4, 3, 4, 5), (4, 2, 3, 3, 3), dict(strides=[2, 2, 2], pads=[1, 1, 1, 1, 1, 1],
                                            output_padding=[1, 0, 1])),
    ((2, 6, 5, 5), (6, 2, 8, 8), dict(strides=[4, 4], pads=[2, 2, 2, 2], group=3)),
    ((1, 2, 4, 4), (2, 3, 3, 3), dict(strides=[2, 2], pads=[3, 3, 3, 3])),
    ((8, 128, 32, 32), (128, 64, 4, 4), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
]


@pytest.mark.parametrize("xs,ws,at", CONVT)
def test_conv_transpose_against_oracle(ops, xs, ws, at):
    rng = np.random.default_rng((int(np.prod(xs)) * 3 + int(np.prod(ws))) % 10007)
    x = rng.standard_normal(xs).astype(np.float32)
    w = (rng.standard_normal(ws) / np.sqrt(ws[0])).astype(np.float32)
    b = rng.standard_normal(ws[1] * at.get("group", 1)).astype(np.float32)
    y = ops.op_conv_transpose(x, w, b, **at)
    ref = oracle.conv_transpose(x, w, b, **at)
    assert y.shape == ref.shape
    assert G.rms_error(y, ref) <= TOL, G.rms_error(y, ref)


INTCONV = [
    # x shape, w shape, x signed, w signed, attrs
    ((1, 3, 9, 9), (4, 3, 3, 3), False, True, dict(pads=[1, 1, 1, 1])),
    ((2, 64, 10, 12), (16, 64, 3, 3), False, True, dict(pads=[1, 2, 0, 1], strides=[1, 2])),
    ((1, 96, 8, 8), (8, 48, 3, 3), True, True, dict(group=2, dilations=[2, 1], pads=[2, 1, 2, 1])),
    ((1, 40, 13), (6, 40, 7), True, False, dict(pads=[3, 3])),                   # 1-D, u8 weights
    ((1, 300, 6, 6), (5, 300, 1, 1), False, False, {}),                          # K = 300 > 256
    ((1, 128, 12, 12), (64, 128, 3, 3), False, True, dict(pads=[1, 1, 1, 1])),   # K = 1152
    # One group: the int8 MFMA GEMM over a byte im2col.  K = 45 (not a
    # multiple of 4), 3-D with strides and dilations, batches with a 5 x 5
    # kernel at stride 2.
    ((1, 5, 9, 9), (4, 5, 3, 3), False, False, dict(pads=[1, 1, 1, 1])),
    ((2, 7, 4, 5, 6), (3, 7, 2, 3, 3), True, True,
     dict(pads=[1, 0, 1, 1, 1, 0], strides=[1, 2, 1], dilations=[2, 1, 1])),
    ((3, 16, 11, 11), (9, 16, 5, 5), False, True,
     dict(pads=[2, 2, 2, 2], strides=[2, 2], dilations=[1, 2])),
]


def _rand_int(rng, shape, signed):
    return (rng.integers(-128, 128, shape).astype(np.int8) if signed
            else rng.integers(0, 256, shape).astype(np.uint8))


@pytest.mark.parametrize("xs,ws,xsg,wsg,at", INTCONV)
@pytest.mark.parametrize("per_channel", [False, True])
def test_conv_integer_bit_exact(ops, xs, ws, xsg, wsg, at, per_channel):
    rng = np.random.default_rng(int(np.prod(xs)) % 9973 + per_channel)
    x = _rand_int(rng, xs, xsg)
    w = _rand_int(rng, ws, wsg)
    xz = _rand_int(rng, (), xsg)
    wz = _rand_int(rng, (ws[0],) if per_channel else (), wsg)
    y = ops.op_conv_integer(x, w, xz, wz, **at)
    ref = oracle.conv_integer(x, w, xz, wz, **at)
    np.testing.assert_array_equal(y, ref)


@pytest.mark.parametrize("wz_value", [0, -5])
def test_conv_integer_uniform_per_channel_zero_points(ops, wz_value):
    # A per-channel zero-point array whose entries are all equal goes to the
    # GEMM as one scalar; the sums must not change.
    rng = np.random.default_rng(0x5EED00D0 + wz_value)
    x = _rand_int(rng, (2, 24, 9, 9), False)
    w = _rand_int(rng, (12, 24, 3, 3), True)
    wz = np.full(12, wz_value, np.int8)
    y = ops.op_conv_integer(x, w, np.uint8(131), wz, pads=[1, 1, 1, 1])
    np.testing.assert_array_equal(y, oracle.conv_integer(x, w, np.uint8(131), wz,
                                                         pads=[1, 1, 1, 1]))


def test_conv_integer_extreme_values_k_2304(ops):
    """Every product at +-255^2 over K = 256 * 9: the largest magnitudes the
    exact fp32 segments and the int32 accumulators have to carry."""
    x = np.full((1, 256, 5, 5), 255, np.uint8)
    w = np.full((3, 256, 3, 3), -128, np.int8)
    w[1] = 127
    y = ops.op_conv_integer(x, w, np.uint8(0), np.array([127, -128, 0], np.int8),
                            pads=[1, 1, 1, 1])
    ref = oracle.conv_integer(x, w, np.uint8(0), np.array([127, -128, 0], np.int8),
                              pads=[1, 1, 1, 1])
    np.testing.assert_array_equal(y, ref)
    assert ref.min() == -255 * 255 * 256 * 9


QLCONV = INTCONV[:4] + INTCONV[6:] + [
    # The ResNet-50 3 x 3 layer the bench times, at two images.
    ((2, 256, 14, 14), (256, 256, 3, 3), False, True, dict(pads=[1, 1, 1, 1])),
]


@pytest.mark.parametrize("xs,ws,xsg,wsg,at", QLCONV)
@pytest.mark.parametrize("signed_out", [False, True])
def test_qlinear_conv_bit_exact(ops, xs, ws, xsg, wsg, at, signed_out):
    rng = np.random.default_rng(int(np.prod(ws)) % 9973 + signed_out)
    x = _rand_int(rng, xs, xsg)
    w = _rand_int(rng, ws, wsg)
    xz = _rand_int(rng, (), xsg)
    wz = _rand_int(rng, (ws[0],), wsg)
    ws_ = rng.uniform(0.002, 0.02, ws[0]).astype(np.float32)
    bias = rng.integers(-2000, 2000, ws[0]).astype(np.int32)
    yz = np.int8(3) if signed_out else np.uint8(128)
    lo, hi = (-128, 127) if signed_out else (0, 255)
    # y_scale from the accumulators' spread, so that most outputs are in range
    acc = oracle.conv_integer(x, w, xz, wz, **at).astype(np.float64)
    ys = np.float32(0.05 * float(np.mean(ws_)) * (float(np.std(acc)) + 1.0) / 40.0)
    args = (x, np.float32(0.05), xz, w, ws_, wz, ys, yz, bias)
    y = ops.op_qlinear_conv(*args, lo=lo, hi=hi, **at)
    ref = oracle.qlinear_conv(*args, lo=lo, hi=hi, **at)
    np.testing.assert_array_equal(y, ref)
    assert 0 < np.mean((ref > lo) & (ref < hi))  # not all saturated


def test_conv_device_entry_points_match_host(ops):
    rng = np.random.default_rng(5)
    D = ops.DeviceBuffer
    x = rng.standard_normal((2, 8, 12, 11)).astype(np.float32)
    w = rng.standard_normal((6, 4, 3, 3)).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    at = dict(strides=[2, 1], pads=[1, 1, 0, 1], group=2)
    want = ops.op_conv(x, w, b, **at)
    xd, wd, bd = (D.from_array(a) for a in (x, w, b))
    yd = D(want.nbytes)
    ops.conv_f32_dev(xd.ptr, x.shape, wd.ptr, w.shape, yd.ptr, bd.ptr, **at)
    np.testing.assert_array_equal(yd.to_array(want.shape, np.float32), want)

    wt = rng.standard_normal((8, 3, 3, 3)).astype(np.float32)
    att = dict(strides=[2, 2], pads=[1, 0, 1, 0], output_padding=[1, 1], group=2)
    want_t = ops.op_conv_transpose(x, wt, None, **att)
    wtd = D.from_array(wt)
    ytd = D(want_t.nbytes)
    ops.conv_transpose_f32_dev(xd.ptr, x.shape, wtd.ptr, wt.shape, ytd.ptr, **att)
    np.testing.assert_array_equal(ytd.to_array(want_t.shape, np.float32), want_t)

    xi = rng.integers(0, 256, (1, 16, 7, 7)).astype(np.uint8)
    wi = rng.integers(-128, 128, (4, 16, 3, 3)).astype(np.int8)
    wz = np.array([1, -2, 3, 0], np.int8)
    want_i = ops.op_conv_integer(xi, wi, np.uint8(7), wz, pads=[1, 1, 1, 1])
    xid, wid = D.from_array(xi), D.from_array(wi)
    yid = D(want_i.size * 4)
    ops.conv_integer_dev(xid.ptr, False, xi.shape, wid.ptr, True, wi.shape, yid.ptr, 7, wz,
                         pads=[1, 1, 1, 1])
    np.testing.assert_array_equal(yid.to_array(want_i.shape, np.int32).astype(np.int64), want_i)

    ws_ = np.array([0.01, 0.02, 0.015, 0.005], np.float32)
    bias = np.array([100, -50, 0, 7], np.int32)
    want_q = ops.op_qlinear_conv(xi, np.float32(0.04), np.uint8(7), wi, ws_, wz,
                                 np.float32(0.3), np.uint8(120), bias, pads=[1, 1, 1, 1],
                                 lo=0, hi=255)
    bqd = D.from_array(bias)
    yqd = D(want_q.size)
    ops.qlinear_conv_dev(xid.ptr, False, xi.shape, 0.04, 7, wid.ptr, True, wi.shape, ws_, wz,
                         0.3, 120, yqd.ptr, bqd.ptr, pads=[1, 1, 1, 1], lo=0, hi=255)
    np.testing.assert_array_equal(yqd.to_array(want_q.shape, np.uint8).astype(np.int64), want_q)
    for buf in (xd, wd, bd, yd, wtd, ytd, xid, wid, yid, bqd, yqd):
        buf.free()


def test_conv_errors(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError, StateError, UnsupportedError
    x = np.zeros((1, 4, 5, 5), np.float32)
    with pytest.raises(ArgumentError):
        ops.op_conv(x, np.zeros((2, 3, 3, 3), np.float32))            # channel mismatch
    with pytest.raises(ArgumentError):
        ops.op_conv(x, np.zeros((3, 2, 3, 3), np.float32), group=2)   # M % group
    with pytest.raises(ArgumentError):
        ops.op_conv(x, np.zeros((2, 4, 7, 7), np.float32))            # kernel > input
    with pytest.raises(ArgumentError):
        ops.op_conv(x, np.zeros((2, 4, 3, 3), np.float32), strides=[0, 1])
    with pytest.raises(StateError):
        ops.op_conv(x, np.zeros((2, 4, 3, 3), np.float32), kernel_shape=[2, 2])
    with pytest.raises(UnsupportedError):
        ops.op_conv_integer(np.zeros((1, 2, 4, 4), np.uint8), np.zeros((3, 2, 1, 1), np.int8),
                            np.uint8(0), np.zeros(2, np.int8))             # zp neither 1 nor M
    with pytest.raises(ArgumentError):
        ops.op_conv(np.zeros((1, 4, 5), np.float32), np.zeros((2, 4, 3, 3), np.float32))
    # empty batch: empty output, no launch
    y = ops.op_conv(np.zeros((0, 4, 5, 5), np.float32), np.zeros((2, 4, 3, 3), np.float32))
    assert y.shape == (0, 2, 3, 3)
