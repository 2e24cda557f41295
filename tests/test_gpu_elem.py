"""Elementwise device ops (Add/Sub/Mul/Div with broadcasting, Sigmoid,
RMSNorm, SkipSimplifiedLayerNormalization) against the oracle and the
reference's fixtures, and a decoder layer's chain kept on the device.

Bars: the binary ops bit-exact (f32 op = the reference's double op rounded
once); Sigmoid and RMSNorm within 1 f32 ulp of the oracle (exp in double
and a parallel double sum of squares, against the reference's sequential
one)."""
import numpy as np
import pytest

import golden_io as G
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


def ulps(a, b):
    a = np.asarray(a, np.float32).ravel().view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).ravel().view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max()) if a.size else 0


@pytest.mark.parametrize("name", ["add_bias_broadcast_lastdim", "add_broadcast_middle"])
def test_add_fixtures(ops, name):
    d = G.load(name)
    a, b = d["arrays"]
    y = ops.op_add(a, b)
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], name)
    np.testing.assert_array_equal(y, oracle.binary_f32("add", a, b))


def test_rmsnorm_pattern_fixture(ops):
    d = G.load("rmsnorm_pattern")
    x, g = d["arrays"]
    y = ops.op_rms_norm(x, g, d["attrs"]["axis"], d["attrs"]["epsilon"])
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], "rmsnorm_pattern")
    assert ulps(y, oracle.rms_norm_f32(x, g, d["attrs"]["axis"], d["attrs"]["epsilon"])) <= 1


def test_skip_simplified_layer_norm_fixture(ops):
    d = G.load("skipsimplifiedlayernorm")
    x, skip, w = d["arrays"]
    y, s = ops.op_skip_simplified_layer_norm(x, skip, w, eps=d["attrs"]["epsilon"])
    G.assert_reference_parity(y, d["want"]["out0"], "out0")
    G.assert_reference_parity(s, d["want"]["out3"], "out3")
    np.testing.assert_array_equal(s, x + skip)


def test_glu_gate_fixture(ops):
    d = G.load("glu_gate")
    (x,) = d["arrays"]
    a, b = np.split(x, 2, axis=d["attrs"]["axis"])
    y = ops.op_mul(a, ops.op_sigmoid(b))
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], "glu_gate")


SHAPES = [((2, 3, 4), (2, 3, 4)), ((2, 3, 4), ()), ((), (5,)), ((2, 1, 4, 3), (5, 1, 3)),
          ((4, 1), (1, 6)), ((3, 5, 8), (8,)), ((3, 5, 8), (3, 5, 1)), ((1, 7), (3, 1, 1)),
          ((2, 0, 3), (1, 3)), ((2, 1, 2, 1, 2, 1, 2), (1, 2, 1, 2, 1, 2, 1)),
          ((512, 2048), (2048,)), ((16, 1, 8192), (16, 1, 8192)), ((1000003,), (1000003,)),
          ((3, 1, 2, 1, 2, 1, 2, 1, 2), (1, 2, 1, 2, 1, 2, 1, 2, 1))]


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("sa,sb", SHAPES)
def test_binary_bitwise(ops, op, sa, sb):
    rng = np.random.default_rng(3)
    a = rng.standard_normal(sa).astype(np.float32)
    b = (rng.standard_normal(sb) + 2.5).astype(np.float32)
    y = getattr(ops, f"op_{op}")(a, b)
    want = oracle.binary_f32(op, a, b)
    assert y.shape == want.shape
    np.testing.assert_array_equal(y, want)


def test_binary_unaligned_and_in_place(ops):
    # Operands at 4-byte (not 16-byte) offsets take the scalar form; the output
    # may alias an input (a residual add in place).
    rng = np.random.default_rng(4)
    n = 4099
    a = rng.standard_normal(n + 1).astype(np.float32)
    b = rng.standard_normal(n + 1).astype(np.float32)
    buf = ops.DeviceBuffer.from_array(np.concatenate([a, b]))
    pa, pb = buf.ptr + 4, buf.ptr + 4 * (n + 2)
    ops.binary_f32_dev("add", pa, (n,), pb, (n,), pa)
    got = buf.to_array((2 * n + 2,), np.float32)
    np.testing.assert_array_equal(got[1:n + 1], a[1:] + b[1:])
    buf.free()


def test_binary_rejects_incompatible_shapes(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError
    with pytest.raises(ArgumentError, match=r"Cannot broadcast shapes \[2, 3\] and \[4\]"):
        ops.op_add(np.zeros((2, 3), np.float32), np.zeros((4,), np.float32))


def test_sigmoid(ops):
    x = np.concatenate([np.linspace(-40, 40, 100001), [0.0, -0.0, 1e-30, 88.0, -88.0, -104.0,
                                                       np.inf, -np.inf, np.nan]]).astype(np.float32)
    y = ops.op_sigmoid(x)
    want = oracle.sigmoid_f32(x)
    fin = ~np.isnan(x)
    assert ulps(y[fin], want[fin]) <= 1
    assert np.isnan(y[-1])


@pytest.mark.parametrize("shape,axis", [((512, 2048), -1), ((1, 1024), -1), ((3, 5000), 1),
                                        ((2, 5, 16), 2), ((3, 4, 6), 0), ((3, 4, 6), 1),
                                        ((7,), 0), ((2, 3, 1), -1), ((4, 300, 8), 1)])
def test_rms_norm(ops, shape, axis):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    g = rng.uniform(0.5, 2.0, shape[-1]).astype(np.float32)
    y = ops.op_rms_norm(x, g, axis, 1e-6)
    assert ulps(y, oracle.rms_norm_f32(x, g, axis, 1e-6)) <= 1


def test_rms_norm_rejects_gamma_of_another_length(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError
    with pytest.raises(ArgumentError, match="RMSNorm gamma length 3 != last dim 4"):
        ops.op_rms_norm(np.zeros((2, 4), np.float32), np.ones(3, np.float32), -1, 1e-5)


@pytest.mark.parametrize("rows,d,with_bias", [(1, 1024, False), (512, 1024, True),
                                              (3, 4100, True)])
def test_skip_rms_norm(ops, rows, d, with_bias):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    skip = rng.standard_normal((rows, d)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, d).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32) if with_bias else None
    y, s = ops.op_skip_simplified_layer_norm(x, skip, g, bias, eps=1e-5)
    s_ref = oracle.binary_f32("add", x, skip)
    np.testing.assert_array_equal(s, s_ref)
    y_ref = oracle.rms_norm_f32(s_ref, g, -1, 1e-5)
    if with_bias:
        y_ref = oracle.binary_f32("add", y_ref, bias)
    assert ulps(y, y_ref) <= 1


@pytest.mark.parametrize("d", [1022, 2046, 4094, 5001, 12000, 20000, 2048])
@pytest.mark.parametrize("offset", [0, 1])
def test_skip_rms_norm_row_plans(ops, d, offset):
    # The row kernel's plans: float4 slots for rows of d % 4 == 0 on 16-byte
    # aligned buffers (1 to 4 slots per thread), one element per slot for
    # other rows or buffers one float off alignment (4 to 16 per thread), and
    # two passes over rows too long for registers (5001 unaligned, 20000).
    rng = np.random.default_rng(8 + d + offset)
    rows = 3
    x = rng.standard_normal((rows, d)).astype(np.float32)
    skip = rng.standard_normal((rows, d)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, d).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32)
    D = ops.DeviceBuffer
    n = rows * d

    def placed(a):  # a's elements from float `offset` of a buffer of n + 1
        buf = np.zeros(n + 1, np.float32)
        buf[offset:offset + n] = a.ravel()
        return D.from_array(buf)

    bufs = [placed(x), placed(skip), placed(np.zeros(n, np.float32)),
            placed(np.zeros(n, np.float32))]
    px, pskip, py, psum = (b.ptr + 4 * offset for b in bufs)
    bg, bb = D.from_array(g), D.from_array(bias)
    ops.skip_rms_norm_f32_dev(px, pskip, (rows, d), bg.ptr, d, bb.ptr, 1e-5, py, psum)
    y, s = (b.to_array(n + 1, np.float32)[offset:offset + n].reshape(rows, d)
            for b in bufs[2:])
    s_ref = oracle.binary_f32("add", x, skip)
    np.testing.assert_array_equal(s, s_ref)
    y_ref = oracle.binary_f32("add", oracle.rms_norm_f32(s_ref, g, -1, 1e-5), bias)
    assert ulps(y, y_ref) <= 1
    for b in (*bufs, bg, bb):
        b.free()


@pytest.mark.parametrize("alias", ["sum=x", "sum=skip", "y=x", "y=skip", "y=sum",
                                   "sum=x,y=skip", "y=x,no-sum"])
def test_skip_rms_norm_in_place(ops, alias):
    # An in-place residual stream: the sum and the normed output written over
    # the inputs.  Each aliasing form must give the separate-buffer results.
    rng = np.random.default_rng(7)
    rows, d = 5, 2100
    x = rng.standard_normal((rows, d)).astype(np.float32)
    skip = rng.standard_normal((rows, d)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, d).astype(np.float32)
    s_ref = oracle.binary_f32("add", x, skip)
    y_ref = oracle.rms_norm_f32(s_ref, g, -1, 1e-5)
    D = ops.DeviceBuffer
    bx, bskip, bg = D.from_array(x), D.from_array(skip), D.from_array(g)
    by, bsum = D(x.nbytes), D(x.nbytes)
    pairs = dict(p.split("=") for p in alias.split(",") if "=" in p)
    ptr = {"x": bx.ptr, "skip": bskip.ptr}
    psum = None if "no-sum" in alias else ptr.get(pairs.get("sum"), bsum.ptr)
    ptr["sum"] = psum
    py = ptr.get(pairs.get("y"), by.ptr)
    ops.skip_rms_norm_f32_dev(bx.ptr, bskip.ptr, (rows, d), bg.ptr, d, None, 1e-5, py, psum)
    out = {}
    for name, b in (("x", bx), ("skip", bskip), ("y", by), ("sum", bsum)):
        out[b.ptr] = b.to_array((rows, d), np.float32)
    assert ulps(out[py], y_ref) <= 1
    if psum is not None:
        if psum != py:
            np.testing.assert_array_equal(out[psum], s_ref)
    for b in (bx, bskip, bg, by, bsum):
        b.free()


@pytest.mark.parametrize("m", [1, 16])
def test_decoder_mlp_chain_on_device(ops, m):
    # The MLP half of a Qwen3-style layer with every intermediate in HBM:
    # h = SkipRMSNorm(x, residual); g, u = MatMulNBits(h) (one grouped
    # launch); a = g * sigmoid(g) * u; y = MatMulNBits(a) + residual sum.
    rng = np.random.default_rng(0x5EED0080 + m)
    hidden, inter, bs = 1024, 3072, 128

    def weight(k, n):
        nb = k // bs
        b = rng.integers(0, 256, (n, nb, bs // 2), dtype=np.uint8)
        s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float32)
        z = rng.integers(0, 256, (n, (nb + 1) // 2), dtype=np.uint8)
        return b, s, z

    hw = {"gate": weight(hidden, inter), "up": weight(hidden, inter), "down": weight(inter, hidden)}
    w = {k: ops.NBitsWeight(*v, k=hidden if k != "down" else inter,
                            n=inter if k != "down" else hidden, block_size=bs)
         for k, v in hw.items()}
    x = rng.standard_normal((m, hidden)).astype(np.float32)
    res = rng.standard_normal((m, hidden)).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    D = ops.DeviceBuffer
    bx, br, bg = D.from_array(x), D.from_array(res), D.from_array(gamma)
    bh, bsum = D(m * hidden * 4), D(m * hidden * 4)
    bgate, bup, bsig, bact = (D(m * inter * 4) for _ in range(4))
    by, bout = D(m * hidden * 4), D(m * hidden * 4)
    ops.skip_rms_norm_f32_dev(bx.ptr, br.ptr, (m, hidden), bg.ptr, hidden, None, 1e-6, bh.ptr,
                              bsum.ptr)
    ops.matmul_nbits_group_dev([w["gate"], w["up"]], bh.ptr, m, [bgate.ptr, bup.ptr])
    ops.sigmoid_f32_dev(bgate.ptr, m * inter, bsig.ptr)
    ops.binary_f32_dev("mul", bgate.ptr, (m, inter), bsig.ptr, (m, inter), bact.ptr)
    ops.binary_f32_dev("mul", bact.ptr, (m, inter), bup.ptr, (m, inter), bact.ptr)
    w["down"].run_dev(bact.ptr, m, by.ptr)
    ops.binary_f32_dev("add", by.ptr, (m, hidden), bsum.ptr, (m, hidden), bout.ptr)
    got = bout.to_array((m, hidden), np.float32)
    # The same chain on the oracle.
    s = oracle.binary_f32("add", x, res)
    h = oracle.rms_norm_f32(s, gamma, -1, 1e-6)
    g = oracle.matmul_nbits(h, *hw["gate"], k=hidden, n=inter, block_size=bs)
    u = oracle.matmul_nbits(h, *hw["up"], k=hidden, n=inter, block_size=bs)
    act = oracle.binary_f32("mul", oracle.binary_f32("mul", g, oracle.sigmoid_f32(g)), u)
    ref = oracle.binary_f32("add", oracle.matmul_nbits(act, *hw["down"], k=inter, n=hidden,
                                                       block_size=bs), s)
    assert G.rms_error(got, ref) <= 1e-3
    for b in (bx, br, bg, bh, bsum, bgate, bup, bsig, bact, by, bout):
        b.free()
    for v in w.values():
        v.release()
