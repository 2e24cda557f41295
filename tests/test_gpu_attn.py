"""Fused attention (_FusedSDPA, MultiHeadAttention) on the GPU against the
oracle and the reference's ORT fixtures.  fp32 path: the task's float bar is
max|d| <= 1e-3 * rms(ref); these tests hold the kernel to 1e-4."""
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


@pytest.mark.parametrize("name", G.names("mha"))
def test_mha_fixture(ops, name):
    d = G.load(name)
    x, at = d["arrays"], d["attrs"]
    bias = x[5] if len(x) > 5 else None
    y = ops.op_multi_head_attention(x[0], x[1], x[2], bias, num_heads=at["num_heads"],
                                    scale=at.get("scale"))
    want = d["want"][d["outputs"][0]]
    G.assert_reference_parity(y, want, name, tolerance=1e-4)


SDPA = [
    # a, b, v, mask
    ((2, 3, 5, 8), (2, 3, 8, 7), (2, 3, 7, 4), (2, 1, 1, 7)),
    ((4, 6, 3), (4, 3, 6), (4, 6, 5), (6, 6)),
    ((2, 1, 5, 8), (1, 3, 8, 9), (2, 3, 9, 4), ()),
    ((3, 7, 16), (16, 7), (7, 16), (7,)),
    ((1, 1, 4), (1, 4, 2), (3, 1, 2, 5), (1, 2)),
    ((2, 4, 130, 64), (2, 4, 64, 300), (2, 4, 300, 48), (2, 1, 130, 300)),  # 2 query tiles, ragged keys
    ((1, 2, 1, 100), (1, 2, 100, 77), (1, 2, 77, 96), (1, 1, 1, 77)),        # one query, D 100, DV 96
    ((1, 1, 33, 128), (1, 1, 128, 65), (1, 1, 65, 128), (33, 65)),           # D = DV = 128
    ((8, 12, 128, 32), (8, 12, 32, 128), (8, 12, 128, 32), (8, 1, 1, 128)),  # MiniLM-shaped
]


@pytest.mark.parametrize("shapes", SDPA)
def test_fused_sdpa_against_oracle(ops, shapes):
    rng = np.random.default_rng(sum(int(np.prod(s)) for s in shapes) % 10007)
    a, b, v, m = (rng.standard_normal(sh).astype(np.float32) for sh in shapes)
    if m.ndim:
        m[m < -1.5] = -10000.0  # BERT-style padding values
    scale = 1.0 / np.sqrt(a.shape[-1])
    y = ops.op_fused_sdpa(a, b, v, m, scale)
    ref = oracle.fused_sdpa(a, b, v, m, scale)
    assert y.shape == ref.shape
    assert G.rms_error(y, ref) <= TOL, G.rms_error(y, ref)
    np.testing.assert_array_equal(ops.op_fused_sdpa(a, b, v, m, scale), y)  # deterministic


def test_fused_sdpa_masked_rows_and_empty_keys(ops):
    rng = np.random.default_rng(11)
    a = rng.standard_normal((2, 40, 16)).astype(np.float32)
    b = rng.standard_normal((2, 16, 70)).astype(np.float32)
    v = rng.standard_normal((2, 70, 8)).astype(np.float32)
    m = np.zeros((40, 70), np.float32)
    m[3, :] = -np.inf                 # fully masked: NaN, as in the reference
    m[5, 33:] = -np.inf               # masked past the first key tile
    m[6, :32] = -np.inf               # first key tile fully masked, the rest not
    y = ops.op_fused_sdpa(a, b, v, m, 0.25)
    ref = oracle.fused_sdpa(a, b, v, m, 0.25)
    np.testing.assert_array_equal(np.isnan(y), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert G.rms_error(y[fin], ref[fin]) <= TOL
    # No keys: an empty softmax row times an empty V is zeros.
    y0 = ops.op_fused_sdpa(a, np.zeros((2, 16, 0), np.float32), np.zeros((2, 0, 8), np.float32),
                           np.zeros((40, 0), np.float32), 0.25)
    assert y0.shape == (2, 40, 8) and not y0.any()


@pytest.mark.parametrize("batch,seq,kv,hidden,heads,bias_heads,scale", [
    (2, 9, 9, 24, 4, 4, 0.35), (1, 130, 70, 64, 2, 1, None), (3, 1, 200, 256, 4, 0, None),
    (32, 128, 128, 384, 12, 0, None)])   # MiniLM self-attention
def test_mha_against_oracle(ops, batch, seq, kv, hidden, heads, bias_heads, scale):
    rng = np.random.default_rng(batch * seq + kv)
    q = rng.standard_normal((batch, seq, hidden)).astype(np.float32)
    k = rng.standard_normal((batch, kv, hidden)).astype(np.float32)
    v = rng.standard_normal((batch, kv, hidden)).astype(np.float32)
    bias = rng.standard_normal((batch, bias_heads, seq, kv)).astype(np.float32) \
        if bias_heads else None
    y = ops.op_multi_head_attention(q, k, v, bias, num_heads=heads, scale=scale)
    ref = oracle.multi_head_attention(q, k, v, bias, num_heads=heads, scale=scale)
    assert G.rms_error(y, ref) <= TOL, G.rms_error(y, ref)


def test_device_entry_points_match_host(ops):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((2, 3, 50, 32)).astype(np.float32)
    b = rng.standard_normal((2, 3, 32, 40)).astype(np.float32)
    v = rng.standard_normal((2, 3, 40, 32)).astype(np.float32)
    m = rng.standard_normal((2, 1, 1, 40)).astype(np.float32)
    host = ops.op_fused_sdpa(a, b, v, m, 0.2)
    bufs = [ops.DeviceBuffer.from_array(x) for x in (a, b, v, m)]
    yd = ops.DeviceBuffer(host.nbytes)
    ops.fused_sdpa_dev(bufs[0].ptr, a.shape, bufs[1].ptr, b.shape, bufs[2].ptr, v.shape,
                       bufs[3].ptr, m.shape, 0.2, yd.ptr)
    np.testing.assert_array_equal(yd.to_array(host.shape, np.float32), host)
    q = rng.standard_normal((2, 20, 64)).astype(np.float32)
    kk = rng.standard_normal((2, 30, 64)).astype(np.float32)
    vv = rng.standard_normal((2, 30, 64)).astype(np.float32)
    bias = rng.standard_normal((2, 4, 20, 30)).astype(np.float32)
    host2 = ops.op_multi_head_attention(q, kk, vv, bias, num_heads=4)
    b2 = [ops.DeviceBuffer.from_array(x) for x in (q, kk, vv, bias)]
    y2 = ops.DeviceBuffer(host2.nbytes)
    ops.multi_head_attention_dev(b2[0].ptr, b2[1].ptr, b2[2].ptr, 2, 20, 30, 64, 4, y2.ptr,
                                 bias_ptr=b2[3].ptr, bias_heads=4)
    np.testing.assert_array_equal(y2.to_array(host2.shape, np.float32), host2)
    for x in bufs + b2 + [yd, y2]:
        x.free()


def test_attention_errors(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError, UnsupportedError
    z = np.zeros
    with pytest.raises(ArgumentError):  # inner dims
        ops.op_fused_sdpa(z((2, 4, 8)), z((2, 7, 5)), z((2, 5, 3)), z((5,)), 1.0)
    with pytest.raises(ArgumentError):  # mask does not broadcast
        ops.op_fused_sdpa(z((2, 4, 8)), z((2, 8, 5)), z((2, 5, 3)), z((3, 5)), 1.0)
    with pytest.raises(UnsupportedError):  # head size above 128
        ops.op_fused_sdpa(z((1, 2, 200)), z((1, 200, 3)), z((1, 3, 4)), z(()), 1.0)
    with pytest.raises(ArgumentError):  # hidden not a multiple of heads
        ops.op_multi_head_attention(z((1, 2, 10)), z((1, 2, 10)), z((1, 2, 10)), num_heads=4)
    with pytest.raises(UnsupportedError):  # bias heads neither 1 nor num_heads
        ops.op_multi_head_attention(z((1, 2, 16)), z((1, 3, 16)), z((1, 3, 16)),
                                    z((1, 2, 2, 3)), num_heads=4)
