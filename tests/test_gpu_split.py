"""Split activations for the decode GEMV written by its input's producer
(mg_skip_rms_norm_f32_split_dev: SkipSimplifiedLayerNormalization or a plain
RMSNorm) and read by mg_matmul_nbits_group_split_dev instead of the GEMV's
own prepass.

Bars: the producer's outputs are bitwise those of the plain ops, and the
GEMV on the split is bitwise the GEMV on the fp32 rows (the split is the
prepass's conversion of the same values), including rows with a non-finite
value; both are checked against the oracle chain to the MatMulNBits bar."""
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


def make_weight(rng, k, n, bs):
    nb = -(-k // bs)
    b = rng.integers(0, 256, (n, nb, bs // 2), dtype=np.uint8)
    s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float32)
    z = rng.integers(0, 256, (n, (nb + 1) // 2), dtype=np.uint8)
    return b, s, z


CASES = [
    # (M, K, bs, N per member): members share K; two members = a sibling group
    (4, 2048, 32, (512, 256)),     # Llama-style q/k/v at M = 4
    (16, 2048, 32, (1024,)),
    (3, 1024, 128, (3072, 3072)),  # Qwen-style gate/up
    (16, 8192, 32, (2048,)),       # down: long rows, K split over workgroups
    (5, 2100, 64, (300,)),         # K not a multiple of 128
    (8, 1000, 256, (130, 70)),     # blocks of 256 (kpad 1024)
]


@pytest.mark.parametrize("m,k,bs,ns", CASES)
@pytest.mark.parametrize("producer", ["skip_norm", "norm"])
def test_split_matches_prepass_bitwise(ops, m, k, bs, ns, producer):
    rng = np.random.default_rng(0x5EED00C0 + m + k + bs + len(producer))
    hw = [make_weight(rng, k, n, bs) for n in ns]
    ws = [ops.NBitsWeight(*h, k=k, n=n, block_size=bs) for h, n in zip(hw, ns)]
    x = rng.standard_normal((m, k)).astype(np.float32)
    x2 = rng.standard_normal((m, k)).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, k).astype(np.float32)
    x[m // 2, k // 3] = 40.0  # an outlier: a different row exponent
    D = ops.DeviceBuffer
    bx, bx2, bg = D.from_array(x), D.from_array(x2), D.from_array(gamma)
    y0, y1, s0, s1 = (D(x.nbytes) for _ in range(4))
    split = D(ops.nbits_split_bytes(k, bs))
    if producer == "skip_norm":
        ops.skip_rms_norm_f32_dev(bx.ptr, bx2.ptr, (m, k), bg.ptr, k, None, 1e-6, y0.ptr, s0.ptr)
        ops.skip_rms_norm_f32_split_dev(bx.ptr, bx2.ptr, (m, k), bg.ptr, k, None, 1e-6, y1.ptr,
                                        s1.ptr, bs, split.ptr)
        np.testing.assert_array_equal(s1.to_array((m, k), np.float32),
                                      s0.to_array((m, k), np.float32))
    else:
        ops.rms_norm_f32_dev(bx.ptr, (m, k), bg.ptr, k, -1, 1e-6, y0.ptr)
        ops.skip_rms_norm_f32_split_dev(bx.ptr, None, (m, k), bg.ptr, k, None, 1e-6, y1.ptr,
                                        None, bs, split.ptr)
    y_ref = y0.to_array((m, k), np.float32)
    np.testing.assert_array_equal(y1.to_array((m, k), np.float32), y_ref)
    outs = {}
    for tag, sp in (("prepass", None), ("split", split.ptr)):
        ys = [D(m * n * 4) for n in ns]
        ops.matmul_nbits_group_split_dev(ws, y1.ptr, sp, m, [b.ptr for b in ys])
        outs[tag] = [b.to_array((m, n), np.float32) for b, n in zip(ys, ns)]
        for b in ys:
            b.free()
    for (b, s, z), n, got, want in zip(hw, ns, outs["split"], outs["prepass"]):
        np.testing.assert_array_equal(got, want)
        cols = np.unique(np.concatenate([np.arange(min(n, 40)), np.arange(n - min(n, 40), n)]))
        ref = oracle.matmul_nbits(y_ref, b[cols], s[cols], z[cols], k=k, n=len(cols),
                                  block_size=bs)
        assert G.rms_error(got[:, cols], ref) <= TOL
    for buf in (bx, bx2, bg, y0, y1, s0, s1, split):
        buf.free()
    for w in ws:
        w.release()


def test_split_with_non_finite_rows_and_other_row_counts(ops):
    # A gamma entry of +Inf puts an Inf into every normalised row, and a NaN
    # input makes its whole row NaN: the split carries them as the prepass
    # does (the same Inf / NaN pattern in the GEMV's output); at M = 1 the
    # GEMV plan does not read the split and must still give the prepass-free
    # result.
    rng = np.random.default_rng(0x5EED00C1)
    k, n, bs = 2048, 700, 32
    h = make_weight(rng, k, n, bs)
    w = ops.NBitsWeight(*h, k=k, n=n, block_size=bs)
    D = ops.DeviceBuffer
    split = D(ops.nbits_split_bytes(k, bs))
    for m in (1, 6, 16):
        a = rng.standard_normal((m, k)).astype(np.float32)
        gamma = rng.uniform(0.5, 1.5, k).astype(np.float32)
        if m > 1:
            gamma[5] = np.inf
            a[m - 1, 9] = np.nan
        ba, bg, by = D.from_array(a), D.from_array(gamma), D(a.nbytes)
        ops.skip_rms_norm_f32_split_dev(ba.ptr, None, (m, k), bg.ptr, k, None, 1e-6, by.ptr,
                                        None, bs, split.ptr)
        o1, o2 = D(m * n * 4), D(m * n * 4)
        ops.matmul_nbits_group_split_dev([w], by.ptr, split.ptr, m, [o1.ptr])
        ops.matmul_nbits_group_dev([w], by.ptr, m, [o2.ptr])
        got = o1.to_array((m, n), np.float32)
        np.testing.assert_array_equal(got, o2.to_array((m, n), np.float32))
        if m > 1:
            assert not np.isfinite(got).any()
            assert np.isnan(got[m - 1]).all()
        for buf in (ba, bg, by, o1, o2):
            buf.free()
    # 17 rows, or rows longer than 8192: too large for a split producer.
    from onnx_runtime_dart_amd.errors import ArgumentError
    a = D(17 * 8200 * 4)
    with pytest.raises(ArgumentError, match="at most 16 rows"):
        ops.skip_rms_norm_f32_split_dev(a.ptr, None, (17, k), a.ptr, k, None, 1e-6, a.ptr, None,
                                        bs, split.ptr)
    with pytest.raises(ArgumentError, match="at most 16 rows"):
        ops.skip_rms_norm_f32_split_dev(a.ptr, None, (2, 8200), a.ptr, 8200, None, 1e-6, a.ptr,
                                        None, bs, split.ptr)
    a.free()
    split.free()
    w.release()
