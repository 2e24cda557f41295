"""The allocation-free MatMulNBits entry point (mg_matmul_nbits_dev_noalloc)
against the allocating one on the GPU: the same kernels and plan, so the
outputs must be bitwise equal; two calls in a row on the shared scratch, the
second smaller, and requests beyond the scratch rejected before any launch."""
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


def _weight(ops, rng, k, n, bs):
    nb = (k + bs - 1) // bs
    b = rng.integers(0, 256, (n, nb, bs // 2), dtype=np.uint8)
    s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float32)
    zp = rng.integers(0, 256, (n, (nb + 1) // 2), dtype=np.uint8)
    return (b, s, zp), ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=bs)


@pytest.mark.parametrize("k,n,bs,ms", [
    (1024, 3072, 128, (512, 100)),   # fp8 prefill, then a smaller prefill
    (3072, 1024, 128, (512, 40)),    # split-K partials in the scratch
    (2048, 512, 32, (16, 4)),        # 16-row decode (activation prepass)
    (1024, 2048, 128, (300, 1)),     # prefill, then the GEMV (no scratch)
])
def test_noalloc_matches_allocating_entry(ops, k, n, bs, ms):
    rng = np.random.default_rng(0x5EED0030 + k + n)
    (b, s, zp), w = _weight(ops, rng, k, n, bs)
    for m in ms:
        a = rng.standard_normal((m, k)).astype(np.float32)
        ad = ops.DeviceBuffer.from_array(a)
        y_ref = ops.DeviceBuffer.from_array(np.full((m, n), np.nan, np.float32))
        y_na = ops.DeviceBuffer.from_array(np.full((m, n), np.nan, np.float32))
        w.run_dev(ad.ptr, m, y_ref.ptr)
        w.run_dev_noalloc(ad.ptr, m, y_na.ptr)
        want = y_ref.to_array((m, n), np.float32)
        got = y_na.to_array((m, n), np.float32)
        np.testing.assert_array_equal(got, want)
        cols = np.arange(0, n, max(1, n // 96))
        ref = oracle.matmul_nbits(a, b[cols], s[cols], zp[cols], k=k, n=len(cols),
                                  block_size=bs)
        assert G.rms_error(got[:, cols], ref) <= TOL
        for buf in (ad, y_ref, y_na):
            buf.free()
    w.release()


def test_noalloc_rejects_requests_beyond_the_scratch(ops):
    from onnx_runtime_dart_amd.errors import ArgumentError
    rng = np.random.default_rng(0x5EED0031)
    _, w = _weight(ops, rng, 1024, 64, 128)
    buf = ops.DeviceBuffer(4096)
    with pytest.raises(ArgumentError, match="scratch"):
        w.run_dev_noalloc(buf.ptr, 1 << 16, buf.ptr)  # 65536 rows: > 32 MiB of workspace
    buf.free()
    w.release()
