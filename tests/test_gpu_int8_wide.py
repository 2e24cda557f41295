"""MatMulInteger on outputs of many column tiles (the Qwen lm_head shape and
its ragged neighbours): ragged M and N, one and two 256-row tiles, K below
and above one 256-k stage and not a multiple of it, every sign combination,
and scalar, per-row and per-column zero points, including per-row zero
points beyond the byte range.  Results are bit-exact against the oracle on
column subsets, and exact int64 row and column sums of the whole output pin
every other element."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


def _cols(n):
    mid = n // 2 - 50
    return np.unique(np.concatenate([np.arange(0, 100), np.arange(mid, mid + 100),
                                     np.arange(n - 130, n)]))


CASES = [
    # (M, K, N, A signed, B signed, a zero point, b zero point)
    (300, 256, 131000 + 37, False, True, "row", "col"),    # ragged M, N; one stage
    (512, 1000, 131072 + 5, True, False, "scalar", "scalar"),  # K padded to 1024
    (200, 512, 262144 + 100, False, False, "none", "col"),  # one row tile of 256
    (512, 1024, 151936, False, True, "row", "none"),        # lm_head shape
    (260, 384, 140000, True, True, "scalar", "col"),        # 4 rows in the second tile
    (512, 1024, 151936, False, True, "wide", "scalar"),     # per-row zp beyond a byte
]


def _zp(rng, mode, n, signed):
    if mode == "none":
        return None
    if mode == "scalar":
        return np.array(rng.integers(-128, 128) if signed else rng.integers(0, 256))
    return rng.integers(-128, 128, n) if signed else rng.integers(0, 256, n)


@pytest.mark.parametrize("m,k,n,sa,sb,azm,bzm", CASES)
def test_wide_matmul_integer_exact(ops, m, k, n, sa, sb, azm, bzm):
    print(f"case m={m} k={k} n={n} sa={sa} sb={sb} azp={azm} bzp={bzm}", flush=True)
    rng = np.random.default_rng(0x5EED00A0 + m + k + n)
    a = rng.integers(-128 if sa else 0, 128 if sa else 256, (m, k)).astype(
        np.int8 if sa else np.uint8)
    b = rng.integers(-128 if sb else 0, 128 if sb else 256, (k, n)).astype(
        np.int8 if sb else np.uint8)
    az = rng.integers(250, 400, m) if azm == "wide" else _zp(rng, azm, m, sa)
    bz = _zp(rng, bzm, n, sb)
    w = ops.Int8Weight(b, bz)
    y = w.matmul_integer(a, az)
    assert y.shape == (m, n)
    cols = _cols(n)
    bzc = None if bz is None else (bz if bz.ndim == 0 else bz[cols])
    np.testing.assert_array_equal(y[:, cols],
                                  oracle.matmul_integer(a, b[:, cols].copy(), az, bzc))
    ac = a.astype(np.int64) - (0 if az is None else np.asarray(az, np.int64).reshape(-1, 1))
    bc = b.astype(np.int64) - (0 if bz is None else np.asarray(bz, np.int64).reshape(1, -1))
    yl = y.astype(np.int64)
    np.testing.assert_array_equal(yl.sum(axis=1), ac @ bc.sum(axis=1))
    np.testing.assert_array_equal(yl.sum(axis=0), ac.sum(axis=0) @ bc)
    w.release()


def test_wide_dev_call_twice_matches_host_call(ops):
    # Device-pointer calls (the session layer's form) on the lm_head shape,
    # two in a row into one output buffer: bitwise the host call's result.
    rng = np.random.default_rng(0x5EED00A1)
    m, k, n = 512, 1024, 151936
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    w = ops.Int8Weight(b, np.array(0))
    ref = w.matmul_integer(a, np.array(128))
    ad = ops.DeviceBuffer.from_array(a)
    yd = ops.DeviceBuffer(m * n * 4)
    for _ in range(2):
        w.matmul_integer_dev(ad.ptr, False, m, yd.ptr, np.array([128], np.int32))
        np.testing.assert_array_equal(yd.to_array((m, n), np.int32), ref)
    ad.free()
    yd.free()
    w.release()
