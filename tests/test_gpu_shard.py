"""Column shards on one GPU: the part of the reference's pool invariant
(parallel_pool_test.dart:27-111: an N-split of the weight gives bitwise the
unsplit result) that a multi-GPU N-split relies on.  Each weight is cut into W
column slices with the pool's rule (n / W each, the first n % W one more,
lib/src/parallel_pool.dart:233-239), every slice runs as its own weight, and
the stitched outputs must equal bitwise the full weight's launch.  The shapes
are ones whose launch plan (tile widths, K split, waves per column group) is
the same for a slice as for the whole weight; that is what makes the float
sums identical."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from onnx_runtime_dart_amd import ops as _ops
    return _ops


def pool_split(n, workers):
    base, rem = divmod(n, workers)
    counts = [base + (1 if w < rem else 0) for w in range(workers)]
    starts = np.cumsum([0] + counts[:-1])
    return list(zip(starts, counts))


@pytest.mark.parametrize("m", [512, 1])
def test_nbits_lm_head_shards(ops, m):
    rng = np.random.default_rng(0x5EED0040 + m)
    k, n, bs, workers = 1024, 151936, 128, 8
    nb = k // bs
    b = rng.integers(0, 256, (n, nb, bs // 2), dtype=np.uint8)
    s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float32)
    zp = rng.integers(0, 256, (n, (nb + 1) // 2), dtype=np.uint8)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=bs)
    full = w(a)
    w.release()
    stitched = np.empty_like(full)
    for c0, cnt in pool_split(n, workers):
        ws = ops.NBitsWeight(b[c0:c0 + cnt], s[c0:c0 + cnt], zp[c0:c0 + cnt], k=k, n=cnt,
                             block_size=bs)
        stitched[:, c0:c0 + cnt] = ws(a)
        ws.release()
    np.testing.assert_array_equal(stitched, full)


def test_int8_lm_head_shards(ops):
    rng = np.random.default_rng(0x5EED0041)
    m, k, n, workers = 512, 1024, 151936, 8
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    w = ops.Int8Weight(b, np.array(0))
    full = w.matmul_integer(a, np.array(128))
    w.release()
    stitched = np.empty_like(full)
    for c0, cnt in pool_split(n, workers):
        ws = ops.Int8Weight(np.ascontiguousarray(b[:, c0:c0 + cnt]), np.array(0))
        stitched[:, c0:c0 + cnt] = ws.matmul_integer(a, np.array(128))
        ws.release()
    np.testing.assert_array_equal(stitched, full)


@pytest.mark.parametrize("workers", [2, 8])
def test_f32_ffn_shards(ops, workers):
    # MiniLM FFN1 (config C3): [4096, 384] x [1536, 384]^T + bias.
    rng = np.random.default_rng(0x5EED0042)
    m, k, n = 4096, 384, 1536
    x = rng.standard_normal((m, k)).astype(np.float32)
    wt = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    c = (rng.standard_normal(n) * 0.02).astype(np.float32)
    fw = ops.F32Weight(wt, trans_b=True)
    full = fw.gemm(x, c)
    fw.release()
    stitched = np.empty_like(full)
    for c0, cnt in pool_split(n, workers):
        fs = ops.F32Weight(np.ascontiguousarray(wt[c0:c0 + cnt]), trans_b=True)
        stitched[:, c0:c0 + cnt] = fs.gemm(x, c[c0:c0 + cnt])
        fs.release()
    np.testing.assert_array_equal(stitched, full)
