"""CPU checks of the fp32 MatMul batch planner (no device): output shapes and
the per-batch operand offsets the kernels use, against numpy broadcasting of
index arrays (lib/src/onnx_ops.dart:1717-1722, :1728-1735, :1742-1764)."""
import numpy as np
import pytest

from onnx_runtime_dart_amd import ops
from onnx_runtime_dart_amd.errors import ArgumentError


def numpy_offsets(a_shape, b_shape):
    """Offsets of every output batch from numpy broadcasting of batch-index
    arrays; the shared-weight collapse gives one batch at offsets 0."""
    m, k = a_shape[-2:]
    n = b_shape[-1]
    ab, bb = tuple(a_shape[:-2]), tuple(b_shape[:-2])
    ob = np.broadcast_shapes(ab, bb)
    if int(np.prod(bb, dtype=np.int64)) == 1 and int(np.prod(ob, dtype=np.int64)) > 1:
        return np.zeros(1, np.int64), np.zeros(1, np.int64)
    ai = np.broadcast_to(np.arange(int(np.prod(ab, dtype=np.int64))).reshape(ab), ob).ravel()
    bi = np.broadcast_to(np.arange(int(np.prod(bb, dtype=np.int64))).reshape(bb), ob).ravel()
    return ai * m * k, bi * k * n


def random_pair(rng, rank_max=7):
    r = int(rng.integers(0, rank_max + 1))
    ob = [int(rng.integers(1, 4)) for _ in range(r)]
    ra = int(rng.integers(0, r + 1))
    rb = int(rng.integers(0, r + 1))
    a = [d if rng.random() < 0.6 else 1 for d in ob[r - ra:]]
    b = [d if rng.random() < 0.6 else 1 for d in ob[r - rb:]]
    m, k, n = (int(x) for x in rng.integers(1, 6, 3))
    return a + [m, k], b + [k, n]


CASES = [
    ([2, 3, 5, 7], [2, 3, 7, 4]),          # equal batch dims (matmul_batched fixture)
    ([32, 12, 128, 32], [32, 12, 32, 128]),  # attention scores
    ([2, 1, 4, 3], [3, 3, 5]),              # [2,1] x [3] -> [2,3]
    ([1, 4, 3], [6, 3, 5]),                 # A broadcast over B's batch
    ([6, 4, 3], [3, 5]),                    # shared-weight collapse
    ([6, 4, 3], [1, 1, 3, 5]),              # collapse through size-1 dims of B
    ([2, 1, 2, 1, 2, 1, 3, 2], [1, 2, 1, 2, 1, 2, 2, 4]),  # 6 alternating dims
    ([2, 1, 2, 1, 2, 1, 2, 1, 3, 2], [1, 2, 1, 2, 1, 2, 1, 2, 2, 4]),  # 8 dims
    ([3, 1, 1, 2, 4, 5], [1, 2, 2, 1, 5, 6]),
    ([1, 1, 2, 3], [1, 1, 3, 2]),
]


@pytest.mark.parametrize("a_shape,b_shape", CASES)
def test_batch_offsets_match_numpy_broadcasting(a_shape, b_shape):
    ao, bo = ops.matmul_f32_batch_offsets(a_shape, b_shape)
    ra, rb = numpy_offsets(a_shape, b_shape)
    np.testing.assert_array_equal(ao, ra)
    np.testing.assert_array_equal(bo, rb)


def test_batch_offsets_random_shapes():
    rng = np.random.default_rng(0x5EED0010)
    for _ in range(400):
        a_shape, b_shape = random_pair(rng)
        ao, bo = ops.matmul_f32_batch_offsets(a_shape, b_shape)
        ra, rb = numpy_offsets(a_shape, b_shape)
        np.testing.assert_array_equal(ao, ra, err_msg=f"{a_shape} x {b_shape}")
        np.testing.assert_array_equal(bo, rb, err_msg=f"{a_shape} x {b_shape}")


def test_batch_offsets_subrange():
    a_shape, b_shape = [2, 1, 2, 1, 2, 1, 3, 2], [1, 2, 1, 2, 1, 2, 2, 4]
    ra, rb = numpy_offsets(a_shape, b_shape)
    ao, bo = ops.matmul_f32_batch_offsets(a_shape, b_shape, 17, 30)
    np.testing.assert_array_equal(ao, ra[17:47])
    np.testing.assert_array_equal(bo, rb[17:47])
    with pytest.raises(ArgumentError):
        ops.matmul_f32_batch_offsets(a_shape, b_shape, 60, 10)


def test_output_shape():
    rng = np.random.default_rng(0x5EED0011)
    for a_shape, b_shape in CASES + [random_pair(rng) for _ in range(100)]:
        want = tuple(np.broadcast_shapes(tuple(a_shape[:-2]), tuple(b_shape[:-2]))) + (
            a_shape[-2], b_shape[-1])
        assert ops.matmul_f32_output_shape(a_shape, b_shape) == want


@pytest.mark.parametrize("a_shape,b_shape", [([2, 4, 3], [3, 4, 5]),   # batch 2 vs 3
                                             ([4, 3], [2, 5]),         # inner dims
                                             ([3], [3, 5])])           # rank 1
def test_planner_rejects_what_the_reference_rejects(a_shape, b_shape):
    with pytest.raises(ArgumentError):
        ops.matmul_f32_output_shape(a_shape, b_shape)
