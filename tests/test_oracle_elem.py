"""The oracle's elementwise restatements (Add/Sub/Mul/Div with broadcasting,
Sigmoid, RMSNorm) against the reference's ORT fixtures and closed forms.

Pins: a float op computed in double and rounded once to f32 equals the
correctly rounded f32 op (53 >= 2 * 24 + 2 bits), so numpy's float32
arithmetic must agree bitwise; RMSNorm against a float64 numpy formula with
gamma broadcast along the last axis for every reduce axis (a gamma indexed
along the reduce axis, or a mean over the wrong axis, fails it)."""
import numpy as np
import pytest

import golden_io as G
import oracle


def ulps(a, b):
    a = np.asarray(a, np.float32).ravel().view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).ravel().view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max()) if a.size else 0


@pytest.mark.parametrize("name", ["add_bias_broadcast_lastdim", "add_broadcast_middle"])
def test_add_fixtures(name):
    d = G.load(name)
    a, b = d["arrays"]
    y = oracle.binary_f32("add", a, b)
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], name)
    np.testing.assert_array_equal(y, a + b)


def test_rmsnorm_pattern_fixture():
    d = G.load("rmsnorm_pattern")
    x, g = d["arrays"]
    y = oracle.rms_norm_f32(x, g, d["attrs"]["axis"], d["attrs"]["epsilon"])
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], "rmsnorm_pattern")


def test_skip_simplified_layer_norm_fixture():
    # SkipSimplifiedLayerNormalization = Add then RMSNorm over the last axis
    # (lib/src/onnx_graph.dart:1793-1813); out3 is the sum.
    d = G.load("skipsimplifiedlayernorm")
    x, skip, w = d["arrays"]
    s = oracle.binary_f32("add", x, skip)
    y = oracle.rms_norm_f32(s, w, -1, d["attrs"]["epsilon"])
    G.assert_reference_parity(y, d["want"]["out0"], "skipsimplifiedlayernorm out0")
    G.assert_reference_parity(s, d["want"]["out3"], "skipsimplifiedlayernorm out3")


def test_glu_gate_fixture():
    # _FusedGlu: a * sigmoid(b) for the two halves of x along axis.
    d = G.load("glu_gate")
    (x,) = d["arrays"]
    a, b = np.split(x, 2, axis=d["attrs"]["axis"])
    y = oracle.binary_f32("mul", a, oracle.sigmoid_f32(b))
    G.assert_reference_parity(y, d["want"][d["outputs"][0]], "glu_gate")


SHAPES = [((2, 3, 4), (2, 3, 4)), ((2, 3, 4), ()), ((), (5,)), ((2, 1, 4, 3), (5, 1, 3)),
          ((4, 1), (1, 6)), ((3, 5, 8), (8,)), ((3, 5, 8), (3, 5, 1)), ((1, 7), (3, 1, 1)),
          ((2, 0, 3), (1, 3)), ((2, 1, 2, 1, 2, 1, 2), (1, 2, 1, 2, 1, 2, 1))]


@pytest.mark.parametrize("op,npop", [("add", np.add), ("sub", np.subtract),
                                     ("mul", np.multiply), ("div", np.divide)])
@pytest.mark.parametrize("sa,sb", SHAPES)
def test_binary_matches_float32_arithmetic(op, npop, sa, sb):
    rng = np.random.default_rng(7)
    a = rng.standard_normal(sa).astype(np.float32)
    b = (rng.standard_normal(sb) + 3).astype(np.float32)
    y = oracle.binary_f32(op, a, b)
    want = npop(a, b)
    assert y.shape == want.shape
    np.testing.assert_array_equal(y, want)


def test_binary_rejects_incompatible_shapes():
    with pytest.raises(oracle.OracleError):
        oracle.binary_f32("add", np.zeros((2, 3), np.float32), np.zeros((4,), np.float32))


def test_sigmoid_closed_form():
    x = np.concatenate([np.linspace(-30, 30, 1001), [0.0, -0.0, 1e-30, 88.0, -88.0, -104.0,
                                                     np.inf, -np.inf]]).astype(np.float32)
    y = oracle.sigmoid_f32(x)
    want = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    assert ulps(y, want) <= 1
    assert set(y[x == 0].tolist()) == {0.5}
    assert y[-2] == 1.0 and y[-1] == 0.0
    assert np.isnan(oracle.sigmoid_f32(np.array([np.nan], np.float32)))[0]


@pytest.mark.parametrize("shape,axis", [((4, 16), -1), ((2, 5, 16), 2), ((3, 4, 6), 0),
                                        ((3, 4, 6), 1), ((7,), 0), ((2, 3, 1), -1)])
def test_rms_norm_closed_form(shape, axis):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(shape).astype(np.float32)
    g = rng.uniform(0.5, 2.0, shape[-1]).astype(np.float32)
    eps = 1e-6
    y = oracle.rms_norm_f32(x, g, axis, eps)
    xd = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xd * xd, axis=axis, keepdims=True) + eps)
    want = (xd * inv * g.astype(np.float64)).astype(np.float32)
    assert ulps(y, want) <= 1


def test_rms_norm_rejects_gamma_of_another_length():
    with pytest.raises(oracle.OracleError):
        oracle.rms_norm_f32(np.zeros((2, 4), np.float32), np.ones(3, np.float32), -1, 1e-5)
