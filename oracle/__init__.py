"""CPU oracle for the matmul operator family — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package, and only as the checker (or the timed CPU baseline).  The
product package ``onnx_runtime_dart_amd`` never imports it.

Thin numpy wrappers over ``oracle/lib/liboracle.so`` (built from oracle.c by
``make -C oracle``); each wrapper mirrors the reference op it restates:

* ``matmul_nbits``         — lib/src/onnx_qlinear_ops.dart:115-228
* ``matmul_integer``       — lib/src/onnx_qlinear_ops.dart:32-81
* ``qlinear_matmul``       — lib/src/onnx_qlinear_ops.dart:85-108
* ``dynamic_quantize_linear`` — lib/src/onnx_ops.dart:3556-3583
* ``matmul_f32``           — lib/src/onnx_ops.dart:1710-1766
* ``gemm_f32``             — lib/src/onnx_ops.dart:2152-2172
* ``matmul_kernel``        — lib/src/gemm_kernel_simd.dart:32-239
* ``fused_sdpa``           — lib/src/onnx_ops.dart:2106-2149
* ``multi_head_attention`` — lib/src/onnx_ops.dart:2019-2098
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "lib" / "liboracle.so"

OK, INVALID_ARGUMENT, UNSUPPORTED = 0, 1, 2


class OracleError(Exception):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: oracle status {status}")
        self.status = status


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


_P = C.c_void_p
_I64 = C.c_int64
_I = C.c_int


def _declare(L):
    L.orc_matmul_kernel.argtypes = [_P, _P, _P, _I64, _I64, _I64]
    L.orc_matmul_kernel.restype = None
    L.orc_matmul_f32.argtypes = [_P, _P, _I, _P, _P, _I, _P]
    L.orc_gemm_f32.argtypes = [_P, _P, _P, _P, _P, _P, _I, C.c_double,
                               C.c_double, _I, _I, _P]
    L.orc_matmul_nbits.argtypes = [_P, _I64, _I64, _I64, _I64, _I64, _P, _P,
                                   _I, _P, _P, _P]
    L.orc_nbits_weight.argtypes = [_I64, _I64, _I64, _I64, _P, _P, _I, _P]
    L.orc_nbits_weight.restype = C.c_float
    L.orc_matmul_integer.argtypes = [_P, _I, _I64, _P, _I, _I64, _I64, _I64,
                                     _I64, _P, _I64, _P, _I64, _P]
    L.orc_qlinear_matmul.argtypes = [_P, _I, _I64, _P, _I, _I64, _I64, _I64,
                                     _I64, C.c_float, _P, _I64, C.c_float, _P,
                                     _I64, C.c_float, C.c_int32, C.c_int32,
                                     C.c_int32, _P]
    L.orc_dynamic_quantize_linear.argtypes = [_P, _I64, _P, _P, _P]
    L.orc_fused_sdpa.argtypes = [_P, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, C.c_double,
                                 _P]
    L.orc_multi_head_attention.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64,
                                           _I, C.c_double, _P]
    L.orc_round_even.argtypes = [C.c_double, _P]
    L.orc_round_even.restype = _I64


def _ptr(x):
    return None if x is None else x.ctypes.data_as(C.c_void_p)


def _shape(a):
    return np.ascontiguousarray(np.array(a.shape if a.ndim else [], dtype=np.int64))


def _check(st, what):
    if st != OK:
        raise OracleError(st, what)


def round_even(v: float) -> int:
    err = C.c_int(0)
    r = lib().orc_round_even(float(v), C.byref(err))
    _check(err.value, "round_even")
    return int(r)


def matmul_kernel(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_kernel(_ptr(a), _ptr(b), _ptr(out), m, k, n)
    return out


def _broadcast(x, y):
    return list(np.broadcast_shapes(tuple(x), tuple(y)))


def matmul_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out_shape = _broadcast(a.shape[:-2], b.shape[:-2]) + [a.shape[-2], b.shape[-1]]
    y = np.empty(out_shape, dtype=np.float32)
    sa, sb = _shape(a), _shape(b)
    _check(lib().orc_matmul_f32(_ptr(a), _ptr(sa), a.ndim, _ptr(b), _ptr(sb),
                                b.ndim, _ptr(y)), "matmul_f32")
    return y


def gemm_f32(a, b, c=None, *, alpha=1.0, beta=1.0, trans_a=False,
             trans_b=False) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m = a.shape[1] if trans_a else a.shape[0]
    n = b.shape[0] if trans_b else b.shape[1]
    y = np.empty((m, n), dtype=np.float32)
    if c is not None:
        c = np.ascontiguousarray(c, dtype=np.float32)
        sc = _shape(c)
    else:
        sc = None
    sa, sb = _shape(a), _shape(b)
    _check(lib().orc_gemm_f32(_ptr(a), _ptr(sa), _ptr(b), _ptr(sb), _ptr(c),
                              _ptr(sc), 0 if c is None else c.ndim,
                              float(np.float32(alpha)), float(np.float32(beta)),
                              int(bool(trans_a)), int(bool(trans_b)), _ptr(y)),
           "gemm_f32")
    return y


def _zp_kind(zp):
    if zp is None:
        return 0, None
    if zp.dtype == np.uint8:
        return 1, np.ascontiguousarray(zp)
    return 2, np.ascontiguousarray(zp, dtype=np.float32)


def matmul_nbits(a, b_q, scales, zero_points=None, *, k, n, bits=4,
                 block_size, bias=None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    kind, zp = _zp_kind(zero_points)
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
    m = a.size // k
    y = np.empty(a.shape[:-1] + (n,), dtype=np.float32)
    _check(lib().orc_matmul_nbits(_ptr(a), m, k, n, bits, block_size,
                                  _ptr(b_q), _ptr(scales), kind, _ptr(zp),
                                  _ptr(bias), _ptr(y)), "matmul_nbits")
    return y


def nbits_dequant(b_q, scales, zero_points=None, *, k, n, block_size):
    """Full dequantized weight [N, K] (the reference's `weight` closure)."""
    b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    kind, zp = _zp_kind(zero_points)
    L = lib()
    w = np.empty((n, k), dtype=np.float32)
    for col in range(n):
        for kk in range(k):
            w[col, kk] = L.orc_nbits_weight(col, kk, k, block_size, _ptr(b_q),
                                            _ptr(scales), kind, _ptr(zp))
    return w


def _zp_arr(z):
    if z is None:
        return None, 0
    z = np.ascontiguousarray(np.asarray(z).astype(np.int32).ravel())
    return z, z.size


def matmul_integer(a, b, a_zp=None, b_zp=None) -> np.ndarray:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.dtype in (np.uint8, np.int8) and b.dtype in (np.uint8, np.int8)
    m, k = a.shape[-2:]
    n = b.shape[-1]
    ab, bb = a.size // (m * k), b.size // (k * n)
    batch = max(ab, bb)
    za, la = _zp_arr(a_zp)
    zb, lb = _zp_arr(b_zp)
    y = np.empty(batch * m * n, dtype=np.int64)
    _check(lib().orc_matmul_integer(_ptr(a), int(a.dtype == np.int8), ab,
                                    _ptr(b), int(b.dtype == np.int8), bb, m, k,
                                    n, _ptr(za), la, _ptr(zb), lb, _ptr(y)),
           "matmul_integer")
    out_batch = a.shape[:-2] if ab >= bb else b.shape[:-2]
    return y.reshape(tuple(out_batch) + (m, n))


def qlinear_matmul(a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, *, lo,
                   hi) -> np.ndarray:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    m, k = a.shape[-2:]
    n = b.shape[-1]
    ab, bb = a.size // (m * k), b.size // (k * n)
    batch = max(ab, bb)
    za, la = _zp_arr(a_zp)
    zb, lb = _zp_arr(b_zp)
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    y = np.empty(batch * m * n, dtype=np.int64)
    _check(lib().orc_qlinear_matmul(
        _ptr(a), int(a.dtype == np.int8), ab, _ptr(b), int(b.dtype == np.int8),
        bb, m, k, n, float(np.float32(a_scale)), _ptr(za), la,
        float(np.float32(b_scale)), _ptr(zb), lb, float(np.float32(y_scale)),
        yz, lo, hi, _ptr(y)), "qlinear_matmul")
    out_batch = a.shape[:-2] if ab >= bb else b.shape[:-2]
    return y.reshape(tuple(out_batch) + (m, n))


def dynamic_quantize_linear(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint8)
    scale = np.zeros(1, dtype=np.float32)
    zp = np.zeros(1, dtype=np.int32)
    _check(lib().orc_dynamic_quantize_linear(_ptr(x), x.size, _ptr(y),
                                             _ptr(scale), _ptr(zp)),
           "dynamic_quantize_linear")
    return y, np.float32(scale[0]), int(zp[0])


__all__ = [n for n in dir() if not n.startswith("_")]
_ = os  # keep import for callers that inspect LIB_PATH via os.path


def fused_sdpa(a, b, v, mask, scale: float) -> np.ndarray:
    a, b, v, mask = (np.ascontiguousarray(x, dtype=np.float32) for x in (a, b, v, mask))
    sb = _broadcast(a.shape[:-2], b.shape[:-2])
    ob = _broadcast(sb, v.shape[:-2])
    y = np.empty(ob + [a.shape[-2], v.shape[-1]], dtype=np.float32)
    _check(lib().orc_fused_sdpa(_ptr(a), _ptr(_shape(a)), a.ndim, _ptr(b), _ptr(_shape(b)),
                                b.ndim, _ptr(v), _ptr(_shape(v)), v.ndim, _ptr(mask),
                                _ptr(_shape(mask)), mask.ndim, float(scale), _ptr(y)),
           "fused_sdpa")
    return y


def multi_head_attention(q, k, v, bias=None, *, num_heads: int, scale=None) -> np.ndarray:
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    batch, seq, hidden = q.shape
    kv_seq = k.shape[1]
    bh = 0
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        bh = bias.shape[1]
    out = np.empty_like(q)
    _check(lib().orc_multi_head_attention(_ptr(q), _ptr(k), _ptr(v), batch, seq, kv_seq, hidden,
                                          num_heads, _ptr(bias), bh, int(scale is not None),
                                          float(scale or 0.0), _ptr(out)),
           "multi_head_attention")
    return out
