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
* ``GemmPool``             — lib/src/parallel_pool.dart:217-261, :299-329
* ``fused_sdpa``           — lib/src/onnx_ops.dart:2106-2149
* ``multi_head_attention`` — lib/src/onnx_ops.dart:2019-2098
* ``group_query_attention`` — lib/src/onnx_ops.dart:1844-2012
* ``rotary_embedding``     — lib/src/onnx_ops.dart:2659-2722
* ``conv``                 — lib/src/onnx_nn_ops.dart:179-817 (+ _resolvePads :38-87)
* ``conv_transpose``       — lib/src/onnx_nn_ops.dart:818-1059
* ``conv_integer``         — lib/src/onnx_qlinear_ops.dart:232-337
* ``qlinear_conv``         — lib/src/onnx_qlinear_ops.dart:339-382
* ``binary_f32``           — lib/src/onnx_ops.dart:26-44, :103-330 (Add/Sub/Mul/Div)
* ``sigmoid_f32``          — lib/src/onnx_ops.dart:2349-2350
* ``rms_norm_f32``         — lib/src/onnx_ops.dart:1771-1815
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# ORACLE_LIBRARY selects another build of oracle.c (the sanitizer build,
# lib/liboracle_san.so, under tests/test_sanitizers.py).
LIB_PATH = Path(os.environ.get("ORACLE_LIBRARY", HERE / "lib" / "liboracle.so"))

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
    L.orc_pool_create.argtypes = [_P, _I64, _I64, C.c_int]
    L.orc_pool_create.restype = C.c_void_p
    L.orc_pool_matmul.argtypes = [C.c_void_p, _P, _I64, _P]
    L.orc_pool_destroy.argtypes = [C.c_void_p]
    L.orc_pool_destroy.restype = None
    L.orc_matmul_f32.argtypes = [_P, _P, _I, _P, _P, _I, _P]
    L.orc_matmul_f64acc.argtypes = [_P, _P, _I, _P, _P, _I, _P]
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
    L.orc_conv.argtypes = [_P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I,
                           C.c_int32, _P, _P]
    L.orc_rotary_embedding.argtypes = [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _I, _P]
    L.orc_rotary_embedding.restype = None
    L.orc_group_query_attention.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P,
                                            _I64, _P, _P, _I64, _I, _I, _P, _I64, _I,
                                            C.c_double, _P, _P, _P]
    L.orc_round_even.argtypes = [C.c_double, _P]
    L.orc_binary_f32.argtypes = [_I, _P, _P, _I, _P, _P, _I, _P, _P]
    L.orc_sigmoid_f32.argtypes = [_P, _I64, _P]
    L.orc_sigmoid_f32.restype = None
    L.orc_rms_norm_f32.argtypes = [_P, _P, _I, _P, _I64, _I64, C.c_double, _P]
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


class GemmPool:
    """The reference's isolate pool for one f32 weight b [k, n]
    (lib/src/parallel_pool.dart:217-261, :299-329) with threads as workers."""

    def __init__(self, b: np.ndarray, workers: int):
        self.b = np.ascontiguousarray(b, dtype=np.float32)
        self.k, self.n = self.b.shape
        self.handle = lib().orc_pool_create(_ptr(self.b), self.k, self.n, int(workers))
        if not self.handle:
            raise OracleError(INVALID_ARGUMENT, "orc_pool_create")

    def matmul(self, a: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        m = a.shape[0]
        y = np.empty((m, self.n), dtype=np.float32)
        _check(lib().orc_pool_matmul(self.handle, _ptr(a), m, _ptr(y)), "pool_matmul")
        return y

    def close(self):
        if self.handle:
            lib().orc_pool_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


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


def matmul_f64acc(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """opMatMul on non-float operands (lib/src/onnx_ops.dart:1753-1762): the
    operands as doubles (getD), a double sum over k per output, f32 result."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    b = np.ascontiguousarray(b, dtype=np.float64)
    out_shape = _broadcast(a.shape[:-2], b.shape[:-2]) + [a.shape[-2], b.shape[-1]]
    y = np.empty(out_shape, dtype=np.float32)
    sa, sb = _shape(a), _shape(b)
    _check(lib().orc_matmul_f64acc(_ptr(a), _ptr(sa), a.ndim, _ptr(b), _ptr(sb),
                                   b.ndim, _ptr(y)), "matmul_f64acc")
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


# ------------------------------------------------------------------ conv

def resolve_pads(in_dims, kernel, strides, dilations, auto_pad="NOTSET", pads=None):
    """_resolvePads (lib/src/onnx_nn_ops.dart:38-87, ceil_mode off): begin /
    end pads and output dims per spatial axis.  Integer division truncates
    towards zero, as Dart's ``~/``."""
    nd = len(in_dims)
    p = [0] * (2 * nd)
    out = [0] * nd
    for k in range(nd):
        window = dilations[k] * (kernel[k] - 1) + 1
        if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
            out[k] = -(-in_dims[k] // strides[k])
            total = max(0, (out[k] - 1) * strides[k] + window - in_dims[k])
            small = total // 2
            p[k] = small if auto_pad == "SAME_UPPER" else total - small
            p[nd + k] = total - p[k]
        elif auto_pad == "VALID":
            out[k] = int((in_dims[k] - window) / strides[k]) + 1
        else:
            p[k] = 0 if pads is None else pads[k]
            p[nd + k] = 0 if pads is None else pads[nd + k]
            out[k] = int((in_dims[k] + p[k] + p[nd + k] - window) / strides[k]) + 1
    return p, out


def _conv_sums(x, x_kind, w, w_kind, n, c, m, group, in_sp, ker, out, st, dl, pb, trans,
               x_zp=0, w_zp=None):
    nd = len(in_sp)
    pad3 = lambda v, fill: [fill] * (3 - nd) + list(v)  # noqa: E731
    arr = lambda v: np.ascontiguousarray(np.array(v, dtype=np.int64))  # noqa: E731
    acc = np.zeros((n, m) + tuple(out), dtype=np.float64)
    wz = None if w_zp is None else np.ascontiguousarray(np.asarray(w_zp, np.int32))
    _check(lib().orc_conv(_ptr(x), x_kind, _ptr(w), w_kind, n, c, m, group,
                          _ptr(arr(pad3(in_sp, 1))), _ptr(arr(pad3(ker, 1))),
                          _ptr(arr(pad3(out, 1))), _ptr(arr(pad3(st, 1))),
                          _ptr(arr(pad3(dl, 1))), _ptr(arr(pad3(pb, 0))), int(trans),
                          int(x_zp), _ptr(wz), _ptr(acc)), "orc_conv")
    return acc


def conv(x, w, bias=None, *, strides=None, pads=None, dilations=None, group=1,
         auto_pad="NOTSET") -> np.ndarray:
    """opConv: sums in double, bias added, one rounding to f32."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    nd = x.ndim - 2
    st = list(strides) if strides is not None else [1] * nd
    dl = list(dilations) if dilations is not None else [1] * nd
    p, out = resolve_pads(list(x.shape[2:]), list(w.shape[2:]), st, dl, auto_pad, pads)
    acc = _conv_sums(x, 0, w, 0, x.shape[0], x.shape[1], w.shape[0], group, list(x.shape[2:]),
                     list(w.shape[2:]), out, st, dl, p[:nd], 0)
    if bias is not None:
        acc += np.asarray(bias, np.float64).reshape((1, -1) + (1,) * nd)
    return acc.astype(np.float32)


def conv_transpose_dims(in_sp, kernel, strides, dilations, output_padding=None,
                        output_shape=None, pads=None):
    """Output dims and begin pads of opConvTranspose
    (lib/src/onnx_nn_ops.dart:976-995)."""
    nd = len(in_sp)
    op = list(output_padding) if output_padding is not None else [0] * nd
    p = list(pads) if pads is not None else [0] * (2 * nd)
    out = [0] * nd
    for k in range(nd):
        full = (in_sp[k] - 1) * strides[k] + dilations[k] * (kernel[k] - 1) + 1 + op[k]
        if output_shape is not None:
            out[k] = output_shape[len(output_shape) - nd + k]
            total = full - out[k]
            p[nd + k] = int(total / 2)
            p[k] = total - p[nd + k]
        else:
            out[k] = full - p[k] - p[nd + k]
    return p[:nd], out


def conv_transpose(x, w, bias=None, *, strides=None, pads=None, dilations=None,
                   output_padding=None, output_shape=None, group=1) -> np.ndarray:
    """opConvTranspose: scatter sums in double, bias added, one rounding."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    nd = x.ndim - 2
    st = list(strides) if strides is not None else [1] * nd
    dl = list(dilations) if dilations is not None else [1] * nd
    pb, out = conv_transpose_dims(list(x.shape[2:]), list(w.shape[2:]), st, dl, output_padding,
                                  output_shape, pads)
    m = w.shape[1] * group
    acc = _conv_sums(x, 0, w, 0, x.shape[0], x.shape[1], m, group, list(x.shape[2:]),
                     list(w.shape[2:]), out, st, dl, pb, 1)
    if bias is not None:
        acc += np.asarray(bias, np.float64).reshape((1, -1) + (1,) * nd)
    return acc.astype(np.float32)


def _kind(a):
    return {np.dtype(np.float32): 0, np.dtype(np.uint8): 1, np.dtype(np.int8): 2}[a.dtype]


def _wz_list(w_zp, m):
    if w_zp is None:
        return [0] * m
    z = np.asarray(w_zp).astype(np.int64).ravel()
    if z.size not in (1, m):
        raise OracleError(UNSUPPORTED, "weight zero point must be scalar or per-channel")
    return [int(z[0 if z.size == 1 else i]) for i in range(m)]


def conv_integer(x, w, x_zp=None, w_zp=None, *, strides=None, pads=None, dilations=None,
                 group=1) -> np.ndarray:
    """opConvInteger: exact sum (x - x_zp)(w - w_zp[m]) as int64."""
    x, w = np.ascontiguousarray(x), np.ascontiguousarray(w)
    nd = x.ndim - 2
    st = list(strides) if strides is not None else [1] * nd
    dl = list(dilations) if dilations is not None else [1] * nd
    p = list(pads) if pads is not None else [0] * (2 * nd)
    _, out = resolve_pads(list(x.shape[2:]), list(w.shape[2:]), st, dl, "NOTSET", p)
    xz = 0 if x_zp is None else int(np.asarray(x_zp).ravel()[0])
    acc = _conv_sums(x, _kind(x), w, _kind(w), x.shape[0], x.shape[1], w.shape[0], group,
                     list(x.shape[2:]), list(w.shape[2:]), out, st, dl, p[:nd], 0, xz,
                     _wz_list(w_zp, w.shape[0]))
    return acc.astype(np.int64)


def qlinear_conv(x, x_scale, x_zp, w, w_scale, w_zp, y_scale, y_zp, bias=None, *,
                 strides=None, pads=None, dilations=None, group=1, lo, hi) -> np.ndarray:
    """opQLinearConv: q = roundHalfEven((acc + bias[m]) * mult[m]) + y_zp,
    clamped; mult = x_scale * w_scale[m] / y_scale in double (the f32 scales
    widened, as Tensor.getD does)."""
    acc = conv_integer(x, w, x_zp, w_zp, strides=strides, pads=pads, dilations=dilations,
                       group=group)
    m = acc.shape[1]
    ws = np.asarray(w_scale, np.float32).ravel()
    xs = float(np.asarray(x_scale, np.float32).ravel()[0])
    ys = float(np.asarray(y_scale, np.float32).ravel()[0])
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    bi = None if bias is None else np.asarray(bias).astype(np.int64).ravel()
    out = np.empty_like(acc)
    for om in range(m):
        mult = xs * float(ws[0 if ws.size == 1 else om]) / ys
        s = acc[:, om] + (0 if bi is None else int(bi[om]))
        q = np.rint(s.astype(np.float64) * mult).astype(np.int64) + yz
        out[:, om] = np.clip(q, lo, hi)
    return out


# ------------------------------------------------------ GroupQueryAttention

def rotary_embedding(x, positions, cos_cache, sin_cache, *, num_heads, interleaved=False):
    """opRotaryEmbedding on [batch, seq, heads * hs] with one position row."""
    x = np.ascontiguousarray(x, np.float32)
    cos_cache = np.ascontiguousarray(cos_cache, np.float32)
    sin_cache = np.ascontiguousarray(sin_cache, np.float32)
    pos = np.ascontiguousarray(np.asarray(positions, np.int64).ravel())
    b, s, hidden = x.shape
    out = np.empty_like(x)
    lib().orc_rotary_embedding(_ptr(x), b, s, num_heads, hidden // num_heads, _ptr(pos),
                               _ptr(cos_cache), _ptr(sin_cache), cos_cache.shape[-1],
                               int(interleaved), _ptr(out))
    return out


def group_query_attention(q, k, v, *, num_heads, kv_num_heads, scale=None, do_rotary=False,
                          rotary_interleaved=False, past_key=None, past_value=None,
                          cos_cache=None, sin_cache=None, attention_bias=None):
    """opGroupQueryAttention -> [output, present_key, present_value]."""
    q, k, v = (np.ascontiguousarray(x, np.float32) for x in (q, k, v))
    b, s, hidden = q.shape
    hs = hidden // num_heads
    past = 0
    if past_key is not None and np.ndim(past_key) == 4:
        past_key = np.ascontiguousarray(past_key, np.float32)
        past_value = np.ascontiguousarray(past_value, np.float32)
        past = past_key.shape[2]
    else:
        past_key = past_value = None
    half = 0
    if do_rotary:
        cos_cache = np.ascontiguousarray(cos_cache, np.float32)
        sin_cache = np.ascontiguousarray(sin_cache, np.float32)
        half = cos_cache.shape[-1]
    bh = 0
    if attention_bias is not None:
        attention_bias = np.ascontiguousarray(attention_bias, np.float32)
        bh = attention_bias.shape[1]
    out = np.empty_like(q)
    pk = np.empty((b, kv_num_heads, past + s, hs), np.float32)
    pv = np.empty_like(pk)
    _check(lib().orc_group_query_attention(
        _ptr(q), _ptr(k), _ptr(v), b, s, hidden, num_heads, kv_num_heads, _ptr(past_key),
        _ptr(past_value), past, _ptr(cos_cache), _ptr(sin_cache), half, int(do_rotary),
        int(rotary_interleaved), _ptr(attention_bias), bh, int(scale is not None),
        float(scale or 0.0), _ptr(out), _ptr(pk), _ptr(pv)), "orc_group_query_attention")
    return [out, pk, pv]


BINARY_OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3}


def binary_f32(op: str, a, b) -> np.ndarray:
    """Add / Sub / Mul / Div of float tensors with broadcasting: op in double
    per element, one rounding to f32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    rank = max(a.ndim, b.ndim)
    out_shape = np.zeros(max(rank, 1), np.int64)
    try:
        shape = np.broadcast_shapes(a.shape, b.shape)
    except ValueError:
        shape = ()
    y = np.empty(max(int(np.prod(shape, dtype=np.int64)), 1), np.float32)
    st = lib().orc_binary_f32(BINARY_OPS[op], _ptr(a), _ptr(np.array(a.shape, np.int64)), a.ndim,
                              _ptr(b), _ptr(np.array(b.shape, np.int64)), b.ndim, _ptr(y),
                              _ptr(out_shape))
    _check(st, "binary_f32")
    return y[:int(np.prod(shape, dtype=np.int64))].reshape(tuple(int(d) for d in out_shape[:rank]))


def sigmoid_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_sigmoid_f32(_ptr(x), x.size, _ptr(y))
    return y


def rms_norm_f32(x, gamma, axis: int, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32).ravel()
    y = np.empty_like(x)
    st = lib().orc_rms_norm_f32(_ptr(x), _ptr(np.array(x.shape, np.int64)), x.ndim, _ptr(g),
                                g.size, axis, eps, _ptr(y))
    _check(st, "rms_norm_f32")
    return y
