"""Host-side operator interface over libmigemm, mirroring the reference ops.

Same names (snake_case of the Dart functions), argument meaning, attribute
defaults and error classes as the reference:

    op_matmul_nbits        <- opMatMulNBits   lib/src/onnx_qlinear_ops.dart:115
    op_matmul_integer      <- opMatMulInteger lib/src/onnx_qlinear_ops.dart:32
    op_qlinear_matmul      <- opQLinearMatMul lib/src/onnx_qlinear_ops.dart:85
    op_dynamic_quantize_linear <- opDynamicQuantizeLinear lib/src/onnx_ops.dart:3556
    op_matmul              <- opMatMul        lib/src/onnx_ops.dart:1710
    op_gemm                <- opGemm          lib/src/onnx_ops.dart:2152
    op_fused_sdpa          <- opFusedSDPA     lib/src/onnx_ops.dart:2106
    op_multi_head_attention <- opMultiHeadAttention lib/src/onnx_ops.dart:2019
    op_group_query_attention <- opGroupQueryAttention lib/src/onnx_ops.dart:1844
    op_conv                <- opConv          lib/src/onnx_nn_ops.dart:179
    op_conv_transpose      <- opConvTranspose lib/src/onnx_nn_ops.dart:818
    op_conv_integer        <- opConvInteger   lib/src/onnx_qlinear_ops.dart:299
    op_qlinear_conv        <- opQLinearConv   lib/src/onnx_qlinear_ops.dart:339

Tensors are numpy arrays on the host; every op runs on the GPU through the
C ABI (there is no CPU path).  Weight handles (NBitsWeight, Int8Weight,
F32Weight) keep prepacked weights resident in HBM across calls, like the
graph's prepacked-weight cache (lib/src/onnx_graph.dart:102-105).
"""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np

from . import _lib
from ._lib import check, lib
from .errors import ArgumentError, StateError, UnsupportedError

MG_ZP_NONE, MG_ZP_UINT4, MG_ZP_FLOAT = 0, 1, 2


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _shape_arr(a):
    return np.ascontiguousarray(np.array(a.shape, dtype=np.int64))


class Context:
    """One mg_ctx: a device, a stream, a grow-only workspace."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib.mg_ctx_create(device, C.byref(h)), "mg_ctx_create")
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            lib.mg_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, hip_stream: int):
        check(lib.mg_ctx_set_stream(self.handle, C.c_void_p(hip_stream)))

    def stream(self) -> int:
        s = C.c_void_p()
        check(lib.mg_ctx_get_stream(self.handle, C.byref(s)))
        return s.value or 0

    def synchronize(self):
        check(lib.mg_ctx_synchronize(self.handle))

    def set_control(self, cancel_flag=None, max_bytes: int = -1):
        """cancel_flag: a numpy int32 array of size 1 (polled before launches)."""
        self._cancel = cancel_flag
        check(lib.mg_ctx_set_control(self.handle, _ptr(cancel_flag), int(max_bytes)))

    def set_profiling(self, enable: bool = True):
        """Per-op device timing of the ops issued on this context (clears
        the records)."""
        check(lib.mg_ctx_set_profiling(self.handle, int(bool(enable))))

    def set_prefill_images(self, enable: bool = True):
        """Whether MatMulNBits weights created on this context from now on
        keep prefill images (default on): the weight's (q - zp) / 2 (q / 2
        with float zero points) as fp6 e2m3 MFMA operands, 3/4 byte per
        weight on top of the packed half byte, for blocks >= 128.  Prefill
        calls on weights with images run the fp6 GEMM, those without the fp8
        GEMM that dequantises each tile (or the fp32 path for float zero
        points).  Both meet the MatMulNBits tolerance; the results differ in
        rounding."""
        check(lib.mg_ctx_set_prefill_images(self.handle, int(bool(enable))))

    def profile_records(self) -> list:
        """[(op type, device ms)] of the profiled ops, in issue order (waits
        for them)."""
        n = C.c_int64(0)
        check(lib.mg_ctx_profile_count(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            op, ms = C.c_char_p(), C.c_float(0.0)
            check(lib.mg_ctx_profile_get(self.handle, i, C.byref(op), C.byref(ms)))
            out.append((op.value.decode(), float(ms.value)))
        return out

    def profile_clear(self):
        check(lib.mg_ctx_profile_clear(self.handle))


class ExecutionProfile:
    """Cumulative per-op-type device timing, as the reference's
    ExecutionProfile keeps per-op wall time (lib/src/onnx_graph.dart:27-86):
    calls_by_op, micros_by_op, per-record `nodes`, and the same report()."""

    def __init__(self):
        self.calls_by_op: dict = {}
        self.micros_by_op: dict = {}
        self.nodes: list = []

    def add(self, ctx: Context, name: str = ""):
        """Folds the context's records in and clears them."""
        for op, ms in ctx.profile_records():
            us = int(round(ms * 1000))
            self.calls_by_op[op] = self.calls_by_op.get(op, 0) + 1
            self.micros_by_op[op] = self.micros_by_op.get(op, 0) + us
            self.nodes.append((name, op, us))
        ctx.profile_clear()

    @property
    def total_micros(self) -> int:
        return sum(self.micros_by_op.values())

    def report(self) -> str:
        ops = sorted(self.micros_by_op, key=lambda o: -self.micros_by_op[o])
        total = self.total_micros
        lines = [f"{'op':<22}{'calls':>7}{'ms':>10}{'share':>8}"]
        for op in ops:
            us = self.micros_by_op[op]
            share = f"{us * 100 / total:.1f}%" if total else ""
            lines.append(f"{op:<22}{self.calls_by_op[op]:>7}{us / 1000:>10.1f}{share:>8}")
        lines.append(f"{'total':<29}{total / 1000:>10.1f}")
        return "\n".join(lines)


_tls = threading.local()


class DeviceBuffer:
    """HBM buffer of the context's device (mg_buffer_alloc), for the _dev ops."""

    def __init__(self, nbytes: int, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib.mg_buffer_alloc(self.ctx.handle, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray, ctx: Context | None = None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes, ctx)
        check(lib.mg_buffer_upload(buf.ctx.handle, C.c_void_p(buf.ptr), _ptr(arr), arr.nbytes))
        return buf

    def to_array(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self.ctx.synchronize()
        check(lib.mg_buffer_download(self.ctx.handle, _ptr(out), C.c_void_p(self.ptr),
                                     out.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib.mg_buffer_free(self.ctx.handle, C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def default_context() -> Context:
    ctx = getattr(_tls, "ctx", None)
    if ctx is None:
        ctx = Context(0)
        _tls.ctx = ctx
    return ctx


# ------------------------------------------------------------------ weights


class _Weight:
    handle = None

    def release(self):
        if self.handle:
            lib.mg_weight_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def info(self):
        k, n, b = C.c_int64(), C.c_int64(), C.c_int64()
        check(lib.mg_weight_info(self.handle, C.byref(k), C.byref(n), C.byref(b)))
        return k.value, n.value, b.value


class TensorSource(C.Structure):
    """mg_tensor_source: a tensor's bytes in host memory or in a file range
    (ONNX external data: location / offset / length)."""
    _fields_ = [("host", C.c_void_p), ("path", C.c_char_p), ("offset", C.c_int64),
                ("length", C.c_int64)]

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "TensorSource":
        src = cls(arr.ctypes.data_as(C.c_void_p), None, 0, arr.nbytes)
        src._keep = arr  # the array must outlive the upload
        return src

    @classmethod
    def from_file(cls, path, offset: int = 0, length: int = 0) -> "TensorSource":
        return cls(None, str(path).encode(), int(offset), int(length))


class NBitsWeight(_Weight):
    """MatMulNBits B/scales/zero_points/bias uploaded and prepacked."""

    @classmethod
    def streamed(cls, b: TensorSource, scales: TensorSource, zero_points: TensorSource = None,
                 *, zp_kind: int = MG_ZP_NONE, k: int, n: int, bits: int = 4,
                 block_size: int, bias=None, has_g_idx=False, chunk_bytes: int = 0,
                 ctx: Context | None = None) -> "NBitsWeight":
        """The load path: B / scales / zero points streamed from host arrays or
        file ranges (mg_weight_nbits_create_streamed), repacked on the GPU."""
        self = cls.__new__(cls)
        self.ctx = ctx or default_context()
        self.k, self.n = int(k), int(n)
        if bias is not None:
            bias = np.asarray(bias)
            if bias.dtype.kind != "f" or bias.shape != (self.n,):
                raise ArgumentError("MatMulNBits: bias must be floating point [N]")
            bias = np.ascontiguousarray(bias, dtype=np.float32)
        h = C.c_void_p()
        check(lib.mg_weight_nbits_create_streamed(
            self.ctx.handle, int(k), int(n), int(bits), int(block_size), C.byref(b),
            C.byref(scales), int(zp_kind), C.byref(zero_points) if zero_points is not None else None,
            _ptr(bias), int(bool(has_g_idx)), int(chunk_bytes), C.byref(h)))
        self.handle = h
        return self

    def __init__(self, b_q, scales, zero_points=None, *, k, n, bits=4, block_size,
                 bias=None, has_g_idx=False, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.k, self.n = int(k), int(n)
        if b_q is None or np.asarray(b_q).dtype != np.uint8:
            raise ArgumentError("MatMulNBits: invalid packed weights or scales")
        b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
        sc = np.asarray(scales)
        if sc.dtype.kind != "f":
            raise ArgumentError("MatMulNBits: invalid packed weights or scales")
        sc = np.ascontiguousarray(sc, dtype=np.float32)
        kind, zp = MG_ZP_NONE, None
        if zero_points is not None:
            zp = np.asarray(zero_points)
            if zp.dtype == np.uint8:
                kind = MG_ZP_UINT4
            elif zp.dtype.kind == "f":
                kind, zp = MG_ZP_FLOAT, zp.astype(np.float32)
            else:
                raise ArgumentError("MatMulNBits: invalid zero_points")
            zp = np.ascontiguousarray(zp)
        if bias is not None:
            bias = np.asarray(bias)
            if bias.dtype.kind != "f":
                raise ArgumentError("MatMulNBits: bias must be floating point [N]")
            bias = np.ascontiguousarray(bias, dtype=np.float32)
        h = C.c_void_p()
        check(lib.mg_weight_nbits_create(
            self.ctx.handle, int(k), int(n), int(bits), int(block_size),
            _ptr(b_q), _ptr(_shape_arr(b_q)), b_q.ndim,
            _ptr(sc), _ptr(_shape_arr(sc)), sc.ndim,
            kind, _ptr(zp), _ptr(_shape_arr(zp)) if zp is not None else None,
            zp.ndim if zp is not None else 0,
            _ptr(bias), _ptr(_shape_arr(bias)) if bias is not None else None,
            bias.ndim if bias is not None else 0, int(bool(has_g_idx)), C.byref(h)))
        self.handle = h

    def __call__(self, a) -> np.ndarray:
        a = np.asarray(a)
        if a.ndim < 1 or a.shape[-1] != self.k or a.dtype.kind != "f":
            raise ArgumentError("MatMulNBits: invalid K, N, block_size or input shape")
        a = np.ascontiguousarray(a, dtype=np.float32)
        m = a.size // self.k
        y = np.empty(a.shape[:-1] + (self.n,), dtype=np.float32)
        if m == 0:
            return y
        check(lib.mg_matmul_nbits(self.ctx.handle, self.handle, _ptr(a), m, _ptr(y)))
        return y

    def run_dev(self, a_ptr: int, m: int, y_ptr: int):
        check(lib.mg_matmul_nbits_dev(self.ctx.handle, self.handle, C.c_void_p(a_ptr), m,
                                      C.c_void_p(y_ptr)))

    def run_dev_noalloc(self, a_ptr: int, m: int, y_ptr: int):
        """run_dev without allocating: the workspace is the library's static
        per-device scratch (calls overlapping on one GPU race)."""
        check(lib.mg_matmul_nbits_dev_noalloc(self.ctx.handle, self.handle, C.c_void_p(a_ptr),
                                              m, C.c_void_p(y_ptr)))


def matmul_nbits_group_dev(weights, a_ptr: int, m: int, y_ptrs, ctx: Context | None = None):
    """Several NBitsWeight sharing K, block size and zero-point form applied to
    one device activation a [m, K]: y_ptrs[i] receives a . W_i^T (one launch
    for decode shapes)."""
    ctx = ctx or weights[0].ctx
    n = len(weights)
    ws = (C.c_void_p * n)(*[w.handle.value if isinstance(w.handle, C.c_void_p) else w.handle
                            for w in weights])
    ys = (C.c_void_p * n)(*[C.c_void_p(p).value for p in y_ptrs])
    check(lib.mg_matmul_nbits_group_dev(ctx.handle, n, ws, C.c_void_p(a_ptr), m, ys))


def matmul_nbits_group_split_dev(weights, a_ptr: int, split_ptr: int | None, m: int, y_ptrs,
                                 ctx: Context | None = None):
    """matmul_nbits_group_dev with the decode GEMV's split activations written
    by a_ptr's producer (skip_rms_norm_f32_split_dev): the GEMV's own
    prepass is skipped; results are bitwise the same."""
    ctx = ctx or weights[0].ctx
    n = len(weights)
    ws = (C.c_void_p * n)(*[w.handle.value if isinstance(w.handle, C.c_void_p) else w.handle
                            for w in weights])
    ys = (C.c_void_p * n)(*[C.c_void_p(p).value for p in y_ptrs])
    check(lib.mg_matmul_nbits_group_split_dev(ctx.handle, n, ws, C.c_void_p(a_ptr),
                                              C.c_void_p(split_ptr) if split_ptr else None, m,
                                              ys))


def nbits_split_bytes(k: int, block_size: int) -> int:
    """Bytes of a split activation buffer for rows of k elements."""
    out = C.c_size_t(0)
    check(lib.mg_nbits_split_bytes(int(k), int(block_size), C.byref(out)))
    return out.value


def _zp_arg(z):
    if z is None:
        return None, 0
    z = np.ascontiguousarray(np.asarray(z).astype(np.int32).ravel())
    return z, z.size


def _q_operand(x, what):
    x = np.asarray(x)
    if x.dtype not in (np.uint8, np.int8):
        raise ArgumentError(f"{what}: 8-bit integer operand expected, got {x.dtype}")
    return np.ascontiguousarray(x), int(x.dtype == np.int8)


class Int8Weight(_Weight):
    """MatMulInteger B [K, N] uploaded with its zero point and column sums."""

    def __init__(self, b, b_zp=None, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        b, self.b_signed = _q_operand(b, "MatMulInteger")
        if b.ndim != 2:
            raise ArgumentError("MatMulInteger: weight must be [K, N]")
        self.k, self.n = b.shape
        zb, lb = _zp_arg(b_zp)
        h = C.c_void_p()
        check(lib.mg_weight_int8_create(self.ctx.handle, _ptr(b), self.b_signed, self.k,
                                        self.n, _ptr(zb), lb, C.byref(h)))
        self.handle = h

    def matmul_integer(self, a, a_zp=None) -> np.ndarray:
        a, sa = _q_operand(a, "MatMulInteger")
        rows = a.size // self.k if self.k else 0
        za, la = _zp_arg(a_zp)
        y = np.empty(a.shape[:-1] + (self.n,), dtype=np.int32)
        check(lib.mg_matmul_integer_w(self.ctx.handle, _ptr(a), sa, rows, a.shape[-1],
                                      _ptr(za), la, self.handle, _ptr(y)))
        return y.astype(np.int64)

    def qlinear_matmul(self, a, a_scale, a_zp, b_scale, y_scale, y_zp, *, lo, hi):
        a, sa = _q_operand(a, "QLinearMatMul")
        rows = a.size // self.k if self.k else 0
        za, la = _zp_arg(a_zp)
        y = np.empty(a.shape[:-1] + (self.n,), dtype=np.int8 if lo < 0 else np.uint8)
        check(lib.mg_qlinear_matmul_w(self.ctx.handle, _ptr(a), sa, rows, a.shape[-1],
                                      float(a_scale), _ptr(za), la, self.handle,
                                      float(b_scale), float(y_scale), int(y_zp), lo, hi,
                                      _ptr(y)))
        return y.astype(np.int64)

    def matmul_integer_dev(self, a_ptr: int, a_signed: bool, rows: int, y_ptr: int,
                           a_zp=None):
        """Device form: a [rows, K] 8-bit and y int32 [rows, N] in HBM; asynchronous
        on the context's stream."""
        za, la = _zp_arg(a_zp)
        check(lib.mg_matmul_integer_w_dev(self.ctx.handle, C.c_void_p(a_ptr), int(a_signed),
                                          rows, self.k, _ptr(za), la, self.handle,
                                          C.c_void_p(y_ptr)))

    def qlinear_matmul_dev(self, a_ptr: int, a_signed: bool, rows: int, a_scale, a_zp,
                           b_scale, y_scale, y_zp, y_ptr: int, *, lo, hi):
        """Device form of qlinear_matmul (y 8-bit [rows, N] in HBM)."""
        za, la = _zp_arg(a_zp)
        check(lib.mg_qlinear_matmul_w_dev(self.ctx.handle, C.c_void_p(a_ptr), int(a_signed),
                                          rows, self.k, float(a_scale), _ptr(za), la,
                                          self.handle, float(b_scale), float(y_scale),
                                          int(y_zp), int(lo), int(hi), C.c_void_p(y_ptr)))

    def matmul_integer_dq_dev(self, a_ptr: int, rows: int, scale_zp_ptr: int, y_ptr: int):
        """MatMulInteger on DynamicQuantizeLinear's device outputs: a uint8
        [rows, K] and the zero point read from scale_zp_ptr on the device."""
        check(lib.mg_matmul_integer_w_dq_dev(self.ctx.handle, C.c_void_p(a_ptr), rows, self.k,
                                             C.c_void_p(scale_zp_ptr), self.handle,
                                             C.c_void_p(y_ptr)))

    def qlinear_matmul_dq_dev(self, a_ptr: int, rows: int, scale_zp_ptr: int, b_scale,
                              y_scale, y_zp, y_ptr: int, *, lo, hi):
        """QLinearMatMul on DynamicQuantizeLinear's device outputs: a_scale and
        a_zp are read from scale_zp_ptr on the device."""
        check(lib.mg_qlinear_matmul_w_dq_dev(self.ctx.handle, C.c_void_p(a_ptr), rows, self.k,
                                             C.c_void_p(scale_zp_ptr), self.handle,
                                             float(b_scale), float(y_scale), int(y_zp),
                                             int(lo), int(hi), C.c_void_p(y_ptr)))


class F32Weight(_Weight):
    """fp32 Gemm/MatMul B uploaded once; trans_b transposes on upload."""

    def __init__(self, b, trans_b=False, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        b = np.ascontiguousarray(b, dtype=np.float32)
        if b.ndim != 2:
            raise ArgumentError("Gemm: weight must be rank 2")
        rows, cols = b.shape
        self.k, self.n = (cols, rows) if trans_b else (rows, cols)
        h = C.c_void_p()
        check(lib.mg_weight_f32_create(self.ctx.handle, _ptr(b), rows, cols,
                                       int(bool(trans_b)), C.byref(h)))
        self.handle = h

    def gemm(self, a, c=None, *, alpha=1.0, beta=1.0) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        rows = a.size // a.shape[-1] if a.size else 0
        y = np.empty(a.shape[:-1] + (self.n,), dtype=np.float32)
        if c is not None:
            c = np.ascontiguousarray(c, dtype=np.float32)
        check(lib.mg_gemm_f32_w(self.ctx.handle, _ptr(a), rows, a.shape[-1], self.handle,
                                float(alpha), float(beta), _ptr(c),
                                _ptr(_shape_arr(c)) if c is not None else None,
                                c.ndim if c is not None else 0, _ptr(y)))
        return y

    def gemm_dev(self, a_ptr: int, rows: int, y_ptr: int, c_ptr: int | None = None,
                 c_shape=None, *, alpha=1.0, beta=1.0):
        """Device form: a [rows, K], y [rows, N] (and C of shape c_shape) in HBM."""
        cs = None if c_shape is None else np.ascontiguousarray(np.array(c_shape, np.int64))
        check(lib.mg_gemm_f32_w_dev(self.ctx.handle, C.c_void_p(a_ptr), rows, self.k,
                                    self.handle, float(alpha), float(beta),
                                    None if c_ptr is None else C.c_void_p(c_ptr),
                                    _ptr(cs), 0 if cs is None else cs.size,
                                    C.c_void_p(y_ptr)))


def matmul_f32_dev(a_ptr: int, a_shape, b_ptr: int, b_shape, y_ptr: int,
                   ctx: Context | None = None):
    """opMatMul on device buffers (numpy broadcasting over leading dims)."""
    ctx = ctx or default_context()
    sa = np.ascontiguousarray(np.array(a_shape, np.int64))
    sb = np.ascontiguousarray(np.array(b_shape, np.int64))
    check(lib.mg_matmul_f32_dev(ctx.handle, C.c_void_p(a_ptr), _ptr(sa), sa.size,
                                C.c_void_p(b_ptr), _ptr(sb), sb.size, C.c_void_p(y_ptr)))


def matmul_f32_output_shape(a_shape, b_shape) -> tuple:
    """Broadcast output shape of opMatMul over these operand shapes (no device)."""
    sa = np.ascontiguousarray(np.array(a_shape, np.int64))
    sb = np.ascontiguousarray(np.array(b_shape, np.int64))
    out = np.zeros(16, np.int64)
    rank = C.c_int32(0)
    check(lib.mg_matmul_f32_output_shape(_ptr(sa), sa.size, _ptr(sb), sb.size, _ptr(out),
                                         C.byref(rank)))
    return tuple(int(v) for v in out[:rank.value])


def matmul_f32_batch_offsets(a_shape, b_shape, first: int = 0, count: int | None = None):
    """Element offsets into A and B of output batches [first, first + count) as
    the fp32 kernels compute them (host-only)."""
    sa = np.ascontiguousarray(np.array(a_shape, np.int64))
    sb = np.ascontiguousarray(np.array(b_shape, np.int64))
    if count is None:
        nb = C.c_int64(0)
        check(lib.mg_matmul_f32_batch_offsets(_ptr(sa), sa.size, _ptr(sb), sb.size, 0, 0,
                                              None, None, C.byref(nb)))
        count = nb.value - first
    ao = np.zeros(max(count, 1), np.int64)
    bo = np.zeros(max(count, 1), np.int64)
    check(lib.mg_matmul_f32_batch_offsets(_ptr(sa), sa.size, _ptr(sb), sb.size, int(first),
                                          int(count), _ptr(ao), _ptr(bo), None))
    return ao[:count], bo[:count]


def dynamic_quantize_linear_dev(x_ptr: int, n: int, y_ptr: int, scale_zp_ptr: int,
                                ctx: Context | None = None):
    """DynamicQuantizeLinear on device: y uint8 [n]; at scale_zp_ptr 12 bytes:
    scale (f32), zp (i32), and an i32 that is 1 when x held Infinity or NaN."""
    ctx = ctx or default_context()
    check(lib.mg_dynamic_quantize_linear_dev(ctx.handle, C.c_void_p(x_ptr), int(n),
                                             C.c_void_p(y_ptr), C.c_void_p(scale_zp_ptr)))


BINARY_OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3}


def binary_f32_dev(op: str, a_ptr: int, a_shape, b_ptr: int, b_shape, y_ptr: int,
                   ctx: Context | None = None):
    """opAdd / opSub / opMul / opDiv on device buffers with broadcasting
    (lib/src/onnx_ops.dart:26-44, :103-330); y holds the broadcast shape."""
    ctx = ctx or default_context()
    sa = np.ascontiguousarray(np.array(a_shape, np.int64))
    sb = np.ascontiguousarray(np.array(b_shape, np.int64))
    check(lib.mg_binary_f32_dev(ctx.handle, BINARY_OPS[op], C.c_void_p(a_ptr), _ptr(sa), sa.size,
                                C.c_void_p(b_ptr), _ptr(sb), sb.size, C.c_void_p(y_ptr)))


def sigmoid_f32_dev(x_ptr: int, n: int, y_ptr: int, ctx: Context | None = None):
    """opSigmoid (lib/src/onnx_ops.dart:2349) on a device buffer of n floats."""
    ctx = ctx or default_context()
    check(lib.mg_sigmoid_f32_dev(ctx.handle, C.c_void_p(x_ptr), int(n), C.c_void_p(y_ptr)))


def rms_norm_f32_dev(x_ptr: int, shape, gamma_ptr: int, gamma_len: int, axis: int, eps: float,
                     y_ptr: int, ctx: Context | None = None):
    """opRMSNorm (lib/src/onnx_ops.dart:1771-1815) on device buffers."""
    ctx = ctx or default_context()
    sh = np.ascontiguousarray(np.array(shape, np.int64))
    check(lib.mg_rms_norm_f32_dev(ctx.handle, C.c_void_p(x_ptr), _ptr(sh), sh.size,
                                  C.c_void_p(gamma_ptr), int(gamma_len), int(axis), float(eps),
                                  C.c_void_p(y_ptr)))


def skip_rms_norm_f32_split_dev(x_ptr: int, skip_ptr: int | None, shape, gamma_ptr: int,
                                gamma_len: int, bias_ptr: int | None, eps: float, y_ptr: int,
                                sum_ptr: int | None, block_size: int, split_ptr: int,
                                ctx: Context | None = None):
    """SkipSimplifiedLayerNormalization (or RMSNorm over the last axis when
    skip_ptr is None) that also writes the decode GEMV's split activations of
    y (rows <= 16, last dim <= 8192)."""
    ctx = ctx or default_context()
    sh = np.ascontiguousarray(np.array(shape, np.int64))
    check(lib.mg_skip_rms_norm_f32_split_dev(
        ctx.handle, C.c_void_p(x_ptr), C.c_void_p(skip_ptr) if skip_ptr else None, _ptr(sh),
        sh.size, C.c_void_p(gamma_ptr), int(gamma_len),
        C.c_void_p(bias_ptr) if bias_ptr else None, float(eps), C.c_void_p(y_ptr),
        C.c_void_p(sum_ptr) if sum_ptr else None, int(block_size), C.c_void_p(split_ptr)))


def skip_rms_norm_f32_dev(x_ptr: int, skip_ptr: int, shape, gamma_ptr: int, gamma_len: int,
                          bias_ptr: int | None, eps: float, y_ptr: int, sum_ptr: int | None,
                          ctx: Context | None = None):
    """SkipSimplifiedLayerNormalization (lib/src/onnx_graph.dart:1793-1813) on
    device buffers: sum = x + skip, y = RMSNorm(sum) (+ bias)."""
    ctx = ctx or default_context()
    sh = np.ascontiguousarray(np.array(shape, np.int64))
    check(lib.mg_skip_rms_norm_f32_dev(ctx.handle, C.c_void_p(x_ptr), C.c_void_p(skip_ptr),
                                       _ptr(sh), sh.size, C.c_void_p(gamma_ptr), int(gamma_len),
                                       C.c_void_p(bias_ptr) if bias_ptr else None, float(eps),
                                       C.c_void_p(y_ptr),
                                       C.c_void_p(sum_ptr) if sum_ptr else None))


# ---------------------------------------------------------------------- ops


def _run_dev(arrays, out_shapes, call, ctx):
    """Uploads arrays, runs call(device pointers..., output pointers...),
    downloads the outputs (float32)."""
    ctx = ctx or default_context()
    ins = [DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32), ctx) for x in arrays]
    outs = [DeviceBuffer(max(int(np.prod(sh, dtype=np.int64)), 1) * 4, ctx) for sh in out_shapes]
    try:
        call(*[b.ptr for b in ins], *[b.ptr for b in outs])
        return [o.to_array(sh, np.float32) for o, sh in zip(outs, out_shapes)]
    finally:
        for b in ins + outs:
            b.free()


def _binary(op, a, b, ctx):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    try:
        shape = np.broadcast_shapes(a.shape, b.shape)
    except ValueError:
        shape = ()  # the library reports the reference's ArgumentError
    return _run_dev([a, b], [shape], lambda pa, pb, py: binary_f32_dev(
        op, pa, a.shape, pb, b.shape, py, ctx), ctx)[0]


def op_add(a, b, ctx: Context | None = None) -> np.ndarray:
    """opAdd on float tensors (lib/src/onnx_ops.dart:402-404)."""
    return _binary("add", a, b, ctx)


def op_sub(a, b, ctx: Context | None = None) -> np.ndarray:
    """opSub on float tensors (lib/src/onnx_ops.dart:444-446)."""
    return _binary("sub", a, b, ctx)


def op_mul(a, b, ctx: Context | None = None) -> np.ndarray:
    """opMul on float tensors (lib/src/onnx_ops.dart:447-449)."""
    return _binary("mul", a, b, ctx)


def op_div(a, b, ctx: Context | None = None) -> np.ndarray:
    """opDiv on float tensors (lib/src/onnx_ops.dart:475-477)."""
    return _binary("div", a, b, ctx)


def op_sigmoid(x, ctx: Context | None = None) -> np.ndarray:
    """opSigmoid (lib/src/onnx_ops.dart:2349-2350)."""
    x = np.asarray(x, np.float32)
    return _run_dev([x], [x.shape], lambda px, py: sigmoid_f32_dev(px, x.size, py, ctx), ctx)[0]


def op_rms_norm(x, gamma, axis: int, eps: float, ctx: Context | None = None) -> np.ndarray:
    """opRMSNorm (lib/src/onnx_ops.dart:1771-1815)."""
    x = np.asarray(x, np.float32)
    g = np.asarray(gamma, np.float32).ravel()
    return _run_dev([x, g], [x.shape], lambda px, pg, py: rms_norm_f32_dev(
        px, x.shape, pg, g.size, axis, eps, py, ctx), ctx)[0]


def op_skip_simplified_layer_norm(x, skip, gamma, bias=None, eps: float = 1e-5,
                                  ctx: Context | None = None):
    """SkipSimplifiedLayerNormalization (lib/src/onnx_graph.dart:1793-1813):
    returns (rmsnorm(x + skip) [+ bias], x + skip)."""
    x = np.asarray(x, np.float32)
    s = np.asarray(skip, np.float32)
    g = np.asarray(gamma, np.float32).ravel()
    ins = [x, s, g] + ([np.asarray(bias, np.float32).ravel()] if bias is not None else [])

    def call(*p):
        px, ps, pg = p[:3]
        pb = p[3] if bias is not None else None
        py, psum = p[-2], p[-1]
        skip_rms_norm_f32_dev(px, ps, x.shape, pg, g.size, pb, eps, py, psum, ctx)

    y, total = _run_dev(ins, [x.shape, x.shape], call, ctx)
    return y, total


def op_matmul_nbits(a, b_q, scales, zero_points=None, *, k, n, bits=4, block_size,
                    bias=None, ctx: Context | None = None) -> np.ndarray:
    """opMatMulNBits (lib/src/onnx_qlinear_ops.dart:115-228)."""
    if bits != 4:
        raise UnsupportedError(f"MatMulNBits: only bits=4 supported, got {bits}")
    a = np.asarray(a)
    if (k <= 0 or n <= 0 or block_size < 16 or block_size & (block_size - 1)
            or a.ndim < 1 or a.shape[-1] != k):
        raise ArgumentError("MatMulNBits: invalid K, N, block_size or input shape")
    w = NBitsWeight(b_q, scales, zero_points, k=k, n=n, bits=bits, block_size=block_size,
                    bias=bias, ctx=ctx)
    try:
        return w(a)
    finally:
        w.release()


# Longest K whose MatMulInteger sums fit int32 for every operand (33025 *
# 255 * 255 < 2^31); longer rows use the int64 entry point.
MAX_K_INT32 = 33025


def op_matmul_integer(a, b, a_zp=None, b_zp=None, ctx: Context | None = None) -> np.ndarray:
    """opMatMulInteger (lib/src/onnx_qlinear_ops.dart:32-81); int64 result."""
    a, sa = _q_operand(a, "MatMulInteger")
    b, sb = _q_operand(b, "MatMulInteger")
    if a.ndim < 2 or b.ndim < 2:
        raise ArgumentError("MatMulInteger: operands must have rank >= 2")
    za, la = _zp_arg(a_zp)
    zb, lb = _zp_arg(b_zp)
    m, n = a.shape[-2], b.shape[-1]
    ab = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    bb = int(np.prod(b.shape[:-2])) if b.ndim > 2 else 1
    out_batch = a.shape[:-2] if ab >= bb else b.shape[:-2]
    ctx = ctx or default_context()
    if a.shape[-1] > MAX_K_INT32:
        # Sums may exceed int32: the int64 form (segments summed in int64).
        y = np.empty(tuple(out_batch) + (m, n), dtype=np.int64)
        check(lib.mg_matmul_integer_i64(ctx.handle, _ptr(a), sa, _ptr(_shape_arr(a)), a.ndim,
                                        _ptr(b), sb, _ptr(_shape_arr(b)), b.ndim, _ptr(za), la,
                                        _ptr(zb), lb, _ptr(y)))
        return y
    y = np.empty(tuple(out_batch) + (m, n), dtype=np.int32)
    check(lib.mg_matmul_integer(ctx.handle, _ptr(a), sa, _ptr(_shape_arr(a)), a.ndim,
                                _ptr(b), sb, _ptr(_shape_arr(b)), b.ndim, _ptr(za), la,
                                _ptr(zb), lb, _ptr(y)))
    return y.astype(np.int64)


def op_qlinear_matmul(a, a_s, a_zp, b, b_s, b_zp, y_s, y_zp, *, lo, hi,
                      ctx: Context | None = None) -> np.ndarray:
    """opQLinearMatMul (lib/src/onnx_qlinear_ops.dart:85-108); int64 result."""
    if np.size(a_s) != 1 or np.size(b_s) != 1 or np.size(y_s) != 1:
        raise UnsupportedError("QLinearMatMul: only per-tensor scales supported")
    a, sa = _q_operand(a, "QLinearMatMul")
    b, sb = _q_operand(b, "QLinearMatMul")
    if a.ndim < 2 or b.ndim < 2:
        raise ArgumentError("MatMulInteger: operands must have rank >= 2")
    za, la = _zp_arg(a_zp)
    zb, lb = _zp_arg(b_zp)
    yz = 0 if y_zp is None else int(np.asarray(y_zp).ravel()[0])
    m, n = a.shape[-2], b.shape[-1]
    ab = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    bb = int(np.prod(b.shape[:-2])) if b.ndim > 2 else 1
    out_batch = a.shape[:-2] if ab >= bb else b.shape[:-2]
    y = np.empty(tuple(out_batch) + (m, n), dtype=np.int8 if lo < 0 else np.uint8)
    ctx = ctx or default_context()
    check(lib.mg_qlinear_matmul(
        ctx.handle, _ptr(a), sa, _ptr(_shape_arr(a)), a.ndim,
        float(np.float32(np.asarray(a_s).ravel()[0])), _ptr(za), la, _ptr(b), sb,
        _ptr(_shape_arr(b)), b.ndim, float(np.float32(np.asarray(b_s).ravel()[0])), _ptr(zb),
        lb, float(np.float32(np.asarray(y_s).ravel()[0])), yz, int(lo), int(hi), _ptr(y)))
    return y.astype(np.int64)


def op_dynamic_quantize_linear(x, ctx: Context | None = None):
    """opDynamicQuantizeLinear (lib/src/onnx_ops.dart:3556-3583) ->
    (y uint8, scale float32, zero point int)."""
    ctx = ctx or default_context()
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint8)
    scale = C.c_float()
    zp = C.c_int32()
    check(lib.mg_dynamic_quantize_linear(ctx.handle, _ptr(x), x.size, _ptr(y),
                                         C.byref(scale), C.byref(zp)))
    return y, np.float32(scale.value), int(zp.value)


def op_matmul(a, b, ctx: Context | None = None) -> np.ndarray:
    """opMatMul (lib/src/onnx_ops.dart:1710-1766), numpy broadcasting.

    Float operands (the reference's Float32List tensors; other float widths
    are taken as f32, as the loader widens fp16) run the fp32 kernel.  When
    either operand is an integer tensor the reference falls back to a double
    sum of getD products per output (:1753-1762): both operands then go to
    the device as doubles (an int64 element's nearest double, as getD) and
    the double-accumulation kernel."""
    a, b = np.asarray(a), np.asarray(b)
    if a.ndim < 2 or b.ndim < 2:
        raise ArgumentError("MatMul: operands must have rank >= 2")
    try:
        batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    except ValueError:
        raise ArgumentError("MatMul: batch dims do not broadcast") from None
    y = np.empty(tuple(batch) + (a.shape[-2], b.shape[-1]), dtype=np.float32)
    ctx = ctx or default_context()
    if a.dtype.kind in "iub" or b.dtype.kind in "iub":
        ad = np.ascontiguousarray(a, dtype=np.float64)
        bd = np.ascontiguousarray(b, dtype=np.float64)
        check(lib.mg_matmul_f64acc(ctx.handle, _ptr(ad), _ptr(_shape_arr(ad)), ad.ndim,
                                   _ptr(bd), _ptr(_shape_arr(bd)), bd.ndim, _ptr(y)))
        return y
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    check(lib.mg_matmul_f32(ctx.handle, _ptr(a), _ptr(_shape_arr(a)), a.ndim, _ptr(b),
                            _ptr(_shape_arr(b)), b.ndim, _ptr(y)))
    return y


def op_gemm(a, b, c=None, *, alpha=1.0, beta=1.0, trans_a=False, trans_b=False,
            ctx: Context | None = None) -> np.ndarray:
    """opGemm (lib/src/onnx_ops.dart:2152-2172)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    if a.ndim != 2 or b.ndim != 2:
        raise ArgumentError("Gemm: A and B must be rank 2")
    m = a.shape[1] if trans_a else a.shape[0]
    n = b.shape[0] if trans_b else b.shape[1]
    y = np.empty((m, n), dtype=np.float32)
    if c is not None:
        c = np.ascontiguousarray(c, dtype=np.float32)
    ctx = ctx or default_context()
    check(lib.mg_gemm_f32(ctx.handle, _ptr(a), _ptr(_shape_arr(a)), _ptr(b),
                          _ptr(_shape_arr(b)), int(bool(trans_a)), int(bool(trans_b)),
                          float(alpha), float(beta), _ptr(c),
                          _ptr(_shape_arr(c)) if c is not None else None,
                          c.ndim if c is not None else 0, _ptr(y)))
    return y


def op_fused_sdpa(a, b, v, mask, scale: float, ctx: Context | None = None) -> np.ndarray:
    """opFusedSDPA (lib/src/onnx_ops.dart:2106-2149):
    MatMul(Softmax(MatMul(a, b) * scale + mask), v); b is K^T [..., D, T]."""
    a, b, v, mask = (np.ascontiguousarray(x, dtype=np.float32) for x in (a, b, v, mask))
    if a.ndim < 2 or b.ndim < 2 or v.ndim < 2:
        raise ArgumentError("_FusedSDPA: operands need rank >= 2")
    try:
        sb = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
        ob = np.broadcast_shapes(sb, v.shape[:-2])
    except ValueError:
        raise ArgumentError("MatMul: batch dims do not broadcast") from None
    y = np.empty(tuple(ob) + (a.shape[-2], v.shape[-1]), dtype=np.float32)
    ctx = ctx or default_context()
    check(lib.mg_fused_sdpa(ctx.handle, _ptr(a), _ptr(_shape_arr(a)), a.ndim, _ptr(b),
                            _ptr(_shape_arr(b)), b.ndim, _ptr(v), _ptr(_shape_arr(v)), v.ndim,
                            _ptr(mask), _ptr(_shape_arr(mask)), mask.ndim, float(scale),
                            _ptr(y)))
    return y


def op_multi_head_attention(q, k, v, attention_bias=None, *, num_heads: int,
                            scale: float | None = None,
                            ctx: Context | None = None) -> np.ndarray:
    """opMultiHeadAttention (lib/src/onnx_ops.dart:2019-2098): q [batch, seq,
    hidden], k / v [batch, kv_seq, hidden], attention_bias [batch, bias_heads,
    seq, kv_seq] or None; scale defaults to 1 / sqrt(hidden / num_heads)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3 or k.shape != v.shape or \
            k.shape[0] != q.shape[0] or k.shape[2] != q.shape[2]:
        raise ArgumentError("MultiHeadAttention: q, k, v must be [batch, seq, hidden]")
    batch, seq, hidden = q.shape
    kv_seq = k.shape[1]
    bias_heads = 0
    if attention_bias is not None:
        attention_bias = np.ascontiguousarray(attention_bias, dtype=np.float32)
        if attention_bias.ndim != 4 or attention_bias.shape[0] != batch or \
                attention_bias.shape[2:] != (seq, kv_seq):
            raise ArgumentError("MultiHeadAttention: bias must be [batch, heads, seq, kv_seq]")
        bias_heads = attention_bias.shape[1]
    y = np.empty_like(q)
    ctx = ctx or default_context()
    check(lib.mg_multi_head_attention(ctx.handle, _ptr(q), _ptr(k), _ptr(v), batch, seq, kv_seq,
                                      hidden, int(num_heads), _ptr(attention_bias), bias_heads,
                                      int(scale is not None),
                                      float(scale if scale is not None else 0.0), _ptr(y)))
    return y


def fused_sdpa_dev(a_ptr: int, a_shape, b_ptr: int, b_shape, v_ptr: int, v_shape,
                   mask_ptr: int, mask_shape, scale: float, y_ptr: int,
                   ctx: Context | None = None):
    """op_fused_sdpa on device buffers (asynchronous on the context's stream)."""
    ctx = ctx or default_context()
    sh = [np.ascontiguousarray(np.array(x, np.int64)) for x in (a_shape, b_shape, v_shape,
                                                                 mask_shape)]
    check(lib.mg_fused_sdpa_dev(ctx.handle, C.c_void_p(a_ptr), _ptr(sh[0]), sh[0].size,
                                C.c_void_p(b_ptr), _ptr(sh[1]), sh[1].size, C.c_void_p(v_ptr),
                                _ptr(sh[2]), sh[2].size, C.c_void_p(mask_ptr), _ptr(sh[3]),
                                sh[3].size, float(scale), C.c_void_p(y_ptr)))


def multi_head_attention_dev(q_ptr: int, k_ptr: int, v_ptr: int, batch: int, seq: int,
                             kv_seq: int, hidden: int, num_heads: int, y_ptr: int,
                             bias_ptr: int = 0, bias_heads: int = 0,
                             scale: float | None = None, ctx: Context | None = None):
    """op_multi_head_attention on device buffers."""
    ctx = ctx or default_context()
    check(lib.mg_multi_head_attention_dev(ctx.handle, C.c_void_p(q_ptr), C.c_void_p(k_ptr),
                                          C.c_void_p(v_ptr), batch, seq, kv_seq, hidden,
                                          int(num_heads),
                                          C.c_void_p(bias_ptr) if bias_ptr else None,
                                          int(bias_heads), int(scale is not None),
                                          float(scale if scale is not None else 0.0),
                                          C.c_void_p(y_ptr)))


def op_group_query_attention(q, k, v, *, num_heads: int, kv_num_heads: int, scale=None,
                            do_rotary: bool = False, rotary_interleaved: bool = False,
                            past_key=None, past_value=None, cos_cache=None, sin_cache=None,
                            attention_bias=None, softcap: float = 0.0, local_window: int = -1,
                            ctx: Context | None = None):
    """opGroupQueryAttention (lib/src/onnx_ops.dart:1844-2012): returns
    [output, present_key, present_value]."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3 or k.shape != v.shape or \
            k.shape[:2] != q.shape[:2]:
        raise ArgumentError("GroupQueryAttention: q, k, v must be [batch, seq, hidden]")
    batch, seq, hidden = q.shape
    if num_heads <= 0 or hidden % num_heads:
        raise ArgumentError("GroupQueryAttention: hidden must be a multiple of num_heads")
    hs = hidden // num_heads
    if kv_num_heads <= 0 or k.shape[2] != kv_num_heads * hs:
        raise ArgumentError("GroupQueryAttention: k and v must be [batch, seq, kv_heads * head_size]")
    past_len = 0
    if past_key is not None:
        past_key = np.ascontiguousarray(past_key, dtype=np.float32)
        past_value = np.ascontiguousarray(past_value, dtype=np.float32)
        if past_key.ndim == 4:
            past_len = past_key.shape[2]
            if past_key.shape != (batch, kv_num_heads, past_len, hs) or \
                    past_value.shape != past_key.shape:
                raise ArgumentError("GroupQueryAttention: past_key / past_value must be "
                                    "[batch, kv_heads, past, head_size]")
        else:
            past_key = past_value = None
    max_pos = half = 0
    if do_rotary:
        if cos_cache is None or sin_cache is None:
            raise ArgumentError("GroupQueryAttention: do_rotary needs cos_cache and sin_cache")
        cos_cache = np.ascontiguousarray(cos_cache, dtype=np.float32)
        sin_cache = np.ascontiguousarray(sin_cache, dtype=np.float32)
        max_pos, half = cos_cache.shape[0], cos_cache.shape[-1]
    total = past_len + seq
    bias_heads = 0
    if attention_bias is not None:
        attention_bias = np.ascontiguousarray(attention_bias, dtype=np.float32)
        if attention_bias.ndim != 4 or attention_bias.shape[0] != batch or \
                attention_bias.shape[2:] != (seq, total):
            raise ArgumentError("GroupQueryAttention: attention_bias must be "
                                "[batch, heads, seq, past + seq]")
        bias_heads = attention_bias.shape[1]
    y = np.empty_like(q)
    pk = np.empty((batch, kv_num_heads, total, hs), np.float32)
    pv = np.empty_like(pk)
    ctx = ctx or default_context()
    check(lib.mg_group_query_attention(
        ctx.handle, _ptr(q), _ptr(k), _ptr(v), batch, seq, hidden, int(num_heads),
        int(kv_num_heads), _ptr(past_key), _ptr(past_value), past_len, _ptr(cos_cache),
        _ptr(sin_cache), max_pos, half, int(bool(do_rotary)), int(bool(rotary_interleaved)),
        _ptr(attention_bias), bias_heads, int(scale is not None),
        float(scale if scale is not None else 0.0), float(softcap), int(local_window), _ptr(y),
        _ptr(pk), _ptr(pv)))
    return [y, pk, pv]


def group_query_attention_dev(q_ptr: int, k_ptr: int, v_ptr: int, batch: int, seq: int,
                              hidden: int, num_heads: int, kv_num_heads: int, y_ptr: int,
                              present_key_ptr: int, present_value_ptr: int, *,
                              past_key_ptr: int = 0, past_value_ptr: int = 0, past_len: int = 0,
                              cos_ptr: int = 0, sin_ptr: int = 0, max_pos: int = 0,
                              half_rot: int = 0, do_rotary: bool = False,
                              rotary_interleaved: bool = False, bias_ptr: int = 0,
                              bias_heads: int = 0, scale=None, ctx: Context | None = None):
    """op_group_query_attention on device buffers (asynchronous)."""
    ctx = ctx or default_context()
    vp = lambda x: C.c_void_p(x) if x else None  # noqa: E731
    check(lib.mg_group_query_attention_dev(
        ctx.handle, vp(q_ptr), vp(k_ptr), vp(v_ptr), batch, seq, hidden, int(num_heads),
        int(kv_num_heads), vp(past_key_ptr), vp(past_value_ptr), past_len, vp(cos_ptr),
        vp(sin_ptr), max_pos, half_rot, int(bool(do_rotary)), int(bool(rotary_interleaved)),
        vp(bias_ptr), bias_heads, int(scale is not None),
        float(scale if scale is not None else 0.0), 0.0, -1, vp(y_ptr), vp(present_key_ptr),
        vp(present_value_ptr)))


# ------------------------------------------------------------ convolution

_AUTO_PAD = {"NOTSET": 0, "SAME_UPPER": 1, "SAME_LOWER": 2, "VALID": 3}


def _i64(v):
    return None if v is None else np.ascontiguousarray(np.array(list(v), dtype=np.int64))


def _check_ranks(op: str, x, w):
    """x and w of one rank, 3 to 5 (lib/src/onnx_nn_ops.dart:196-201); the C
    ABI takes that one rank for both."""
    if x.ndim != w.ndim or not 3 <= x.ndim <= 5:
        raise ArgumentError(f"{op}: x and w must have the same rank, 3 to 5")


def _check_kernel_shape(op: str, kernel_shape, w):
    """The dispatcher's kernel_shape check (lib/src/onnx_graph.dart:2438-2445)."""
    if kernel_shape is not None and list(kernel_shape) != list(w.shape[2:]):
        raise StateError(f"{op} kernel_shape {list(kernel_shape)} does not match weight "
                         f"shape {list(w.shape[2:])}.")


def conv_output_shape(x_shape, w_shape, *, strides=None, pads=None, dilations=None, group=1,
                      auto_pad="NOTSET") -> tuple:
    """Output shape of a Conv (pads resolved as lib/src/onnx_nn_ops.dart:38-87)."""
    xs, ws = _i64(x_shape), _i64(w_shape)
    if auto_pad not in _AUTO_PAD:
        raise ArgumentError(f"Conv: unknown auto_pad {auto_pad}")
    y = np.zeros(max(xs.size, 1), np.int64)
    st, pd, dl = _i64(strides), _i64(pads), _i64(dilations)
    check(lib.mg_conv_output_shape(_ptr(xs), xs.size, _ptr(ws), _ptr(st), _ptr(pd), _ptr(dl),
                                   int(group), _AUTO_PAD[auto_pad], _ptr(y)))
    return tuple(int(v) for v in y)


def op_conv(x, w, bias=None, *, strides=None, pads=None, dilations=None, group: int = 1,
            auto_pad: str = "NOTSET", kernel_shape=None, ctx: Context | None = None):
    """opConv (lib/src/onnx_nn_ops.dart:179-817): x [N, C, *spatial] (1 to 3
    spatial dims), w [M, C / group, *kernel], bias [M] or None."""
    x, w = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, w))
    _check_ranks("Conv", x, w)
    _check_kernel_shape("Conv", kernel_shape, w)
    ys = conv_output_shape(x.shape, w.shape, strides=strides, pads=pads, dilations=dilations,
                           group=group, auto_pad=auto_pad)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    if b is not None and b.size != w.shape[0]:
        raise ArgumentError("Conv: bias must have one value per output channel")
    y = np.empty(ys, np.float32)
    st, pd, dl = _i64(strides), _i64(pads), _i64(dilations)
    ctx = ctx or default_context()
    check(lib.mg_conv_f32(ctx.handle, _ptr(x), _ptr(_shape_arr(x)), x.ndim, _ptr(w),
                          _ptr(_shape_arr(w)), _ptr(b), _ptr(st), _ptr(pd), _ptr(dl), int(group),
                          _AUTO_PAD[auto_pad], _ptr(y)))
    return y


def conv_transpose_output_shape(x_shape, w_shape, *, strides=None, pads=None, dilations=None,
                                output_padding=None, output_shape=None, group=1) -> tuple:
    """Output shape of a ConvTranspose (lib/src/onnx_nn_ops.dart:976-995)."""
    xs, ws = _i64(x_shape), _i64(w_shape)
    y = np.zeros(max(xs.size, 1), np.int64)
    os_ = _i64(output_shape)
    check(lib.mg_conv_transpose_output_shape(
        _ptr(xs), xs.size, _ptr(ws), _ptr(_i64(strides)), _ptr(_i64(pads)),
        _ptr(_i64(dilations)), _ptr(_i64(output_padding)), _ptr(os_),
        0 if os_ is None else os_.size, int(group), _ptr(y)))
    return tuple(int(v) for v in y)


def op_conv_transpose(x, w, bias=None, *, strides=None, pads=None, dilations=None,
                      output_padding=None, output_shape=None, group: int = 1,
                      kernel_shape=None, ctx: Context | None = None):
    """opConvTranspose (lib/src/onnx_nn_ops.dart:818-1059): w [C, M / group,
    *kernel]; output_shape (spatial dims, or the full shape) sets the pads."""
    x, w = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, w))
    _check_ranks("ConvTranspose", x, w)
    _check_kernel_shape("ConvTranspose", kernel_shape, w)
    ys = conv_transpose_output_shape(x.shape, w.shape, strides=strides, pads=pads,
                                     dilations=dilations, output_padding=output_padding,
                                     output_shape=output_shape, group=group)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    if b is not None and b.size != ys[1]:
        raise ArgumentError("ConvTranspose: bias must have one value per output channel")
    y = np.empty(ys, np.float32)
    os_ = _i64(output_shape)
    ctx = ctx or default_context()
    check(lib.mg_conv_transpose_f32(
        ctx.handle, _ptr(x), _ptr(_shape_arr(x)), x.ndim, _ptr(w), _ptr(_shape_arr(w)), _ptr(b),
        _ptr(_i64(strides)), _ptr(_i64(pads)), _ptr(_i64(dilations)),
        _ptr(_i64(output_padding)), _ptr(os_), 0 if os_ is None else os_.size, int(group),
        _ptr(y)))
    return y


def _int_operand(a, what: str):
    a = np.ascontiguousarray(a)
    if a.dtype not in (np.uint8, np.int8):
        raise ArgumentError(f"{what} must be uint8 or int8")
    return a, int(a.dtype == np.int8)


def _zp_list(z):
    if z is None:
        return None, 0
    z = np.ascontiguousarray(np.asarray(z).astype(np.int32).ravel())
    return z, z.size


def _scalar_int(z) -> int:
    return 0 if z is None else int(np.asarray(z).ravel()[0])


def op_conv_integer(x, w, x_zero_point=None, w_zero_point=None, *, strides=None, pads=None,
                    dilations=None, group: int = 1, ctx: Context | None = None):
    """opConvInteger (lib/src/onnx_qlinear_ops.dart:299-337): exact
    sum (x - x_zp)(w - w_zp[m]); returns int64 like the reference's
    Tensor.int64 (the library computes int32)."""
    x, xs = _int_operand(x, "ConvInteger: x")
    w, wsg = _int_operand(w, "ConvInteger: w")
    _check_ranks("ConvInteger", x, w)
    wz, nwz = _zp_list(w_zero_point)
    ys = conv_output_shape(x.shape, w.shape, strides=strides, pads=pads, dilations=dilations,
                           group=group)
    y = np.empty(ys, np.int32)
    ctx = ctx or default_context()
    check(lib.mg_conv_integer(ctx.handle, _ptr(x), xs, _ptr(_shape_arr(x)), x.ndim, _ptr(w), wsg,
                              _ptr(_shape_arr(w)), _scalar_int(x_zero_point), _ptr(wz), nwz,
                              _ptr(_i64(strides)), _ptr(_i64(pads)), _ptr(_i64(dilations)),
                              int(group), _ptr(y)))
    return y.astype(np.int64)


def op_qlinear_conv(x, x_scale, x_zero_point, w, w_scale, w_zero_point, y_scale, y_zero_point,
                    bias=None, *, strides=None, pads=None, dilations=None, group: int = 1,
                    lo: int, hi: int, ctx: Context | None = None):
    """opQLinearConv (lib/src/onnx_qlinear_ops.dart:339-382); lo / hi are
    [-128, 127] when the y_zero_point initializer is int8, else [0, 255]
    (lib/src/onnx_graph.dart:2936,2952-2953).  Returns int64 values."""
    x, xs = _int_operand(x, "QLinearConv: x")
    w, wsg = _int_operand(w, "QLinearConv: w")
    _check_ranks("QLinearConv", x, w)
    wz, nwz = _zp_list(w_zero_point)
    wsc = np.ascontiguousarray(np.asarray(w_scale, dtype=np.float32).ravel())
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias).astype(np.int32).ravel())
    ys = conv_output_shape(x.shape, w.shape, strides=strides, pads=pads, dilations=dilations,
                           group=group)
    y = np.empty(ys, np.uint8)
    ctx = ctx or default_context()
    check(lib.mg_qlinear_conv(
        ctx.handle, _ptr(x), xs, _ptr(_shape_arr(x)), x.ndim,
        float(np.asarray(x_scale, np.float32).ravel()[0]), _scalar_int(x_zero_point), _ptr(w),
        wsg, _ptr(_shape_arr(w)), _ptr(wsc), wsc.size, _ptr(wz), nwz,
        float(np.asarray(y_scale, np.float32).ravel()[0]), _scalar_int(y_zero_point), _ptr(b),
        _ptr(_i64(strides)), _ptr(_i64(pads)), _ptr(_i64(dilations)), int(group), int(lo),
        int(hi), _ptr(y)))
    return (y.view(np.int8) if lo < 0 else y).astype(np.int64)


def conv_f32_dev(x_ptr: int, x_shape, w_ptr: int, w_shape, y_ptr: int, bias_ptr: int = 0, *,
                 strides=None, pads=None, dilations=None, group: int = 1,
                 auto_pad: str = "NOTSET", ctx: Context | None = None):
    """op_conv on device buffers (asynchronous on the context's stream)."""
    ctx = ctx or default_context()
    xs, ws = _i64(x_shape), _i64(w_shape)
    check(lib.mg_conv_f32_dev(ctx.handle, C.c_void_p(x_ptr), _ptr(xs), xs.size,
                              C.c_void_p(w_ptr), _ptr(ws), C.c_void_p(bias_ptr) if bias_ptr else None,
                              _ptr(_i64(strides)), _ptr(_i64(pads)), _ptr(_i64(dilations)),
                              int(group), _AUTO_PAD[auto_pad], C.c_void_p(y_ptr)))


def conv_transpose_f32_dev(x_ptr: int, x_shape, w_ptr: int, w_shape, y_ptr: int,
                           bias_ptr: int = 0, *, strides=None, pads=None, dilations=None,
                           output_padding=None, output_shape=None, group: int = 1,
                           ctx: Context | None = None):
    """op_conv_transpose on device buffers."""
    ctx = ctx or default_context()
    xs, ws, os_ = _i64(x_shape), _i64(w_shape), _i64(output_shape)
    check(lib.mg_conv_transpose_f32_dev(
        ctx.handle, C.c_void_p(x_ptr), _ptr(xs), xs.size, C.c_void_p(w_ptr), _ptr(ws),
        C.c_void_p(bias_ptr) if bias_ptr else None, _ptr(_i64(strides)), _ptr(_i64(pads)),
        _ptr(_i64(dilations)), _ptr(_i64(output_padding)), _ptr(os_),
        0 if os_ is None else os_.size, int(group), C.c_void_p(y_ptr)))


def conv_integer_dev(x_ptr: int, x_signed: bool, x_shape, w_ptr: int, w_signed: bool, w_shape,
                     y_ptr: int, x_zero_point: int = 0, w_zero_point=None, *, strides=None,
                     pads=None, dilations=None, group: int = 1, ctx: Context | None = None):
    """op_conv_integer on device buffers; y is int32."""
    ctx = ctx or default_context()
    xs, ws = _i64(x_shape), _i64(w_shape)
    wz, nwz = _zp_list(w_zero_point)
    check(lib.mg_conv_integer_dev(ctx.handle, C.c_void_p(x_ptr), int(x_signed), _ptr(xs),
                                  xs.size, C.c_void_p(w_ptr), int(w_signed), _ptr(ws),
                                  int(x_zero_point), _ptr(wz), nwz, _ptr(_i64(strides)),
                                  _ptr(_i64(pads)), _ptr(_i64(dilations)), int(group),
                                  C.c_void_p(y_ptr)))


def qlinear_conv_dev(x_ptr: int, x_signed: bool, x_shape, x_scale: float, x_zero_point: int,
                     w_ptr: int, w_signed: bool, w_shape, w_scale, w_zero_point,
                     y_scale: float, y_zero_point: int, y_ptr: int, bias_ptr: int = 0, *,
                     strides=None, pads=None, dilations=None, group: int = 1, lo: int, hi: int,
                     ctx: Context | None = None):
    """op_qlinear_conv on device buffers; y is bytes."""
    ctx = ctx or default_context()
    xs, ws = _i64(x_shape), _i64(w_shape)
    wz, nwz = _zp_list(w_zero_point)
    wsc = np.ascontiguousarray(np.asarray(w_scale, dtype=np.float32).ravel())
    check(lib.mg_qlinear_conv_dev(
        ctx.handle, C.c_void_p(x_ptr), int(x_signed), _ptr(xs), xs.size, float(x_scale),
        int(x_zero_point), C.c_void_p(w_ptr), int(w_signed), _ptr(ws), _ptr(wsc), wsc.size,
        _ptr(wz), nwz, float(y_scale), int(y_zero_point),
        C.c_void_p(bias_ptr) if bias_ptr else None, _ptr(_i64(strides)), _ptr(_i64(pads)),
        _ptr(_i64(dilations)), int(group), int(lo), int(hi), C.c_void_p(y_ptr)))


def library_path() -> str:
    return str(_lib.LIB_PATH)
