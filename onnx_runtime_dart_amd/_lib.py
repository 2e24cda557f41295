"""ctypes binding of libmigemm.so (declarations: include/migemm.h).

The library is the only compute path: if it is missing or fails to load,
importing this module raises, and nothing falls back to CPU arithmetic.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

from .errors import raise_for_status

PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("MIGEMM_LIBRARY", PKG / "lib" / "libmigemm.so"))

_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_F = C.c_float
_SZ = C.c_size_t
_PP = C.POINTER(C.c_void_p)

# name -> argtypes (all return mg_status = int32 unless listed in _RESTYPE)
SIGNATURES = {
    "mg_last_error": [],
    "mg_last_error_budget": [_P, _P],
    "mg_version": [],
    "mg_ctx_create": [_I32, _PP],
    "mg_ctx_destroy": [_P],
    "mg_ctx_set_stream": [_P, _P],
    "mg_ctx_get_stream": [_P, _PP],
    "mg_ctx_synchronize": [_P],
    "mg_ctx_set_control": [_P, _P, _I64],
    "mg_ctx_set_profiling": [_P, _I32],
    "mg_ctx_set_prefill_images": [_P, _I32],
    "mg_ctx_profile_count": [_P, _P],
    "mg_ctx_profile_get": [_P, _I64, _P, _P],
    "mg_ctx_profile_clear": [_P],
    "mg_buffer_alloc": [_P, _SZ, _PP],
    "mg_buffer_free": [_P, _P],
    "mg_buffer_upload": [_P, _P, _P, _SZ],
    "mg_buffer_download": [_P, _P, _P, _SZ],
    "mg_weight_nbits_create": [_P, _I64, _I64, _I64, _I64, _P, _P, _I32, _P, _P, _I32,
                               _I32, _P, _P, _I32, _P, _P, _I32, _I32, _PP],
    "mg_matmul_nbits": [_P, _P, _P, _I64, _P],
    "mg_matmul_nbits_dev": [_P, _P, _P, _I64, _P],
    "mg_matmul_nbits_dev_noalloc": [_P, _P, _P, _I64, _P],
    "mg_matmul_nbits_group_dev": [_P, _I32, _P, _P, _I64, _P],
    "mg_matmul_nbits_group_split_dev": [_P, _I32, _P, _P, _P, _I64, _P],
    "mg_nbits_split_bytes": [_I64, _I64, _P],
    "mg_skip_rms_norm_f32_split_dev": [_P, _P, _P, _P, _I32, _P, _I64, _P, C.c_double, _P, _P,
                                       _I64, _P],
    "mg_weight_int8_create": [_P, _P, _I32, _I64, _I64, _P, _I64, _PP],
    "mg_matmul_integer": [_P, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I64, _P, _I64, _P],
    "mg_matmul_integer_i64": [_P, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I64, _P, _I64,
                              _P],
    "mg_matmul_integer_w": [_P, _P, _I32, _I64, _I64, _P, _I64, _P, _P],
    "mg_matmul_integer_w_dev": [_P, _P, _I32, _I64, _I64, _P, _I64, _P, _P],
    "mg_qlinear_matmul": [_P, _P, _I32, _P, _I32, _F, _P, _I64, _P, _I32, _P, _I32, _F, _P,
                          _I64, _F, _I32, _I32, _I32, _P],
    "mg_qlinear_matmul_w": [_P, _P, _I32, _I64, _I64, _F, _P, _I64, _P, _F, _F, _I32, _I32,
                            _I32, _P],
    "mg_qlinear_matmul_w_dev": [_P, _P, _I32, _I64, _I64, _F, _P, _I64, _P, _F, _F, _I32,
                                _I32, _I32, _P],
    "mg_dynamic_quantize_linear": [_P, _P, _I64, _P, _P, _P],
    "mg_dynamic_quantize_linear_dev": [_P, _P, _I64, _P, _P],
    "mg_binary_f32_dev": [_P, _I32, _P, _P, _I32, _P, _P, _I32, _P],
    "mg_sigmoid_f32_dev": [_P, _P, _I64, _P],
    "mg_rms_norm_f32_dev": [_P, _P, _P, _I32, _P, _I64, _I64, C.c_double, _P],
    "mg_skip_rms_norm_f32_dev": [_P, _P, _P, _P, _I32, _P, _I64, _P, C.c_double, _P, _P],
    "mg_matmul_integer_w_dq_dev": [_P, _P, _I64, _I64, _P, _P, _P],
    "mg_qlinear_matmul_w_dq_dev": [_P, _P, _I64, _I64, _P, _P, _F, _F, _I32, _I32, _I32, _P],
    "mg_fused_sdpa": [_P, _P, _P, _I32, _P, _P, _I32, _P, _P, _I32, _P, _P, _I32, _F, _P],
    "mg_fused_sdpa_dev": [_P, _P, _P, _I32, _P, _P, _I32, _P, _P, _I32, _P, _P, _I32, _F, _P],
    "mg_multi_head_attention": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P, _I32, _I32,
                                _F, _P],
    "mg_multi_head_attention_dev": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P, _I32,
                                    _I32, _F, _P],
    "mg_conv_output_shape": [_P, _I32, _P, _P, _P, _P, _I32, _I32, _P],
    "mg_conv_f32": [_P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _P],
    "mg_conv_f32_dev": [_P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _P],
    "mg_conv_transpose_output_shape": [_P, _I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _P],
    "mg_conv_transpose_f32": [_P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32,
                              _P],
    "mg_conv_transpose_f32_dev": [_P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I32,
                                  _I32, _P],
    "mg_conv_integer": [_P, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I64, _P, _P, _P,
                        _I32, _P],
    "mg_conv_integer_dev": [_P, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I64, _P, _P, _P,
                            _I32, _P],
    "mg_qlinear_conv": [_P, _P, _I32, _P, _I32, _F, _I32, _P, _I32, _P, _P, _I64, _P, _I64,
                        _F, _I32, _P, _P, _P, _P, _I32, _I32, _I32, _P],
    "mg_qlinear_conv_dev": [_P, _P, _I32, _P, _I32, _F, _I32, _P, _I32, _P, _P, _I64, _P,
                            _I64, _F, _I32, _P, _P, _P, _P, _I32, _I32, _I32, _P],
    "mg_weight_nbits_create_streamed": [_P, _I64, _I64, _I64, _I64, _P, _P, _I32, _P, _P, _I32,
                                        _I64, _PP],
    "mg_group_query_attention": [_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _P, _P, _I64,
                                 _P, _P, _I64, _I64, _I32, _I32, _P, _I32, _I32, _F, _F, _I32,
                                 _P, _P, _P],
    "mg_group_query_attention_dev": [_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _P, _P,
                                     _I64, _P, _P, _I64, _I64, _I32, _I32, _P, _I32, _I32, _F,
                                     _F, _I32, _P, _P, _P],
    "mg_matmul_f32": [_P, _P, _P, _I32, _P, _P, _I32, _P],
    "mg_matmul_f64acc": [_P, _P, _P, _I32, _P, _P, _I32, _P],
    "mg_matmul_f32_dev": [_P, _P, _P, _I32, _P, _P, _I32, _P],
    "mg_matmul_f32_output_shape": [_P, _I32, _P, _I32, _P, _P],
    "mg_matmul_f32_batch_offsets": [_P, _I32, _P, _I32, _I64, _I64, _P, _P, _P],
    "mg_gemm_f32": [_P, _P, _P, _P, _P, _I32, _I32, _F, _F, _P, _P, _I32, _P],
    "mg_weight_f32_create": [_P, _P, _I64, _I64, _I32, _PP],
    "mg_gemm_f32_w": [_P, _P, _I64, _I64, _P, _F, _F, _P, _P, _I32, _P],
    "mg_gemm_f32_w_dev": [_P, _P, _I64, _I64, _P, _F, _F, _P, _P, _I32, _P],
    "mg_weight_release": [_P],
    "mg_weight_info": [_P, C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64)],
}
_RESTYPE = {"mg_last_error": C.c_char_p, "mg_version": C.c_char_p}


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; run `python onnx_runtime_dart_amd/csrc/build.py` "
            "(or __graft_entry__.build()) first — there is no CPU fallback")
    lib = C.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, C.c_int32)
    return lib


lib = _load()


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib.mg_last_error().decode(errors="replace")
        budget = None
        if status == 3:
            req, lim = C.c_int64(0), C.c_int64(0)
            if lib.mg_last_error_budget(C.byref(req), C.byref(lim)):
                budget = (req.value, lim.value)
        raise_for_status(status, msg or what, budget)
