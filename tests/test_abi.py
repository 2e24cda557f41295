"""CPU-side checks of the drop-in boundary: the built library loads, exports
every entry point include/migemm.h declares, and the host-side operator layer
raises the reference's error classes before touching a device."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "migemm.h"
LIB = ROOT / "onnx_runtime_dart_amd" / "lib" / "libmigemm.so"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_operator_family():
    syms = declared_symbols()
    for s in ["mg_matmul_nbits", "mg_matmul_integer", "mg_qlinear_matmul",
              "mg_dynamic_quantize_linear", "mg_matmul_f32", "mg_gemm_f32",
              "mg_weight_nbits_create", "mg_ctx_create", "mg_last_error"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "run onnx_runtime_dart_amd/csrc/build.py first"
    lib = ctypes.CDLL(str(LIB))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_covers_every_symbol():
    from onnx_runtime_dart_amd import _lib
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_version_and_last_error_without_device():
    from onnx_runtime_dart_amd import _lib
    assert _lib.lib.mg_version() == b"0.1.0"
    assert isinstance(_lib.lib.mg_last_error(), bytes)


def test_status_codes_map_to_reference_exceptions():
    from onnx_runtime_dart_amd import errors as E
    for st, cls in [(1, E.ArgumentError), (2, E.UnsupportedError),
                    (4, E.OnnxCancelledException), (5, E.StateError)]:
        with pytest.raises(cls):
            E.raise_for_status(st, "x")
    # MG_OUT_OF_MEMORY: the byte budget carries the reference exception's
    # fields; a device allocator failure is a StateError.
    with pytest.raises(E.OnnxMemoryLimitException) as ei:
        E.raise_for_status(3, "x", (100, 16))
    assert (ei.value.required_bytes, ei.value.limit_bytes) == (100, 16)
    with pytest.raises(E.StateError):
        E.raise_for_status(3, "hipMalloc: out of memory")


def test_budget_query_without_a_failure():
    from onnx_runtime_dart_amd import _lib
    req = ctypes.c_int64(-1)
    assert _lib.lib.mg_last_error_budget(ctypes.byref(req), None) in (0, 1)


def test_host_validation_precedes_device_work():
    # Errors the reference raises before any arithmetic are raised here
    # before a context is created (no GPU in this container).
    from onnx_runtime_dart_amd import ops
    from onnx_runtime_dart_amd.errors import ArgumentError, UnsupportedError
    a = np.zeros((2, 64), np.float32)
    b = np.zeros((4, 2, 16), np.uint8)
    s = np.zeros(8, np.float32)
    with pytest.raises(UnsupportedError):  # onnx_qlinear_ops.dart:126-128
        ops.op_matmul_nbits(a, b, s, k=64, n=4, bits=8, block_size=32)
    with pytest.raises(ArgumentError):  # :129-136 block_size not a power of two
        ops.op_matmul_nbits(a, b, s, k=64, n=4, block_size=24)
    with pytest.raises(ArgumentError):  # a.shape.last != K
        ops.op_matmul_nbits(a, b, s, k=32, n=4, block_size=32)
    with pytest.raises(UnsupportedError):  # onnx_qlinear_ops.dart:88-90
        ops.op_qlinear_matmul(np.zeros((2, 2), np.uint8), np.ones(2), None,
                              np.zeros((2, 2), np.uint8), 1.0, None, 1.0, None,
                              lo=0, hi=255)


def test_no_kernel_uses_scratch_memory():
    """Every kernel keeps its state in registers and LDS: a stack copy (an
    escaped kernel argument, a non-inlined helper, a dynamically indexed
    array) costs scratch traffic on every access."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "mg_build", ROOT / "onnx_runtime_dart_amd" / "csrc" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if not list(mod.BUILD.glob("*.usage.txt")):
        pytest.skip("no resource report: run onnx_runtime_dart_amd/csrc/build.py")
    assert mod.kernels_with_scratch() == []


def test_every_entry_point_rejects_null_arguments():
    # Every status-returning entry point called with null pointers and zero
    # sizes returns a status (MG_OK for the release / destroy of nothing,
    # MG_INVALID_ARGUMENT otherwise) without touching a device or memory it
    # was not given.  Under tests/test_sanitizers.py this runs on the host
    # code built with AddressSanitizer and UndefinedBehaviorSanitizer.
    import ctypes as C
    from onnx_runtime_dart_amd import _lib
    ok_on_null = {"mg_weight_release", "mg_ctx_destroy", "mg_last_error_budget"}
    for name, argtypes in sorted(_lib.SIGNATURES.items()):
        if name in _lib._RESTYPE:
            continue
        args = [None if (t in (C.c_void_p, _lib._PP) or
                         (isinstance(t, type) and issubclass(t, C._Pointer))) else 0
                for t in argtypes]
        st = getattr(_lib.lib, name)(*args)
        assert st == (0 if name in ok_on_null else 1) or (name == "mg_last_error_budget"
                                                          and st in (0, 1)), (name, st)
