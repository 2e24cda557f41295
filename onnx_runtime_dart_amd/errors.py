"""Exceptions mirroring the ones the reference ops throw, keyed by mg_status.

ArgumentError / UnsupportedError / StateError are Dart core errors thrown by
lib/src/onnx_qlinear_ops.dart and lib/src/onnx_graph.dart; the two Onnx*
exceptions come from lib/src/execution_control.dart.
"""
from __future__ import annotations


class ArgumentError(ValueError):
    """MG_INVALID_ARGUMENT"""


class UnsupportedError(NotImplementedError):
    """MG_UNSUPPORTED"""


class OnnxMemoryLimitException(MemoryError):
    """MG_OUT_OF_MEMORY"""


class OnnxCancelledException(Exception):
    """MG_CANCELLED"""


class StateError(RuntimeError):
    """MG_DEVICE_ERROR"""


_BY_STATUS = {
    1: ArgumentError,
    2: UnsupportedError,
    3: OnnxMemoryLimitException,
    4: OnnxCancelledException,
    5: StateError,
}


def raise_for_status(status: int, message: str) -> None:
    raise _BY_STATUS.get(status, StateError)(message)
