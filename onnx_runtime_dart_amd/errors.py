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
    """MG_OUT_OF_MEMORY from the byte budget, with the reference exception's
    fields (lib/src/execution_control.dart:12-19).  A device allocator
    failure is a StateError instead."""

    def __init__(self, message: str = "", required_bytes: int = 0, limit_bytes: int = 0):
        super().__init__(message)
        self.required_bytes = required_bytes
        self.limit_bytes = limit_bytes


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


def raise_for_status(status: int, message: str, budget=None) -> None:
    """budget: (required, limit) when an MG_OUT_OF_MEMORY came from the byte
    budget; None for a device allocator failure (-> StateError)."""
    if status == 3 and budget is None:
        raise StateError(message)
    if status == 3:
        raise OnnxMemoryLimitException(message, *budget)
    raise _BY_STATUS.get(status, StateError)(message)
