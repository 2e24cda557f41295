"""MI355X (gfx950) matrix-multiply operators for onnx_runtime_dart.

The compute lives in ``lib/libmigemm.so`` (HIP kernels behind the C ABI of
``include/migemm.h``); ``ops`` mirrors the reference's operator functions on
top of it.  Importing ``ops`` loads the library and fails loudly if it has not
been built — there is no CPU fallback.
"""
from .errors import (ArgumentError, OnnxCancelledException, OnnxMemoryLimitException,
                     StateError, UnsupportedError)

__all__ = ["ArgumentError", "UnsupportedError", "OnnxMemoryLimitException",
           "OnnxCancelledException", "StateError"]
