"""ctypes binding of the HIP library ``sophia_amd/_lib/libsophia_kda.so``.

The library exports the C ABI declared in ``include/sophia_kda.h`` and
``include/sophia_decoder.h``.  torch is
imported first so that the library binds to the HIP runtime torch already
loaded (same soname), which keeps torch streams and device pointers valid for
the kernels.  There is no fallback: if the library is missing or fails to
load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

from ._abi import SIGNATURES, bind  # noqa: F401  (the ctypes table of the C ABI)
from ._abi import (  # noqa: F401
    SOPHIA_OK,
    SOPHIA_ERR_INVALID,
    SOPHIA_ERR_HIP,
    SOPHIA_ERR_WORKSPACE,
    DTYPE_F32,
    DTYPE_BF16,
    QK_L2NORM,
    GATE_IN_KERNEL,
    BETA_SIGMOID,
    SCAN_NO_SEGMENTS,
    BWD_RECURRENT,
    BWD_GRAD_BF16,
)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libsophia_kda.so")

_lib = None
_lock = threading.Lock()


class SophiaNativeError(RuntimeError):
    """Raised when the HIP library is missing or an entry point fails."""


def lib():
    """The loaded library (loads it on first use; raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise SophiaNativeError(
                    f"sophia_amd HIP library not found at {LIB_PATH}; build it with "
                    "`python -m sophia_amd.build` (hipcc, gfx950)")
            _lib = bind(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    return _lib


def last_error() -> str:
    msg = lib().sophia_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != SOPHIA_OK:
        raise SophiaNativeError(f"{what} failed (code {rc}): {last_error()}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise RuntimeError(f"sophia_amd kernels take float32 or bfloat16 tensors, got {dtype}")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
