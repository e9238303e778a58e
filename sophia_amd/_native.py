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

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libsophia_kda.so")

SOPHIA_OK = 0
SOPHIA_ERR_INVALID = 1
SOPHIA_ERR_HIP = 2
SOPHIA_ERR_WORKSPACE = 3

DTYPE_F32 = 0
DTYPE_BF16 = 1

QK_L2NORM = 1
GATE_IN_KERNEL = 2
BETA_SIGMOID = 4
SCAN_NO_SEGMENTS = 8
BWD_RECURRENT = 16

# Every symbol of include/sophia_kda.h and include/sophia_decoder.h, with its
# ctypes signature.
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_u32 = ctypes.c_uint
_sz = ctypes.c_size_t
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "sophia_last_error": (ctypes.c_char_p, []),
    "sophia_abi_version": (_i32, []),
    "sophia_short_conv_fwd": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _i32,
                                     _i64, _i32, _i32, _i32, _i32, _vp]),
    "sophia_short_conv_step": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _i32,
                                      _i32, _i32, _vp]),
    "sophia_short_conv_bwd_workspace_size": (_sz, [_i64, _i32, _i32]),
    "sophia_short_conv_bwd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp,
                                     _i32, _i64, _i32, _i32, _i32, _vp, _vp, _sz, _vp]),
    "sophia_kda_chunk_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "sophia_kda_chunk_fwd": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _i32,
                                    _vp, _vp, _f32, _f32, _u32, _vp, _vp, _i32, _i64, _i32, _i32,
                                    _vp, _vp, _i32, _vp, _vp, _i64, _vp, _sz, _vp]),
    "sophia_kda_chunk_fwd_no_alloc": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64,
                                             _i32, _vp, _vp, _f32, _f32, _u32, _vp, _vp, _i32, _i64,
                                             _i32, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _vp]),
    "sophia_kda_decode_step": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _i32,
                                      _vp, _vp, _f32, _f32, _u32, _vp, _i32, _vp, _i32, _i32, _i32,
                                      _i32, _vp, _i64, _vp]),
    "sophia_kda_decode_conv_step": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i64, _i32,
                                           _vp, _i64, _i32, _vp, _vp, _f32, _f32, _u32, _vp, _i32,
                                           _vp, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "sophia_kda_chunk_bwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "sophia_kda_chunk_bwd": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _i32,
                                    _vp, _vp, _f32, _f32, _u32, _vp, _i32, _i64, _i32, _i32,
                                    _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _vp, _vp, _sz, _vp]),
    "sophia_attn_res_mix": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _vp, _vp,
                                   _f32, _vp, _f32, _vp, _i64, _i64, _i32, _i32, _vp]),
    "sophia_situ_glu": (_i32, [_vp, _i64, _vp, _i64, _i64, _i32, _f32, _f32, _i32, _vp]),
    "sophia_gated_head_norm": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _f32, _vp, _i64, _i64, _i32,
                                      _i32, _i32, _vp]),
    "sophia_gated_head_norm_bwd_workspace_size": (_sz, [_i64, _i32, _i32]),
    "sophia_gated_head_norm_bwd": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _i64, _vp, _f32, _vp, _i64,
                                          _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _sz, _vp]),
    "sophia_mla_decode_workspace_size": (_sz, [_i64, _i32, _i32]),
    "sophia_causal_attention": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32,
                                       _i64, _i64, _i32, _i32, _i32, _f32, _i32, _vp]),
    "sophia_mla_decode_attn": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _f32, _vp,
                                      _i64, _i32, _i64, _i32, _i32, _i32, _vp, _sz, _vp]),
}

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
            handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
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
