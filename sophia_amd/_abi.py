"""The C ABI of ``libsophia_kda.so`` as a ctypes table, with no torch import.

Status codes, element types and flag bits of include/sophia_kda.h and every
entry point of include/sophia_kda.h and include/sophia_decoder.h with its
ctypes signature.  ``sophia_amd._native`` binds the library through this
table; the CPU tests also bind a host-sanitized build of the library with it
(torch is not loaded into that process).
"""

from __future__ import annotations

import ctypes

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
BWD_GRAD_BF16 = 32

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
    "sophia_kda_conv_chunk_fwd": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _vp, _i64, _i32,
                                         _vp, _i64, _i32, _vp, _vp, _f32, _f32, _u32, _vp, _vp, _i32,
                                         _i64, _i32, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _sz, _vp]),
    "sophia_mla_latent_norms": (_i32, [_vp, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _f32, _vp, _f32,
                                       _vp, _i32, _i32, _i64, _vp, _i32, _vp, _vp, _vp, _vp, _vp]),
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



def bind(path: str, mode: int = ctypes.DEFAULT_MODE) -> ctypes.CDLL:
    """Load the library at ``path`` and set every entry point's signature."""
    handle = ctypes.CDLL(path, mode=mode)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle
