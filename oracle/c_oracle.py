"""ctypes binding of the C oracle (oracle/kda_ref.c).  Test infrastructure only."""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build as _build

_LIB = None
QK_L2NORM, GATE, BETA_SIGMOID = 1, 2, 4


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_build.LIB_PATH):
            _build.build()
        lib = ctypes.CDLL(_build.LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        ip = ctypes.POINTER(ctypes.c_int32)
        lib.oracle_kda_varlen_f32.argtypes = [fp, fp, fp, fp, fp, fp, fp, ctypes.c_float,
                                              ctypes.c_float, ctypes.c_int, ip, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp,
                                              fp, ctypes.c_int]
        lib.oracle_kda_varlen_f32.restype = ctypes.c_int
        lib.oracle_kda_varlen_bwd_f32.argtypes = [fp, fp, fp, fp, fp, fp, fp, ctypes.c_float,
                                                  ctypes.c_float, ctypes.c_int, ip, ctypes.c_int,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, fp, fp,
                                                  fp, fp, fp, fp, fp, fp, fp, fp, fp, ctypes.c_int]
        lib.oracle_kda_varlen_bwd_f32.restype = ctypes.c_int
        lib.oracle_max_threads.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def max_threads() -> int:
    return int(_lib().oracle_max_threads())


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a, ctype=ctypes.c_float):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctype))


def kda_varlen(q, k, v, g, beta, cu_seqlens, *, A_log=None, dt_bias=None, lower_bound=-5.0,
               initial_states=None, use_qk_l2norm=True, use_gate=True, use_beta_sigmoid=True,
               scale=None, nthreads=0):
    """Same contract as kda_oracle.kda_varlen, fp32, in C."""
    q, k, v, g, beta = (_f32(x) for x in (q, k, v, g, beta))
    total, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    n = int(cu.shape[0]) - 1
    if scale is None:
        scale = key_dim ** -0.5
    flags = (QK_L2NORM if use_qk_l2norm else 0) | (GATE if use_gate else 0) | (
        BETA_SIGMOID if use_beta_sigmoid else 0)
    a_log = _f32(A_log) if use_gate else None
    dtb = _f32(dt_bias) if use_gate else None
    h0 = _f32(initial_states)
    o = np.zeros((total, heads, value_dim), dtype=np.float32)
    ht = np.zeros((n, heads, key_dim, value_dim), dtype=np.float32)
    rc = _lib().oracle_kda_varlen_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(a_log),
                                      _ptr(dtb), float(lower_bound), float(scale), flags,
                                      _ptr(cu, ctypes.c_int32), n, heads, key_dim, value_dim,
                                      _ptr(h0), _ptr(o), _ptr(ht), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle_kda_varlen_f32 failed with {rc}")
    return o, ht


def kda_varlen_bwd(q, k, v, g, beta, cu_seqlens, d_out, *, d_final_states=None, A_log=None,
                   dt_bias=None, lower_bound=-5.0, initial_states=None, use_qk_l2norm=True,
                   use_gate=True, use_beta_sigmoid=True, scale=None, nthreads=0):
    """Same contract as kda_oracle.kda_varlen_bwd, fp32, in C."""
    q, k, v, g, beta, d_out = (_f32(x) for x in (q, k, v, g, beta, d_out))
    total, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    n = int(cu.shape[0]) - 1
    if scale is None:
        scale = key_dim ** -0.5
    flags = (QK_L2NORM if use_qk_l2norm else 0) | (GATE if use_gate else 0) | (
        BETA_SIGMOID if use_beta_sigmoid else 0)
    a_log = _f32(A_log) if use_gate else None
    dtb = _f32(dt_bias) if use_gate else None
    h0 = _f32(initial_states)
    dht = _f32(d_final_states)
    out = {name: np.zeros(shape, dtype=np.float32) for name, shape in (
        ("dq", q.shape), ("dk", k.shape), ("dv", v.shape), ("dg", g.shape), ("dbeta", beta.shape),
        ("dh0", (n, heads, key_dim, value_dim)))}
    da = np.zeros((n, heads), dtype=np.float32)
    dbias = np.zeros((n, heads, key_dim), dtype=np.float32)
    rc = _lib().oracle_kda_varlen_bwd_f32(
        _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(a_log), _ptr(dtb), float(lower_bound),
        float(scale), flags, _ptr(cu, ctypes.c_int32), n, heads, key_dim, value_dim, _ptr(h0),
        _ptr(d_out), _ptr(dht), _ptr(out["dq"]), _ptr(out["dk"]), _ptr(out["dv"]), _ptr(out["dg"]),
        _ptr(out["dbeta"]), _ptr(out["dh0"]), _ptr(da), _ptr(dbias), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle_kda_varlen_bwd_f32 failed with {rc}")
    if use_gate:
        out["dA_log"] = da.sum(axis=0)
        out["ddt_bias"] = dbias.sum(axis=0).reshape(heads * key_dim)
    return out
