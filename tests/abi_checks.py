"""Host-side checks of the C ABI, shared by tests/test_abi.py (the built
library, through sophia_amd._native) and tests/test_abi_sanitized.py (a build
with the host code under ASan/UBSan, in a process without torch).  No call
here launches a kernel: each returns at a size query or an argument check.
"""

from __future__ import annotations

import ctypes
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declarations() -> dict[str, int]:
    """name -> number of parameters, for every function the headers declare."""
    decls = {}
    for header in HEADERS:
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(sophia_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            name, params = m.group(1), m.group(2).strip()
            assert name not in decls, f"{name} declared twice"
            decls[name] = 0 if params in ("", "void") else len(params.split(","))
    return decls


def check_exports(path: str, signatures: dict) -> None:
    """The library at ``path`` exports every declared symbol, and the ctypes
    table has one signature per declaration with the same argument count."""
    handle = ctypes.CDLL(path)
    decls = declarations()
    for name, nparams in decls.items():
        assert hasattr(handle, name), f"{name} not exported"
        assert name in signatures, f"{name} has no ctypes signature"
        assert len(signatures[name][1]) == nparams, f"{name}: argument count differs"
    assert set(signatures) == set(decls)


def check_host_side(lib, nat) -> None:
    """Size queries and argument validation of every entry point (host side only:
    each call returns before any launch).  ``nat`` holds the status codes and a
    ``last_error()``."""
    assert lib.sophia_abi_version() >= 100
    # 8 sequences, 17,408 tokens, 16 heads: header + one record per (chunk, head).
    ws = lib.sophia_kda_chunk_workspace_size(17408, 8, 16, 128)
    assert ws > 0
    assert lib.sophia_kda_chunk_workspace_size(2 * 17408, 8, 16, 128) > ws
    assert lib.sophia_kda_chunk_workspace_size(17408, 8, 16, 64) == 0
    assert lib.sophia_kda_chunk_workspace_size(100, 0, 16, 128) == 0
    # head_dim 64 is rejected on the host before any launch.
    rc = lib.sophia_kda_decode_step(None, None, None, 2048, 1, None, 2048, 0, None, 16, 0, None,
                                    None, 1.0, -5.0, 7, None, 1, None, 1, 1, 16, 64, None, 2048,
                                    None)
    assert rc == nat.SOPHIA_ERR_INVALID
    assert "head_dim" in nat.last_error()
    rc = lib.sophia_short_conv_fwd(None, 6144, None, 6144, 1, None, None, 0, None, None, 1, 10,
                                   6143, 4, 0, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID
    assert "channels" in nat.last_error()
    rc = lib.sophia_kda_chunk_fwd(None, None, None, 2048, 1, None, 2048, 0, None, 16, 0, None,
                                  None, 1.0, -6.0, 7, None, None, 1, 0, 16, 128, None, None, 0,
                                  None, None, 2048, None, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID
    # A host copy of the offsets that is not non-decreasing within [0, total].
    host = (ctypes.c_int32 * 3)(0, 70, 40)
    rc = lib.sophia_kda_chunk_fwd(16, 32, 48, 2048, 1, 64, 2048, 0, 80, 16, 0, None, None, 1.0,
                                  -5.0, 1, 96, ctypes.addressof(host), 2, 100, 16, 128, None,
                                  None, 0, None, 256, 2048, 512, 1 << 30, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "cu_seqlens_host" in nat.last_error()
    # The fused-conv prefill: kernel size 4 and bf16 rows only; rows whose
    # stride is not a multiple of 8 elements cannot be copied whole.
    conv = lambda *a: lib.sophia_kda_conv_chunk_fwd(*a)  # noqa: E731
    cargs = [16, 32, 48, 6160, 1, 64, 128, 4, 0, 80, 2048, 0, 96, 16, 0, None, None, 1.0, -5.0, 1, 112,
             None, 2, 100, 16, 128, None, None, 0, None, 256, 2048, 512, 1 << 30, None]
    a = list(cargs)
    a[7] = 3
    assert conv(*a) == nat.SOPHIA_ERR_INVALID and "kernel_size" in nat.last_error()
    a = list(cargs)
    a[4] = 0
    assert conv(*a) == nat.SOPHIA_ERR_INVALID and "bf16" in nat.last_error()
    a = list(cargs)
    a[5] = 68
    assert conv(*a) == nat.SOPHIA_ERR_INVALID and "conv_weight" in nat.last_error()
    a = list(cargs)
    a[3] = 6164
    assert conv(*a) == nat.SOPHIA_ERR_INVALID and "stride" in nat.last_error()
    # Decoder kernels: dim not a multiple of 8, too deep, too wide, misaligned.
    mix = lambda *a: lib.sophia_attn_res_mix(*a)  # noqa: E731
    rc = mix(None, 1536, None, 0, None, 0, None, 0, 0, 0, None, None, 1e-5, None, 1e-5, None,
             1536, 4, 1532, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "dim" in nat.last_error()
    rc = mix(None, 1536, None, 0, None, 0, None, 0, 0, 16, None, None, 1e-5, None, 1e-5, None,
             1536, 4, 1536, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "n_blocks" in nat.last_error()
    rc = mix(None, 8192, None, 0, None, 0, None, 0, 0, 0, None, None, 1e-5, None, 1e-5, None,
             8192, 4, 8192, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "dim" in nat.last_error()
    rc = mix(8, 1536, None, 0, None, 0, None, 0, 0, 0, 16, 32, 1e-5, None, 1e-5, 64, 1536, 4,
             1536, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "aligned" in nat.last_error()
    # A residual needs somewhere to write the new partial block.
    rc = mix(16, 1536, 32, 1536, None, 0, None, 0, 0, 0, 48, 64, 1e-5, None, 1e-5, 80, 1536, 4,
             1536, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "partial_out" in nat.last_error()
    # No rows: nothing to launch, no pointer needed.
    assert mix(None, 1536, None, 0, None, 0, None, 3 * 1536, 1536, 3, None, None, 1e-5, None,
               1e-5, None, 1536, 0, 1536, 1, None) == nat.SOPHIA_OK
    rc = lib.sophia_situ_glu(None, 7936, None, 3968, 4, 3964, 4.0, 25.0, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "hidden" in nat.last_error()
    rc = lib.sophia_situ_glu(None, 7936, None, 3968, 4, 3968, 0.0, 25.0, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID
    # Non-null addresses that are never dereferenced: the stride check fails first.
    rc = lib.sophia_situ_glu(16, 3968, 32, 3968, 4, 3968, 4.0, 25.0, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "stride" in nat.last_error()
    rc = lib.sophia_gated_head_norm(16, 2048, 1, 32, 2048, None, 1e-5, 48, 2048, 4, 16, 96, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "head_dim" in nat.last_error()
    rc = lib.sophia_gated_head_norm(16, 2048, 1, 40, 2048, None, 1e-5, 48, 2048, 4, 16, 128, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "aligned" in nat.last_error()
    rc = lib.sophia_gated_head_norm(16, 2048, 1, 32, 2047, None, 1e-5, 48, 2048, 4, 16, 128, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "stride" in nat.last_error()
    rc = lib.sophia_gated_head_norm(16, 2048, 1, 32, 2048, None, 1e-5, 48, 2048, 4, 16, 128, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "dtype" in nat.last_error()
    # MLA decode: rank 96 and 17 heads are rejected; splits need a workspace.
    assert lib.sophia_mla_decode_workspace_size(240, 128, 1) == 0
    assert lib.sophia_mla_decode_workspace_size(240, 128, 3) == 240 * 3 * 16 * 130 * 4
    rc = lib.sophia_mla_decode_attn(16, 2048, 1, 32, 2048 * 96, 8, 2048, 48, 64, 0.1, 80, 2048, 1, 4,
                                    16, 96, 1, None, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "rank" in nat.last_error()
    rc = lib.sophia_mla_decode_attn(16, 4096, 1, 32, 2048 * 128, 8, 2048, 48, 64, 0.1, 80, 4096, 1,
                                    4, 17, 128, 1, None, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "heads" in nat.last_error()
    rc = lib.sophia_mla_decode_attn(16, 2048, 1, 32, 2048 * 128, 8, 2048, 48, 64, 0.1, 80, 2048, 1, 4,
                                    16, 128, 3, None, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "workspace" in nat.last_error()
    # Causal attention: bf16 and head_dim 128 only.
    rc = lib.sophia_causal_attention(16, 2048, 32, 2048, 48, 2048, 64, 2048, 80, None, 2, 100, 0, 64,
                                     16, 128, 0.08, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "bf16" in nat.last_error()
    rc = lib.sophia_causal_attention(16, 1024, 32, 1024, 48, 1024, 64, 1024, 80, None, 2, 100, 0, 64,
                                     16, 64, 0.08, 1, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "head_dim" in nat.last_error()
    # KDA backward: size query, head_dim, gate-parameter outputs without the
    # gate, short workspace (all rejected before any launch).
    bws = lib.sophia_kda_chunk_bwd_workspace_size(1000, 3, 16, 128)
    assert bws > lib.sophia_kda_chunk_bwd_workspace_size(500, 3, 16, 128) > 0
    assert lib.sophia_kda_chunk_bwd_workspace_size(1000, 3, 16, 64) == 0
    assert lib.sophia_kda_chunk_bwd_workspace_size(1000, 0, 16, 128) == 0
    bwd = lambda *a: lib.sophia_kda_chunk_bwd(*a)  # noqa: E731
    args = [16, 32, 48, 2048, 1, 64, 2048, 0, 80, 16, 0, None, None, 0.08, -5.0, 0, 96, 3, 1000,
            16, 128, None, 112, 2048, 1, None, 128, 144, 160, 176, 192, None, None, None, 256,
            bws, None]
    a = list(args)
    a[20] = 64
    assert bwd(*a) == nat.SOPHIA_ERR_INVALID and "head_dim" in nat.last_error()
    a = list(args)
    a[32] = 240
    assert bwd(*a) == nat.SOPHIA_ERR_INVALID and "dA_log" in nat.last_error()
    a = list(args)
    a[35] = bws - 1
    assert bwd(*a) == nat.SOPHIA_ERR_WORKSPACE
    a = list(args)
    a[3] = 2047
    assert bwd(*a) == nat.SOPHIA_ERR_INVALID and "stride" in nat.last_error()
    # ShortConv backward: channels, short workspace; gated-norm backward:
    # head_dim, a norm weight without a workspace.
    cws = lib.sophia_short_conv_bwd_workspace_size(1000, 6144, 4)
    assert cws >= 8 * 6144 * 4 * 4 and lib.sophia_short_conv_bwd_workspace_size(1000, 6144, 5) == 0
    rc = lib.sophia_short_conv_bwd(16, 6144, 32, 6144, 48, 6144, 1, 64, None, 0, None, 80, 1, 1000, 6142, 4, 0,
                                   96, 128, cws, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "channels" in nat.last_error()
    rc = lib.sophia_short_conv_bwd(16, 6144, 32, 6144, 48, 6144, 1, 64, None, 0, None, 80, 1, 1000, 6144, 4, 0,
                                   96, 128, cws - 4, None)
    assert rc == nat.SOPHIA_ERR_WORKSPACE
    gws = lib.sophia_gated_head_norm_bwd_workspace_size(100, 16, 128)
    assert gws > 0
    gnb = lambda *a: lib.sophia_gated_head_norm_bwd(*a)  # noqa: E731
    rc = gnb(16, 2048, 32, 2048, 1, 48, 2048, None, 1e-5, 64, 2048, 80, 2048, None, 100, 4, 512, 1, None, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "head_dim" in nat.last_error()
    rc = gnb(16, 2048, 32, 2048, 1, 48, 2048, 96, 1e-5, 64, 2048, 80, 2048, 112, 100, 16, 128, 1, None, 0, None)
    assert rc == nat.SOPHIA_ERR_INVALID and "workspace" in nat.last_error()
