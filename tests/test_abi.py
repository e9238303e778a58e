"""The C-ABI library loads and exports every entry point that the headers
under include/ declare, with the argument counts the ctypes binding uses.  CPU only: the calls made here are host-side (version, workspace-size
query, argument validation) and never launch a kernel.
"""

from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def _declarations() -> dict[str, int]:
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


def _lib():
    from sophia_amd import _native
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("HIP library not built (run `python -m sophia_amd.build`)")
    return _native


def test_header_declares_the_entry_points():
    decls = _declarations()
    for name in ("sophia_short_conv_fwd", "sophia_short_conv_step", "sophia_kda_chunk_fwd",
                 "sophia_kda_chunk_workspace_size", "sophia_kda_decode_step",
                 "sophia_last_error", "sophia_abi_version", "sophia_attn_res_mix",
                 "sophia_situ_glu", "sophia_gated_head_norm", "sophia_mla_decode_attn",
                 "sophia_mla_decode_workspace_size", "sophia_causal_attention"):
        assert name in decls, name


def test_library_exports_every_declared_symbol():
    nat = _lib()
    handle = ctypes.CDLL(nat.LIB_PATH)
    decls = _declarations()
    for name, nparams in decls.items():
        assert hasattr(handle, name), f"{name} not exported"
        assert name in nat.SIGNATURES, f"{name} has no ctypes signature"
        assert len(nat.SIGNATURES[name][1]) == nparams, f"{name}: argument count differs"
    assert set(nat.SIGNATURES) == set(decls)


def test_host_side_queries_and_validation():
    nat = _lib()
    lib = nat.lib()
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


def test_ops_reject_cpu_tensors():
    import torch
    from sophia_amd import ops
    x = torch.zeros(4, 16, 128)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.kda_chunk_fwd(x, x, x, x, torch.zeros(4, 16), torch.tensor([0, 4], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.kda_decode_step(x, x, x, x, torch.zeros(4, 16), torch.zeros(4, 16, 128, 128))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.kda_chunk_bwd(x, x, x, x, torch.zeros(4, 16), torch.tensor([0, 4], dtype=torch.int32), x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.short_conv_fwd(torch.zeros(4, 8), torch.zeros(8, 4),
                           torch.tensor([0, 4], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attn_res_mix(torch.zeros(4, 64), torch.zeros(4, 2, 64), torch.ones(64),
                         torch.zeros(64), 1e-5)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.situ_glu(torch.zeros(4, 64), 4.0, 25.0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.gated_head_norm(torch.zeros(4, 256), torch.zeros(4, 256), 2, 128)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.mla_decode_attn(torch.zeros(4, 2, 32), torch.zeros(4, 8, 32),
                            torch.zeros(4, dtype=torch.int32), torch.zeros(4, dtype=torch.int64), 0.1)
