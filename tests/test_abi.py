"""The C-ABI library loads and exports every entry point that the headers
under include/ declare, with the argument counts the ctypes binding uses.  CPU only: the calls made here are host-side (version, workspace-size
query, argument validation) and never launch a kernel.
"""

from __future__ import annotations

import os

import pytest

import abi_checks



def _lib():
    from sophia_amd import _native
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("HIP library not built (run `python -m sophia_amd.build`)")
    return _native


def test_header_declares_the_entry_points():
    decls = abi_checks.declarations()
    for name in ("sophia_short_conv_fwd", "sophia_short_conv_step", "sophia_kda_chunk_fwd",
                 "sophia_kda_chunk_workspace_size", "sophia_kda_decode_step",
                 "sophia_last_error", "sophia_abi_version", "sophia_attn_res_mix",
                 "sophia_situ_glu", "sophia_gated_head_norm", "sophia_mla_decode_attn",
                 "sophia_mla_decode_workspace_size", "sophia_causal_attention",
                 "sophia_short_conv_bwd", "sophia_gated_head_norm_bwd"):
        assert name in decls, name


def test_library_exports_every_declared_symbol():
    nat = _lib()
    abi_checks.check_exports(nat.LIB_PATH, nat.SIGNATURES)


def test_host_side_queries_and_validation():
    nat = _lib()
    abi_checks.check_host_side(nat.lib(), nat)


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
