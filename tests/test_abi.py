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
                 "sophia_short_conv_bwd", "sophia_gated_head_norm_bwd", "sophia_kda_conv_chunk_fwd"):
        assert name in decls, name


def test_header_constants_match_the_binding():
    """Every status code, element type and flag bit #defined in
    include/sophia_kda.h has the value the ctypes table binds."""
    import re
    from sophia_amd import _abi
    path = os.path.join(os.path.dirname(__file__), "..", "include", "sophia_kda.h")
    defs = {m.group(1): int(m.group(2)) for m in
            re.finditer(r"^#define SOPHIA_(\w+) (\d+)u?\b", open(path).read(), re.M)}
    names = {"OK": "SOPHIA_OK", "ERR_INVALID": "SOPHIA_ERR_INVALID", "ERR_HIP": "SOPHIA_ERR_HIP",
             "ERR_WORKSPACE": "SOPHIA_ERR_WORKSPACE", "DTYPE_F32": "DTYPE_F32", "DTYPE_BF16": "DTYPE_BF16",
             "KDA_QK_L2NORM": "QK_L2NORM", "KDA_GATE_IN_KERNEL": "GATE_IN_KERNEL",
             "KDA_BETA_SIGMOID": "BETA_SIGMOID", "KDA_SCAN_NO_SEGMENTS": "SCAN_NO_SEGMENTS",
             "KDA_BWD_RECURRENT": "BWD_RECURRENT", "KDA_BWD_GRAD_BF16": "BWD_GRAD_BF16"}
    assert set(defs) == set(names), sorted(set(defs) ^ set(names))
    for hname, pname in names.items():
        assert defs[hname] == getattr(_abi, pname), hname
    flags = [v for k, v in defs.items() if k.startswith("KDA_")]
    assert len(set(flags)) == len(flags) and all(f & (f - 1) == 0 for f in flags)


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
