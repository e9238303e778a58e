"""The prefill entry point that allocates nothing (sophia_kda_chunk_fwd_no_alloc),
called through the C ABI, against sophia_kda_chunk_fwd with a workspace.

Both run the same kernels, so outputs and final states must be bit-identical.
Two calls in a row (the second with a smaller batch) check that the static
scratch left by the first call does not leak into the second.  A batch too
large for the static scratch is rejected on the host with
SOPHIA_ERR_WORKSPACE before any launch.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")

def _case(dev, lens, heads, seed):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lens)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32)
    q = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(dev)
    k = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(dev)
    z = (torch.randn(total, heads, 128, generator=gen) * 2.0).to(dev)
    b = torch.randn(total, heads, generator=gen).to(dev)
    a_log = (torch.randn(heads, generator=gen) * 0.5).to(dev)
    dtb = (torch.randn(heads * 128, generator=gen) - 4.0).to(dev)
    h0 = (torch.randn(len(lens), heads, 128, 128, generator=gen) * 0.05).to(dev)
    return dict(q=q, k=k, v=v, z=z, b=b, a_log=a_log, dtb=dtb, h0=h0, cu=cu.to(dev), cu_cpu=cu,
                total=total, n=len(lens), heads=heads)

def _call(c, *, no_alloc: bool, host_offsets: bool):
    from sophia_amd import _native as nat
    lib = nat.lib()
    total, n, heads = c["total"], c["n"], c["heads"]
    o = torch.full((total, heads, 128), 7.0, dtype=torch.bfloat16, device=c["q"].device)
    state = c["h0"].clone()
    stream = nat.stream_handle(c["q"].device)
    flags = nat.QK_L2NORM | nat.GATE_IN_KERNEL | nat.BETA_SIGMOID
    host = c["cu_cpu"].data_ptr() if host_offsets else None
    common = (nat.ptr(c["q"]), nat.ptr(c["k"]), nat.ptr(c["v"]), heads * 128, nat.DTYPE_BF16,
              nat.ptr(c["z"]), heads * 128, nat.DTYPE_F32, nat.ptr(c["b"]), heads, nat.DTYPE_F32,
              nat.ptr(c["a_log"]), nat.ptr(c["dtb"]), 128 ** -0.5, -5.0, flags, nat.ptr(c["cu"]),
              host, n, total, heads, 128, nat.ptr(state), nat.ptr(state), n, None, nat.ptr(o),
              heads * 128)
    if no_alloc:
        rc = lib.sophia_kda_chunk_fwd_no_alloc(*common, stream)
        nat.check(rc, "sophia_kda_chunk_fwd_no_alloc")
    else:
        need = int(lib.sophia_kda_chunk_workspace_size(total, n, heads, 128))
        ws = torch.empty(need + 256, dtype=torch.uint8, device=c["q"].device)
        addr = ws.data_ptr() + (-ws.data_ptr()) % 256
        rc = lib.sophia_kda_chunk_fwd(*common, addr, need, stream)
        nat.check(rc, "sophia_kda_chunk_fwd")
        torch.cuda.synchronize()
        del ws
    torch.cuda.synchronize()
    return o, state

def test_no_alloc_prefill_matches_workspace_prefill_twice():
    dev = _dev()
    big = _case(dev, [900, 1, 64, 700, 300], 16, seed=1)     # 33 chunks x 16 heads
    small = _case(dev, [129, 17], 16, seed=2)                # 4 chunks x 16 heads
    for case, host in ((big, True), (small, False)):
        o_ref, s_ref = _call(case, no_alloc=False, host_offsets=host)
        o, s = _call(case, no_alloc=True, host_offsets=host)
        assert torch.equal(o, o_ref), "outputs differ"
        assert torch.equal(s, s_ref), "final states differ"
        assert bool(torch.isfinite(o.float()).all())
    # the small call again right after the big one, through the same scratch
    o_ref, s_ref = _call(small, no_alloc=False, host_offsets=False)
    o, s = _call(small, no_alloc=True, host_offsets=False)
    assert torch.equal(o, o_ref) and torch.equal(s, s_ref)

def test_no_alloc_prefill_rejects_batches_beyond_the_static_scratch():
    from sophia_amd import _native as nat
    dev = _dev()
    lib = nat.lib()
    limit = 64 << 20
    heads, n = 16, 1
    total = 64 * 60                                          # 61 chunks x 16 heads > 903 records
    assert int(lib.sophia_kda_chunk_workspace_size(total, n, heads, 128)) > limit
    x = torch.zeros(1, dtype=torch.bfloat16, device=dev)
    cu = torch.tensor([0, total], dtype=torch.int32, device=dev)
    p = nat.ptr(x)
    rc = lib.sophia_kda_chunk_fwd_no_alloc(p, p, p, heads * 128, nat.DTYPE_BF16, p, heads * 128,
                                           nat.DTYPE_F32, p, heads, nat.DTYPE_F32, None, None,
                                           0.088, -5.0, 0, nat.ptr(cu), None, n, total, heads, 128,
                                           None, None, 0, None, p, heads * 128,
                                           nat.stream_handle(dev))
    assert rc == nat.SOPHIA_ERR_WORKSPACE
    assert "static buffer" in nat.last_error()
