"""Host-side argument checks of the torch-facing ops, and the call forms of
the reference's seam.

Every mis-sized tensor must raise RuntimeError on the host before a kernel
is launched (the reference's custom ops raise RuntimeError on bad arguments,
ml/training/pretrain/engine/sm120_concurrent_ffn.py:49-59).  The varlen call
form of FlashKDA (``chunk_kda(..., cu_seqlens=..., cu_seqlens_cpu=...)``,
sm120_concurrent_ffn.py:375-423) and a host ``cu_seqlens`` are checked
against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import kda_oracle as ko

pytestmark = pytest.mark.gpu

REL_TOL = 2e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _np(t):
    return t.detach().float().cpu().numpy()


def _inputs(dev, total, heads, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(dev)
    k = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(dev)
    g = (torch.rand(total, heads, 128, generator=gen) * -5.0).to(dev)
    beta = torch.rand(total, heads, generator=gen).to(dev)
    return q, k, v, g, beta


def test_chunk_fwd_rejects_mis_sized_tensors():
    from sophia_amd import ops
    dev = _dev()
    q, k, v, g, beta = _inputs(dev, 100, 2)
    cu = torch.tensor([0, 60, 100], dtype=torch.int32, device=dev)
    kw = dict(use_gate=False, use_beta_sigmoid=False)
    with pytest.raises(RuntimeError, match="out has 99 rows"):
        ops.kda_chunk_fwd(q, k, v, g, beta, cu, out=torch.empty(99, 2, 128, dtype=torch.bfloat16,
                                                                  device=dev), **kw)
    with pytest.raises(RuntimeError, match="beta has 99 rows"):
        ops.kda_chunk_fwd(q, k, v, g, beta[:99], cu, **kw)
    with pytest.raises(RuntimeError, match="state_slots must hold 2"):
        ops.kda_chunk_fwd(q, k, v, g, beta, cu, final_state=torch.zeros(4, 2, 128, 128, device=dev),
                          state_slots=torch.tensor([0, 1, 2], dtype=torch.int32, device=dev), **kw)
    with pytest.raises(RuntimeError, match="out must have q's dtype"):
        ops.kda_chunk_fwd(q, k, v, g, beta, cu, out=torch.empty(100, 2, 128, device=dev), **kw)
    with pytest.raises(RuntimeError):
        ops.kda_chunk_fwd(q, k, v[:99], g, beta, cu, **kw)


def test_decode_step_rejects_mis_sized_tensors():
    from sophia_amd import ops
    dev = _dev()
    q, k, v, g, beta = _inputs(dev, 4, 2)
    state = torch.zeros(6, 2, 128, 128, device=dev)
    kw = dict(use_gate=False, use_beta_sigmoid=False)
    for name, bad in (("k", (q, k[:3], v, g, beta)), ("v", (q, k, v[:3], g, beta)),
                      ("g", (q, k, v, g[:3], beta)), ("beta", (q, k, v, g, beta[:3]))):
        with pytest.raises(RuntimeError, match=f"{name} has 3 rows"):
            ops.kda_decode_step(*bad, state, **kw)
    with pytest.raises(RuntimeError, match="out has 5 rows"):
        ops.kda_decode_step(q, k, v, g, beta, state,
                            out=torch.empty(5, 2, 128, dtype=torch.bfloat16, device=dev), **kw)
    with pytest.raises(RuntimeError, match="state_slots must hold 4"):
        ops.kda_decode_step(q, k, v, g, beta, state,
                            state_slots=torch.tensor([0, 1], dtype=torch.int32, device=dev), **kw)
    assert bool((state == 0).all())  # nothing ran


def test_short_conv_rejects_mis_sized_tensors():
    from sophia_amd import ops
    dev = _dev()
    x = torch.randn(30, 64, device=dev)
    w = torch.randn(64, 4, device=dev)
    cu = torch.tensor([0, 10, 30], dtype=torch.int32, device=dev)
    cs = torch.zeros(3, 64, 3, device=dev)
    with pytest.raises(RuntimeError, match="out has 29 rows"):
        ops.short_conv_fwd(x, w, cu, out=torch.empty(29, 64, device=dev))
    with pytest.raises(RuntimeError, match="state_slots must hold 2"):
        ops.short_conv_fwd(x, w, cu, conv_state=cs, write_history=True,
                           state_slots=torch.tensor([0], dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError, match="out has 2 rows"):
        ops.short_conv_step(x[:3], w, cs, out=torch.empty(2, 64, device=dev))
    with pytest.raises(RuntimeError, match="fewer slots"):
        ops.short_conv_step(x[:4], w, cs)
    with pytest.raises(RuntimeError, match="state_slots must hold 3"):
        ops.short_conv_step(x[:3], w, cs, state_slots=torch.tensor([0, 1], dtype=torch.int32,
                                                                     device=dev))


def test_chunk_kda_varlen_call_form_matches_oracle():
    """ops.chunk_kda with FlashKDA's packed varlen arguments: q/k/v/g
    [1, total, H, 128], beta [1, total, H], device cu_seqlens plus the host
    copy cu_seqlens_cpu, gate / beta sigmoid / l2norm in the kernel, initial
    state per sequence, final state returned."""
    from sophia_amd import ops
    dev = _dev()
    rng = np.random.default_rng(40)
    lens = [300, 1, 129, 64, 0, 77]
    cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, heads, n = int(cu_np[-1]), 4, len(lens)
    bf = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16).to(dev)
    q, k, v = (bf(rng.standard_normal((1, total, heads, 128))) for _ in range(3))
    z = torch.tensor(rng.standard_normal((1, total, heads, 128)) * 2.0, dtype=torch.float32, device=dev)
    b = torch.tensor(rng.standard_normal((1, total, heads)), dtype=torch.float32, device=dev)
    a_log = torch.tensor(rng.standard_normal(heads) * 0.5, dtype=torch.float32)
    dtb = torch.tensor(ko.inverse_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), heads * 128))),
                       dtype=torch.float32)
    h0 = (rng.standard_normal((n, heads, 128, 128)) * 0.05).astype(np.float32)
    cu_cpu = torch.tensor(cu_np)
    o, ht = ops.chunk_kda(q, k, v, z, b, initial_state=torch.tensor(h0, device=dev),
                          output_final_state=True, use_qk_l2norm_in_kernel=True,
                          use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, safe_gate=True,
                          lower_bound=-5.0, A_log=a_log, dt_bias=dtb,
                          cu_seqlens=cu_cpu.to(dev), cu_seqlens_cpu=cu_cpu, chunk_size=64)
    assert tuple(o.shape) == (1, total, heads, 128) and o.dtype == torch.bfloat16
    assert tuple(ht.shape) == (n, heads, 128, 128) and ht.dtype == torch.float32
    o_ref, h_ref = c_oracle.kda_varlen(_np(q)[0], _np(k)[0], _np(v)[0], _np(z)[0], _np(b)[0], cu_np,
                                       A_log=a_log.numpy(), dt_bias=dtb.numpy(), initial_states=h0)
    assert _rel(_np(o)[0], o_ref) < REL_TOL
    assert _rel(_np(ht), h_ref) < REL_TOL
    # a host cu_seqlens alone: moved to the device and also used as the host copy
    o2, ht2 = ops.chunk_kda(q, k, v, z, b, initial_state=torch.tensor(h0, device=dev),
                            output_final_state=True, use_qk_l2norm_in_kernel=True,
                            use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                            safe_gate=True, lower_bound=-5.0, A_log=a_log, dt_bias=dtb,
                            cu_seqlens=cu_cpu)
    assert torch.equal(o, o2) and torch.equal(ht, ht2)


def test_kda_chunk_fwd_host_cu_seqlens_matches_oracle():
    """ops.kda_chunk_fwd given cu_seqlens on the host (the documented host
    path): the offsets move to the device and the host copy plans the launch."""
    from sophia_amd import ops
    dev = _dev()
    lens = [200, 5, 64]
    cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v, g, beta = _inputs(dev, int(cu_np[-1]), 2, seed=3)
    kw = dict(use_gate=False, use_beta_sigmoid=False)
    st = torch.zeros(3, 2, 128, 128, device=dev)
    o = ops.kda_chunk_fwd(q, k, v, g, beta, torch.tensor(cu_np), final_state=st, **kw)
    o_ref, h_ref = c_oracle.kda_varlen(_np(q), _np(k), _np(v), _np(g), _np(beta), cu_np, **kw)
    assert _rel(_np(o), o_ref) < REL_TOL and _rel(_np(st), h_ref) < REL_TOL


def test_chunk_kda_allow_neg_eigval_matches_oracle():
    """allow_neg_eigval with the beta sigmoid in the kernel: beta = 2 sigmoid(b)
    (sm120_concurrent_ffn.py:240-244).  Forward against the fp32 C oracle given
    that beta; the gradient of the raw b against the float64 oracle backward
    times 2 s (1 - s)."""
    from sophia_amd import ops
    dev = _dev()
    rng = np.random.default_rng(41)
    lens = [130, 70]
    cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, heads = int(cu_np[-1]), 2
    f32 = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)
    q, k, v = (f32(rng.standard_normal((1, total, heads, 128))) for _ in range(3))
    g = f32(rng.uniform(-1.0, 0.0, (1, total, heads, 128)))
    b = f32(rng.standard_normal((1, total, heads)) * 1.5).requires_grad_(True)
    cu_cpu = torch.tensor(cu_np)
    o, ht = ops.chunk_kda(q, k, v, g, b, output_final_state=True, use_qk_l2norm_in_kernel=True,
                          use_beta_sigmoid_in_kernel=True, allow_neg_eigval=True, safe_gate=True,
                          lower_bound=-5.0, cu_seqlens=cu_cpu.to(dev), cu_seqlens_cpu=cu_cpu)
    beta_eff = 2.0 / (1.0 + np.exp(-_np(b)[0].astype(np.float64)))
    assert beta_eff.max() > 1.5      # the case reaches negative eigenvalues of I - beta k k^T
    o_ref, h_ref = c_oracle.kda_varlen(_np(q)[0], _np(k)[0], _np(v)[0], _np(g)[0], beta_eff, cu_np,
                                       use_qk_l2norm=True, use_gate=False, use_beta_sigmoid=False)
    assert _rel(_np(o)[0], o_ref) < REL_TOL
    assert _rel(_np(ht), h_ref) < REL_TOL
    w = torch.tensor(rng.standard_normal((1, total, heads, 128)), dtype=torch.float32, device=dev)
    (o * w).sum().backward()
    ref = ko.kda_varlen_bwd(_np(q)[0], _np(k)[0], _np(v)[0], _np(g)[0], beta_eff, cu_np, _np(w)[0],
                            use_qk_l2norm=True, use_gate=False, use_beta_sigmoid=False)
    s = beta_eff / 2.0
    db_ref = ref["dbeta"] * 2.0 * s * (1.0 - s)
    # the autograd path runs the chunk form of the backward (bf16 MFMA
    # operands in its chunk scans): the bound of test_gpu_kda_bwd's chunk tests
    assert _rel(_np(b.grad)[0], db_ref) < 1.5e-2


def test_chunk_kda_state_v_first_is_the_transposed_state():
    """state_v_first: states in and out as [N, H, V, K].  Bit-equal to the
    default layout with the states transposed, forward and initial-state
    gradient."""
    from sophia_amd import ops
    dev = _dev()
    rng = np.random.default_rng(42)
    lens = [100, 37]
    cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, heads, n = int(cu_np[-1]), 2, len(lens)
    f32 = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)
    q, k, v = (f32(rng.standard_normal((1, total, heads, 128))) for _ in range(3))
    g = f32(rng.uniform(-2.0, 0.0, (1, total, heads, 128)))
    b = f32(rng.uniform(0.0, 1.0, (1, total, heads)))
    h0 = f32(rng.standard_normal((n, heads, 128, 128)) * 0.1)
    cu_cpu = torch.tensor(cu_np)
    kw = dict(output_final_state=True, use_qk_l2norm_in_kernel=True, safe_gate=True, lower_bound=-5.0,
              cu_seqlens=cu_cpu.to(dev), cu_seqlens_cpu=cu_cpu)
    o1, h1 = ops.chunk_kda(q, k, v, g, b, initial_state=h0, **kw)
    o2, h2 = ops.chunk_kda(q, k, v, g, b, initial_state=h0.transpose(-1, -2).contiguous(),
                           state_v_first=True, **kw)
    assert torch.equal(o1, o2) and torch.equal(h1, h2.transpose(-1, -2))
    a1 = h0.clone().requires_grad_(True)
    a2 = h0.transpose(-1, -2).contiguous().requires_grad_(True)
    w = f32(rng.standard_normal((1, total, heads, 128)))
    (ops.chunk_kda(q, k, v, g, b, initial_state=a1, **kw)[0] * w).sum().backward()
    (ops.chunk_kda(q, k, v, g, b, initial_state=a2, state_v_first=True, **kw)[0] * w).sum().backward()
    assert torch.equal(a1.grad, a2.grad.transpose(-1, -2))
