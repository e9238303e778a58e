"""GPU parity at the exact shapes the benchmarks time.

The launch plan of the chunk prefill (value-column slices per (sequence,
head), scan order) depends on the batch: the 8-sequence packed batch of the
prefill benchmark with its host offsets, and the 16 x 1,024-token prefill of
the continuous-batching decoder step with device offsets, each run a kernel
variant that small test batches never reach.  These tests run those exact
calls and compare every sequence's output and final state with the fp32
oracle (tolerance per tensor: max|y - y_ref| / max|y_ref| <= 2e-2).

The backward benchmark's call (the same batch, a bf16 output gradient) is
checked here too, the chunk form against the fp32 recurrent form.

Also here: a long slow-decay prefill (gates drawn the way SophiaKDA's
initialisation draws them, ml/runtime/model/attention.py:101-106: A_log = 0,
dt log-uniform in [1e-3, 1e-1], so g = -5 sigmoid(z + dt_bias) is mostly in
[-0.5, -0.005], the long-memory regime where state errors persist).
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


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _per_sequence(o, o_ref, st, h_ref, cu, what):
    worst = 0.0
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        if b > a:
            e = _rel(o[a:b], o_ref[a:b])
            assert e < REL_TOL, f"{what}: sequence {s} output {e:.3e}"
            worst = max(worst, e)
        e = _rel(st[s], h_ref[s])
        assert e < REL_TOL, f"{what}: sequence {s} state {e:.3e}"
        worst = max(worst, e)
    print(f"{what}: worst relative error {worst:.3e}", flush=True)
    return worst


def test_prefill_benchmark_batch_matches_oracle():
    """The prefill benchmark's call: 8 sequences of U[256, 4096] tokens
    (seed 0: 12,450 tokens), 16 heads, bf16 q/k/v, fp32 g in [-5, 0] and
    beta, zero initial state, host offsets passed -- the call behind the
    headline number, with its final states written."""
    import bench
    from sophia_amd import ops
    dev = _dev()
    lengths = bench.prefill_lengths()
    inp = bench.make_prefill_inputs(torch, dev, lengths)
    n = len(lengths)
    state = torch.full((n, bench.HEADS, 128, 128), -3.0, device=dev)
    o = ops.kda_chunk_fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["cu"],
                          use_gate=False, use_beta_sigmoid=False, final_state=state,
                          cu_seqlens_cpu=inp["cu_cpu"])
    torch.cuda.synchronize()
    cu = inp["cu_cpu"].numpy()
    o_ref, h_ref = c_oracle.kda_varlen(_np(inp["q"]), _np(inp["k"]), _np(inp["v"]), _np(inp["g"]),
                                       _np(inp["beta"]), cu, use_gate=False, use_beta_sigmoid=False)
    _per_sequence(_np(o), o_ref, _np(state), h_ref, cu, "prefill benchmark batch")
    # the same call with device offsets only (another launch plan) is bit-identical
    state2 = torch.zeros_like(state)
    o2 = ops.kda_chunk_fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["cu"],
                           use_gate=False, use_beta_sigmoid=False, final_state=state2)
    assert torch.equal(o, o2) and torch.equal(state, state2)


def test_backward_benchmark_batch_matches_recurrent_form():
    """The backward benchmark's call: the prefill benchmark's batch and flags
    (l2norm in the kernel, precomputed log-decay and beta) with a bf16 output
    gradient drawn as the benchmark draws it; the chunk form (the default, the
    call behind the backward figure, with its launch plan for this batch)
    against the fp32 per-token recurrent form (itself within 1e-5 of the
    float64 oracle on smaller batches), every gradient within 1.5e-2."""
    import bench
    from sophia_amd import ops
    dev = _dev()
    lengths = bench.prefill_lengths()
    inp = bench.make_prefill_inputs(torch, dev, lengths)
    total = int(sum(lengths))
    gen = torch.Generator().manual_seed(12)
    d_out = torch.randn((total, bench.HEADS, bench.DIM), generator=gen).to(torch.bfloat16).to(dev)

    def grads(recurrent):
        return ops.kda_chunk_bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["cu"], d_out,
                                 use_qk_l2norm=True, use_gate=False, use_beta_sigmoid=False,
                                 cu_seqlens_cpu=inp["cu_cpu"], recurrent=recurrent)

    got, want = grads(False), grads(True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), got, want):
        a, b = a.double().cpu(), b.double().cpu()
        assert bool(torch.isfinite(a).all()), name
        err = float((a - b).abs().max()) / max(float(b.abs().max()), 1e-30)
        print(f"backward benchmark batch {name}: rel err {err:.2e}", flush=True)
        assert err <= 1.5e-2, f"{name}: {err:.3e}"


def test_mixed_step_prefill_shape_matches_oracle():
    """The KDA prefill of the decoder's continuous-batching step: 16 sequences
    of 1,024 tokens, 16 heads, gate computed in the kernel from bf16 decay
    logits, beta sigmoid in the kernel, device offsets only, states in
    scattered cache slots."""
    from sophia_amd import ops
    dev = _dev()
    rng = np.random.default_rng(31)
    n, length, heads = 16, 1024, 16
    total = n * length
    cu = np.arange(0, total + 1, length, dtype=np.int32)
    bf = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16).to(dev)
    q = bf(rng.standard_normal((total, heads, 128)))
    k = bf(rng.standard_normal((total, heads, 128)))
    v = bf(rng.standard_normal((total, heads, 128)))
    z = bf(rng.standard_normal((total, heads, 128)) * 2.0)
    b = bf(rng.standard_normal((total, heads)))
    a_log = (rng.standard_normal(heads) * 0.5).astype(np.float32)
    dtb = ko.inverse_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), heads * 128))).astype(np.float32)
    slots = rng.permutation(24)[:n].astype(np.int32)
    state = torch.full((24, heads, 128, 128), -1.0, device=dev)
    o = ops.kda_chunk_fwd(q, k, v, z, b, torch.tensor(cu, device=dev), A_log=torch.tensor(a_log),
                          dt_bias=torch.tensor(dtb), use_gate=True, use_beta_sigmoid=True,
                          final_state=state, state_slots=torch.tensor(slots, device=dev))
    torch.cuda.synchronize()
    o_ref, h_ref = c_oracle.kda_varlen(_np(q), _np(k), _np(v), _np(z), _np(b), cu, A_log=a_log,
                                       dt_bias=dtb)
    st = _np(state)
    _per_sequence(_np(o), o_ref, st[slots], h_ref, cu, "mixed-step prefill shape")
    untouched = np.setdiff1d(np.arange(24), slots)
    assert np.all(st[untouched] == -1.0)


def test_slow_decay_long_prefill_drift():
    """8,192 tokens x 16 heads with the gate of a freshly initialised mixer
    (A_log = 0, dt_bias = inverse_softplus(dt), dt log-uniform in [1e-3, 1e-1],
    decay logits z ~ N(0, 0.5^2)), bf16 q/k/v, a nonzero initial state: the
    state keeps most of its memory across all 128 chunks, so any per-chunk
    rounding of the state would accumulate here."""
    from sophia_amd import ops
    dev = _dev()
    gen = torch.Generator().manual_seed(32)
    total, heads = 8192, 16
    q = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16)
    z = torch.randn(total, heads, 128, generator=gen) * 0.5
    b = torch.randn(total, heads, generator=gen)
    a_log = torch.zeros(heads)
    lo, hi = np.log(1e-3), np.log(1e-1)
    dt = torch.exp(torch.rand(heads * 128, generator=gen) * (hi - lo) + lo).clamp_min(1e-4)
    dtb = dt + torch.log(-torch.expm1(-dt))
    h0 = torch.randn(1, heads, 128, 128, generator=gen) * 0.05
    g_np = ko.kda_gate(z.numpy(), a_log.numpy(), dtb.numpy(), -5.0)
    assert float(np.median(g_np)) > -0.6  # the long-memory regime
    state = h0.to(dev)
    cu = np.array([0, total], dtype=np.int32)
    o = ops.kda_chunk_fwd(q.to(dev), k.to(dev), v.to(dev), z.to(dev), b.to(dev),
                          torch.tensor(cu, device=dev), A_log=a_log, dt_bias=dtb,
                          initial_state=state, final_state=state)
    torch.cuda.synchronize()
    o_ref, h_ref = c_oracle.kda_varlen(_np(q), _np(k), _np(v), z.numpy(), b.numpy(), cu,
                                       A_log=a_log.numpy(), dt_bias=dtb.numpy(),
                                       initial_states=h0.numpy())
    o_np = _np(o)
    e_o, e_h = _rel(o_np, o_ref), _rel(_np(state), h_ref)
    # the last 1,024 tokens alone, where drift would be largest
    e_tail = _rel(o_np[-1024:], o_ref[-1024:])
    print(f"slow-decay drift over {total} tokens: output {e_o:.3e} (last 1,024: {e_tail:.3e}), "
          f"state {e_h:.3e}", flush=True)
    assert e_o < REL_TOL and e_tail < REL_TOL and e_h < REL_TOL
