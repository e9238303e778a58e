"""The prefill with its ShortConv fused in (sophia_kda_conv_chunk_fwd) against
the two launches it replaces: sophia_short_conv_fwd over the q | k | v
channels (write_history=1) followed by sophia_kda_chunk_fwd on the conv
outputs.  The fused kernel forms each conv output with the same fused
multiply-adds and SiLU and rounds it to bf16 as the separate conv writes it,
so outputs, final states and the new conv histories must be equal bit for
bit.  The separate launches are themselves checked against the oracle
(test_gpu_kernels.py, test_gpu_bench_shapes.py).
"""

from __future__ import annotations

import pytest
import torch

from sophia_amd import ops

pytestmark = pytest.mark.gpu

D = 128
DEV = "cuda"


def _case(cu, heads, *, seed, slots, n_slots, pad=16, g_dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    total, inner = cu[-1], heads * D
    width = 3 * inner + pad                       # row stride: a multiple of 8, as the fused projection's
    x = (torch.randn(total, width, generator=gen) * 1.5).to(torch.bfloat16)
    taps = (torch.randn(3 * inner, 4, generator=gen) * 0.5).to(torch.bfloat16).float()
    conv_state = torch.randn(n_slots, 3 * inner, 3, generator=gen)
    g = torch.randn(total, heads, D, generator=gen).to(g_dtype)
    beta = torch.randn(total, heads, generator=gen).to(torch.bfloat16)
    state = torch.randn(n_slots, heads, D, D, generator=gen) * 0.05
    gate = dict(A_log=(torch.rand(heads, generator=gen) * 2 - 1).to(DEV),
                dt_bias=(torch.randn(heads * D, generator=gen) * 0.5).to(DEV))
    sl = None if slots is None else torch.tensor(slots, dtype=torch.int32, device=DEV)
    return (x.to(DEV), taps.to(DEV), conv_state.to(DEV), g.to(DEV), beta.to(DEV), state.to(DEV),
            gate, sl)


def _both(cu, heads, *, seed, slots, n_slots, read, host_offsets=True, g_dtype=torch.bfloat16):
    x, taps, cs, g, beta, st, gate, sl = _case(cu, heads, seed=seed, slots=slots, n_slots=n_slots,
                                               g_dtype=g_dtype)
    inner = heads * D
    cu_d = torch.tensor(cu, dtype=torch.int32, device=DEV)
    cu_h = torch.tensor(cu, dtype=torch.int32) if host_offsets else None
    xq = x[:, :3 * inner]
    # separate launches
    cs1, st1 = cs.clone(), st.clone()
    y = torch.empty((cu[-1], 3 * inner), dtype=torch.bfloat16, device=DEV)
    ops.short_conv_fwd(xq, taps, cu_d, conv_state=cs1, state_slots=sl, read_history=read,
                       write_history=True, out=y, weight_rounded=True)
    o1 = ops.kda_chunk_fwd(y[:, :inner].unflatten(1, (heads, D)), y[:, inner:2 * inner].unflatten(1, (heads, D)),
                           y[:, 2 * inner:].unflatten(1, (heads, D)), g, beta, cu_d,
                           initial_state=st1 if read else None, final_state=st1, state_slots=sl,
                           cu_seqlens_cpu=cu_h, **gate)
    # fused
    cs2, st2 = cs.clone(), st.clone()
    o2 = ops.kda_conv_chunk_fwd(x[:, :3 * inner], taps, cs2, g, beta, cu_d, read_history=read,
                                initial_state=st2 if read else None, final_state=st2, state_slots=sl,
                                cu_seqlens_cpu=cu_h, **gate)
    torch.cuda.synchronize()
    return (o1, st1, cs1), (o2, st2, cs2), cs


def _assert_bitwise(a, b, what):
    assert a.dtype == b.dtype and a.shape == b.shape, what
    ia = a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32)
    ib = b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)
    n_diff = int((ia != ib).sum())
    print(f"{what}: {n_diff} of {a.numel()} elements differ", flush=True)
    assert n_diff == 0, what


@pytest.mark.parametrize("read", [False, True])
@pytest.mark.parametrize("g_dtype", [torch.bfloat16, torch.float32])
def test_fused_conv_prefill_equals_separate_launches(read, g_dtype):
    """Ragged batch: one-token and two-token sequences (the new history mixes
    the old one and the rows), an empty sequence, a sequence crossing a chunk
    boundary by 3 rows (its second chunk's first rows take the last rows of the
    first chunk), two multi-chunk sequences, one slot out of range (no history
    read or written, zero state); 3 heads."""
    cu = [0, 1, 3, 3, 70, 200, 330]
    slots = [5, 2, 7, 0, 99, 3]
    (o1, st1, cs1), (o2, st2, cs2), cs0 = _both(cu, 3, seed=11, slots=slots, n_slots=8, read=read,
                                                g_dtype=g_dtype)
    assert torch.isfinite(o1.float()).all()
    _assert_bitwise(o2, o1, "o")
    _assert_bitwise(st2, st1, "final states")
    _assert_bitwise(cs2, cs1, "conv histories")
    # the histories of the slots no sequence uses are untouched
    for s in (1, 4, 6):
        _assert_bitwise(cs2[s], cs0[s], f"conv history of unused slot {s}")


def test_fused_conv_prefill_without_host_offsets_or_slots():
    """Device-only offsets and the default slots (sequence s in slot s)."""
    cu = [0, 64, 64, 190]
    (o1, st1, cs1), (o2, st2, cs2), _ = _both(cu, 2, seed=12, slots=None, n_slots=3, read=True,
                                              host_offsets=False)
    _assert_bitwise(o2, o1, "o")
    _assert_bitwise(st2, st1, "final states")
    _assert_bitwise(cs2, cs1, "conv histories")


def test_fused_conv_prefill_at_the_mixed_step_shape():
    """The mixed step's prefill rows: 16 sequences of 1,024 tokens, 16 heads,
    bf16 decay logits with the gate in the kernel, fresh slots."""
    cu = [1024 * i for i in range(17)]
    slots = list(range(16, 32))
    (o1, st1, cs1), (o2, st2, cs2), _ = _both(cu, 16, seed=13, slots=slots, n_slots=32, read=False)
    _assert_bitwise(o2, o1, "o")
    _assert_bitwise(st2, st1, "final states")
    _assert_bitwise(cs2, cs1, "conv histories")


def test_fused_conv_prefill_rejects_rows_it_cannot_copy_whole():
    """Rows whose stride is not a multiple of 8 elements cannot be copied into
    LDS as whole lines: the call is refused on the host, before any launch."""
    cu = [0, 40]
    x, taps, cs, g, beta, st, gate, _ = _case(cu, 1, seed=14, slots=None, n_slots=1, pad=4)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ops.kda_conv_chunk_fwd(x[:, :3 * D], taps, cs, g, beta, torch.tensor(cu, dtype=torch.int32),
                               final_state=st, **gate)
    with pytest.raises(RuntimeError, match="bf16"):
        ops.kda_conv_chunk_fwd(x[:, :3 * D].float(), taps, cs, g, beta, torch.tensor(cu, dtype=torch.int32),
                               final_state=st, **gate)


@pytest.mark.parametrize("seed", list(range(8)))
def test_fused_conv_prefill_random_batches(seed):
    """Seeded random sweep: 1-12 sequences of 0-300 tokens (some empty, some of
    1-3 tokens, whose new history mixes old history and rows; every fourth case
    one sequence of 8,200-8,800 tokens, which the host plan cuts into segments
    of 64 chunks), 1-4 heads, fp32 or bf16 decay logits, the three in-kernel
    switches (l2 norm, gate, beta sigmoid), shuffled slots with one out of
    range, histories read or not, host offsets or device offsets alone.
    Outputs, final states and histories equal the two separate launches bit
    for bit; slots no sequence uses keep their histories."""
    import numpy as np
    rng = np.random.default_rng(500 + seed)
    n = int(rng.integers(1, 13))
    lens = rng.integers(0, 301, size=n)
    lens[rng.random(n) < 0.15] = 0
    lens[rng.random(n) < 0.15] = rng.integers(1, 4)
    if seed % 4 == 0:
        n, lens = 1, np.array([int(rng.integers(8200, 8801))])
    heads = int(rng.integers(1, 5))
    g_dt = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    l2, gated, bsig = bool(rng.random() < 0.7), bool(rng.random() < 0.6), bool(rng.random() < 0.6)
    read, host = bool(rng.random() < 0.6), seed % 3 != 2
    n_slots = n + 3
    slots = [int(s) for s in rng.permutation(n_slots)[:n]]
    if n > 1:
        slots[int(rng.integers(0, n))] = n_slots + 5        # out of range: no history, zero state
    cu = [0] + np.cumsum(lens).tolist()
    print(f"case {seed}: lens={lens.tolist()} heads={heads} g={g_dt} l2={l2} gate={gated} "
          f"beta_sigmoid={bsig} read={read} host_offsets={host} slots={slots}", flush=True)
    x, taps, cs, g, beta, st, gate, sl = _case(cu, heads, seed=seed, slots=slots, n_slots=n_slots,
                                               g_dtype=g_dt)
    if not gated:
        g = -torch.rand(g.shape, device=DEV).mul(4.0).to(g_dt)   # log-decays in [-4, 0]
        gate = {}
    flags = dict(use_qk_l2norm=l2, use_gate=gated, use_beta_sigmoid=bsig)
    if not l2:
        # unnormalised keys: small pre-conv k rows keep |k|^2 well under 1, so
        # that the delta rule's state stays bounded
        x[:, heads * D:2 * heads * D] *= 0.05
    if not bsig:
        beta = torch.sigmoid(beta.float()).to(beta.dtype)
    inner = heads * D
    cu_d = torch.tensor(cu, dtype=torch.int32, device=DEV)
    cu_h = torch.tensor(cu, dtype=torch.int32) if host else None
    cs1, st1 = cs.clone(), st.clone()
    y = torch.empty((cu[-1], 3 * inner), dtype=torch.bfloat16, device=DEV)
    ops.short_conv_fwd(x[:, :3 * inner], taps, cu_d, conv_state=cs1, state_slots=sl, read_history=read,
                       write_history=True, out=y, weight_rounded=True)
    o1 = ops.kda_chunk_fwd(y[:, :inner].unflatten(1, (heads, D)), y[:, inner:2 * inner].unflatten(1, (heads, D)),
                           y[:, 2 * inner:].unflatten(1, (heads, D)), g, beta, cu_d,
                           initial_state=st1 if read else None, final_state=st1, state_slots=sl,
                           cu_seqlens_cpu=cu_h, **gate, **flags)
    cs2, st2 = cs.clone(), st.clone()
    o2 = ops.kda_conv_chunk_fwd(x[:, :3 * inner], taps, cs2, g, beta, cu_d, read_history=read,
                                initial_state=st2 if read else None, final_state=st2, state_slots=sl,
                                cu_seqlens_cpu=cu_h, **gate, **flags)
    torch.cuda.synchronize()
    assert torch.isfinite(o1.float()).all()
    _assert_bitwise(o2, o1, "o")
    _assert_bitwise(st2, st1, "final states")
    _assert_bitwise(cs2, cs1, "conv histories")
    for s in sorted(set(range(n_slots)) - set(slots)):
        _assert_bitwise(cs2[s], cs[s], f"conv history of unused slot {s}")
