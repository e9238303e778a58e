"""KDA backward on the GPU (sophia_kda_chunk_bwd and the autograd path).

Gradients from the HIP kernels are compared with the oracle's float64
backward (kda_varlen_bwd, itself pinned by finite differences and by torch
autograd in test_oracle_kda_bwd.py) on the same inputs, with the error
measured as max|hip - oracle| / max|oracle| per tensor.  Two forms:
  * the recurrent form (SOPHIA_KDA_BWD_RECURRENT), fp32 arithmetic: bound
    1e-5 (measured about 2e-7; a dropped term or a wrong sign shows as an
    error of order 1);
  * the chunk form (the default, the autograd path), bf16 MFMA operands in
    its two chunk scans as in the forward, fp32 elsewhere: bound 1.5e-2
    (measured 0.4e-3 to 9.4e-3 on every gradient, dA_log and ddt_bias
    included).
At larger sizes the gradients are checked through properties that do not
need the oracle: linearity in the output cotangent, and the chunk form
against the fp32 recurrent form.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as ko
from sophia_amd import ops  # noqa: F401  (registers torch.ops.sophia)

from kda_autograd_ref import kda_packed_grads

pytestmark = pytest.mark.gpu

D = 128
TOL = 1e-5
TOL_CHUNK = 1.5e-2


def _rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _inputs(cu, heads, *, seed, gated, dtype, h0=True, dht=True, gb_dtype=torch.float32):
    """Seeded inputs; ``gb_dtype`` is the dtype of g and beta (bf16 as the
    reference's training seam passes decay_logits / beta_logits; the oracle
    then gets the bf16-rounded values)."""
    gen = torch.Generator().manual_seed(seed)
    total, n = cu[-1], len(cu) - 1

    def rnd(*shape, scale=1.0):
        return torch.randn(*shape, generator=gen) * scale

    inp = {
        "q": rnd(total, heads, D).to(dtype),
        "k": rnd(total, heads, D).to(dtype),
        "v": rnd(total, heads, D).to(dtype),
    }
    if gated:
        inp["g"] = rnd(total, heads, D)
        inp["beta"] = rnd(total, heads)
        inp["A_log"] = torch.rand(heads, generator=gen) * 2 - 1
        inp["dt_bias"] = rnd(heads * D, scale=0.5)
    else:
        inp["q"] = torch.nn.functional.normalize(inp["q"].float(), dim=-1).to(dtype)
        inp["k"] = torch.nn.functional.normalize(inp["k"].float(), dim=-1).to(dtype)
        inp["g"] = -5.0 * torch.rand(total, heads, D, generator=gen)
        inp["beta"] = torch.rand(total, heads, generator=gen)
    inp["g"] = inp["g"].to(gb_dtype)
    inp["beta"] = inp["beta"].to(gb_dtype)
    inp["h0"] = rnd(n, heads, D, D, scale=0.1) if h0 else None
    d_out = rnd(total, heads, D).to(dtype)
    d_final = rnd(n, heads, D, D, scale=0.1) if dht else None
    flags = dict(use_qk_l2norm=gated, use_gate=gated, use_beta_sigmoid=gated)
    return inp, d_out, d_final, flags


def _hip(inp, cu, d_out, d_final, flags, recurrent=True, host_offsets=True):
    dev = "cuda"
    cu_t = torch.tensor(cu, dtype=torch.int32)
    res = torch.ops.sophia.kda_chunk_bwd(
        inp["q"].to(dev), inp["k"].to(dev), inp["v"].to(dev), inp["g"].to(dev),
        inp["beta"].to(dev), cu_t.to(dev), d_out.to(dev),
        None if inp.get("A_log") is None else inp["A_log"].to(dev),
        None if inp.get("dt_bias") is None else inp["dt_bias"].to(dev), D ** -0.5, -5.0,
        flags["use_qk_l2norm"], flags["use_gate"], flags["use_beta_sigmoid"],
        None if inp["h0"] is None else inp["h0"].to(dev),
        None if d_final is None else d_final.to(dev), cu_t if host_offsets else None, recurrent)
    names = ("q", "k", "v", "g", "beta", "h0", "A_log", "dt_bias")
    return {name: t.cpu().numpy() for name, t in zip(names, res)}


def _oracle(inp, cu, d_out, d_final, flags):
    f64 = lambda t: None if t is None else t.double().numpy()  # noqa: E731
    r = ko.kda_varlen_bwd(f64(inp["q"]), f64(inp["k"]), f64(inp["v"]), f64(inp["g"]),
                          f64(inp["beta"]), cu, f64(d_out), d_final_states=f64(d_final),
                          initial_states=f64(inp["h0"]), A_log=f64(inp.get("A_log")),
                          dt_bias=f64(inp.get("dt_bias")), **flags)
    out = {"q": r["dq"], "k": r["dk"], "v": r["dv"], "g": r["dg"], "beta": r["dbeta"],
           "h0": r["dh0"]}
    if flags["use_gate"]:
        out["A_log"], out["dt_bias"] = r["dA_log"], r["ddt_bias"]
    return out


def _compare(got, want, what, tol=TOL):
    for name, ref in want.items():
        assert np.all(np.isfinite(got[name])), f"{what}: d{name} not finite"
        err = _rel(got[name], ref)
        print(f"{what} d{name}: rel err {err:.2e}", flush=True)
        assert err <= tol, f"{what}: d{name} rel err {err:.3e}"


@pytest.mark.parametrize("gated,dtype", [(True, torch.float32), (True, torch.bfloat16),
                                         (False, torch.float32)])
def test_bwd_matches_oracle_ragged(gated, dtype):
    """Ragged packed batch: an empty sequence, partial and full chunks, a
    sequence crossing two chunk boundaries, initial and final-state terms."""
    cu = [0, 37, 37, 166, 230]
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=5, gated=gated, dtype=dtype)
    _compare(_hip(inp, cu, d_out, d_final, flags), _oracle(inp, cu, d_out, d_final, flags),
             f"ragged gated={gated} {dtype}")


def test_bwd_matches_oracle_long_sequence():
    """One 1,000-token sequence (16 chunks, the reverse chain crosses every
    checkpoint), gate-logit inputs, no initial state."""
    cu = [0, 1000]
    inp, d_out, d_final, flags = _inputs(cu, 1, seed=9, gated=True, dtype=torch.bfloat16,
                                         h0=False, dht=False)
    _compare(_hip(inp, cu, d_out, d_final, flags), _oracle(inp, cu, d_out, d_final, flags),
             "long")


def test_bwd_matches_torch_autograd_restatement():
    """The HIP gradients against torch.autograd of the float64 torch
    restatement (no shared code with the oracle or the kernels)."""
    cu = [0, 9, 24]
    inp, d_out, d_final, flags = _inputs(cu, 1, seed=13, gated=True, dtype=torch.float32)
    got = _hip(inp, cu, d_out, d_final, flags)
    ref = kda_packed_grads({name: (None if t is None else t.double())
                            for name, t in inp.items()}, cu, d_out.double(),
                           d_final.double(), **flags)
    _compare(got, ref, "torch autograd")


def test_bwd_is_deterministic():
    cu = [0, 100, 300]
    inp, d_out, d_final, flags = _inputs(cu, 4, seed=17, gated=True, dtype=torch.bfloat16)
    a = _hip(inp, cu, d_out, d_final, flags)
    b = _hip(inp, cu, d_out, d_final, flags)
    for name in a:
        np.testing.assert_array_equal(a[name], b[name])


def test_bwd_linear_in_cotangent_at_size():
    """8 sequences of 256..1,100 tokens, 16 heads (the mixer's head count):
    grads(a do1 + b do2) == a grads(do1) + b grads(do2) for every input."""
    gen = torch.Generator().manual_seed(23)
    lens = torch.randint(256, 1100, (8,), generator=gen).tolist()
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    inp, d1, f1, flags = _inputs(cu, 16, seed=29, gated=True, dtype=torch.bfloat16)
    _, d2, f2, _ = _inputs(cu, 16, seed=31, gated=True, dtype=torch.bfloat16)
    d1, d2 = d1.float(), d2.float()
    a, b = 0.75, -1.25
    g1 = _hip(inp, cu, d1, f1, flags)
    g2 = _hip(inp, cu, d2, f2, flags)
    g12 = _hip(inp, cu, a * d1 + b * d2, a * f1 + b * f2, flags)
    for name in g1:
        want = a * g1[name].astype(np.float64) + b * g2[name].astype(np.float64)
        err = _rel(g12[name], want)
        print(f"linearity d{name}: rel err {err:.2e}", flush=True)
        assert np.all(np.isfinite(g12[name]))
        assert err <= 1e-4, f"d{name}: {err:.3e}"


@pytest.mark.parametrize("gb_dtype", [torch.float32, torch.bfloat16])
def test_autograd_through_chunk_kda(gb_dtype):
    """ops.chunk_kda / flash_kda with requires_grad inputs: loss.backward()
    fills every leaf's .grad in its own shape and dtype with the oracle's
    gradients (through the chunk form).  bf16 g and beta are what the
    reference's training seam passes (decay_logits, beta_logits)."""
    cu = [0, 70, 150]
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=37, gated=True, dtype=torch.bfloat16, gb_dtype=gb_dtype)
    dev = "cuda"
    leaves = {name: t.to(dev).clone().requires_grad_(True) for name, t in inp.items()}
    o, ht = ops.flash_kda(
        leaves["q"][None], leaves["k"][None], leaves["v"][None], leaves["g"][None],
        leaves["beta"][None], leaves["A_log"], leaves["dt_bias"], initial_state=leaves["h0"],
        output_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
        use_beta_sigmoid_in_kernel=True, cu_seqlens=torch.tensor(cu, dtype=torch.int32),
        lower_bound=-5.0)
    assert o.shape == (1, cu[-1], 2, D) and o.dtype == torch.bfloat16
    loss = (o.float() * d_out.to(dev)[None].float()).sum() + (ht * d_final.to(dev)).sum()
    loss.backward()
    want = _oracle(inp, cu, d_out, d_final, flags)
    for name, leaf in leaves.items():
        assert leaf.grad is not None and leaf.grad.shape == leaf.shape
        assert leaf.grad.dtype == leaf.dtype
    got = {name: leaf.grad.float().cpu().numpy() for name, leaf in leaves.items()}
    # the autograd path runs the chunk form
    for name, ref in want.items():
        tol = TOL_CHUNK
        err = _rel(got[name], ref)
        print(f"autograd d{name}: rel err {err:.2e}", flush=True)
        assert err <= tol, f"d{name}: {err:.3e}"


def test_no_grad_path_unchanged():
    """Without requires_grad, chunk_kda takes the forward-only op and returns
    the same output as the autograd path."""
    cu = [0, 90]
    inp, _, _, _ = _inputs(cu, 2, seed=41, gated=True, dtype=torch.bfloat16, h0=False)
    dev = "cuda"
    args = [inp[n].to(dev)[None] for n in ("q", "k", "v", "g", "beta")]
    kw = dict(use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, A_log=inp["A_log"].to(dev),
              dt_bias=inp["dt_bias"].to(dev), output_final_state=True)
    o1, h1 = ops.chunk_kda(*args, **kw)
    q = args[0].clone().requires_grad_(True)
    o2, h2 = ops.chunk_kda(q, *args[1:], **kw)
    assert o2.requires_grad and not o1.requires_grad
    torch.testing.assert_close(o1, o2.detach(), rtol=0, atol=0)
    torch.testing.assert_close(h1, h2.detach(), rtol=0, atol=0)


# ---- the chunk form -----------------------------------------------------------
@pytest.mark.parametrize("gated,dtype,gb_dtype", [
    (True, torch.float32, torch.float32), (True, torch.bfloat16, torch.float32),
    (False, torch.float32, torch.float32), (False, torch.bfloat16, torch.float32),
    (True, torch.bfloat16, torch.bfloat16), (False, torch.bfloat16, torch.bfloat16)])
def test_chunk_bwd_matches_oracle_ragged(gated, dtype, gb_dtype):
    """The chunk form on a ragged batch: an empty sequence, partial and full
    chunks, initial and final-state terms; g and beta in fp32 or in bf16 (the
    training seam's dtype: the bf16 g/beta instantiations of the intra and
    gradient kernels and the gate kernels' bf16 loads)."""
    cu = [0, 37, 37, 166, 230]
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=5, gated=gated, dtype=dtype, gb_dtype=gb_dtype)
    _compare(_hip(inp, cu, d_out, d_final, flags, recurrent=False),
             _oracle(inp, cu, d_out, d_final, flags), f"chunk ragged gated={gated} {dtype} g/beta {gb_dtype}",
             TOL_CHUNK)


@pytest.mark.parametrize("gated,gb_dtype", [(True, torch.float32), (False, torch.float32),
                                            (True, torch.bfloat16), (False, torch.bfloat16)])
def test_chunk_bwd_matches_oracle_long_sequence(gated, gb_dtype):
    """One 1,000-token sequence: 16 chunk steps of each chunk scan."""
    cu = [0, 1000]
    inp, d_out, d_final, flags = _inputs(cu, 1, seed=9, gated=gated, dtype=torch.bfloat16,
                                         h0=False, dht=False, gb_dtype=gb_dtype)
    _compare(_hip(inp, cu, d_out, d_final, flags, recurrent=False),
             _oracle(inp, cu, d_out, d_final, flags), f"chunk long gated={gated} g/beta {gb_dtype}", TOL_CHUNK)


@pytest.mark.parametrize("recurrent", [False, True])
def test_bwd_rows_outside_the_sequences_get_zero_gradients(recurrent):
    """Offsets that stop before the last row (cu[-1] < total) and start after
    row 0, given on the device only (so the host cannot check them): the rows
    no sequence covers hold NaN inputs and NaN output gradients, yet get zero
    gradients and add nothing to dA_log / ddt_bias; the covered rows match the
    oracle on the sequences alone."""
    cu = [0, 37, 166]
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=83, gated=True, dtype=torch.bfloat16,
                                         gb_dtype=torch.bfloat16)
    want = _oracle(inp, cu, d_out, d_final, flags)
    lead, tail = 5, 29
    total = cu[-1] + lead + tail

    def pad(t):
        out = torch.full((total,) + tuple(t.shape[1:]), float("nan"), dtype=t.dtype)
        out[lead:lead + cu[-1]] = t
        return out

    padded = {name: (pad(t) if name in ("q", "k", "v", "g", "beta") else t) for name, t in inp.items()}
    cu_p = [c + lead for c in cu]
    got = _hip(padded, cu_p, pad(d_out), d_final, flags, recurrent=recurrent, host_offsets=False)
    inside = slice(lead, lead + cu[-1])
    for name in ("q", "k", "v", "g", "beta"):
        outside = np.concatenate([got[name][:lead], got[name][lead + cu[-1]:]])
        assert np.array_equal(outside, np.zeros_like(outside)), f"d{name} outside the sequences"
        got[name] = got[name][inside]
    _compare(got, want, f"padded batch recurrent={recurrent}", TOL if recurrent else TOL_CHUNK)


@pytest.mark.parametrize("recurrent", [False, True])
def test_bf16_gradients_are_the_fp32_gradients_rounded(recurrent):
    """grad_dtype=torch.bfloat16 (SOPHIA_KDA_BWD_GRAD_BF16, the call the
    autograd function makes for bf16 q, k, v): dq, dk, dv equal the fp32
    call's gradients rounded to nearest even, bit for bit, on a padded batch
    with device-only offsets (the rows outside the sequences zero in bf16
    too); dg, dbeta, dh0, dA_log and ddt_bias are the fp32 call's, bit for
    bit."""
    cu = [0, 37, 37, 166, 230]
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=91, gated=True, dtype=torch.bfloat16,
                                         gb_dtype=torch.bfloat16)
    lead, tail = 3, 21
    total = cu[-1] + lead + tail
    dev = "cuda"

    def pad(t):
        out = torch.full((total,) + tuple(t.shape[1:]), float("nan"), dtype=t.dtype)
        out[lead:lead + cu[-1]] = t
        return out.to(dev)

    cu_d = torch.tensor([c + lead for c in cu], dtype=torch.int32, device=dev)
    args = [pad(inp[n]) for n in ("q", "k", "v", "g", "beta")] + [cu_d, pad(d_out)]
    kw = dict(A_log=inp["A_log"].to(dev), dt_bias=inp["dt_bias"].to(dev), initial_state=inp["h0"].to(dev),
              d_final_state=d_final.to(dev), recurrent=recurrent, **flags)
    f32 = ops.kda_chunk_bwd(*args, **kw)
    b16 = ops.kda_chunk_bwd(*args, grad_dtype=torch.bfloat16, **kw)
    torch.cuda.synchronize()
    for i, name in enumerate(("q", "k", "v")):
        assert b16[i].dtype == torch.bfloat16 and b16[i].shape == f32[i].shape
        assert f32[i].dtype == torch.float32
        assert torch.isfinite(f32[i]).all(), f"d{name}"
        assert torch.equal(b16[i].view(torch.int16), f32[i].to(torch.bfloat16).view(torch.int16)), f"d{name}"
        outside = torch.cat([b16[i][:lead], b16[i][lead + cu[-1]:]])
        assert torch.equal(outside.view(torch.int16), torch.zeros_like(outside.view(torch.int16))), f"d{name}"
    for i, name in zip(range(3, 8), ("g", "beta", "h0", "A_log", "dt_bias")):
        assert b16[i].dtype == torch.float32
        assert torch.equal(b16[i].view(torch.int32), f32[i].view(torch.int32)), f"d{name}"
    with pytest.raises(RuntimeError, match="grad_dtype"):
        ops.kda_chunk_bwd(*args, grad_dtype=torch.float16, **kw)


def test_chunk_bwd_matches_torch_autograd_restatement():
    cu = [0, 9, 24, 90]
    inp, d_out, d_final, flags = _inputs(cu, 1, seed=13, gated=True, dtype=torch.float32)
    got = _hip(inp, cu, d_out, d_final, flags, recurrent=False)
    ref = kda_packed_grads({name: (None if t is None else t.double())
                            for name, t in inp.items()}, cu, d_out.double(),
                           d_final.double(), **flags)
    _compare(got, ref, "chunk vs torch autograd", TOL_CHUNK)


def test_chunk_bwd_more_sequences_than_the_ranked_plan():
    """20 sequences: past the 16 that the two chunk scans rank longest first on
    the device, they take the chains in packing order.  Empty, one-token and
    multi-chunk sequences mixed, against the oracle."""
    rng = np.random.default_rng(71)
    lens = rng.integers(0, 200, size=20)
    lens[[3, 11]] = 0
    lens[7] = 1
    lens[15] = 260
    cu = [0] + np.cumsum(lens).tolist()
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=71, gated=True, dtype=torch.bfloat16)
    _compare(_hip(inp, cu, d_out, d_final, flags, recurrent=False),
             _oracle(inp, cu, d_out, d_final, flags), "chunk 20 sequences", TOL_CHUNK)


def test_chunk_bwd_slow_decay_and_one_token_sequences():
    """Log-decays near 0 (long memory: the reverse scan carries dS through
    every chunk nearly undamped), beta = 0 rows, and sequences of 1 and 64
    tokens beside longer ones."""
    cu = [0, 1, 65, 65, 300, 301]
    inp, d_out, d_final, flags = _inputs(cu, 2, seed=43, gated=False, dtype=torch.bfloat16)
    inp["g"] = inp["g"] * 1e-3
    inp["beta"][::7] = 0.0
    _compare(_hip(inp, cu, d_out, d_final, flags, recurrent=False),
             _oracle(inp, cu, d_out, d_final, flags), "chunk slow decay", TOL_CHUNK)


def test_chunk_bwd_is_deterministic():
    cu = [0, 100, 300]
    inp, d_out, d_final, flags = _inputs(cu, 4, seed=17, gated=True, dtype=torch.bfloat16)
    a = _hip(inp, cu, d_out, d_final, flags, recurrent=False)
    b = _hip(inp, cu, d_out, d_final, flags, recurrent=False)
    for name in a:
        np.testing.assert_array_equal(a[name], b[name])


def test_chunk_bwd_graph_replays_equal_eager():
    """The chunk backward captured in a HIP graph (outputs and workspace from
    the graph's pool, host offsets given): three replays, with eager backward
    calls on another cotangent and synchronisations between them, each equal
    bit for bit to the eager call."""
    cu = [0, 100, 300, 301, 520]
    inp, d_out, d_final, flags = _inputs(cu, 4, seed=61, gated=True, dtype=torch.bfloat16)
    dev = "cuda"
    t = {name: x.to(dev) for name, x in inp.items()}
    d_out_d, d_final_d = d_out.to(dev), d_final.to(dev)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=dev)
    cu_h = torch.tensor(cu, dtype=torch.int32)

    def call(do):
        return ops.kda_chunk_bwd(t["q"], t["k"], t["v"], t["g"], t["beta"], cu_d, do, A_log=t["A_log"],
                                 dt_bias=t["dt_bias"], initial_state=t["h0"], d_final_state=d_final_d,
                                 cu_seqlens_cpu=cu_h, **flags)

    want = [x.clone() for x in call(d_out_d)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(d_out_d)   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = call(d_out_d)
    other = (d_out_d.float() * -0.5 + 0.25).to(d_out_d.dtype)
    names = ("dq", "dk", "dv", "dg", "dbeta", "dh0", "dA_log", "ddt_bias")
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, w_, g_ in zip(names, want, outs):
            assert torch.equal(w_, g_), f"replay {rep}: {name} differs from the eager call"
        print(f"replay {rep}: all gradients bitwise equal", flush=True)
        call(other)
        torch.cuda.synchronize()


def test_chunk_bwd_matches_recurrent_at_size():
    """8 sequences of 256..1,100 tokens, 16 heads: the chunk form against the
    fp32 recurrent form (where the float64 oracle would take minutes)."""
    gen = torch.Generator().manual_seed(47)
    lens = torch.randint(256, 1100, (8,), generator=gen).tolist()
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    inp, d_out, d_final, flags = _inputs(cu, 16, seed=53, gated=True, dtype=torch.bfloat16)
    want = _hip(inp, cu, d_out, d_final, flags, recurrent=True)
    got = _hip(inp, cu, d_out, d_final, flags, recurrent=False)
    _compare(got, want, "chunk vs recurrent", TOL_CHUNK)


def test_chunk_bwd_sequence_order_is_immaterial():
    """The backward's two chunk scans take the chains longest first (for up to
    16 sequences) and, with that order, thinner value-column slices over two
    rounds of work-groups.  The same sequences packed in the reverse order
    must give each token and each sequence bit-identical gradients: every
    chain's arithmetic depends only on its own sequence."""
    lens = [70, 900, 0, 1500, 257, 64, 1]
    heads = 4
    cu = [0] + list(np.cumsum(lens))
    inp, d_out, d_final, flags = _inputs(cu, heads, seed=21, gated=False, dtype=torch.bfloat16)
    got = _hip(inp, cu, d_out, d_final, flags, recurrent=False)
    order = list(range(len(lens)))[::-1]
    rows = [np.arange(cu[i], cu[i + 1]) for i in order]
    perm = np.concatenate(rows)
    cu_r = [0] + list(np.cumsum([lens[i] for i in order]))
    inp_r = {k: (None if t is None else (t[perm] if k not in ("h0",) else t[order]))
             for k, t in inp.items()}
    got_r = _hip(inp_r, cu_r, d_out[perm], d_final[order], flags, recurrent=False)
    for name in ("q", "k", "v", "g", "beta"):
        assert np.array_equal(got[name][perm], got_r[name]), f"d{name} differs with the order"
    assert np.array_equal(got["h0"][order], got_r["h0"]), "dh0 differs with the order"


def test_chunk_bwd_long_slow_decay_sequence():
    """One 16,384-token sequence (256 chunk steps in each scan), 4 heads,
    with the gate of a freshly initialised mixer in the kernel (A_log = 0,
    dt_bias = inverse_softplus(dt), dt log-uniform in [1e-3, 1e-1], decay
    logits z ~ N(0, 0.5^2); ml/runtime/model/attention.py:101-106): the state
    and its gradient keep most of their memory across the whole chain, so a
    per-chunk rounding in either scan would accumulate.  Chunk form against
    the fp32 recurrent form, dA_log and ddt_bias (sums over all tokens)
    included."""
    gen = torch.Generator().manual_seed(61)
    total, heads = 16384, 4
    lo, hi = np.log(1e-3), np.log(1e-1)
    dt = torch.exp(torch.rand(heads * D, generator=gen) * (hi - lo) + lo).clamp_min(1e-4)
    inp = {
        "q": torch.randn(total, heads, D, generator=gen).to(torch.bfloat16),
        "k": torch.randn(total, heads, D, generator=gen).to(torch.bfloat16),
        "v": torch.randn(total, heads, D, generator=gen).to(torch.bfloat16),
        "g": torch.randn(total, heads, D, generator=gen) * 0.5,
        "beta": torch.randn(total, heads, generator=gen),
        "A_log": torch.zeros(heads),
        "dt_bias": dt + torch.log(-torch.expm1(-dt)),
        "h0": torch.randn(1, heads, D, D, generator=gen) * 0.05,
    }
    g_np = ko.kda_gate(inp["g"].numpy(), inp["A_log"].numpy(), inp["dt_bias"].numpy(), -5.0)
    assert float(np.median(g_np)) > -0.6  # the long-memory regime
    d_out = torch.randn(total, heads, D, generator=gen).to(torch.bfloat16)
    d_final = torch.randn(1, heads, D, D, generator=gen) * 0.05
    flags = dict(use_qk_l2norm=True, use_gate=True, use_beta_sigmoid=True)
    cu = [0, total]
    want = _hip(inp, cu, d_out, d_final, flags, recurrent=True)
    got = _hip(inp, cu, d_out, d_final, flags, recurrent=False)
    _compare(got, want, "chunk vs recurrent, 16 k slow-decay tokens", TOL_CHUNK)
    # the first 1,024 tokens, whose gradients come through the whole reverse chain
    for name in ("q", "k", "v", "g"):
        err = _rel(got[name][:1024], want[name][:1024])
        print(f"first 1,024 tokens d{name}: rel err {err:.2e}", flush=True)
        assert err <= TOL_CHUNK
