"""The sophia:: custom ops under torch.compile.

The KDA kernels are registered as ``torch.library`` custom ops with fake
implementations and ``mutates_args`` (the reference's convention for its own
kernels, ml/training/pretrain/engine/sm120_concurrent_ffn.py:62-104).  Checked
here: ``torch.library.opcheck`` on each op (schema, fake tensor, aliasing),
and ``torch.compile(fullgraph=True)`` -- no graph break anywhere -- of the
FLA-signature seam (``ops.chunk_kda``) and of the whole ``SophiaKDA.forward``
(prefill, then cached decode steps), matching eager bit for bit.  The
``aot_eager`` backend traces through dynamo and AOT autograd without
generating kernels of its own, so the same HIP kernels run in both.
"""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _kda_args(dev, total=70, heads=2, seed=0):
    gen = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=gen)
    return dict(q=mk(total, heads, 128).to(torch.bfloat16).to(dev),
                k=mk(total, heads, 128).to(torch.bfloat16).to(dev),
                v=mk(total, heads, 128).to(torch.bfloat16).to(dev),
                g=(mk(total, heads, 128) * 2).to(dev), beta=mk(total, heads).to(dev),
                A_log=(mk(heads) * 0.3).to(dev), dt_bias=(mk(heads * 128) - 3).to(dev))


def test_opcheck_custom_ops():
    from sophia_amd import torch_ops  # noqa: F401  (registers the ops)
    dev = _dev()
    a = _kda_args(dev)
    cu = torch.tensor([0, 50, 70], dtype=torch.int32, device=dev)
    state = torch.randn(3, 2, 128, 128, device=dev) * 0.05
    h0 = torch.randn(2, 2, 128, 128, device=dev) * 0.05
    ops_ = torch.ops.sophia
    torch.library.opcheck(ops_.kda_chunk_fwd.default,
                          (a["q"], a["k"], a["v"], a["g"], a["beta"], cu, a["A_log"], a["dt_bias"],
                           0.088, -5.0, True, True, True, h0, state[:2].clone(), False, None,
                           cu.cpu()))
    torch.library.opcheck(ops_.kda_chunk_fwd.default,
                          (a["q"], a["k"], a["v"], a["g"], a["beta"], cu, a["A_log"], a["dt_bias"],
                           0.088, -5.0, True, True, True, None, state.clone(), True,
                           torch.tensor([2, 0], dtype=torch.int32, device=dev), None))
    torch.library.opcheck(ops_.kda_decode_step.default,
                          (a["q"][:3], a["k"][:3], a["v"][:3], a["g"][:3], a["beta"][:3],
                           state.clone(), a["A_log"], a["dt_bias"], 0.088, -5.0, True, True, True,
                           None, True))
    x = torch.randn(70, 96, device=dev).to(torch.bfloat16)
    w = torch.randn(96, 4, device=dev) * 0.3
    cs = torch.randn(2, 96, 3, device=dev)
    torch.library.opcheck(ops_.short_conv_fwd.default, (x, w, cu, cs.clone(), None, True, True, False))
    torch.library.opcheck(ops_.short_conv_step.default, (x[:2], w, cs.clone(), None, True, False))
    gate = torch.randn(70, 256, device=dev).to(torch.bfloat16)
    o = torch.randn(70, 2, 128, device=dev)
    torch.library.opcheck(ops_.gated_head_norm.default, (o, gate, torch.rand(128, device=dev) + 0.5,
                                                         2, 128, 1e-5))


def test_compiled_chunk_kda_seam_matches_eager():
    """The FLA-signature prefill seam compiles with no graph break."""
    from sophia_amd import ops
    dev = _dev()
    a = _kda_args(dev, total=200, heads=4, seed=1)
    shape = lambda t: t.unsqueeze(0)
    cu = torch.tensor([0, 130, 200], dtype=torch.int32, device=dev)
    h0 = torch.randn(2, 4, 128, 128, device=dev) * 0.05

    def seam(q, k, v, g, beta, h0):
        return ops.chunk_kda(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                             use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                             use_beta_sigmoid_in_kernel=True, safe_gate=True, lower_bound=-5.0,
                             A_log=a["A_log"], dt_bias=a["dt_bias"], cu_seqlens=cu)

    args = (shape(a["q"]), shape(a["k"]), shape(a["v"]), shape(a["g"]), shape(a["beta"]), h0)
    o_e, h_e = seam(*args)
    compiled = torch.compile(seam, backend="aot_eager", fullgraph=True)
    o_c, h_c = compiled(*args)
    assert torch.equal(o_c, o_e) and torch.equal(h_c, h_e)


def test_compiled_mixer_forward_matches_eager():
    """SophiaKDA.forward (prefill of 70 tokens, then three cached decode
    steps) under torch.compile(fullgraph=True) equals the eager module: same
    outputs, same recurrent and conv caches."""
    from sophia_amd.config import ModelArgs
    from sophia_amd.kda import SophiaKDA
    dev = _dev()
    torch.manual_seed(3)
    args = ModelArgs(dim=256, num_heads=2, max_batch_size=2)
    eager = SophiaKDA(args).to(dev).eval()
    twin = copy.deepcopy(eager)
    compiled = torch.compile(twin, backend="aot_eager", fullgraph=True)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(2, 73, 256, generator=gen).to(dev)
    with torch.no_grad():
        outs_e = [eager(x[:, :70], start_pos=0)]
        outs_c = [compiled(x[:, :70], start_pos=0)]
        for t in range(70, 73):
            outs_e.append(eager(x[:, t:t + 1], start_pos=t))
            outs_c.append(compiled(x[:, t:t + 1], start_pos=t))
    for i, (e, c) in enumerate(zip(outs_e, outs_c)):
        assert torch.equal(e, c), f"step {i} differs"
    assert torch.equal(eager.recurrent_state, twin.recurrent_state)
    assert torch.equal(eager.conv_state, twin.conv_state)
