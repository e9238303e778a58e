"""Training through the mixer on the GPU: the ShortConv and gated-norm backward
kernels, their autograd registration, and the whole SophiaKDA module's
parameter gradients.

References are float64 torch autograd (tests/mixer_autograd_ref.py, pinned
against the numpy oracle on the CPU), on the same inputs rounded as the
kernels see them.  Errors are max|hip - ref| / max|ref| per tensor.  Bounds:
  * ShortConv and gated norm alone: fp32 1e-5 (fp32 arithmetic, other
    summation order); bf16 outputs 1e-2 (one bf16 rounding of each output,
    2^-8 relative), the fp32 weight gradients 1e-4;
  * the whole mixer: 1.5e-2, the KDA backward's own bound (its chunk form
    runs bf16 MFMA operands; the other gradients pass through it).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mixer_autograd_ref import mixer_forward_ref, short_conv_ref

pytestmark = pytest.mark.gpu

TOL_MIXER = 1.5e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _rel(a, b) -> float:
    a = torch.as_tensor(a).double().cpu()
    b = torch.as_tensor(b).double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kernel", [4, 2])
@pytest.mark.parametrize("with_history", [False, True])
def test_short_conv_backward_matches_float64_autograd(dtype, kernel, with_history):
    """Ragged packed batch (empty, one-token, two-token, 130-token sequences:
    sequence starts inside row groups and a sequence across the 128-row group
    boundary), x a column slice of a wider row (strided), cache slots, and
    five rows past the last sequence (their dx must be zero)."""
    from sophia_amd import ops
    dev = _dev()
    gen = torch.Generator().manual_seed(11 + kernel)
    lens = [5, 1, 0, 2, 40, 3, 130, 17]
    cu = [0] + np.cumsum(lens).tolist()
    total, pad, channels = cu[-1], 5, 96
    wide = torch.randn(total + pad, channels + 32, generator=gen).to(dtype)
    x = wide[:, 16:16 + channels]
    dy = torch.randn(total + pad, channels, generator=gen).to(dtype)
    w = torch.randn(channels, kernel, generator=gen) * 0.5
    slots = torch.tensor([6, 0, 3, 1, 5, 2, 7, 4], dtype=torch.int32)
    hist = torch.randn(8, channels, kernel - 1, generator=gen) if with_history else None
    cu_t = torch.tensor(cu, dtype=torch.int32)
    dx, dw = ops.short_conv_bwd(dy.to(dev), x.to(dev), w.to(dev), cu_t.to(dev),
                                conv_state=None if hist is None else hist.to(dev),
                                state_slots=slots.to(dev), read_history=with_history)
    torch.cuda.synchronize()
    assert dx.dtype == dtype and dw.dtype == torch.float32
    w_r = w.to(dtype).double().requires_grad_(True)   # the taps the kernels use
    dx_ref = torch.zeros(total, channels, dtype=torch.float64)
    for s in range(len(lens)):
        a, b = cu[s], cu[s + 1]
        if a == b:
            continue
        xs = x[a:b].double().clone().requires_grad_(True)
        h = None
        if with_history:
            h = hist[int(slots[s])].to(dtype).double()[None]
        y = short_conv_ref(xs[None], w_r, h)
        (y[0] * dy[a:b].double()).sum().backward()
        dx_ref[a:b] = xs.grad
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    err_x, err_w = _rel(dx[:total], dx_ref), _rel(dw, w_r.grad)
    print(f"short_conv bwd {dtype} K={kernel} hist={with_history}: dx {err_x:.2e} dw {err_w:.2e}", flush=True)
    assert err_x <= tol and err_w <= 1e-4
    assert bool((dx[total:] == 0).all()), "rows past the last sequence"


def test_short_conv_autograd_and_opcheck():
    """sophia::short_conv under autograd gives the backward op's gradients,
    and torch.library.opcheck accepts the op (schema, fake, autograd)."""
    from sophia_amd import ops, torch_ops
    dev = _dev()
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(70, 64, generator=gen).to(dev, torch.bfloat16).requires_grad_(True)
    w = (torch.randn(64, 4, generator=gen) * 0.4).to(dev).requires_grad_(True)
    cu = torch.tensor([0, 33, 70], dtype=torch.int32, device=dev)
    y = torch_ops.short_conv(x, w, cu, None, None, False, False)
    dy = torch.randn(70, 64, generator=gen).to(dev, torch.bfloat16)
    (y.float() * dy.float()).sum().backward()
    dx, dw = ops.short_conv_bwd(dy, x.detach(), w.detach(), cu)
    assert torch.equal(x.grad, dx) and torch.equal(w.grad, dw)
    torch.library.opcheck(torch.ops.sophia.short_conv.default,
                          (x.detach().requires_grad_(True), w.detach().requires_grad_(True), cu, None, None,
                           False, False))


@pytest.mark.parametrize("o_dtype,dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                           (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("with_norm", [True, False])
def test_gated_head_norm_backward_matches_float64_autograd(o_dtype, dtype, with_norm):
    """37 rows x 3 heads x 128; the gate a column slice of a wider row; an fp32
    o with a bf16 gate is rounded to bf16 first, as the forward does (its
    gradient passes the rounding unchanged)."""
    from sophia_amd import ops
    dev = _dev()
    gen = torch.Generator().manual_seed(3)
    rows, heads, hd, eps = 37, 3, 128, 1e-5
    o = (torch.randn(rows, heads * hd, generator=gen) * 2.0).to(o_dtype)
    wide = torch.randn(rows, heads * hd + 64, generator=gen).to(dtype)
    gate = wide[:, 64:]
    dy = torch.randn(rows, heads * hd, generator=gen).to(dtype)
    w = torch.rand(hd, generator=gen) + 0.5 if with_norm else None
    d_o, d_g, d_w = ops.gated_head_norm_bwd(dy.to(dev), o.to(dev), gate.to(dev), heads, hd,
                                            norm_weight=None if w is None else w.to(dev), eps=eps)
    torch.cuda.synchronize()
    assert d_o.dtype == o_dtype and d_g.dtype == dtype and d_o.shape == o.shape and d_g.shape == gate.shape
    o64 = o.double().requires_grad_(True)
    o_in = o64.to(dtype).double() if o_dtype != dtype else o64   # the forward's rounding; identity gradient
    o_in = o64 + (o_in - o64).detach()
    g64 = gate.double().requires_grad_(True)
    w64 = None if w is None else w.double().requires_grad_(True)
    v = o_in.view(rows, heads, hd)
    if w64 is not None:
        v = torch.nn.functional.rms_norm(v, (hd,), w64, eps)
    y = v.reshape(rows, heads * hd) * torch.sigmoid(g64)
    (y * dy.double()).sum().backward()
    tol_o = 1e-5 if o_dtype == torch.float32 else 1e-2
    tol_g = 1e-5 if dtype == torch.float32 else 1e-2
    errs = {"o": _rel(d_o, o64.grad), "gate": _rel(d_g, g64.grad)}
    if w64 is not None:
        errs["w"] = _rel(d_w, w64.grad)
    print(f"gated_head_norm bwd o {o_dtype} gate {dtype} norm={with_norm}: "
          + " ".join(f"d{k} {e:.2e}" for k, e in errs.items()), flush=True)
    assert errs["o"] <= tol_o and errs["gate"] <= tol_g
    if w64 is not None:
        assert errs["w"] <= 1e-4
    else:
        assert d_w is None


def _trained_like(module, gen):
    """Move A_log, dt_bias and the norm weight off their init values."""
    with torch.no_grad():
        module.A_log.copy_(torch.randn(module.A_log.shape, generator=gen) * 0.4)
        module.dt_bias.add_(torch.randn(module.dt_bias.shape, generator=gen) * 0.3)
        module.output_norm.weight.copy_(torch.rand(module.output_norm.weight.shape, generator=gen) + 0.5)
        for conv in (module.q_conv, module.k_conv, module.v_conv):
            conv.weight.mul_(10.0)   # taps of order 0.2 instead of 0.02: the conv matters


@pytest.mark.parametrize("seqlen", [70, 9])
def test_mixer_parameter_gradients_match_float64_autograd(seqlen):
    """sophia_amd.kda.SophiaKDA in training (no caches, fp32 activations):
    loss.backward() through the fused projection, the ShortConv backward
    kernel, the KDA chunk backward, the gated-norm backward kernel and o_proj
    gives every parameter's gradient, and x's, within 1.5e-2 of float64 torch
    autograd through mixer_autograd_ref (attention.py:373-420)."""
    from sophia_amd.config import ModelArgs
    from sophia_amd.kda import SophiaKDA
    dev = _dev()
    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(21)
    module = SophiaKDA(ModelArgs(dim=64, num_heads=2, head_dim=128, use_cache=False))
    _trained_like(module, gen)
    module = module.to(dev).train()
    x = torch.randn(2, seqlen, 64, generator=gen)
    r = torch.randn(2, seqlen, 64, generator=gen)
    xd = x.to(dev).requires_grad_(True)
    y = module(xd)
    (y * r.to(dev)).sum().backward()
    params = {name: p.detach().cpu().double().requires_grad_(True) for name, p in module.named_parameters()}
    x64 = x.double().requires_grad_(True)
    y64 = mixer_forward_ref(params, x64, heads=2)
    assert _rel(y.detach(), y64.detach()) <= 2e-2
    (y64 * r.double()).sum().backward()
    worst = 0.0
    for name, p in module.named_parameters():
        assert p.grad is not None, f"{name} got no gradient"
        err = _rel(p.grad, params[name].grad)
        worst = max(worst, err)
        print(f"T={seqlen} d{name}: rel err {err:.2e}", flush=True)
        assert err <= TOL_MIXER, name
    err_x = _rel(xd.grad, x64.grad)
    print(f"T={seqlen} dx: rel err {err_x:.2e} (worst parameter {worst:.2e})", flush=True)
    assert err_x <= TOL_MIXER
