"""install_mi355x_kda on a model shaped like the reference's.

The stand-in classes below reproduce only what the installer relies on: the
reference mixer's seam (``_fla_chunk_kda()`` / ``_fla_fused_recurrent_kda()``
called with the keyword arguments of ml/runtime/model/attention.py:330-365,
the final state copied back into ``recurrent_state``, attention.py:398-410)
and the reference conv's ``forward(x, *, history=None)`` contract
(attention.py:32-60).  Before the install the seam raises (flash-linear-
attention absent, attention.py:296-312); after it, prefill and decode match
the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

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
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def _np(t):
    return t.detach().float().cpu().numpy()


class CausalDepthwiseConv1d(nn.Module):
    """Stand-in with the reference conv's attributes and call contract."""

    def __init__(self, channels, kernel_size):
        super().__init__()
        self.channels, self.kernel_size = channels, kernel_size
        self.weight = nn.Parameter(torch.randn(channels, kernel_size) * 0.3)

    def forward(self, x, *, history=None):
        raise RuntimeError("unpatched conv")


class SeamShapedMixer(nn.Module):
    """Calls its KDA kernels the way the reference mixer's _run_kda does."""

    def __init__(self, heads, batch):
        super().__init__()
        self.num_heads, self.head_dim, self.lower_bound, self.use_cache = heads, 128, -5.0, True
        self.A_log = nn.Parameter(torch.randn(heads) * 0.3)
        self.dt_bias = nn.Parameter(torch.randn(heads * 128) - 3.0)
        self.register_buffer("recurrent_state", torch.zeros(batch, heads, 128, 128))
        self.conv = CausalDepthwiseConv1d(64, 4)

    @staticmethod
    def _fla_chunk_kda():
        raise RuntimeError("CUDA Sophia KDA training requires flash-linear-attention>=0.5.2")

    @staticmethod
    def _fla_fused_recurrent_kda():
        raise RuntimeError("CUDA Sophia KDA decoding requires flash-linear-attention>=0.5.2")

    def core(self, q, k, v, z, b, *, start_pos):
        bsz = int(q.size(0))
        initial = self.recurrent_state[:bsz] if start_pos > 0 else None
        common = dict(q=q, k=k, v=v, g=z, beta=b, use_qk_l2norm_in_kernel=True,
                      use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                      lower_bound=self.lower_bound, A_log=self.A_log, dt_bias=self.dt_bias)
        if int(q.size(1)) == 1 and initial is not None:
            out, final = self._fla_fused_recurrent_kda()(initial_state=initial,
                                                         output_final_state=True, **common)
        else:
            out, final = self._fla_chunk_kda()(initial_state=initial,
                                               output_final_state=self.use_cache, safe_gate=True,
                                               **common)
        with torch.no_grad():
            self.recurrent_state[:bsz].copy_(final.detach().float())
        return out


def test_installer_patches_the_seam_and_matches_oracle():
    from sophia_amd.install import install_mi355x_kda
    dev = _dev()
    torch.manual_seed(0)
    model = SeamShapedMixer(heads=2, batch=2).to(dev)
    rng = np.random.default_rng(1)
    bsz, steps = 2, 53
    bf = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16).to(dev)
    q, k, v = (bf(rng.standard_normal((bsz, steps, 2, 128))) for _ in range(3))
    z = torch.tensor(rng.standard_normal((bsz, steps, 2, 128)), dtype=torch.float32, device=dev)
    b = torch.tensor(rng.standard_normal((bsz, steps, 2)), dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="flash-linear-attention"):
        model.core(q[:, :50], k[:, :50], v[:, :50], z[:, :50], b[:, :50], start_pos=0)
    x = bf(rng.standard_normal((bsz, 9, 64)))
    with pytest.raises(RuntimeError, match="unpatched"):
        model.conv(x)

    assert install_mi355x_kda(model) == {"conv": 1, "mixer": 1}
    with torch.no_grad():
        outs = [model.core(q[:, :50], k[:, :50], v[:, :50], z[:, :50], b[:, :50], start_pos=0)]
        for t in range(50, steps):
            sl = slice(t, t + 1)
            outs.append(model.core(q[:, sl], k[:, sl], v[:, sl], z[:, sl], b[:, sl], start_pos=t))
    o = _np(torch.cat(outs, 1))
    a_log, dtb = _np(model.A_log), _np(model.dt_bias)
    for s in range(bsz):
        sl = slice(s, s + 1)
        o_ref, h_ref = ko.kda_recurrent(_np(q[sl]), _np(k[sl]), _np(v[sl]), _np(z[sl]), _np(b[sl]),
                                        A_log=a_log, dt_bias=dtb, dtype=np.float64)
        assert _rel(o[s], o_ref[0]) < REL_TOL
        assert _rel(_np(model.recurrent_state[s]), h_ref[0]) < REL_TOL

    # the patched conv follows the reference contract, history included
    hist = bf(rng.standard_normal((bsz, 64, 3)))
    y, nxt = model.conv(x, history=hist)
    w = _np(model.conv.weight.to(torch.bfloat16))
    for s in range(bsz):
        y_ref, h_ref = ko.short_conv(_np(x[s:s + 1]).astype(np.float64), w.astype(np.float64),
                                     _np(hist[s:s + 1]).astype(np.float64))
        np.testing.assert_allclose(_np(y[s]), y_ref[0], rtol=1e-2, atol=1e-2)
        np.testing.assert_allclose(_np(nxt[s]), h_ref[0], rtol=0, atol=0)
    assert y.dtype == x.dtype and nxt.dtype == x.dtype and tuple(nxt.shape) == (bsz, 64, 3)


def test_installed_seam_trains():
    """The installed conv and KDA seam under autograd, as the reference's
    training plugin uses them (sm120_concurrent_ffn.py:199-207,425-430): the
    conv's dx and dweight and the core's gradients of q, k, v, the decay
    logits, beta, A_log and dt_bias against float64 torch autograd (the conv
    through torch's conv1d, the core through the explicit-matrix recurrence)."""
    from mixer_autograd_ref import short_conv_ref
    from kda_autograd_ref import kda_packed_forward
    from sophia_amd.install import install_mi355x_kda
    dev = _dev()
    torch.manual_seed(2)
    model = SeamShapedMixer(heads=2, batch=2).to(dev)
    assert install_mi355x_kda(model) == {"conv": 1, "mixer": 1}
    gen = torch.Generator().manual_seed(9)
    # conv
    x = torch.randn(2, 45, 64, generator=gen).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y, nxt = model.conv(xd)
    ry = torch.randn(2, 45, 64, generator=gen)
    (y.float() * ry.to(dev)).sum().backward()
    x64 = x.double().requires_grad_(True)
    w64 = model.conv.weight.detach().cpu().to(torch.bfloat16).double().requires_grad_(True)
    # the gradient reaching the bf16 y is ry rounded to bf16
    (short_conv_ref(x64, w64) * ry.to(torch.bfloat16).double()).sum().backward()
    assert _rel(_np(xd.grad), x64.grad.numpy()) < 1e-2
    assert _rel(_np(model.conv.weight.grad), w64.grad.numpy()) < 1e-4
    assert torch.equal(nxt.detach(), xd.detach().transpose(1, 2)[..., -3:])
    # core through the seam
    bsz, steps = 2, 90
    q, k, v = (torch.randn(bsz, steps, 2, 128, generator=gen).to(torch.bfloat16) for _ in range(3))
    z = torch.randn(bsz, steps, 2, 128, generator=gen)
    b = torch.randn(bsz, steps, 2, generator=gen)
    leaves = [t.to(dev).requires_grad_(True) for t in (q, k, v, z, b)]
    out = model.core(*leaves, start_pos=0)
    ro = torch.randn(bsz, steps, 2, 128, generator=gen)
    (out.float() * ro.to(dev)).sum().backward()
    ref_leaves = [t.double().reshape(bsz * steps, *t.shape[2:]).requires_grad_(True) for t in (q, k, v, z, b)]
    a64 = model.A_log.detach().cpu().double().requires_grad_(True)
    d64 = model.dt_bias.detach().cpu().double().requires_grad_(True)
    o64, _ = kda_packed_forward(*ref_leaves, [0, steps, 2 * steps], A_log=a64, dt_bias=d64)
    (o64 * ro.to(torch.bfloat16).double().reshape(bsz * steps, 2, 128)).sum().backward()
    for name, got, want in zip("qkvzb", leaves, ref_leaves):
        err = _rel(_np(got.grad).reshape(want.grad.shape), want.grad.numpy())
        print(f"seam d{name}: rel err {err:.2e}", flush=True)
        assert err < 1.5e-2, name
    # dA_log = sum dz (z + dt_bias) and ddt_bias = sum_t dz over 180 tokens x
    # 128 channels, with heavy cancellation: checked as the chain rule applied
    # to the kernel's own dz (pinned just above against float64), to 1e-4 of
    # the sum of the absolute terms; the direct error is printed.
    dz = leaves[3].grad.double().cpu().reshape(bsz * steps, 2, 128)
    zb = z.double().reshape(bsz * steps, 2, 128) + model.dt_bias.detach().cpu().double().view(1, 2, 128)
    terms_a, terms_b = dz * zb, dz
    for got, terms, dims, name, ref in ((model.A_log.grad, terms_a, (0, 2), "A_log", a64.grad),
                                        (model.dt_bias.grad, terms_b, (0,), "dt_bias", d64.grad)):
        want = terms.sum(dims).reshape(-1)
        mass = terms.abs().sum(dims).reshape(-1)
        gap = float(((got.double().cpu() - want).abs() / mass).max())
        print(f"seam d{name}: chain-rule gap {gap:.2e} of the term mass; vs float64 rel err "
              f"{_rel(_np(got), ref.numpy()):.2e}", flush=True)
        assert gap < 1e-4, name
