"""Float64 torch restatement of the KDA mixer forward, differentiated by autograd.

Follows SophiaKDA.forward without caches (ml/runtime/model/attention.py:373-420):
the q/k/v projections, the three ShortConvs (CausalDepthwiseConv1d.forward,
attention.py:32-60, as torch's conv1d over cat(zero history, x)), the decay
and beta projections, the KDA core (the explicit-matrix restatement of
kda_autograd_ref), RMSNorm per head (torch's rms_norm, the routine
ml/runtime/model/ops.py:49-64 calls) times sigmoid(output_gate(x)), and
o_proj.  torch.autograd supplies every gradient, so it shares no code with
the HIP backward kernels.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from kda_autograd_ref import kda_packed_forward


def short_conv_ref(x: torch.Tensor, weight: torch.Tensor, history: torch.Tensor | None = None) -> torch.Tensor:
    """x [B, T, C], weight [C, K], history [B, C, K-1] or None -> silu(conv) [B, T, C]."""
    bsz, _, channels = x.shape
    hist_len = int(weight.shape[1]) - 1
    xc = x.transpose(1, 2)
    if history is None:
        history = xc.new_zeros((bsz, channels, hist_len))
    seq = torch.cat((history, xc), dim=-1)
    return F.silu(F.conv1d(seq, weight.unsqueeze(1), groups=channels).transpose(1, 2))


def mixer_forward_ref(p: dict, x: torch.Tensor, *, heads: int, head_dim: int = 128,
                      lower_bound: float = -5.0, norm_eps: float = 1e-5) -> torch.Tensor:
    """p: float64 tensors keyed by SophiaKDA's parameter names; x [B, T, dim]."""
    bsz, seqlen, _ = x.shape

    def lin(t, name):
        return t @ p[name].T

    q = short_conv_ref(lin(x, "q_proj.weight"), p["q_conv.weight"])
    k = short_conv_ref(lin(x, "k_proj.weight"), p["k_conv.weight"])
    v = short_conv_ref(lin(x, "v_proj.weight"), p["v_conv.weight"])
    z = lin(lin(x, "decay_down.weight"), "decay_up.weight")
    b = lin(x, "beta_proj.weight")
    rows = bsz * seqlen
    cu = list(range(0, rows + 1, seqlen))
    o, _ = kda_packed_forward(q.reshape(rows, heads, head_dim), k.reshape(rows, heads, head_dim),
                              v.reshape(rows, heads, head_dim), z.reshape(rows, heads, head_dim),
                              b.reshape(rows, heads), cu, A_log=p["A_log"], dt_bias=p["dt_bias"],
                              lower_bound=lower_bound, use_qk_l2norm=True, use_gate=True,
                              use_beta_sigmoid=True)
    gate = torch.sigmoid(lin(x, "output_gate.weight")).view(bsz, seqlen, heads, head_dim)
    o = F.rms_norm(o.view(bsz, seqlen, heads, head_dim), (head_dim,), p["output_norm.weight"], norm_eps) * gate
    return lin(o.reshape(bsz, seqlen, heads * head_dim), "o_proj.weight")
