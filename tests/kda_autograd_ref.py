"""Float64 torch restatement of the packed KDA prefill, differentiated by autograd.

Independent of the oracle's hand-written backward: the forward is written
again with torch ops (the explicit-matrix form of the update,
S_t = (I - b k k^T) Diag(a) S_{t-1} + b k v^T) and torch.autograd supplies
every gradient, so the two backward paths share no code.
"""

from __future__ import annotations

import torch


def kda_packed_forward(q, k, v, g, beta, cu, *, A_log=None, dt_bias=None, initial_states=None,
                       lower_bound=-5.0, use_qk_l2norm=True, use_gate=True,
                       use_beta_sigmoid=True, scale=None):
    """q, k, g: [T, H, K]; v: [T, H, V]; beta: [T, H]; cu: list of offsets.
    Returns (o [T, H, V], finals [N, H, K, V])."""
    total, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    if scale is None:
        scale = key_dim ** -0.5
    if use_qk_l2norm:
        q = torch.nn.functional.normalize(q, dim=-1, eps=1e-12)
        k = torch.nn.functional.normalize(k, dim=-1, eps=1e-12)
    q = q * scale
    if use_gate:
        logd = lower_bound * torch.sigmoid(
            torch.exp(A_log).view(1, heads, 1) * (g + dt_bias.view(1, heads, key_dim)))
    else:
        logd = g
    alpha = torch.exp(logd)
    b = torch.sigmoid(beta) if use_beta_sigmoid else beta
    eye = torch.eye(key_dim, dtype=q.dtype)
    outs, finals = [], []
    for s in range(len(cu) - 1):
        if initial_states is None:
            S = torch.zeros(heads, key_dim, value_dim, dtype=q.dtype)
        else:
            S = initial_states[s]
        for t in range(cu[s], cu[s + 1]):
            kk = k[t]
            proj = eye - b[t].view(heads, 1, 1) * kk.unsqueeze(-1) * kk.unsqueeze(-2)
            S = torch.matmul(proj, alpha[t].unsqueeze(-1) * S) \
                + b[t].view(heads, 1, 1) * kk.unsqueeze(-1) * v[t].unsqueeze(-2)
            outs.append(torch.einsum("hd,hdv->hv", q[t], S))
        finals.append(S)
    o = torch.stack(outs) if outs else q.new_zeros((0, heads, value_dim))
    return o, torch.stack(finals)


def kda_packed_grads(inputs: dict, cu, d_out, d_final, **flags) -> dict:
    """Gradients of sum(o * d_out) + sum(finals * d_final) with respect to
    every tensor in ``inputs`` (float64 leaves are made here)."""
    leaves = {name: torch.as_tensor(val, dtype=torch.float64).clone().requires_grad_(True)
              for name, val in inputs.items() if val is not None}
    o, finals = kda_packed_forward(leaves["q"], leaves["k"], leaves["v"], leaves["g"],
                                   leaves["beta"], cu, A_log=leaves.get("A_log"),
                                   dt_bias=leaves.get("dt_bias"),
                                   initial_states=leaves.get("h0"), **flags)
    loss = (o * torch.as_tensor(d_out, dtype=torch.float64)).sum()
    if d_final is not None:
        loss = loss + (finals * torch.as_tensor(d_final, dtype=torch.float64)).sum()
    loss.backward()
    return {name: leaf.grad.numpy() for name, leaf in leaves.items()}
