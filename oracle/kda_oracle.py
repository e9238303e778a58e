"""CPU oracle for the KDA mixer hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
module: it is the reference that ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` compare the HIP path against.

It is a plain numpy restatement of the reference's CPU path for Kimi Delta
Attention (``ml/runtime/model/attention.py`` in Arain119/Sophia): the
ShortConv, the gate / beta / q,k normalisation, the per-token delta-rule
recurrence (``_reference_kda``) and the mixer module glue
(``SophiaKDA.forward``).  Every function cites the reference lines it follows.

Arithmetic runs in the dtype of the arrays handed in (float32 reproduces the
reference's fp32 CPU run; float64 is used by the tests that pin this oracle
against closed forms).

Parity status of each function (what pins it; see tests/test_oracle_*.py):

* ``short_conv``       -- pinned: numpy.convolve per channel, history carry.
* ``kda_gate``         -- pinned: closed form of the sigmoid bound, pad logit.
* ``inverse_softplus`` -- pinned: softplus(inverse_softplus(dt)) == dt.
* ``l2_normalize``     -- pinned: unit norm, zero vector stays zero.
* ``kda_recurrent``    -- pinned: explicit-matrix form of the update
  S_t = (I - b k k^T) Diag(a) S_{t-1} + b k v^T built with numpy.outer and
  numpy.diag, hand-worked 2x2 step, beta=0 pure decay, orthonormal-key
  write/read, alpha=1/beta=1 projection property.
* ``kda_varlen``       -- pinned: packed run == each sequence run alone.
* ``kda_varlen_bwd``   -- pinned: central finite differences of
  ``kda_varlen`` in float64 for every input (q, k, v, g, beta, the initial
  state, A_log, dt_bias), with and without the in-kernel norms, gate and
  beta sigmoid, and torch.autograd through an independent float64 torch
  restatement of the recurrence.
* ``rms_norm``         -- pinned: unit RMS after normalisation.
* ``mixer_forward``    -- pinned by the reference's own module invariants
  (causality, cached decode == full prompt, split prefill == one shot,
  padded row == unpadded row, stateless run leaves caches untouched).
"""

from __future__ import annotations

import numpy as np

# attention.py:17 -- logit written into decay and beta at pad positions.
PAD_LOGIT = -1.0e4


def _errstate():
    # sigmoid(-1e4) overflows exp() on purpose: the reference relies on
    # sigmoid saturating to exactly 0 there (attention.py:394-397).
    return np.errstate(over="ignore", under="ignore")


def sigmoid(x: np.ndarray) -> np.ndarray:
    """torch.sigmoid restated: 1 / (1 + exp(-x))."""
    x = np.asarray(x)
    one = np.array(1.0, dtype=x.dtype)
    with _errstate():
        return one / (one + np.exp(-x))


def silu(x: np.ndarray) -> np.ndarray:
    """functional.silu, used at attention.py:60."""
    return x * sigmoid(x)


def inverse_softplus(value: np.ndarray) -> np.ndarray:
    """attention.py:20-21: value + log(-expm1(-value))."""
    return value + np.log(-np.expm1(-value))


def l2_normalize(x: np.ndarray, eps: float = 1e-12) -> np.ndarray:
    """functional.normalize(x, p=2, dim=-1) as used at attention.py:270-273."""
    norm = np.sqrt(np.sum(x * x, axis=-1, keepdims=True))
    return x / np.maximum(norm, np.array(eps, dtype=x.dtype))


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """RMSNorm (ops.py:49-64, functional.rms_norm over the last dim)."""
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + np.array(eps, dtype=x.dtype)) * weight.astype(x.dtype)


def short_conv(x: np.ndarray, weight: np.ndarray, history: np.ndarray | None = None):
    """CausalDepthwiseConv1d.forward (attention.py:32-60).

    x: [B, T, C]; weight: [C, K]; history: [B, C, K-1] or None (zeros).
    Returns (silu(y) [B, T, C], next_history [B, C, K-1]) where
    y[b, t, c] = sum_j weight[c, j] * seq[b, c, t + j] and
    seq = cat(history, x^T) along time.  weight[:, K-1] multiplies the
    current token, weight[:, 0] the oldest one.
    """
    bsz, seqlen, channels = x.shape
    kernel = int(weight.shape[1])
    hist_len = kernel - 1
    xc = np.transpose(x, (0, 2, 1))
    if history is None:
        history = np.zeros((bsz, channels, hist_len), dtype=x.dtype)
    seq = np.concatenate((history.astype(x.dtype), xc), axis=-1) if hist_len > 0 else xc
    w = weight.astype(x.dtype)
    out = np.zeros((bsz, channels, seqlen), dtype=x.dtype)
    for j in range(kernel):
        out += w[None, :, j : j + 1] * seq[:, :, j : j + seqlen]
    next_history = seq[..., seq.shape[-1] - hist_len :] if hist_len > 0 else seq[..., :0]
    return silu(np.transpose(out, (0, 2, 1))), next_history


def kda_gate(decay_logits: np.ndarray, A_log: np.ndarray, dt_bias: np.ndarray,
             lower_bound: float) -> np.ndarray:
    """Per-channel log-decay g (attention.py:275-279).

    g = lower_bound * sigmoid(exp(A_log[h]) * (z + dt_bias[h, :])) for
    z: [..., H, K], A_log: [H], dt_bias: [H*K].
    """
    heads = A_log.shape[0]
    head_dim = decay_logits.shape[-1]
    dtype = decay_logits.dtype
    scale = np.exp(A_log.astype(dtype)).reshape((1,) * (decay_logits.ndim - 2) + (heads, 1))
    bias = dt_bias.astype(dtype).reshape((1,) * (decay_logits.ndim - 2) + (heads, head_dim))
    return np.array(lower_bound, dtype=dtype) * sigmoid(scale * (decay_logits + bias))


def kda_recurrent(q, k, v, g, beta, *, A_log=None, dt_bias=None, lower_bound=-5.0,
                  initial_state=None, use_qk_l2norm=True, use_gate=True,
                  use_beta_sigmoid=True, scale=None, dtype=np.float32):
    """SophiaKDA._reference_kda (attention.py:260-294), per-token loop.

    q, k: [B, T, H, K]; v: [B, T, H, V]; g: [B, T, H, K] (decay logits when
    use_gate, else log-decay); beta: [B, T, H] (logits when use_beta_sigmoid).
    initial_state: [B, H, K, V] or None (zeros).
    Returns (o [B, T, H, V], final_state [B, H, K, V]) in ``dtype``.

    The flags mirror the kernel-side switches of the reference's
    chunk_kda call (attention.py:349-365); their defaults reproduce
    _reference_kda exactly (normalise q and k, scale q by K^-1/2, gate and
    beta sigmoid applied).
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    g = np.asarray(g, dtype=dtype)
    beta = np.asarray(beta, dtype=dtype)
    bsz, seqlen, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    if scale is None:
        scale = key_dim ** -0.5
    if use_qk_l2norm:
        q = l2_normalize(q)
        k = l2_normalize(k)
    q = q * np.array(scale, dtype=dtype)
    if use_gate:
        log_decay = kda_gate(g, np.asarray(A_log), np.asarray(dt_bias), lower_bound)
    else:
        log_decay = g
    alpha = np.exp(log_decay)
    if use_beta_sigmoid:
        beta = sigmoid(beta)
    if initial_state is None:
        state = np.zeros((bsz, heads, key_dim, value_dim), dtype=dtype)
    else:
        state = np.array(initial_state, dtype=dtype, copy=True)
    out = np.zeros((bsz, seqlen, heads, value_dim), dtype=dtype)
    for t in range(seqlen):
        state = state * alpha[:, t][..., None]
        prediction = np.einsum("bhd,bhdv->bhv", k[:, t], state)
        correction = (v[:, t] - prediction) * beta[:, t][..., None]
        state = state + k[:, t][..., None] * correction[..., None, :]
        out[:, t] = np.einsum("bhd,bhdv->bhv", q[:, t], state)
    return out, state


def kda_varlen(q, k, v, g, beta, cu_seqlens, *, initial_states=None, **kw):
    """Packed ragged batch: each sequence of ``cu_seqlens`` run on its own.

    q, k: [sum_T, H, K]; v: [sum_T, H, V]; g: [sum_T, H, K]; beta: [sum_T, H];
    cu_seqlens: [N+1] int offsets; initial_states: [N, H, K, V] or None.
    This is the contract of the reference's varlen seam
    (sm120_concurrent_ffn.py:209-268, cu_seqlens + chunk_indices): state
    resets at every sequence boundary.
    Returns (o [sum_T, H, V], final_states [N, H, K, V]).
    """
    dtype = kw.get("dtype", np.float32)
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    n = len(cu) - 1
    heads, key_dim = q.shape[1], q.shape[2]
    value_dim = v.shape[2]
    out = np.zeros((q.shape[0], heads, value_dim), dtype=dtype)
    finals = np.zeros((n, heads, key_dim, value_dim), dtype=dtype)
    for s in range(n):
        a, b = cu[s], cu[s + 1]
        h0 = None if initial_states is None else initial_states[s : s + 1]
        if b == a:
            finals[s] = 0 if h0 is None else h0[0]
            continue
        o, ht = kda_recurrent(q[None, a:b], k[None, a:b], v[None, a:b], g[None, a:b],
                              beta[None, a:b], initial_state=h0, **kw)
        out[a:b] = o[0]
        finals[s] = ht[0]
    return out, finals


def kda_varlen_bwd(q, k, v, g, beta, cu_seqlens, d_out, *, d_final_states=None,
                   initial_states=None, A_log=None, dt_bias=None, lower_bound=-5.0,
                   use_qk_l2norm=True, use_gate=True, use_beta_sigmoid=True, scale=None,
                   dtype=np.float64):
    """Gradients of ``kda_varlen`` (the packed prefill) by the chain rule.

    This is what FlashKDAFunction.backward returns
    (ml/training/pretrain/engine/sm120_concurrent_ffn.py:301-373: the
    chunk_kda_train_bwd call, then l2norm_bwd and fused_beta_sigmoid_bwd),
    restated per token from the forward recurrence of ``kda_recurrent``:
    with q^ = scale q/|q|, k^ = k/|k|, alpha = e^g,
      S~ = Diag(alpha) S_{t-1}, p = k^T S~, u = beta (v - p),
      S_t = S~ + k^ u^T, o_t = S_t^T q^,
    the reverse step is
      dS += q^ do^T; dq^ = S_t do; du = dS^T k^; dv = beta du;
      dbeta = du . (v - p); dp = -beta du; dk^ = dS u + S~ dp;
      dS~ = dS + k^ dp^T; dalpha = rowsum(dS~ o S_{t-1}); dS_{t-1} = Diag(alpha) dS~,
    followed by the backward of the norms, the gate
    g = lb sigmoid(e^A_log (z + dt_bias)) and the beta sigmoid.

    Shapes as ``kda_varlen``; d_out: [sum_T, H, V]; d_final_states:
    [N, H, K, V] or None.  Returns a dict of dq, dk, dv, dg, dbeta, dh0
    (gradients of the inputs as passed, dg of the logits when ``use_gate``),
    and dA_log [H], ddt_bias [H*K] when ``use_gate``.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    g = np.asarray(g, dtype=dtype)
    beta = np.asarray(beta, dtype=dtype)
    d_out = np.asarray(d_out, dtype=dtype)
    total, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    if scale is None:
        scale = key_dim ** -0.5
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    n = len(cu) - 1
    # forward pieces, all tokens at once
    if use_qk_l2norm:
        nq = np.maximum(np.sqrt(np.sum(q * q, axis=-1, keepdims=True)), dtype(1e-12))
        nk = np.maximum(np.sqrt(np.sum(k * k, axis=-1, keepdims=True)), dtype(1e-12))
        qh, kh = q / nq * scale, k / nk
    else:
        qh, kh = q * scale, k
    if use_gate:
        ea = np.exp(np.asarray(A_log, dtype=dtype)).reshape(1, heads, 1)
        zb = g + np.asarray(dt_bias, dtype=dtype).reshape(1, heads, key_dim)
        sg = sigmoid(ea * zb)
        logd = lower_bound * sg
    else:
        logd = g
    alpha = np.exp(logd)
    bt = sigmoid(beta) if use_beta_sigmoid else beta
    dqh = np.zeros_like(qh)
    dkh = np.zeros_like(kh)
    dalpha = np.zeros_like(alpha)
    dv = np.zeros_like(v)
    dbt = np.zeros_like(bt)
    dh0 = np.zeros((n, heads, key_dim, value_dim), dtype=dtype)
    for s in range(n):
        a, b = cu[s], cu[s + 1]
        S = (np.zeros((heads, key_dim, value_dim), dtype=dtype) if initial_states is None
             else np.array(initial_states[s], dtype=dtype))
        states, preds = [S], []
        for t in range(a, b):
            St = S * alpha[t][..., None]
            p = np.einsum("hd,hdv->hv", kh[t], St)
            S = St + kh[t][..., None] * (bt[t][:, None] * (v[t] - p))[:, None, :]
            states.append(S)
            preds.append(p)
        dS = (np.zeros((heads, key_dim, value_dim), dtype=dtype) if d_final_states is None
              else np.array(d_final_states[s], dtype=dtype))
        for i in range(b - a - 1, -1, -1):
            t = a + i
            prev, cur, p = states[i], states[i + 1], preds[i]
            do = d_out[t]
            dS = dS + qh[t][..., None] * do[:, None, :]
            dqh[t] = np.einsum("hdv,hv->hd", cur, do)
            du = np.einsum("hdv,hd->hv", dS, kh[t])
            vp = v[t] - p
            u = bt[t][:, None] * vp
            dv[t] = bt[t][:, None] * du
            dbt[t] = np.sum(du * vp, axis=-1)
            dp = -bt[t][:, None] * du
            st = prev * alpha[t][..., None]
            dkh[t] = np.einsum("hdv,hv->hd", dS, u) + np.einsum("hdv,hv->hd", st, dp)
            dst = dS + kh[t][..., None] * dp[:, None, :]
            dalpha[t] = np.sum(dst * prev, axis=-1)
            dS = dst * alpha[t][..., None]
        dh0[s] = dS
    # norms: y = x / n, dx = (dy - y (y . dy)) / n (n held constant when clamped)
    if use_qk_l2norm:
        def norm_bwd(x, nx, dy):
            y = x / nx
            unclamped = np.sqrt(np.sum(x * x, axis=-1, keepdims=True)) >= 1e-12
            proj = np.where(unclamped, y * np.sum(y * dy, axis=-1, keepdims=True), 0.0)
            return (dy - proj) / nx
        dq = norm_bwd(q, nq, dqh * scale)
        dk = norm_bwd(k, nk, dkh)
    else:
        dq, dk = dqh * scale, dkh
    dlogd = dalpha * alpha
    out = {"dv": dv, "dh0": dh0, "dq": dq, "dk": dk}
    if use_gate:
        dz = dlogd * lower_bound * sg * (1.0 - sg) * ea
        out["dg"] = dz
        out["ddt_bias"] = dz.sum(axis=0).reshape(heads * key_dim)
        out["dA_log"] = (dz * zb).sum(axis=(0, 2))
    else:
        out["dg"] = dlogd
    out["dbeta"] = dbt * bt * (1.0 - bt) if use_beta_sigmoid else dbt
    return out


def kda_decode_step(q, k, v, g, beta, state, **kw):
    """One recurrent step for B sequences (the fused_recurrent_kda call at
    attention.py:330-348): q,k: [B, H, K]; v: [B, H, V]; g: [B, H, K];
    beta: [B, H]; state: [B, H, K, V].  Returns (o [B, H, V], new_state)."""
    o, ht = kda_recurrent(q[:, None], k[:, None], v[:, None], g[:, None], beta[:, None],
                          initial_state=state, **kw)
    return o[:, 0], ht


def linear(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """RuntimeLinear.forward (runtime_linear.py:32-33) without bias."""
    return x @ weight.T.astype(x.dtype)


def mixer_forward(params: dict, x: np.ndarray, *, start_pos: int = 0, cache: dict | None = None,
                  pad_mask: np.ndarray | None = None, num_heads: int = 16, head_dim: int = 128,
                  lower_bound: float = -5.0, norm_eps: float = 1e-5):
    """SophiaKDA.forward (attention.py:373-420) restated.

    params: numpy arrays keyed by the reference's parameter names
    (``q_proj.weight``, ``q_conv.weight``, ``decay_down.weight``, ...,
    ``A_log``, ``dt_bias``, ``output_gate.weight``, ``output_norm.weight``,
    ``o_proj.weight``).  cache: None (use_cache=False) or a dict holding
    ``recurrent`` [maxB, H, K, V] and ``conv`` [maxB, 3, H*K, K_conv-1]
    arrays, updated in place as the reference's buffers are.
    pad_mask: [B, T] bool (True = real token), honoured only at start_pos 0
    (attention.py:379).
    """
    dtype = x.dtype
    bsz, seqlen, _ = x.shape
    use_cache = cache is not None
    pm = pad_mask if (pad_mask is not None and int(start_pos) == 0) else None
    if pm is not None:
        x = x * pm[:, :seqlen].astype(dtype)[..., None]
    q = linear(x, params["q_proj.weight"])
    k = linear(x, params["k_proj.weight"])
    v = linear(x, params["v_proj.weight"])
    # _short_convolution (attention.py:226-258)
    outs = []
    for idx, (name, val) in enumerate((("q_conv", q), ("k_conv", k), ("v_conv", v))):
        hist = cache["conv"][:bsz, idx] if (use_cache and int(start_pos) > 0) else None
        y, nh = short_conv(val, params[f"{name}.weight"], hist)
        outs.append((y, nh))
    if use_cache:
        for idx, (_, nh) in enumerate(outs):
            cache["conv"][:bsz, idx] = nh.astype(cache["conv"].dtype)
    q, k, v = (o[0].reshape(bsz, seqlen, num_heads, head_dim) for o in outs)
    decay = linear(linear(x, params["decay_down.weight"]), params["decay_up.weight"])
    decay = decay.reshape(bsz, seqlen, num_heads, head_dim)
    beta_logits = linear(x, params["beta_proj.weight"])
    if pm is not None:
        drop = ~pm[:, :seqlen].astype(bool)
        decay = np.where(drop[:, :, None, None], np.array(PAD_LOGIT, dtype=dtype), decay)
        beta_logits = np.where(drop[:, :, None], np.array(PAD_LOGIT, dtype=dtype), beta_logits)
    h0 = cache["recurrent"][:bsz] if (use_cache and int(start_pos) > 0) else None
    o, final = kda_recurrent(q, k, v, decay, beta_logits, A_log=params["A_log"],
                             dt_bias=params["dt_bias"], lower_bound=lower_bound,
                             initial_state=h0, dtype=dtype)
    if use_cache:
        cache["recurrent"][:bsz] = final.astype(cache["recurrent"].dtype)
    if "output_gate.weight" in params:
        gate_logits = linear(x, params["output_gate.weight"])
    else:
        gate_logits = linear(linear(x, params["output_gate_down.weight"]),
                             params["output_gate_up.weight"])
    gate = sigmoid(gate_logits).reshape(bsz, seqlen, num_heads, head_dim)
    o = rms_norm(o.astype(dtype), params["output_norm.weight"], norm_eps) * gate
    return linear(o.reshape(bsz, seqlen, num_heads * head_dim), params["o_proj.weight"])


__all__ = [
    "PAD_LOGIT",
    "inverse_softplus",
    "kda_decode_step",
    "kda_gate",
    "kda_recurrent",
    "kda_varlen",
    "kda_varlen_bwd",
    "l2_normalize",
    "linear",
    "mixer_forward",
    "rms_norm",
    "short_conv",
    "sigmoid",
    "silu",
]
