"""CPU oracle for the Sophia hybrid decoder around the KDA mixer -- TEST
INFRASTRUCTURE ONLY (imported by tests/ alone; the product never imports it).

A numpy restatement of the reference's runtime decoder:

* ``mla_forward``   -- SophiaMLA.forward (ml/runtime/model/attention.py:609-657):
  NoPE multi-head latent attention, q = q_up(RMSNorm(q_down x)), latent =
  RMSNorm(kv_down x) cached per position, k/v = k_up/v_up(latent), causal
  softmax attention with scale d^-1/2, output gated by sigmoid(output_gate x).
* ``ffn_forward``   -- FeedForward (ml/runtime/model/blocks.py:12-27): SiTU-GLU.
* ``attn_res_mix``  -- AttentionResidualMixer (blocks.py:30-48).
* ``block_forward`` -- SophiaBlock.forward (blocks.py:51-87).
* ``decoder_forward`` -- Transformer._run_main_layers / forward
  (ml/runtime/model/transformer.py:169-207; ops.py:66-77): embedding, the
  [KDA, KDA, KDA, MLA] layers, the output mixer, final RMSNorm, tied head.

The KDA mixer itself is ``kda_oracle.mixer_forward``.  Parameters are numpy
arrays keyed by the reference's state_dict names.  Parity status: pinned by
the closed-form checks in tests/test_oracle_decoder.py (softmax attention ==
explicit loops, causal prefix invariance, AttnRes with zero query weight ==
uniform mean, SiTU-GLU at small inputs == the GLU it approximates).
"""

from __future__ import annotations

import numpy as np

from . import kda_oracle as ko


def linear(x, w):
    return x @ w.T.astype(x.dtype)


def mla_forward(params: dict, prefix: str, x: np.ndarray, *, start_pos: int = 0,
                cache: np.ndarray | None = None, num_heads: int, head_dim: int = 128,
                norm_eps: float = 1e-5) -> np.ndarray:
    """SophiaMLA.forward (attention.py:609-657) without padding.

    x: [B, T, dim]; cache: [maxB, maxT, kv_rank] latent cache updated in place
    at positions start_pos .. start_pos + T (None: use_cache off, keys are the
    current tokens only).  Causal over the whole cached span (lower-right).
    """
    p = lambda name: params[f"{prefix}.{name}"]
    bsz, seqlen, _ = x.shape
    q = linear(ko.rms_norm(linear(x, p("q_down.weight")), p("q_norm.weight"), norm_eps),
               p("q_up.weight")).reshape(bsz, seqlen, num_heads, head_dim)
    latent = ko.rms_norm(linear(x, p("kv_down.weight")), p("kv_norm.weight"), norm_eps)
    if cache is not None:
        end = start_pos + seqlen
        cache[:bsz, start_pos:end] = latent
        latent_full = cache[:bsz, :end].astype(x.dtype)
    else:
        latent_full = latent
    klen = latent_full.shape[1]
    k = linear(latent_full, p("k_up.weight")).reshape(bsz, klen, num_heads, head_dim)
    v = linear(latent_full, p("v_up.weight")).reshape(bsz, klen, num_heads, head_dim)
    scores = np.einsum("bqhd,bkhd->bhqk", q, k) * (head_dim ** -0.5)
    offset = klen - seqlen
    allow = np.tril(np.ones((seqlen, klen), dtype=bool), k=offset)
    scores = np.where(allow[None, None], scores, -np.inf)
    scores = scores - scores.max(axis=-1, keepdims=True)
    prob = np.exp(scores)
    prob = prob / prob.sum(axis=-1, keepdims=True)
    out = np.einsum("bhqk,bkhd->bqhd", prob, v)
    gate = ko.sigmoid(linear(x, p("output_gate.weight"))).reshape(out.shape)
    return linear((out * gate).reshape(bsz, seqlen, num_heads * head_dim), p("o_proj.weight"))


def ffn_forward(params: dict, prefix: str, x: np.ndarray, *, gate_softcap: float = 4.0,
                up_softcap: float = 25.0) -> np.ndarray:
    """FeedForward.forward (blocks.py:23-27): SiTU-GLU with tanh soft caps."""
    gu = linear(x, params[f"{prefix}.gate_up_proj.weight"])
    hidden = gu.shape[-1] // 2
    gate, up = gu[..., :hidden], gu[..., hidden:]
    bounded_gate = gate_softcap * np.tanh(gate / gate_softcap)
    bounded_up = up_softcap * np.tanh(up / up_softcap)
    return linear(bounded_gate * ko.sigmoid(gate) * bounded_up,
                  params[f"{prefix}.down_proj.weight"])


def attn_res_mix(params: dict, prefix: str, partial: np.ndarray, completed: np.ndarray, *,
                 norm_eps: float = 1e-5) -> np.ndarray:
    """AttentionResidualMixer.forward (blocks.py:38-48): softmax over the depth
    axis of [completed blocks..., partial] with scores RMSNorm(value) . query."""
    values = np.concatenate([completed, partial[:, :, None]], axis=2)
    keys = ko.rms_norm(values, params[f"{prefix}.norm.weight"], norm_eps)
    scores = keys @ params[f"{prefix}.query.weight"][0].astype(values.dtype)
    scores = scores - scores.max(axis=2, keepdims=True)
    weights = np.exp(scores)
    weights = weights / weights.sum(axis=2, keepdims=True)
    return (weights[..., None] * values).sum(axis=2)


def block_forward(params: dict, layer: int, partial, completed, *, start_pos: int,
                  caches: dict | None, cfg: dict):
    """SophiaBlock.forward (blocks.py:66-87)."""
    pre = f"layers.{layer}"
    attn_input = attn_res_mix(params, f"{pre}.attn_residual", partial, completed,
                              norm_eps=cfg["norm_eps"])
    normed = ko.rms_norm(attn_input, params[f"{pre}.attn_norm.weight"], cfg["norm_eps"])
    if layer % 4 == 3:
        mixed = mla_forward(params, f"{pre}.attn", normed, start_pos=start_pos,
                            cache=None if caches is None else caches[layer]["latent"],
                            num_heads=cfg["num_heads"], norm_eps=cfg["norm_eps"])
    else:
        kda_params = {k[len(pre) + 6:]: v for k, v in params.items() if k.startswith(pre + ".attn.")}
        mixed = ko.mixer_forward(kda_params, normed, start_pos=start_pos,
                                 cache=None if caches is None else caches[layer],
                                 num_heads=cfg["num_heads"], norm_eps=cfg["norm_eps"])
    if layer % cfg["attn_res_block_size"] == 0:
        completed = np.concatenate([completed, partial[:, :, None]], axis=2)
        partial = mixed
    else:
        partial = partial + mixed
    ffn_input = attn_res_mix(params, f"{pre}.ffn_residual", partial, completed,
                             norm_eps=cfg["norm_eps"])
    partial = partial + ffn_forward(
        params, f"{pre}.ffn", ko.rms_norm(ffn_input, params[f"{pre}.ffn_norm.weight"], cfg["norm_eps"]),
        gate_softcap=cfg["situ_gate_softcap"], up_softcap=cfg["situ_up_softcap"])
    return partial, completed


def decoder_forward(params: dict, ids: np.ndarray, *, start_pos: int = 0, caches=None,
                    cfg: dict, dtype=np.float64) -> np.ndarray:
    """Transformer.forward (transformer.py:169-207): logits [B, T, vocab]."""
    hidden = params["tok_embeddings.weight"].astype(dtype)[ids]
    completed = np.zeros(hidden.shape[:2] + (0, hidden.shape[2]), dtype=dtype)
    for layer in range(cfg["n_layers"]):
        hidden, completed = block_forward(params, layer, hidden, completed, start_pos=start_pos,
                                          caches=caches, cfg=cfg)
    hidden = attn_res_mix(params, "output_attn_residual", hidden, completed,
                          norm_eps=cfg["norm_eps"])
    return linear(ko.rms_norm(hidden, params["norm.weight"], cfg["norm_eps"]),
                  params["output.weight"])


def new_caches(cfg: dict, batch: int, max_len: int, dtype=np.float64) -> dict:
    """Zeroed per-layer caches in the reference's layouts (attention.py:122-143,449-456)."""
    inner = cfg["num_heads"] * 128
    caches = {}
    for layer in range(cfg["n_layers"]):
        if layer % 4 == 3:
            caches[layer] = {"latent": np.zeros((batch, max_len, cfg["mla_kv_rank"]), dtype=dtype)}
        else:
            caches[layer] = {"recurrent": np.zeros((batch, cfg["num_heads"], 128, 128), dtype=dtype),
                             "conv": np.zeros((batch, 3, inner, cfg["short_conv_kernel"] - 1), dtype=dtype)}
    return caches


__all__ = ["attn_res_mix", "block_forward", "decoder_forward", "ffn_forward", "mla_forward",
           "new_caches"]
