"""Pins the decoder part of the CPU oracle (oracle/decoder_oracle.py) against
closed forms and independent computations.  CPU only, float64."""

from __future__ import annotations

import numpy as np

from oracle import decoder_oracle as do
from oracle import kda_oracle as ko

CFG = dict(n_layers=4, num_heads=2, norm_eps=1e-5, attn_res_block_size=4, situ_gate_softcap=4.0,
           situ_up_softcap=25.0, mla_kv_rank=16, short_conv_kernel=4)


def _params(rng, dim=32, heads=2, vocab=40, ffn=24, q_rank=12, kv_rank=16, layers=4):
    inner = heads * 128
    p = {"tok_embeddings.weight": rng.standard_normal((vocab, dim)) * 0.5,
         "norm.weight": 1 + 0.1 * rng.standard_normal(dim),
         "output_attn_residual.norm.weight": np.ones(dim),
         "output_attn_residual.query.weight": rng.standard_normal((1, dim)) * 0.1}
    p["output.weight"] = p["tok_embeddings.weight"]
    for i in range(layers):
        pre = f"layers.{i}"
        for name in ("attn_norm", "ffn_norm"):
            p[f"{pre}.{name}.weight"] = np.ones(dim)
        for name in ("attn_residual", "ffn_residual"):
            p[f"{pre}.{name}.norm.weight"] = np.ones(dim)
            p[f"{pre}.{name}.query.weight"] = rng.standard_normal((1, dim)) * 0.1
        p[f"{pre}.ffn.gate_up_proj.weight"] = rng.standard_normal((2 * ffn, dim)) * 0.2
        p[f"{pre}.ffn.down_proj.weight"] = rng.standard_normal((dim, ffn)) * 0.2
        a = f"{pre}.attn"
        if i % 4 == 3:
            shapes = {"q_down": (q_rank, dim), "q_up": (inner, q_rank), "kv_down": (kv_rank, dim),
                      "k_up": (inner, kv_rank), "v_up": (inner, kv_rank),
                      "output_gate": (inner, dim), "o_proj": (dim, inner)}
            for name, shp in shapes.items():
                p[f"{a}.{name}.weight"] = rng.standard_normal(shp) * 0.1
            p[f"{a}.q_norm.weight"] = np.ones(q_rank)
            p[f"{a}.kv_norm.weight"] = np.ones(kv_rank)
        else:
            for name in ("q_proj", "k_proj", "v_proj", "output_gate"):
                p[f"{a}.{name}.weight"] = rng.standard_normal((inner, dim)) * 0.1
            for name in ("q_conv", "k_conv", "v_conv"):
                p[f"{a}.{name}.weight"] = rng.standard_normal((inner, 4)) * 0.3
            p[f"{a}.decay_down.weight"] = rng.standard_normal((8, dim)) * 0.1
            p[f"{a}.decay_up.weight"] = rng.standard_normal((inner, 8)) * 0.1
            p[f"{a}.beta_proj.weight"] = rng.standard_normal((heads, dim)) * 0.1
            p[f"{a}.A_log"] = np.zeros(heads)
            p[f"{a}.dt_bias"] = ko.inverse_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), inner)))
            p[f"{a}.output_norm.weight"] = np.ones(128)
            p[f"{a}.o_proj.weight"] = rng.standard_normal((dim, inner)) * 0.1
    return p


def test_mla_matches_explicit_attention_loops():
    rng = np.random.default_rng(0)
    p = _params(rng)
    x = rng.standard_normal((1, 7, 32))
    y = do.mla_forward(p, "layers.3.attn", x, num_heads=2)
    a = lambda n: p[f"layers.3.attn.{n}.weight"]
    q = ko.rms_norm(x @ a("q_down").T, a("q_norm"), 1e-5) @ a("q_up").T
    lat = ko.rms_norm(x @ a("kv_down").T, a("kv_norm"), 1e-5)
    k, v = lat @ a("k_up").T, lat @ a("v_up").T
    out = np.zeros((7, 256))
    for h in range(2):
        sl = slice(128 * h, 128 * h + 128)
        for t in range(7):
            s = np.array([q[0, t, sl] @ k[0, j, sl] / np.sqrt(128) for j in range(t + 1)])
            w = np.exp(s - s.max())
            w /= w.sum()
            out[t, sl] = sum(w[j] * v[0, j, sl] for j in range(t + 1))
    gate = 1 / (1 + np.exp(-(x[0] @ a("output_gate").T)))
    np.testing.assert_allclose(y[0], (out * gate) @ a("o_proj").T, rtol=1e-10, atol=1e-12)


def test_mla_cached_decode_equals_full_and_is_causal():
    rng = np.random.default_rng(1)
    p = _params(rng)
    x = rng.standard_normal((2, 9, 32))
    full = do.mla_forward(p, "layers.3.attn", x, num_heads=2)
    cache = np.zeros((2, 16, 16))
    steps = [do.mla_forward(p, "layers.3.attn", x[:, :5], num_heads=2, cache=cache, start_pos=0)]
    for t in range(5, 9):
        steps.append(do.mla_forward(p, "layers.3.attn", x[:, t:t + 1], num_heads=2, cache=cache,
                                    start_pos=t))
    np.testing.assert_allclose(np.concatenate(steps, 1), full, rtol=1e-10, atol=1e-12)
    x2 = x.copy()
    x2[:, 6:] += 1.0
    np.testing.assert_array_equal(do.mla_forward(p, "layers.3.attn", x2, num_heads=2)[:, :6],
                                  full[:, :6])


def test_attn_res_zero_query_is_uniform_mean():
    rng = np.random.default_rng(2)
    p = {"m.norm.weight": np.ones(8), "m.query.weight": np.zeros((1, 8))}
    partial = rng.standard_normal((2, 3, 8))
    completed = rng.standard_normal((2, 3, 4, 8))
    y = do.attn_res_mix(p, "m", partial, completed)
    np.testing.assert_allclose(y, (completed.sum(2) + partial) / 5, rtol=1e-12)
    # with no completed block the mix is the identity
    np.testing.assert_allclose(do.attn_res_mix(p, "m", partial, completed[:, :, :0]), partial)


def test_ffn_hand_worked_and_small_input_limit():
    # one hidden unit: gate 2, up 3 -> 4 tanh(0.5) * sigmoid(2) * 25 tanh(0.12)
    p = {"f.gate_up_proj.weight": np.array([[2.0], [3.0]]), "f.down_proj.weight": np.array([[1.0]])}
    y = do.ffn_forward(p, "f", np.array([[1.0]]))
    expect = 4 * np.tanh(0.5) * (1 / (1 + np.exp(-2.0))) * 25 * np.tanh(3 / 25)
    np.testing.assert_allclose(y, [[expect]], rtol=1e-14)
    rng = np.random.default_rng(3)
    p = {"f.gate_up_proj.weight": rng.standard_normal((8, 5)) * 1e-3,
         "f.down_proj.weight": rng.standard_normal((5, 4))}
    x = rng.standard_normal((3, 5))
    gu = x @ p["f.gate_up_proj.weight"].T
    glu = (gu[:, :4] * (1 / (1 + np.exp(-gu[:, :4]))) * gu[:, 4:]) @ p["f.down_proj.weight"].T
    np.testing.assert_allclose(do.ffn_forward(p, "f", x), glu, rtol=1e-5)


def test_decoder_cached_decode_equals_full_prompt_and_causality():
    """The reference's own invariants (test_sophia_runtime_forward.py:140-168)
    on the restated decoder."""
    rng = np.random.default_rng(4)
    p = _params(rng)
    ids = rng.integers(0, 40, size=(2, 12))
    full = do.decoder_forward(p, ids, cfg=CFG)
    caches = do.new_caches(CFG, 2, 16)
    steps = [do.decoder_forward(p, ids[:, :8], start_pos=0, caches=caches, cfg=CFG)]
    for t in range(8, 12):
        steps.append(do.decoder_forward(p, ids[:, t:t + 1], start_pos=t, caches=caches, cfg=CFG))
    np.testing.assert_allclose(np.concatenate(steps, 1), full, rtol=1e-9, atol=1e-11)
    ids2 = ids.copy()
    ids2[:, 9:] = (ids2[:, 9:] + 1) % 40
    np.testing.assert_array_equal(do.decoder_forward(p, ids2, cfg=CFG)[:, :9], full[:, :9])
