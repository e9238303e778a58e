"""Pins the CPU oracle (oracle/kda_oracle.py) against closed forms, hand-worked
cases, independent library routines and brute force.  CPU only.

Each check is chosen so that a plausible restatement mistake fails it: decay
applied on the value axis instead of the key axis, prediction taken before
the decay, beta applied to the value instead of the correction, conv taps
reversed, history not carried, sequence boundaries leaking state.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kda_oracle as ko
from oracle import c_oracle
import chunk_model


def _rng(seed=0):
    return np.random.default_rng(seed)


# ----------------------------------------------------------------- ShortConv
def test_conv_matches_numpy_convolve_per_channel():
    rng = _rng(1)
    x = rng.standard_normal((2, 9, 5))
    w = rng.standard_normal((5, 4))
    hist = rng.standard_normal((2, 5, 3))
    y, nh = ko.short_conv(x, w, hist)
    for b in range(2):
        for c in range(5):
            seq = np.concatenate([hist[b, c], x[b, :, c]])
            # numpy.convolve flips its second argument: flip the taps back so
            # w[c, 3] multiplies the newest sample.
            ref = np.convolve(seq, w[c, ::-1], mode="valid")
            np.testing.assert_allclose(y[b, :, c], ref / (1 + np.exp(-ref)), rtol=1e-12)
            np.testing.assert_array_equal(nh[b, c], seq[-3:])


def test_conv_history_carry_equals_one_shot():
    rng = _rng(2)
    x = rng.standard_normal((3, 11, 4))
    w = rng.standard_normal((4, 4))
    full, hist_full = ko.short_conv(x, w)
    y1, h1 = ko.short_conv(x[:, :5], w)
    y2, h2 = ko.short_conv(x[:, 5:6], w, h1)     # one-token step
    y3, h3 = ko.short_conv(x[:, 6:], w, h2)
    np.testing.assert_allclose(np.concatenate([y1, y2, y3], axis=1), full, rtol=1e-12)
    np.testing.assert_array_equal(h3, hist_full)


def test_conv_short_sequence_history_keeps_old_entries():
    x = np.array([[[7.0]]])                      # B=1, T=1, C=1
    w = np.array([[0.0, 0.0, 0.0, 1.0]])
    hist = np.array([[[1.0, 2.0, 3.0]]])
    _, nh = ko.short_conv(x, w, hist)
    np.testing.assert_array_equal(nh, [[[2.0, 3.0, 7.0]]])


def test_conv_kernel_one_has_empty_history():
    # reference test: tests/tests/test_sophia_runtime_forward.py:253-258
    y, h = ko.short_conv(_rng(3).standard_normal((2, 3, 4)), np.ones((4, 1)))
    assert y.shape == (2, 3, 4)
    assert h.shape == (2, 4, 0)


# --------------------------------------------------------------- gate / misc
def test_gate_is_bounded_and_pad_logit_is_identity():
    rng = _rng(4)
    z = rng.standard_normal((3, 2, 8)).astype(np.float32) * 10
    a_log = rng.standard_normal(2).astype(np.float32)
    dtb = rng.standard_normal(16).astype(np.float32)
    g = ko.kda_gate(z, a_log, dtb, -5.0)
    # fp32 sigmoid saturates to 1 for large logits, so the bound is closed.
    assert np.all(g >= -5.0) and np.all(g <= 0.0)
    pad = np.full((1, 2, 8), ko.PAD_LOGIT, dtype=np.float32)
    gp = ko.kda_gate(pad, a_log, np.zeros(16, np.float32), -5.0)
    assert np.all(gp == 0.0) and np.all(np.exp(gp) == 1.0)
    assert ko.sigmoid(np.float32(ko.PAD_LOGIT)) == 0.0
    # closed form at z + dt_bias = 0: sigmoid(0) = 1/2 -> g = lower_bound / 2
    g0 = ko.kda_gate(np.zeros((1, 1, 4)), np.zeros(1), np.zeros(4), -5.0)
    np.testing.assert_allclose(g0, -2.5)


def test_inverse_softplus_roundtrip():
    dt = np.exp(_rng(5).uniform(np.log(1e-3), np.log(1e-1), 64))
    np.testing.assert_allclose(np.log1p(np.exp(ko.inverse_softplus(dt))), dt, rtol=1e-10)


def test_l2_normalize_and_rms_norm():
    x = _rng(6).standard_normal((5, 7))
    np.testing.assert_allclose(np.linalg.norm(ko.l2_normalize(x), axis=-1), 1.0, rtol=1e-12)
    assert np.all(ko.l2_normalize(np.zeros((1, 4))) == 0.0)
    y = ko.rms_norm(x, np.ones(7), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, rtol=1e-12)


# --------------------------------------------------------------- recurrence
def _raw(q, k, v, g, beta, h0=None):
    """Run the oracle with every in-kernel transform switched off."""
    return ko.kda_recurrent(q, k, v, g, beta, initial_state=h0, use_qk_l2norm=False,
                            use_gate=False, use_beta_sigmoid=False, scale=1.0, dtype=np.float64)


def test_single_step_by_hand_2x2():
    # S0 = [[1,2],[3,4]], alpha = (0.5, 0.25), k = (0.6, 0.8), beta = 0.5,
    # v = (1, 2), q = (1, 0).  Worked by hand:
    #   Diag(alpha) S0 = [[0.5, 1.0], [0.75, 1.0]]
    #   prediction = k^T (.)  = (0.9, 1.4)
    #   correction = (v - prediction) * beta = (0.05, 0.3)
    #   S1 = [[0.53, 1.18], [0.79, 1.24]],  o = S1^T q = (0.53, 1.18)
    s0 = np.array([[[[1.0, 2.0], [3.0, 4.0]]]])
    q = np.array([1.0, 0.0]).reshape(1, 1, 1, 2)
    k = np.array([0.6, 0.8]).reshape(1, 1, 1, 2)
    v = np.array([1.0, 2.0]).reshape(1, 1, 1, 2)
    g = np.log(np.array([0.5, 0.25])).reshape(1, 1, 1, 2)
    beta = np.array([0.5]).reshape(1, 1, 1)
    o, s1 = _raw(q, k, v, g, beta, s0)
    np.testing.assert_allclose(s1[0, 0], [[0.53, 1.18], [0.79, 1.24]], rtol=1e-12)
    np.testing.assert_allclose(o[0, 0, 0], [0.53, 1.18], rtol=1e-12)


def test_matches_explicit_matrix_form_of_equation_1():
    # S_t = (I - b_t k_t k_t^T) Diag(a_t) S_{t-1} + b_t k_t v_t^T, o_t = S_t^T q_t
    rng = _rng(7)
    key_dim, value_dim, steps = 6, 5, 9
    q = rng.standard_normal((1, steps, 1, key_dim))
    k = ko.l2_normalize(rng.standard_normal((1, steps, 1, key_dim)))
    v = rng.standard_normal((1, steps, 1, value_dim))
    g = rng.uniform(-5, 0, (1, steps, 1, key_dim))
    beta = rng.uniform(0, 1, (1, steps, 1))
    s = rng.standard_normal((key_dim, value_dim))
    o_ref = []
    o, st = _raw(q, k, v, g, beta, s[None, None])
    for t in range(steps):
        kk = k[0, t, 0]
        m = (np.eye(key_dim) - beta[0, t, 0] * np.outer(kk, kk)) @ np.diag(np.exp(g[0, t, 0]))
        s = m @ s + beta[0, t, 0] * np.outer(kk, v[0, t, 0])
        o_ref.append(s.T @ q[0, t, 0])
    np.testing.assert_allclose(o[0, :, 0], np.array(o_ref), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(st[0, 0], s, rtol=1e-10, atol=1e-12)


def test_beta_zero_is_pure_decay():
    rng = _rng(8)
    steps, key_dim = 7, 4
    s0 = rng.standard_normal((1, 1, key_dim, 3))
    q = rng.standard_normal((1, steps, 1, key_dim))
    g = rng.uniform(-2, 0, (1, steps, 1, key_dim))
    o, st = _raw(q, rng.standard_normal((1, steps, 1, key_dim)),
                 rng.standard_normal((1, steps, 1, 3)), g, np.zeros((1, steps, 1)), s0)
    decay = np.exp(np.cumsum(g[0, :, 0], axis=0))           # [steps, K]
    np.testing.assert_allclose(st[0, 0], decay[-1][:, None] * s0[0, 0], rtol=1e-12)
    for t in range(steps):
        np.testing.assert_allclose(o[0, t, 0], (decay[t][:, None] * s0[0, 0]).T @ q[0, t, 0],
                                   rtol=1e-10)


def test_orthonormal_keys_write_then_read_exactly():
    # alpha = 1, beta = 1 and orthonormal keys: each write stores v_j under
    # key e_j, and a query e_j reads it back unchanged.
    key_dim, value_dim = 4, 3
    rng = _rng(9)
    basis, _ = np.linalg.qr(rng.standard_normal((key_dim, key_dim)))
    vals = rng.standard_normal((key_dim, value_dim))
    k = basis.T.reshape(1, key_dim, 1, key_dim)
    q = np.concatenate([k, k], axis=1)
    kk = np.concatenate([k, k], axis=1)
    v = np.concatenate([vals, np.zeros_like(vals)], axis=0).reshape(1, 2 * key_dim, 1, value_dim)
    beta = np.concatenate([np.ones(key_dim), np.zeros(key_dim)]).reshape(1, 2 * key_dim, 1)
    o, _ = _raw(q, kk, v, np.zeros((1, 2 * key_dim, 1, key_dim)), beta)
    np.testing.assert_allclose(o[0, key_dim:, 0], vals, atol=1e-12)


def test_delta_rule_overwrites_same_key():
    # beta = 1, alpha = 1: writing v1 then v2 under the same unit key leaves v2.
    k = np.array([0.0, 1.0]).reshape(1, 1, 1, 2).repeat(2, axis=1)
    v = np.array([[1.0, -1.0], [5.0, 7.0]]).reshape(1, 2, 1, 2)
    o, st = _raw(k, k, v, np.zeros((1, 2, 1, 2)), np.ones((1, 2, 1)))
    np.testing.assert_allclose(o[0, 1, 0], [5.0, 7.0], atol=1e-12)
    np.testing.assert_allclose(st[0, 0], [[0, 0], [5.0, 7.0]], atol=1e-12)


def test_reference_defaults_normalise_and_scale():
    # The default flags reproduce _reference_kda: q, k normalised, q * K^-1/2.
    rng = _rng(10)
    shape = (1, 5, 2, 8)
    q, k, z = (rng.standard_normal(shape) for _ in range(3))
    v = rng.standard_normal((1, 5, 2, 8))
    bl = rng.standard_normal((1, 5, 2))
    a_log, dtb = rng.standard_normal(2), rng.standard_normal(16)
    o, st = ko.kda_recurrent(q, k, v, z, bl, A_log=a_log, dt_bias=dtb, dtype=np.float64)
    g = ko.kda_gate(z, a_log, dtb, -5.0)
    o2, st2 = _raw(ko.l2_normalize(q) * 8 ** -0.5, ko.l2_normalize(k), v, g, ko.sigmoid(bl))
    np.testing.assert_allclose(o, o2, rtol=1e-12)
    np.testing.assert_allclose(st, st2, rtol=1e-12)


def test_varlen_equals_each_sequence_alone_and_resets_state():
    rng = _rng(11)
    lens = [3, 1, 0, 7, 2]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, heads, dim = int(cu[-1]), 2, 4
    q, k, g = (rng.standard_normal((total, heads, dim)) for _ in range(3))
    v = rng.standard_normal((total, heads, dim))
    beta = rng.standard_normal((total, heads))
    h0 = rng.standard_normal((len(lens), heads, dim, dim))
    kw = dict(A_log=np.zeros(heads), dt_bias=rng.standard_normal(heads * dim), dtype=np.float64)
    o, ht = ko.kda_varlen(q, k, v, g, beta, cu, initial_states=h0, **kw)
    for s in range(len(lens)):
        a, b = cu[s], cu[s + 1]
        if a == b:
            np.testing.assert_array_equal(ht[s], h0[s])
            continue
        o1, h1 = ko.kda_recurrent(q[None, a:b], k[None, a:b], v[None, a:b], g[None, a:b],
                                  beta[None, a:b], initial_state=h0[s : s + 1], **kw)
        np.testing.assert_array_equal(o[a:b], o1[0])
        np.testing.assert_array_equal(ht[s], h1[0])


def test_c_oracle_matches_numpy_oracle():
    rng = _rng(12)
    lens = [17, 64, 1, 130]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, heads, dim = int(cu[-1]), 3, 16
    f = np.float32
    q, k, z = (rng.standard_normal((total, heads, dim)).astype(f) for _ in range(3))
    v = rng.standard_normal((total, heads, dim)).astype(f)
    bl = rng.standard_normal((total, heads)).astype(f)
    h0 = rng.standard_normal((len(lens), heads, dim, dim)).astype(f) * 0.1
    a_log = rng.standard_normal(heads).astype(f) * 0.3
    dtb = rng.standard_normal(heads * dim).astype(f)
    kw = dict(A_log=a_log, dt_bias=dtb, lower_bound=-5.0)
    o1, h1 = ko.kda_varlen(q, k, v, z, bl, cu, initial_states=h0, dtype=np.float64, **kw)
    o2, h2 = c_oracle.kda_varlen(q, k, v, z, bl, cu, initial_states=h0, **kw)
    np.testing.assert_allclose(o2, o1, rtol=2e-4, atol=2e-5)
    np.testing.assert_allclose(h2, h1, rtol=2e-4, atol=2e-5)


# -------------------------------------------- chunk algorithm of the kernels
@pytest.mark.parametrize("seed,length,lo", [(0, 1, -5.0), (1, 16, -5.0), (2, 63, -5.0),
                                            (3, 64, -1.0), (4, 65, -5.0), (5, 200, -0.5),
                                            (6, 129, -5.0)])
def test_chunk_algorithm_equals_recurrence(seed, length, lo):
    rng = _rng(100 + seed)
    dim = 16
    qn = ko.l2_normalize(rng.standard_normal((length, dim))) * dim ** -0.5
    kn = ko.l2_normalize(rng.standard_normal((length, dim)))
    v = rng.standard_normal((length, dim))
    g = rng.uniform(lo, 0.0, (length, dim))
    if seed % 2 == 0:
        g[: min(length, 20)] = -5.0                 # saturated decay: e^-80 per sub-block
    beta = rng.uniform(0, 1, length)
    s0 = rng.standard_normal((dim, dim))
    o_ref, s_ref = _raw(qn[None, :, None], kn[None, :, None], v[None, :, None],
                        g[None, :, None], beta[None, :, None], s0[None, None])
    o, s1 = chunk_model.kda_chunked(qn, kn, v, g, beta, s0)
    np.testing.assert_allclose(o, o_ref[0, :, 0], rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(s1, s_ref[0, 0], rtol=1e-9, atol=1e-11)


def test_gate_head_scale_closed_form():
    """A_log = ln 2 doubles the logit: g = lb * sigmoid(2 (z + b)).  At
    z + b = ln(3) / 2 that is lb * sigmoid(ln 3) = 3/4 lb exactly, while a
    dropped exp(A_log) would give lb * sigmoid(ln(3) / 2) = lb * sqrt(3) / (1 + sqrt(3))."""
    heads, d = 2, 4
    z = np.full((1, heads, d), np.log(3.0) / 2 - 0.25)
    dtb = np.full(heads * d, 0.25)
    a_log = np.array([np.log(2.0), 0.0])
    g = ko.kda_gate(z, a_log, dtb, -5.0)
    np.testing.assert_allclose(g[0, 0], -5.0 * 0.75, rtol=1e-6)
    np.testing.assert_allclose(g[0, 1], -5.0 * np.sqrt(3.0) / (1.0 + np.sqrt(3.0)), rtol=1e-6)
    # a head-wide A_log of ln 4 with z + b = ln(3) / 4: sigmoid(ln 3) again
    g4 = ko.kda_gate(np.full((1, 1, d), np.log(3.0) / 4), np.array([np.log(4.0)]), np.zeros(d), -2.0)
    np.testing.assert_allclose(g4, -1.5, rtol=1e-6)


def test_rms_norm_weight_matches_torch():
    """rms_norm with a non-unit weight and eps against torch's functional rms_norm
    (the routine the reference's RMSNorm calls, ml/runtime/model/ops.py:49-64)."""
    import torch

    rng = _rng(21)
    x = rng.standard_normal((6, 128)) * 3.0
    w = rng.uniform(0.25, 2.0, 128)
    for eps in (1e-5, 1e-6, 0.5):
        ref = torch.nn.functional.rms_norm(torch.tensor(x), (128,), torch.tensor(w), eps).numpy()
        np.testing.assert_allclose(ko.rms_norm(x, w, eps), ref, rtol=1e-12, atol=1e-12)
    # a scaled weight scales the output channel by channel
    np.testing.assert_allclose(ko.rms_norm(x, 2.0 * w, 1e-5), 2.0 * ko.rms_norm(x, w, 1e-5), rtol=1e-12)


def _epilogue_params(rng, heads=2, hd=8, gate_scale=0.0):
    """A tiny mixer (dim == inner, o_proj = identity) whose output is the
    epilogue RMSNorm(o) * sigmoid(x Wg^T) itself."""
    inner = heads * hd
    p = {name: rng.standard_normal((inner, inner)) * 0.3 for name in ("q_proj.weight", "k_proj.weight",
                                                                       "v_proj.weight")}
    for name in ("q_conv", "k_conv", "v_conv"):
        p[f"{name}.weight"] = rng.standard_normal((inner, 4)) * 0.4
    p["decay_down.weight"] = rng.standard_normal((4, inner)) * 0.2
    p["decay_up.weight"] = rng.standard_normal((inner, 4)) * 0.2
    p["beta_proj.weight"] = rng.standard_normal((heads, inner)) * 0.3
    p["A_log"] = np.zeros(heads)
    p["dt_bias"] = ko.inverse_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), inner)))
    p["output_gate.weight"] = rng.standard_normal((inner, inner)) * gate_scale
    p["output_norm.weight"] = rng.uniform(0.5, 1.5, hd)
    p["o_proj.weight"] = np.eye(inner)
    return p


def _unit_ms_defect(y, gate, w, heads, hd):
    """max over (token, head) of |mean((y / (gate * w))^2) - 1|."""
    unit = (y / gate).reshape(-1, heads, hd) / w
    return np.abs((unit ** 2).mean(-1) - 1.0).max()


@pytest.mark.parametrize("gate_scale", [0.0, 1.5])
def test_mixer_epilogue_is_norm_then_sigmoid_gate(gate_scale):
    """attention.py:411-420: y = o_proj(RMSNorm_head(o; w) * sigmoid(x Wg^T)).
    With o_proj = I and a tiny eps, y / (sigmoid(x Wg^T) * w) is o scaled to unit
    mean square in every (token, head).  Mistakes planted in a copy of the
    epilogue (gate before the norm, sigmoid dropped, norm over the whole row,
    norm weight dropped) each break that.  With Wg = 0 the gate is exactly 1/2."""
    heads, hd = 2, 8
    rng = _rng(31)
    p = _epilogue_params(rng, heads, hd, gate_scale)
    w = p["output_norm.weight"]
    x = rng.standard_normal((1, 7, heads * hd))
    y = ko.mixer_forward(p, x, num_heads=heads, head_dim=hd, norm_eps=1e-14)
    logits = x @ p["output_gate.weight"].T
    gate = ko.sigmoid(logits)
    if gate_scale == 0.0:
        np.testing.assert_array_equal(gate, 0.5)
    assert _unit_ms_defect(y, gate, w, heads, hd) < 1e-9
    # the recurrence's output, up to a positive scale per (token, head); the
    # heads are given unequal scales, as raw outputs have
    o = ((y / gate).reshape(1, 7, heads, hd) / w) * np.array([0.7, 2.9])[:, None]
    gate4 = gate.reshape(1, 7, heads, hd)
    planted = {
        "dropped norm weight": (ko.rms_norm(o, np.ones(hd), 1e-14) * gate4),
        "whole-row norm": (o / np.sqrt((o ** 2).mean((-2, -1), keepdims=True)) * w * gate4),
    }
    if gate_scale:
        assert np.ptp(gate4, axis=-1).min() > 0.1   # the gate varies over channels
        planted["gate before the norm"] = ko.rms_norm(o * gate4, w, 1e-14)
        planted["sigmoid dropped"] = ko.rms_norm(o, w, 1e-14) * logits.reshape(1, 7, heads, hd)
    for name, bad in planted.items():
        assert _unit_ms_defect(bad.reshape(y.shape), gate, w, heads, hd) > 1e-2, name
    # o_proj = P is P applied to the same epilogue output
    proj = rng.standard_normal((heads * hd - 3, heads * hd))
    q = dict(p, **{"o_proj.weight": proj})
    np.testing.assert_allclose(ko.mixer_forward(q, x, num_heads=heads, head_dim=hd, norm_eps=1e-14),
                               y @ proj.T, rtol=1e-10, atol=1e-12)
