"""The float64 torch mixer restatement (tests/mixer_autograd_ref.py), which the
GPU training tests differentiate, against the numpy oracle's mixer_forward
(oracle/kda_oracle.py, pinned in test_oracle_kda.py): two independent
restatements of attention.py:373-420 must agree to float64 rounding.  And
its ShortConv against numpy.convolve per channel."""

from __future__ import annotations

import numpy as np
import torch

from oracle import kda_oracle as ko
from mixer_autograd_ref import mixer_forward_ref, short_conv_ref


def _params(rng, dim=24, heads=2, rank=8):
    inner = heads * 128
    p = {name: rng.standard_normal((inner, dim)) * 0.2 for name in
         ("q_proj.weight", "k_proj.weight", "v_proj.weight", "output_gate.weight")}
    for name in ("q_conv", "k_conv", "v_conv"):
        p[f"{name}.weight"] = rng.standard_normal((inner, 4)) * 0.4
    p["decay_down.weight"] = rng.standard_normal((rank, dim)) * 0.2
    p["decay_up.weight"] = rng.standard_normal((inner, rank)) * 0.2
    p["beta_proj.weight"] = rng.standard_normal((heads, dim)) * 0.3
    p["A_log"] = rng.standard_normal(heads) * 0.3
    p["dt_bias"] = ko.inverse_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), inner)))
    p["output_norm.weight"] = rng.uniform(0.5, 1.5, 128)
    p["o_proj.weight"] = rng.standard_normal((dim, inner)) * 0.2
    return p


def test_torch_mixer_restatement_equals_numpy_oracle():
    rng = np.random.default_rng(7)
    p = _params(rng)
    x = rng.standard_normal((2, 19, 24))
    want = ko.mixer_forward(p, x, num_heads=2, head_dim=128)
    got = mixer_forward_ref({k: torch.tensor(v) for k, v in p.items()}, torch.tensor(x), heads=2).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-11)


def test_torch_short_conv_restatement_equals_numpy_convolve():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((1, 11, 5))
    w = rng.standard_normal((5, 4))
    hist = rng.standard_normal((1, 5, 3))
    got = short_conv_ref(torch.tensor(x), torch.tensor(w), torch.tensor(hist)).numpy()
    for c in range(5):
        seq = np.concatenate([hist[0, c], x[0, :, c]])
        conv = np.convolve(seq, w[c][::-1], mode="valid")   # w[c, 3] multiplies the newest sample
        np.testing.assert_allclose(got[0, :, c], conv / (1 + np.exp(-conv)), rtol=1e-12, atol=1e-14)
