"""Pins the oracle's KDA backward (kda_varlen_bwd) on the CPU.

Two independent checks, both in float64:
  * central finite differences of the oracle's own forward (kda_varlen) for
    every input element of a small packed batch, in both flag settings;
  * torch.autograd through a separate torch restatement of the recurrence
    (tests/kda_autograd_ref.py), which shares no code with the oracle.
A planted mistake in the backward (a dropped term, a sign) fails both.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kda_oracle as ko

from kda_autograd_ref import kda_packed_grads

K = V = 4
H = 2
CU = [0, 3, 3, 8]          # includes an empty sequence


def _case(seed: int, gated: bool):
    rng = np.random.default_rng(seed)
    total, n = CU[-1], len(CU) - 1
    inp = {
        "q": rng.standard_normal((total, H, K)),
        "k": rng.standard_normal((total, H, K)),
        "v": rng.standard_normal((total, H, V)),
        "beta": rng.standard_normal((total, H)),
        "h0": rng.standard_normal((n, H, K, V)) * 0.5,
    }
    if gated:
        inp["g"] = rng.standard_normal((total, H, K))
        inp["A_log"] = rng.uniform(-1.0, 1.0, H)
        inp["dt_bias"] = rng.standard_normal(H * K) * 0.5
    else:
        inp["g"] = -rng.uniform(0.0, 1.0, (total, H, K))     # log-decay in [-1, 0]
        inp["beta"] = rng.uniform(0.1, 0.9, (total, H))
    d_out = rng.standard_normal((total, H, V))
    d_final = rng.standard_normal((n, H, K, V))
    flags = dict(use_qk_l2norm=gated, use_gate=gated, use_beta_sigmoid=gated)
    return inp, d_out, d_final, flags


def _loss(inp, d_out, d_final, flags):
    o, fin = ko.kda_varlen(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], CU,
                           initial_states=inp["h0"], A_log=inp.get("A_log"),
                           dt_bias=inp.get("dt_bias"), dtype=np.float64, **flags)
    return float(np.sum(o * d_out) + np.sum(fin * d_final))


def _oracle_grads(inp, d_out, d_final, flags):
    r = ko.kda_varlen_bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], CU, d_out,
                          d_final_states=d_final, initial_states=inp["h0"],
                          A_log=inp.get("A_log"), dt_bias=inp.get("dt_bias"), **flags)
    names = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "h0": "dh0",
             "A_log": "dA_log", "dt_bias": "ddt_bias"}
    return {name: r[key] for name, key in names.items() if name in inp}


@pytest.mark.parametrize("gated", [True, False])
def test_backward_matches_finite_differences(gated):
    inp, d_out, d_final, flags = _case(11 if gated else 12, gated)
    grads = _oracle_grads(inp, d_out, d_final, flags)
    eps = 1e-6
    for name, val in inp.items():
        fd = np.zeros_like(val)
        flat, fd_flat = val.reshape(-1), fd.reshape(-1)
        for i in range(flat.size):
            keep = flat[i]
            flat[i] = keep + eps
            up = _loss(inp, d_out, d_final, flags)
            flat[i] = keep - eps
            down = _loss(inp, d_out, d_final, flags)
            flat[i] = keep
            fd_flat[i] = (up - down) / (2 * eps)
        np.testing.assert_allclose(grads[name].reshape(fd.shape), fd, rtol=1e-6, atol=1e-7,
                                   err_msg=f"d{name}")


@pytest.mark.parametrize("gated", [True, False])
def test_backward_matches_torch_autograd(gated):
    inp, d_out, d_final, flags = _case(21 if gated else 22, gated)
    grads = _oracle_grads(inp, d_out, d_final, flags)
    ref = kda_packed_grads(inp, CU, d_out, d_final, **flags)
    for name in inp:
        np.testing.assert_allclose(grads[name], ref[name], rtol=1e-10, atol=1e-12,
                                   err_msg=f"d{name}")


def test_backward_without_final_gradient_is_output_only():
    """d_final_states=None equals a zero final-state gradient."""
    inp, d_out, _, flags = _case(31, True)
    a = _oracle_grads(inp, d_out, None, flags)
    b = _oracle_grads(inp, d_out, np.zeros((len(CU) - 1, H, K, V)), flags)
    for name in a:
        np.testing.assert_array_equal(a[name], b[name])


def test_dropped_final_state_term_is_caught():
    """A backward that forgets the final-state gradient (a dropped term) is
    rejected by the same finite-difference tolerance."""
    inp, d_out, d_final, flags = _case(41, False)
    bad = _oracle_grads(inp, d_out, None, flags)["v"]
    eps = 1e-6
    val = inp["v"].reshape(-1)
    keep = val[0]
    val[0] = keep + eps
    up = _loss(inp, d_out, d_final, flags)
    val[0] = keep - eps
    down = _loss(inp, d_out, d_final, flags)
    val[0] = keep
    fd0 = (up - down) / (2 * eps)
    assert abs(bad.reshape(-1)[0] - fd0) > 1e-3


def test_c_backward_matches_numpy_backward():
    """The C restatement of the backward (the CPU baseline of bench.py's
    backward leg) equals the numpy float64 backward to fp32 rounding."""
    from oracle import c_oracle
    rng = np.random.default_rng(51)
    cu = [0, 20, 20, 75, 100]
    heads, kd, vd = 2, 16, 24
    total = cu[-1]
    for gated in (True, False):
        q = rng.standard_normal((total, heads, kd))
        k = rng.standard_normal((total, heads, kd))
        v = rng.standard_normal((total, heads, vd))
        g = rng.standard_normal((total, heads, kd)) if gated else -rng.uniform(0, 1, (total, heads, kd))
        beta = rng.standard_normal((total, heads)) if gated else rng.uniform(0, 1, (total, heads))
        a_log = rng.uniform(-1, 1, heads)
        dt_bias = rng.standard_normal(heads * kd) * 0.5
        h0 = rng.standard_normal((4, heads, kd, vd)) * 0.3
        d_out = rng.standard_normal((total, heads, vd))
        d_fin = rng.standard_normal((4, heads, kd, vd)) * 0.3
        kw = dict(use_qk_l2norm=gated, use_gate=gated, use_beta_sigmoid=gated, A_log=a_log,
                  dt_bias=dt_bias, initial_states=h0, d_final_states=d_fin)
        want = ko.kda_varlen_bwd(q, k, v, g, beta, cu, d_out, **kw)
        got = c_oracle.kda_varlen_bwd(q, k, v, g, beta, cu, d_out, **kw)
        assert set(got) == set(want)
        for name in want:
            err = np.max(np.abs(got[name] - want[name])) / max(np.max(np.abs(want[name])), 1e-30)
            assert err < 1e-4, f"gated={gated} {name}: {err:.2e}"
