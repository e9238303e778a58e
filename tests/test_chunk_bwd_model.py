"""The chunked backward (tests/chunk_bwd_model.py) against the oracle's
per-token reverse recurrence (oracle.kda_oracle.kda_varlen_bwd): two
independent derivations of the same gradients must agree to float64
rounding.  Small head dims keep it fast; the chunk length is the kernels' 64.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kda_oracle as ko
from tests import chunk_bwd_model as cbm


def _case(total, key_dim, value_dim, seed, g_lo=-5.0, g_hi=0.0):
    rng = np.random.default_rng(seed)
    qn = rng.standard_normal((total, key_dim)) / np.sqrt(key_dim)
    kn = rng.standard_normal((total, key_dim))
    kn /= np.linalg.norm(kn, axis=1, keepdims=True)
    v = rng.standard_normal((total, value_dim))
    g = rng.uniform(g_lo, g_hi, (total, key_dim))
    beta = rng.uniform(0.0, 1.0, total)
    s0 = rng.standard_normal((key_dim, value_dim)) * 0.5
    do = rng.standard_normal((total, value_dim))
    dsf = rng.standard_normal((key_dim, value_dim)) * 0.5
    return qn, kn, v, g, beta, s0, do, dsf


def _oracle(qn, kn, v, g, beta, s0, do, dsf):
    total = qn.shape[0]
    cu = np.array([0, total])
    r = ko.kda_varlen_bwd(qn[:, None], kn[:, None], v[:, None], g[:, None], beta[:, None], cu,
                          do[:, None], d_final_states=dsf[None, None], initial_states=s0[None, None],
                          use_qk_l2norm=False, use_gate=False, use_beta_sigmoid=False, scale=1.0)
    return (r["dq"][:, 0], r["dk"][:, 0], r["dv"][:, 0], r["dg"][:, 0], r["dbeta"][:, 0],
            r["dh0"][0, 0])


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


@pytest.mark.parametrize("total,seed", [(64, 0), (150, 1), (200, 2), (1, 3)])
def test_chunked_backward_equals_recurrent_backward(total, seed):
    args = _case(total, 16, 8, seed)
    got = cbm.kda_chunked_bwd(*args)
    ref = _oracle(*args)
    names = ("dq", "dk", "dv", "dg", "dbeta", "dh0")
    for name, a, b in zip(names, got, ref):
        assert _rel(a, b) < 1e-9, (name, _rel(a, b))


def test_chunked_backward_slow_decay_and_zero_beta_rows():
    """Long memory (g near 0) and some beta = 0 rows (no write)."""
    qn, kn, v, g, beta, s0, do, dsf = _case(130, 8, 8, 7, g_lo=-1e-3, g_hi=0.0)
    beta[::5] = 0.0
    got = cbm.kda_chunked_bwd(qn, kn, v, g, beta, s0, do, dsf)
    ref = _oracle(qn, kn, v, g, beta, s0, do, dsf)
    for a, b in zip(got, ref):
        assert _rel(a, b) < 1e-9


def test_reverse_chunk_scan_step_needs_no_state():
    """dS0 of a chunk from dS1 and dO alone equals the full chunk backward's."""
    qn, kn, v, g, beta, s0, do, dsf = _case(64, 16, 8, 11)
    _, _, ctx = cbm.chunk_forward(qn, kn, v, g, beta, s0)
    ds0_full = cbm.chunk_backward(ctx, do, dsf)[-1]
    ctx2 = dict(ctx, s0=np.full_like(s0, np.nan))        # the state must not be read
    ds0 = cbm.chunk_dstate(ctx2, do, dsf)
    assert _rel(ds0, ds0_full) < 1e-12


@pytest.mark.parametrize("g_lo,seed", [(-5.0, 21), (-1e-3, 22), (-0.5, 23)])
def test_factored_decay_products_equal_the_chunk_backward(g_lo, seed):
    """The sub-block-factored products (no factor above e^80) give the same
    chunk gradients as the whole-chunk exponentials, for a full and a partial
    chunk, including the strongest decay (cumulative log-decay -320)."""
    for c in (64, 37):
        qn, kn, v, g, beta, s0, do, dsf = _case(c, 16, 8, seed, g_lo=g_lo, g_hi=0.0)
        _, _, ctx = cbm.chunk_forward(qn, kn, v, g, beta, s0)
        ref = cbm.chunk_backward(ctx, do, dsf)
        got = cbm.chunk_backward_factored(ctx, do, dsf)
        for a, b in zip(got, ref):
            assert _rel(a, b) < 1e-10


def test_factored_decay_products_are_fp32_safe():
    """In float32 the factored products stay finite at the strongest decay and
    match float64 to fp32 rounding (the whole-chunk e^-G would overflow)."""
    qn, kn, v, g, beta, s0, do, dsf = _case(64, 16, 8, 31, g_lo=-5.0, g_hi=-4.0)
    _, _, ctx = cbm.chunk_forward(qn, kn, v, g, beta, s0)
    rng = np.random.default_rng(32)
    rows = np.arange(64)
    dA_qk = np.where(rows[:, None] >= rows[None, :], rng.standard_normal((64, 64)), 0.0)
    dP = np.where(rows[:, None] > rows[None, :], rng.standard_normal((64, 64)), 0.0)
    ref = cbm.decay_products_factored(ctx, dA_qk, dP)
    ctx32 = {key: ctx[key].astype(np.float32) for key in ("qn", "kn", "G")}
    with np.errstate(over="raise", invalid="raise"):
        got = cbm.decay_products_factored(ctx32, dA_qk.astype(np.float32), dP.astype(np.float32))
    assert np.exp(-ctx["G"].min()) > np.finfo(np.float32).max   # e^-G alone overflows fp32
    for a, b in zip(got, ref):
        assert np.all(np.isfinite(a))
        assert _rel(a, b) < 1e-4


@pytest.mark.parametrize("total,seed,g_lo", [(64, 11, -5.0), (45, 12, -0.5), (64, 13, -0.05)])
def test_gradient_kernel_identities(total, seed, g_lo):
    """The per-chunk gradient kernel forms neither dW nor dT: since
    U = T (Xu - Xw S0), dT = dW Xw^T + dU Xu^T = dU (T^-1 U)^T, so
    tril_strict(-T^T dT T^T) = tril_strict(-T^T Y) with Y the strictly lower
    part of dU U^T (the only part the strict result reads), and
    T^T dW = -(T^T dU) S0^T.  The plausible slips (U dU^T for dU U^T, T for
    T^T) break the equality."""
    qn, kn, v, g, beta, s0, do, dsf = _case(total, 32, 24, seed, g_lo=g_lo)
    o, s1, ctx = cbm.chunk_forward(qn, kn, v, g, beta, s0)
    do = cbm._pad(do, cbm.CHUNK - total)
    dU = ctx["A_qk"].T @ do + ctx["Kbar"] @ dsf
    T, U, strict = ctx["T"], ctx["U"], ctx["strict"]
    dW = -dU @ s0.T
    dT = dW @ ctx["Xw"].T + dU @ ctx["Xu"].T
    want = np.where(strict, -T.T @ dT @ T.T, 0.0)
    got = np.where(strict, -T.T @ np.where(strict, dU @ U.T, 0.0), 0.0)
    assert _rel(got, want) < 1e-11
    assert _rel(-(T.T @ dU) @ s0.T, T.T @ dW) < 1e-11
    for bad in (np.where(strict, -T.T @ np.where(strict, U @ dU.T, 0.0), 0.0),
                np.where(strict, -T @ np.where(strict, dU @ U.T, 0.0), 0.0)):
        assert _rel(bad, want) > 1e-3
