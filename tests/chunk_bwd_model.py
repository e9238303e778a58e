"""Float64 numpy model of a chunked (C = 64) KDA backward.

A design model, not the oracle: it differentiates the chunk form of
``chunk_model.py`` by hand, so that a chunk-parallel backward can be checked
against the per-token reverse recurrence of the oracle
(``oracle.kda_oracle.kda_varlen_bwd``) on the CPU.  The HIP backward in
``sophia_amd/csrc/kda_bwd.hip`` runs the per-token recurrence; this model is
the specification of the chunked form that replaces its per-token work with
matrix products.

Per chunk, with the within-chunk cumulative log-decay G, Gamma = G[C-1],
Kg = K e^G, Kn = K e^-G, Qg = Q e^G, Kbar = K e^(Gamma - G):

  forward   A_kk = tril_strict(Diag(beta) Kg Kn^T), A_qk = tril(Qg Kn^T),
            T = (I + A_kk)^-1, W = T Diag(beta) Kg, Ut = T Diag(beta) V,
            U = Ut - W S0, O = Qg S0 + A_qk U, S1 = Diag(e^Gamma) S0 + Kbar^T U
  backward  dU = A_qk^T dO + Kbar dS1
            dS0 = Diag(e^Gamma) dS1 + Qg^T dO - W^T dU      (the reverse chunk scan)
            dA_qk = tril(dO U^T), dQg = dO S0^T, dW = -dU S0^T, dKbar = U dS1^T
            dT = dW (Diag(beta) Kg)^T + dU (Diag(beta) V)^T,
            dA_kk = tril_strict(-T^T dT T^T), then the products back to Q, K, V,
            beta and G, and dg = reverse cumsum of dG plus dGamma on every row.

``chunk_backward`` forms the exponentials over a whole chunk (float64 holds
e^320).  ``chunk_backward_factored`` is the form fp32 kernels need: the
products through A_qk and A_kk take the forward's per-16-token sub-block
factors (``decay_products_factored``), so no factor exceeds e^80, and every
other exponential it forms is at most 1.
"""

from __future__ import annotations

import numpy as np

CHUNK = 64


def _pad(x, pad):
    return np.concatenate([x, np.zeros((pad,) + x.shape[1:], dtype=x.dtype)], axis=0)


def chunk_forward(qn, kn, v, g, beta, s0):
    """Forward of one chunk (rows past c zero-padded).  Returns (o [c, V],
    s1 [K, V], ctx) with the intermediates the backward reads."""
    c = qn.shape[0]
    pad = CHUNK - c
    qn, kn, v, g, beta = (_pad(np.asarray(x, dtype=np.float64), pad) for x in (qn, kn, v, g, beta))
    G = np.cumsum(g, axis=0)
    gam = G[-1]
    eg, eng = np.exp(G), np.exp(-G)
    Kg, Kn, Qg = kn * eg, kn * eng, qn * eg
    Kbar = kn * np.exp(gam[None, :] - G)
    rows = np.arange(CHUNK)
    strict = rows[:, None] > rows[None, :]
    incl = rows[:, None] >= rows[None, :]
    P = np.where(strict, Kg @ Kn.T, 0.0)
    A_kk = beta[:, None] * P
    A_qk = np.where(incl, Qg @ Kn.T, 0.0)
    T = np.linalg.inv(np.eye(CHUNK) + A_kk)
    Xw = beta[:, None] * Kg
    Xu = beta[:, None] * v
    W = T @ Xw
    Ut = T @ Xu
    U = Ut - W @ s0
    o = Qg @ s0 + A_qk @ U
    s1 = np.exp(gam)[:, None] * s0 + Kbar.T @ U
    ctx = dict(c=c, qn=qn, kn=kn, v=v, beta=beta, G=G, gam=gam, Kg=Kg, Kn=Kn, Qg=Qg, Kbar=Kbar,
               A_qk=A_qk, P=P, T=T, Xw=Xw, Xu=Xu, W=W, U=U, s0=s0, strict=strict, incl=incl)
    return o[:c], s1, ctx


def chunk_dstate(ctx, do, ds1):
    """The reverse chunk-scan step alone: dS0 from dS1 and the chunk's dO
    (needs no forward state)."""
    do = _pad(np.asarray(do, dtype=np.float64), CHUNK - ctx["c"])
    dU = ctx["A_qk"].T @ do + ctx["Kbar"] @ ds1
    return np.exp(ctx["gam"])[:, None] * ds1 + ctx["Qg"].T @ do - ctx["W"].T @ dU


def chunk_backward(ctx, do, ds1):
    """Gradients of one chunk given dO [c, V] and dS1 [K, V]: (dqn, dkn, dv,
    dg, dbeta) for its c rows and dS0."""
    c = ctx["c"]
    do = _pad(np.asarray(do, dtype=np.float64), CHUNK - c)
    s0, U, T, W = ctx["s0"], ctx["U"], ctx["T"], ctx["W"]
    beta, v, kn, qn = ctx["beta"], ctx["v"], ctx["kn"], ctx["qn"]
    Kg, Kn, Qg, Kbar, A_qk = ctx["Kg"], ctx["Kn"], ctx["Qg"], ctx["Kbar"], ctx["A_qk"]
    gam = ctx["gam"]

    dU = A_qk.T @ do + Kbar @ ds1
    ds0 = np.exp(gam)[:, None] * ds1 + Qg.T @ do - W.T @ dU
    dA_qk = np.where(ctx["incl"], do @ U.T, 0.0)
    dQg = do @ s0.T
    dW = -dU @ s0.T
    dKbar = U @ ds1.T
    dgam = np.sum(ds1 * s0, axis=1) * np.exp(gam)          # through Diag(e^Gamma) S0
    # W = T Xw, Ut = T Xu (dUt = dU)
    dT = dW @ ctx["Xw"].T + dU @ ctx["Xu"].T
    dXw = T.T @ dW
    dXu = T.T @ dU
    dv = beta[:, None] * dXu
    dbeta = np.sum(dXu * v, axis=1) + np.sum(dXw * Kg, axis=1)
    dKg = beta[:, None] * dXw
    # T = (I + A_kk)^-1
    dA_kk = np.where(ctx["strict"], -T.T @ dT @ T.T, 0.0)
    # A_kk = tril_strict(Diag(beta) Kg Kn^T)
    P = Kg @ Kn.T
    dbeta += np.sum(dA_kk * P, axis=1)
    dKg += beta[:, None] * (dA_kk @ Kn)
    dKn = (beta[:, None] * dA_kk).T @ Kg
    # A_qk = tril(Qg Kn^T)
    dQg += dA_qk @ Kn
    dKn += dA_qk.T @ Qg
    # elementwise: Kg = K e^G, Kn = K e^-G, Qg = Q e^G, Kbar = K e^(Gamma - G)
    eG = np.exp(ctx["G"])
    dkn = dKg * eG + dKn / eG + dKbar * np.exp(gam[None, :] - ctx["G"])
    dqn = dQg * eG
    dG = dKg * Kg - dKn * Kn + dQg * Qg - dKbar * Kbar
    dgam = dgam + np.sum(dKbar * Kbar, axis=0)
    # G = cumsum(g), Gamma = G[C-1]
    dg = np.cumsum(dG[::-1], axis=0)[::-1] + dgam[None, :]
    return dqn[:c], dkn[:c], dv[:c], dg[:c], dbeta[:c], ds0


def kda_chunked_bwd(qn, kn, v, g, beta, s0, do, ds_final=None):
    """One sequence: qn, kn [T, K] (already scaled / normalised); v [T, V];
    g [T, K] log-decay; beta [T]; s0 [K, V]; do [T, V]; ds_final [K, V] or
    None.  Returns (dqn, dkn, dv, dg, dbeta, ds0).

    A forward pass keeps each chunk's entering state, a reverse pass carries
    dS across chunks; every chunk's gradients then depend only on its own
    S0, dS1 and dO (computed here in the reverse pass, in parallel on a GPU)."""
    total, key_dim = qn.shape
    value_dim = v.shape[1]
    state = np.array(s0, dtype=np.float64)
    ctxs = []
    for start in range(0, total, CHUNK):
        stop = min(total, start + CHUNK)
        _, state, ctx = chunk_forward(qn[start:stop], kn[start:stop], v[start:stop], g[start:stop],
                                      beta[start:stop], state)
        ctxs.append((start, stop, ctx))
    ds = np.zeros((key_dim, value_dim)) if ds_final is None else np.array(ds_final, dtype=np.float64)
    out = [np.zeros((total, key_dim)), np.zeros((total, key_dim)), np.zeros((total, value_dim)),
           np.zeros((total, key_dim)), np.zeros(total)]
    for start, stop, ctx in reversed(ctxs):
        dq_c, dk_c, dv_c, dg_c, db_c, ds = chunk_backward(ctx, do[start:stop], ds)
        for arr, part in zip(out, (dq_c, dk_c, dv_c, dg_c, db_c)):
            arr[start:stop] = part
    return (*out, ds)


SUB = 16


def _factors(G):
    """Sub-block reference points of chunk_model.py: ref[s] = G[16 s - 1]
    (ref[0] = 0), and the per-row factors a = e^(G - ref[blk]) <= 1,
    bq = e^(ref[blk] - G) <= e^80, d = e^(ref[blk + 1] - G) <= 1."""
    key_dim = G.shape[1]
    ref = np.zeros((5, key_dim))
    for s in range(1, 5):
        ref[s] = G[SUB * s - 1]
    blk = np.arange(CHUNK) // SUB
    a = np.exp(G - ref[blk])
    bq = np.exp(ref[blk] - G)
    d = np.exp(ref[blk + 1] - G)
    return ref, a, bq, d


def decay_products_factored(ctx, dA_qk, dP):
    """The gradient products through A_qk = tril(Qg Kn^T) and P = Kg Kn^T (the
    unmasked A_kk / beta) with no factor above e^80, as fp32 kernels form them.

    For r in sub-block i and j in sub-block b <= i,
    e^(G_r - G_j) = a_r f_ib d_j with f_ib = e^(ref_i - ref_(b+1)) <= 1 (b < i),
    and a_r bq_j on the diagonal blocks.  Returns (dq_e, dk_e, dG_e): the
    contributions of dA_qk and dP to dq, dk and dG, equal to
    dQg += dA_qk Kn, dKg += dP Kn, dKn = dA_qk^T Qg + dP^T Kg taken through
    Qg = Q e^G, Kg = K e^G, Kn = K e^-G."""
    qn, kn, G = ctx["qn"], ctx["kn"], ctx["G"]
    ref, a, bq, d = _factors(G)
    QS, KS = qn * a, kn * a             # <= |q|, |k|
    KB, KD = kn * bq, kn * d            # KB only on diagonal blocks
    dq_p = np.zeros_like(qn)            # sum_j dA_qk[r, j] k_j e^(G_r - G_j)
    dkg_p = np.zeros_like(kn)           # sum_j dP[r, j] k_j e^(G_r - G_j)
    dkq = np.zeros_like(kn)             # sum_r dA_qk[r, j] q_r e^(G_r - G_j)
    dkk = np.zeros_like(kn)             # sum_r dP[r, j] k_r e^(G_r - G_j)
    for i in range(4):
        ri = slice(SUB * i, SUB * i + SUB)
        for b in range(i + 1):
            rb = slice(SUB * b, SUB * b + SUB)
            Aq, Ak = dA_qk[ri, rb], dP[ri, rb]
            if b == i:
                dq_p[ri] += a[ri] * (Aq @ KB[rb])
                dkg_p[ri] += a[ri] * (Ak @ KB[rb])
                dkq[rb] += bq[rb] * (Aq.T @ QS[ri])
                dkk[rb] += bq[rb] * (Ak.T @ KS[ri])
            else:
                f = np.exp(ref[i] - ref[b + 1])[None, :]
                dq_p[ri] += a[ri] * f * (Aq @ KD[rb])
                dkg_p[ri] += a[ri] * f * (Ak @ KD[rb])
                dkq[rb] += d[rb] * f * (Aq.T @ QS[ri])
                dkk[rb] += d[rb] * f * (Ak.T @ KS[ri])
    dq_e = dq_p
    dk_e = dkg_p + dkq + dkk
    dG_e = qn * dq_p + kn * dkg_p - kn * (dkq + dkk)
    return dq_e, dk_e, dG_e


def chunk_backward_factored(ctx, do, ds1):
    """chunk_backward with the A_qk / A_kk products through the sub-block
    factors (decay_products_factored) instead of e^G and e^-G over the chunk;
    every other exponential it forms is at most 1."""
    c = ctx["c"]
    do = _pad(np.asarray(do, dtype=np.float64), CHUNK - c)
    s0, U, T, W = ctx["s0"], ctx["U"], ctx["T"], ctx["W"]
    beta, v, kn = ctx["beta"], ctx["v"], ctx["kn"]
    Kg, Qg, Kbar, A_qk = ctx["Kg"], ctx["Qg"], ctx["Kbar"], ctx["A_qk"]
    G, gam = ctx["G"], ctx["gam"]
    dU = A_qk.T @ do + Kbar @ ds1
    ds0 = np.exp(gam)[:, None] * ds1 + Qg.T @ do - W.T @ dU
    dA_qk = np.where(ctx["incl"], do @ U.T, 0.0)
    dQg = do @ s0.T
    dW = -dU @ s0.T
    dKbar = U @ ds1.T
    dgam = np.sum(ds1 * s0, axis=1) * np.exp(gam)
    dT = dW @ ctx["Xw"].T + dU @ ctx["Xu"].T
    dXw = T.T @ dW
    dXu = T.T @ dU
    dv = beta[:, None] * dXu
    dbeta = np.sum(dXu * v, axis=1) + np.sum(dXw * Kg, axis=1)
    dA_kk = np.where(ctx["strict"], -T.T @ dT @ T.T, 0.0)
    A_kk_over_beta = ctx["P"]
    # A_kk = Diag(beta) P (strict): dbeta from P = A_kk / beta without dividing
    dbeta += np.sum(dA_kk * A_kk_over_beta, axis=1)
    dP = beta[:, None] * dA_kk
    dq_e, dk_e, dG_e = decay_products_factored(ctx, dA_qk, dP)
    eG = np.exp(G)                      # <= 1
    dKg = beta[:, None] * dXw
    dqn = dQg * eG + dq_e
    dkn = dKg * eG + dKbar * np.exp(gam[None, :] - G) + dk_e
    dG = dKg * Kg + dQg * Qg - dKbar * Kbar + dG_e
    dgam = dgam + np.sum(dKbar * Kbar, axis=0)
    dg = np.cumsum(dG[::-1], axis=0)[::-1] + dgam[None, :]
    return dqn[:c], dkn[:c], dv[:c], dg[:c], dbeta[:c], ds0
