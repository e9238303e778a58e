"""Float64 numpy model of the chunk-64 KDA prefill algorithm run by the HIP kernels.

This is a design model, not the oracle: it restates, step by step and with the
same exponent factorisation, what ``sophia_amd/csrc/kda_chunk.hip`` computes,
so that the algorithm itself can be checked against the per-token recurrence
of the oracle on the CPU.

Per chunk of C=64 tokens (zero-padded at the tail of a sequence) with the
within-chunk inclusive cumulative log-decay G[r] = sum_{t<=r} g[t]:

* U  = T (beta V) - T (beta K e^G) S0  with T = (I + A_kk)^-1,
  A_kk[r, j] = beta_r sum_c k_rc k_jc exp(G_rc - G_jc), j < r;
* O  = (Q e^G) S0 + A_qk U,  A_qk[r, j] = sum_c q_rc k_jc exp(G_rc - G_jc), j <= r;
* S1 = Diag(e^{G_C}) S0 + (K e^{G_C - G})^T U.

Exponents are never formed as exp(G_r) * exp(-G_j) over a whole chunk: with
g >= -5 a 64-token cumulative decay reaches e^-320.  The chunk is cut into
four 16-token sub-blocks with reference points ref[s] = G[16 s - 1]
(ref[0] = 0, ref[4] = G_C).  Every factor is then either <= 1 (safe: it can
only underflow when the true product is negligible) or, on the diagonal
sub-blocks only, <= e^80 (finite in fp32 and bf16).
"""

from __future__ import annotations

import numpy as np

CHUNK = 64
SUB = 16


def chunk_states(qn, kn, v, g, beta, s0):
    """One chunk.  qn (scaled+normalised), kn: [c, K]; v: [c, V]; g: log-decay
    [c, K]; beta: [c]; s0: [K, V].  Returns (o [c, V], s1 [K, V])."""
    c = qn.shape[0]
    key_dim = qn.shape[1]
    pad = CHUNK - c

    def padded(x):
        return np.concatenate([x, np.zeros((pad,) + x.shape[1:], dtype=x.dtype)], axis=0)

    qn, kn, v, g, beta = (padded(x) for x in (qn, kn, v, g, beta))
    G = np.cumsum(g, axis=0)
    ref = np.zeros((5, key_dim))
    for s in range(1, 5):
        ref[s] = G[SUB * s - 1]
    blk = np.arange(CHUNK) // SUB
    a = np.exp(G - ref[blk])                      # <= 1
    b = np.exp(ref[blk] - G)                      # in [1, e^80]
    d = b * np.exp(ref[blk + 1] - ref[blk])       # <= 1
    QS, KS, KB, KD = qn * a, kn * a, kn * b, kn * d
    A_qk = np.zeros((CHUNK, CHUNK))
    A_kk = np.zeros((CHUNK, CHUNK))
    for i in range(4):
        ri = slice(SUB * i, SUB * i + SUB)
        for j in range(i + 1):
            rj = slice(SUB * j, SUB * j + SUB)
            if i == j:
                qa, ka, kb = QS[ri], KS[ri], KB[rj]
            else:
                f = np.exp(ref[i] - ref[j + 1])   # <= 1
                qa, ka, kb = QS[ri] * f, KS[ri] * f, KD[rj]
            A_qk[ri, rj] = qa @ kb.T
            A_kk[ri, rj] = ka @ kb.T
    rows = np.arange(CHUNK)
    A_qk = np.where(rows[:, None] >= rows[None, :], A_qk, 0.0)
    A_kk = np.where(rows[:, None] > rows[None, :], A_kk, 0.0) * beta[:, None]
    T = np.linalg.inv(np.eye(CHUNK) + A_kk)
    eref = np.exp(ref[blk])
    W = T @ (beta[:, None] * KS * eref)
    Ut = T @ (beta[:, None] * v)
    Qbar = QS * eref
    Kbar = KD * np.exp(ref[4][None, :] - ref[blk + 1])
    gamma = np.exp(ref[4])
    U = Ut - W @ s0
    o = Qbar @ s0 + A_qk @ U
    s1 = gamma[:, None] * s0 + Kbar.T @ U
    return o[:c], s1


def kda_chunked(qn, kn, v, g, beta, s0):
    """Whole sequence: qn, kn [T, K]; v [T, V]; g [T, K] log-decay; beta [T];
    s0 [K, V].  Returns (o [T, V], final state)."""
    total = qn.shape[0]
    out = np.zeros((total, v.shape[1]))
    state = np.array(s0, dtype=np.float64)
    for start in range(0, total, CHUNK):
        stop = min(total, start + CHUNK)
        o, state = chunk_states(qn[start:stop], kn[start:stop], v[start:stop], g[start:stop],
                                beta[start:stop], state)
        out[start:stop] = o
    return out, state
