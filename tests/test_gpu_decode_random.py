"""Seeded random sweep of the recurrent decode step against the oracle.

Each case draws a batch of 1-300 one-token rows, 1-5 heads, bf16 or fp32
q/k/v, fp32 or bf16 decay, the three in-kernel switches, states in shuffled
slots of a larger cache (one row with a slot out of range: output 0, no state
touched), and reading the state or starting from zero (``read_state``).
Outputs must match the float64 oracle to max|y - y_ref| / max|y_ref| <= 2e-2
and the updated states to 1e-4; slots no row uses keep their bits.  The case
parameters are printed before each launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as ko

pytestmark = pytest.mark.gpu


def _rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("seed", list(range(10)))
def test_random_decode_step_matches_oracle(seed):
    from sophia_amd import ops
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(2000 + seed)
    batch = int(rng.integers(1, 301))
    heads = int(rng.choice([1, 2, 3, 5]))
    qkv_dt = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    g_dt = torch.float32 if rng.random() < 0.7 else torch.bfloat16
    l2, gate, bsig = (bool(rng.random() < 0.7), bool(rng.random() < 0.5), bool(rng.random() < 0.5))
    read = seed % 4 != 3
    print(f"case {seed}: batch={batch} heads={heads} qkv={qkv_dt} g={g_dt} l2={l2} gate={gate} "
          f"beta_sigmoid={bsig} read_state={read}", flush=True)
    shape = (batch, heads, 128)
    q = torch.tensor(rng.standard_normal(shape), dtype=torch.float32)
    k = torch.tensor(rng.standard_normal(shape), dtype=torch.float32)
    v = torch.tensor(rng.standard_normal(shape), dtype=torch.float32)
    if not l2:
        q, k = q / np.sqrt(128.0), k / np.sqrt(128.0)
    if gate:
        g = torch.tensor(rng.standard_normal(shape) * 2.0, dtype=torch.float32)
        a_log = torch.tensor(rng.standard_normal(heads) * 0.5, dtype=torch.float32)
        dtb = torch.tensor(ko.inverse_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), heads * 128))),
                           dtype=torch.float32)
    else:
        g = torch.tensor(rng.uniform(-5.0, 0.0, shape), dtype=torch.float32)
        a_log = dtb = None
    beta = torch.tensor(rng.standard_normal((batch, heads)) if bsig else rng.uniform(0, 1, (batch, heads)),
                        dtype=torch.float32)
    q, k, v = (t.to(qkv_dt) for t in (q, k, v))
    g = g.to(g_dt)
    n_slots = batch + 3
    slots = rng.permutation(n_slots)[:batch].astype(np.int32)
    off = int(rng.integers(0, batch))
    slots[off] = -1                                   # no cache slot for this row
    cache = (rng.standard_normal((n_slots, heads, 128, 128)) * 0.1).astype(np.float32)
    state = torch.tensor(cache, device=dev)
    o = ops.kda_decode_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), state,
                            A_log=None if a_log is None else a_log.to(dev),
                            dt_bias=None if dtb is None else dtb.to(dev), use_qk_l2norm=l2, use_gate=gate,
                            use_beta_sigmoid=bsig, state_slots=torch.tensor(slots, device=dev),
                            read_state=read)
    torch.cuda.synchronize()
    rows = [b for b in range(batch) if b != off]
    h0 = np.stack([cache[slots[b]] if read else np.zeros_like(cache[0]) for b in rows])
    kw = dict(use_qk_l2norm=l2, use_gate=gate, use_beta_sigmoid=bsig)
    if gate:
        kw.update(A_log=a_log.numpy(), dt_bias=dtb.numpy())
    o_ref, h_ref = ko.kda_decode_step(_np(q)[rows], _np(k)[rows], _np(v)[rows], _np(g)[rows],
                                      _np(beta)[rows], h0, **kw)
    o_np, s_np = _np(o), _np(state)
    assert _rel(o_np[rows], o_ref) < 2e-2
    assert np.all(o_np[off] == 0.0)
    assert _rel(s_np[slots[rows]], h_ref) < 1e-4
    for s in sorted(set(range(n_slots)) - {int(x) for x in slots[rows]}):
        assert np.array_equal(s_np[s], cache[s])
