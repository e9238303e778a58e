"""Seeded random sweep of ShortConv (packed prefill and one-token step) against the oracle.

Each prefill case draws a packed ragged batch (1-24 sequences of 0-300 tokens,
some empty and some shorter than the history), 8-6,144 channels, kernel sizes
1-4, bf16 or fp32, rows of x and of the output that are views of wider
buffers, histories in shuffled slots of a larger cache (one sequence without a
slot: it starts from zero and writes nothing), and each of read/write history
on or off.  Each step case draws 1-300 rows with the same choices (kernel
sizes 2-4).  Outputs must match the float64 oracle to max|y - y_ref| /
max|y_ref| <= 1e-5 (fp32) or 8e-3 (bf16, one rounding of the output); the
written histories are copies of input samples and must be bit-exact; slots no
sequence uses keep their bits.  The case parameters are printed before each
launch.
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
    if b.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _np(t):
    return t.detach().float().cpu().numpy()


def _rows_view(rng, rows: int, channels: int, dtype, dev):
    """A [rows, channels] view with a row stride of channels + 8 j and a
    column offset of 8 i (16-byte aligned for both dtypes), or a dense tensor."""
    if rng.random() < 0.5:
        return torch.empty((rows, channels), dtype=dtype, device=dev)
    pad = 8 * int(rng.integers(1, 4))
    off = 8 * int(rng.integers(0, pad // 8 + 1))
    big = torch.full((rows, channels + pad), float("nan"), dtype=dtype, device=dev)
    return big[:, off:off + channels]


def _tol(dtype) -> float:
    return 1e-5 if dtype == torch.float32 else 8e-3


@pytest.mark.parametrize("seed", list(range(10)))
def test_random_short_conv_prefill_matches_oracle(seed):
    from sophia_amd import ops
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(3000 + seed)
    channels = int(rng.choice([8, 64, 96, 1000, 6144]))
    kernel = int(rng.integers(1, 5))
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    n = int(rng.integers(1, 25))
    max_len = 60 if channels == 6144 else 300
    lens = rng.integers(0, max_len + 1, size=n)
    lens[rng.random(n) < 0.15] = 0
    lens[rng.random(n) < 0.15] = 1
    if seed == 9:
        lens[:] = 0                                   # an empty batch still shifts the histories
    use_state = kernel > 1
    read = bool(use_state and rng.random() < 0.7)
    write = bool(use_state and rng.random() < 0.7)
    cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total = int(cu_np[-1])
    print(f"case {seed}: n={n} total={total} channels={channels} kernel={kernel} dtype={dtype} "
          f"read_history={read} write_history={write}", flush=True)
    x_host = torch.tensor(rng.standard_normal((total, channels)), dtype=torch.float32).to(dtype)
    w = torch.tensor(rng.standard_normal((channels, kernel)) * 0.5, dtype=torch.float32)
    x = _rows_view(rng, total, channels, dtype, dev)
    x.copy_(x_host.to(dev))
    out = _rows_view(rng, total, channels, dtype, dev)
    n_slots = n + 2
    slots = rng.permutation(n_slots)[:n].astype(np.int32)
    no_slot = int(rng.integers(0, n))
    slots[no_slot] = -1 if rng.random() < 0.5 else n_slots + 1
    hist_len = kernel - 1
    cache = rng.standard_normal((n_slots, channels, hist_len)).astype(np.float32)
    state = torch.tensor(cache, device=dev) if use_state else None
    y = ops.short_conv_fwd(x, w.to(dev), torch.tensor(cu_np, device=dev), conv_state=state,
                           state_slots=torch.tensor(slots, device=dev) if use_state else None,
                           read_history=read, write_history=write, out=out)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr()
    xf = _np(x_host).astype(np.float64)
    wf = _np(w.to(dtype)).astype(np.float64)
    y_np = _np(y)
    expect = cache.copy()
    for s, (a, b) in enumerate(zip(cu_np[:-1], cu_np[1:])):
        has_slot = 0 <= slots[s] < n_slots
        hist = None
        if read and has_slot:
            hist = _np(torch.tensor(cache[slots[s]][None]).to(dtype)).astype(np.float64)
        yr, nh = ko.short_conv(xf[None, a:b], wf, hist)
        assert _rel(y_np[a:b], yr[0]) <= _tol(dtype), s
        if write and has_slot:
            expect[slots[s]] = nh[0].astype(np.float32)
    if use_state:
        assert np.array_equal(_np(state), expect)


@pytest.mark.parametrize("seed", list(range(8)))
def test_random_short_conv_step_matches_oracle(seed):
    from sophia_amd import ops
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(4000 + seed)
    channels = int(rng.choice([8, 64, 96, 1000, 6144]))
    kernel = int(rng.integers(2, 5))
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    batch = int(rng.integers(1, 301))
    read = seed % 4 != 3
    print(f"case {seed}: batch={batch} channels={channels} kernel={kernel} dtype={dtype} "
          f"read_history={read}", flush=True)
    x_host = torch.tensor(rng.standard_normal((batch, channels)), dtype=torch.float32).to(dtype)
    w = torch.tensor(rng.standard_normal((channels, kernel)) * 0.5, dtype=torch.float32)
    x = _rows_view(rng, batch, channels, dtype, dev)
    x.copy_(x_host.to(dev))
    out = _rows_view(rng, batch, channels, dtype, dev)
    n_slots = batch + 3
    slots = rng.permutation(n_slots)[:batch].astype(np.int32)
    no_slot = int(rng.integers(0, batch))
    slots[no_slot] = -1
    cache = rng.standard_normal((n_slots, channels, kernel - 1)).astype(np.float32)
    state = torch.tensor(cache, device=dev)
    y = ops.short_conv_step(x, w.to(dev), state, state_slots=torch.tensor(slots, device=dev),
                            read_history=read, out=out)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr()
    hist = np.zeros((batch, channels, kernel - 1), dtype=np.float64)
    if read:
        rows = [b for b in range(batch) if b != no_slot]
        hist[rows] = _np(torch.tensor(cache[slots[rows]]).to(dtype))
    yr, nh = ko.short_conv(_np(x_host)[:, None].astype(np.float64), _np(w.to(dtype)).astype(np.float64),
                           hist)
    assert _rel(_np(y), yr[:, 0]) <= _tol(dtype)
    expect = cache.copy()
    for b in range(batch):
        if b != no_slot:
            expect[slots[b]] = nh[b].astype(np.float32)
    assert np.array_equal(_np(state), expect)
