"""GPU parity of the whole KDA mixer module (sophia_amd.kda.SophiaKDA) against
the oracle's restatement of the reference module (attention.py:373-420), and
the reference's own module invariants re-expressed for the GPU path:
cached decode == full prompt (test_sophia_runtime_forward.py:154-168), split
prefill == one shot (test_sophia_incremental_cache.py:65-88), padded row ==
unpadded row (attention.py:379-397), stateless run leaves the caches zero
(test_dynamic_batch_capacity.py:74-96), cache snapshot round trip
(test_dynamic_batch_capacity.py:120-141), packed == per sequence.

Tolerance (stated by the task): max|y - y_ref| / max|y_ref| <= 2e-2 against the
fp32 oracle, for outputs and final states.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as ko

pytestmark = pytest.mark.gpu

REL_TOL = 2e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _module(dev, *, max_batch=2, use_cache=True, seed=42, dim=1536, heads=16):
    from sophia_amd.config import ModelArgs
    from sophia_amd.kda import SophiaKDA
    torch.manual_seed(seed)
    args = ModelArgs(dim=dim, num_heads=heads, max_batch_size=max_batch, use_cache=use_cache)
    mod = SophiaKDA(args).to(dev)
    params = {k: _np(v) for k, v in mod.state_dict().items()}
    return mod, params


def _oracle(params, x, **kw):
    heads = params["A_log"].shape[0]
    return ko.mixer_forward({k: v.astype(np.float64) for k, v in params.items()},
                            x.astype(np.float64), num_heads=heads, **kw)


def test_mixer_forward_config1_matches_oracle():
    """B=1, T=512, hidden 1536, 16 x 128, seed 42, x ~ N(0,1), fp32 (config 1)."""
    dev = _dev()
    mod, params = _module(dev, max_batch=1)
    x = torch.randn(1, 512, 1536, generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        y = mod(x.to(dev), start_pos=0)
    cache = {"recurrent": np.zeros((1, 16, 128, 128)), "conv": np.zeros((1, 3, 2048, 3))}
    y_ref = _oracle(params, _np(x), cache=cache)
    err_y = _rel(_np(y), y_ref)
    err_s = _rel(_np(mod.recurrent_state[:1]), cache["recurrent"])
    err_c = _rel(_np(mod.conv_state[:1]), cache["conv"])
    print(f"config 1 mixer: output {err_y:.2e}, state {err_s:.2e}, conv cache {err_c:.2e}")
    assert err_y < REL_TOL and err_s < REL_TOL
    assert err_c < 1e-5


def test_cached_decode_matches_full_prompt():
    dev = _dev()
    mod, params = _module(dev, max_batch=2, dim=256, heads=2)
    gen = torch.Generator().manual_seed(1)
    total, prompt = 150, 140
    x = torch.randn(2, total, 256, generator=gen)
    with torch.no_grad():
        outs = [mod(x[:, :prompt].to(dev), start_pos=0)]
        for t in range(prompt, total):
            outs.append(mod(x[:, t:t + 1].to(dev), start_pos=t))
    y = torch.cat(outs, dim=1)
    cache = {"recurrent": np.zeros((2, 2, 128, 128)), "conv": np.zeros((2, 3, 256, 3))}
    y_ref = _oracle(params, _np(x), cache=cache)
    assert _rel(_np(y), y_ref) < REL_TOL
    assert _rel(_np(mod.recurrent_state[:2]), cache["recurrent"]) < REL_TOL
    assert _rel(_np(mod.conv_state[:2]), cache["conv"]) < 1e-5


def test_split_prefill_matches_one_shot():
    dev = _dev()
    mod, _ = _module(dev, max_batch=1, dim=256, heads=2)
    x = torch.randn(1, 200, 256, generator=torch.Generator().manual_seed(2)).to(dev)
    with torch.no_grad():
        full = mod(x, start_pos=0)
        state_full = mod.recurrent_state.clone()
        mod.reset()
        a = mod(x[:, :77], start_pos=0)
        b = mod(x[:, 77:], start_pos=77)
    assert _rel(_np(torch.cat([a, b], 1)), _np(full)) < REL_TOL
    assert _rel(_np(mod.recurrent_state), _np(state_full)) < REL_TOL


def test_padded_row_matches_unpadded_row():
    from sophia_amd.kda import set_pad_mask
    dev = _dev()
    mod, _ = _module(dev, max_batch=2, dim=256, heads=2)
    gen = torch.Generator().manual_seed(3)
    real, pad = 90, 23
    seq = torch.randn(1, real, 256, generator=gen)
    batch = torch.cat([torch.cat([torch.randn(1, pad, 256, generator=gen), seq], 1),
                       torch.randn(1, real + pad, 256, generator=gen)], 0).to(dev)
    mask = torch.ones(2, real + pad, dtype=torch.bool, device=dev)
    mask[0, :pad] = False
    with torch.no_grad():
        set_pad_mask(mod, mask)
        y_pad = mod(batch, start_pos=0)
        state_pad = mod.recurrent_state[0].clone()
        set_pad_mask(mod, None)
        mod.reset()
        y_one = mod(seq.to(dev), start_pos=0)
    assert _rel(_np(y_pad[0, pad:]), _np(y_one[0])) < REL_TOL
    assert _rel(_np(state_pad), _np(mod.recurrent_state[0])) < REL_TOL


def test_stateless_run_leaves_caches_zero_and_snapshot_roundtrip():
    dev = _dev()
    mod, _ = _module(dev, max_batch=2, use_cache=False, dim=256, heads=2)
    x = torch.randn(2, 40, 256, generator=torch.Generator().manual_seed(4)).to(dev)
    with torch.no_grad():
        mod(x, start_pos=0)
    assert torch.count_nonzero(mod.recurrent_state) == 0
    assert torch.count_nonzero(mod.conv_state) == 0

    mod2, _ = _module(dev, max_batch=2, dim=256, heads=2)
    with torch.no_grad():
        mod2(x, start_pos=0)
    snap = mod2.cache_snapshot(device="cpu", batch_size=2, cache_pos=None)
    rec, conv = mod2.recurrent_state.clone(), mod2.conv_state.clone()
    mod2.reset()
    assert torch.count_nonzero(mod2.recurrent_state) == 0
    mod2.load_cache_snapshot(snap)
    assert torch.equal(mod2.recurrent_state, rec) and torch.equal(mod2.conv_state, conv)


def test_packed_forward_matches_each_sequence_alone():
    """forward_packed over a ragged batch with explicit cache slots equals
    running each sequence alone through forward().  The KDA kernels are
    bit-exact under packing (test_gpu_kernels.py::test_chunk_prefill_packing_is_exact);
    here the projection GEMMs see different row counts, so their fp32 results
    may differ in the last bit and flip a bf16 rounding of an MFMA operand:
    the bound is 5e-3 rather than bitwise."""
    dev = _dev()
    mod, _ = _module(dev, max_batch=6, dim=256, heads=2)
    lens = [37, 1, 130, 64]
    slots = [4, 0, 2, 5]
    gen = torch.Generator().manual_seed(5)
    xs = [torch.randn(n, 256, generator=gen) for n in lens]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    with torch.no_grad():
        mod.reset()
        y = mod.forward_packed(torch.cat(xs).to(dev), cu,
                               state_slots=torch.tensor(slots, dtype=torch.int32, device=dev),
                               use_state=False)
        packed_states = mod.recurrent_state.clone()
        packed_conv = mod.conv_state.clone()
        for s, (xi, slot) in enumerate(zip(xs, slots)):
            ref_mod, _ = _module(dev, max_batch=1, dim=256, heads=2)
            ref_mod.load_state_dict(mod.state_dict())
            yi = ref_mod(xi[None].to(dev), start_pos=0)
            a, b = int(cu[s]), int(cu[s + 1])
            assert _rel(_np(y[a:b]), _np(yi[0])) < 5e-3, f"sequence {s}"
            assert _rel(_np(packed_states[slot]), _np(ref_mod.recurrent_state[0])) < 5e-3
            assert _rel(_np(packed_conv[slot]), _np(ref_mod.conv_state[0])) < 1e-5
    untouched = [i for i in range(6) if i not in slots]
    assert torch.count_nonzero(packed_states[untouched]) == 0


def test_packed_decode_step_matches_forward_decode():
    """forward_packed with one token per sequence (decode kernels, cache slots)
    equals the reference-shaped forward(x[:, t:t+1], start_pos=t)."""
    dev = _dev()
    mod, _ = _module(dev, max_batch=3, dim=256, heads=2)
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(3, 21, 256, generator=gen).to(dev)
    with torch.no_grad():
        mod(x[:, :20], start_pos=0)
        rec, conv = mod.recurrent_state.clone(), mod.conv_state.clone()
        y_ref = mod(x[:, 20:21], start_pos=20)
        rec_ref, conv_ref = mod.recurrent_state.clone(), mod.conv_state.clone()
        mod.recurrent_state.copy_(rec)
        mod.conv_state.copy_(conv)
        cu = torch.arange(0, 4, dtype=torch.int32, device=dev)
        y = mod.forward_packed(x[:, 20], cu, max_seqlen=1)
    assert _rel(_np(y), _np(y_ref[:, 0])) < 1e-5
    assert _rel(_np(mod.recurrent_state), _np(rec_ref)) < 1e-5
    assert torch.equal(mod.conv_state, conv_ref)


def test_mixer_with_trained_parameter_values_matches_oracle():
    """Config-1 shape with A_log, dt_bias and the output norm weight drawn away
    from their init values (a trained state_dict's situation): the per-head
    gate scale exp(A_log) and the RMSNorm weight enter the comparison."""
    from trained_params import perturb_like_trained
    dev = _dev()
    mod, _ = _module(dev, max_batch=1, seed=7)
    touched = perturb_like_trained(mod, seed=8)
    assert {"A_log", "dt_bias", "output_norm.weight"} <= set(touched)
    params = {k: _np(v) for k, v in mod.state_dict().items()}
    assert np.ptp(params["A_log"]) > 0.5 and np.ptp(params["output_norm.weight"]) > 0.5
    x = torch.randn(1, 512, 1536, generator=torch.Generator().manual_seed(9))
    with torch.no_grad():
        y = mod(x.to(dev), start_pos=0)
    cache = {"recurrent": np.zeros((1, 16, 128, 128)), "conv": np.zeros((1, 3, 2048, 3))}
    y_ref = _oracle(params, _np(x), cache=cache)
    err_y = _rel(_np(y), y_ref)
    err_s = _rel(_np(mod.recurrent_state[:1]), cache["recurrent"])
    print(f"trained-value mixer: output {err_y:.2e}, state {err_s:.2e}")
    assert err_y < REL_TOL and err_s < REL_TOL
