"""GPU parity of the hybrid decoder (sophia_amd.decoder) against the oracle's
restatement of the reference decoder (transformer.py:169-207, blocks.py,
attention.py:423-657), on a small seeded configuration in fp32, plus the
continuous-batching mixed step and its HIP-graph capture.

Tolerance: max|y - y_ref| / max|y_ref| <= 2e-2 on the logits against the
float64 oracle.  Graph replays are checked against the eager step at the same
cache state, with eager work and host synchronisation between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decoder_oracle as do

pytestmark = pytest.mark.gpu

REL_TOL = 2e-2
SMALL = dict(vocab_size=512, n_layers=4, ffn_hidden=320, mla_q_rank=64, mla_kv_rank=32, dim=256,
             num_heads=2, max_seq_len=128, max_batch_size=6)


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def _np(t):
    return t.detach().float().cpu().numpy()


def _model(dev, seed=0, **over):
    from sophia_amd.config import ModelArgs
    from sophia_amd.decoder import Transformer
    torch.manual_seed(seed)
    args = ModelArgs(**{**SMALL, **over})
    model = Transformer(args)
    # non-zero residual queries so the depth mixing is exercised
    with torch.no_grad():
        for m in model.modules():
            if m.__class__.__name__ == "AttentionResidualMixer":
                m.query.weight.normal_(0.0, 0.05)
    model = model.to(dev)
    params = {k: _np(v).astype(np.float64) for k, v in model.state_dict().items()}
    cfg = dict(n_layers=4, num_heads=2, norm_eps=1e-5, attn_res_block_size=4,
               situ_gate_softcap=4.0, situ_up_softcap=25.0, mla_kv_rank=int(args.mla_kv_rank),
               short_conv_kernel=4)
    return model, params, cfg


def test_decoder_forward_matches_oracle_and_cached_decode():
    dev = _dev()
    model, params, cfg = _model(dev)
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        logits = model(ids.to(dev), start_pos=0)
        model.reset_runtime_cache()
        steps = [model(ids[:, :33].to(dev), start_pos=0)]
        for t in range(33, 40):
            steps.append(model(ids[:, t:t + 1].to(dev), start_pos=t))
    ref = do.decoder_forward(params, ids.numpy(), cfg=cfg)
    err = _rel(_np(logits), ref)
    print(f"decoder logits rel err {err:.2e}")
    assert err < REL_TOL
    assert _rel(_np(torch.cat(steps, 1)), ref) < REL_TOL
    with pytest.raises(ValueError):
        model(ids[:, :2].to(dev), start_pos=3)   # transformer.py:150-153
    # the reference's call forms: forward(input_ids, attention_mask, start_pos), forward_full
    with torch.no_grad():
        model.reset_runtime_cache()
        again = model(ids.to(dev), None, 0)
        full = model.forward_full(ids.to(dev), attention_mask=torch.ones(2, 40, device=dev), start_pos=0)
    assert torch.equal(again, logits) and torch.equal(full, logits)


def test_forward_with_last_hidden_and_replay_with_cache():
    """The runtime host's entry points (runtime_host.py:115-170):
    forward_with_last_hidden gives forward's logits (every position, or the
    last one) and the last position's final depth mix, whose head
    (output(norm(.))) is that position's logits; replay_with_cache of a prompt
    and then of several tokens after it (one at a time) gives the one-pass
    logits."""
    dev = _dev()
    model, _, _ = _model(dev, seed=11)
    ids = torch.randint(0, 512, (2, 30), generator=torch.Generator().manual_seed(12)).to(dev)
    with torch.no_grad():
        model.reset_runtime_cache()
        full = model(ids, start_pos=0)
        model.reset_runtime_cache()
        logits, last = model.forward_with_last_hidden(ids, 0)
        model.reset_runtime_cache()
        last_only, _ = model.forward_with_last_hidden(ids, 0, return_all_logits=False)
        head = model.output(model.norm(last))
        model.reset_runtime_cache()
        a, _ = model.replay_with_cache(ids[:, :20], 0)
        b, last_b = model.replay_with_cache(ids[:, 20:], 20)
    assert logits.shape == full.shape and tuple(last.shape) == (2, 256) and tuple(last_only.shape) == (2, 512)
    assert _rel(_np(logits), _np(full)) < 1e-4
    assert _rel(_np(last_only), _np(full[:, -1])) < 1e-4
    assert _rel(_np(head), _np(full[:, -1])) < 1e-4
    err = _rel(_np(torch.cat([a, b], 1)), _np(full))
    print(f"replayed prompt + 10 cached tokens vs one pass: {err:.2e}", flush=True)
    assert tuple(b.shape) == (2, 10, 512) and err < 5e-3
    assert _rel(_np(last_b), _np(last)) < 5e-3


def _mixed_case(dev, model):
    """Three running sequences (histories of 37, 12 and 1 tokens in slots 0-2)
    and two new 30-token sequences (slots 3, 4)."""
    gen = torch.Generator().manual_seed(2)
    hist = [torch.randint(0, 512, (n,), generator=gen) for n in (37, 12, 1)]
    new_tok = torch.randint(0, 512, (3,), generator=gen)
    prefill = torch.randint(0, 512, (2, 30), generator=gen)
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=dev)
    with torch.no_grad():
        model.reset_runtime_cache()
        for slot, h in enumerate(hist):
            model.forward_mixed(h[None].to(dev), torch.empty(0, dtype=torch.long, device=dev),
                                prefill_slots=i32([slot]), decode_slots=i32([]),
                                decode_pos=torch.empty(0, dtype=torch.long, device=dev),
                                max_decode_len=1)
    step = dict(prefill_ids=prefill.to(dev), decode_ids=new_tok.to(dev),
                prefill_slots=i32([3, 4]), decode_slots=i32([0, 1, 2]),
                decode_pos=torch.tensor([37, 12, 1], dtype=torch.long, device=dev))
    full = [prefill[0], prefill[1]] + [torch.cat([h, new_tok[i:i + 1]]) for i, h in enumerate(hist)]
    return step, full


def _snapshot(model):
    return [(layer.attn.recurrent_state.clone(), layer.attn.conv_state.clone())
            if layer.layer_type == "kda" else (layer.attn.latent_cache.clone(),)
            for layer in model.layers]


def _restore(model, snap):
    for layer, s in zip(model.layers, snap):
        if layer.layer_type == "kda":
            layer.attn.recurrent_state.copy_(s[0])
            layer.attn.conv_state.copy_(s[1])
        else:
            layer.attn.latent_cache.copy_(s[0])


def test_mixed_step_matches_each_sequence_run_alone():
    dev = _dev()
    model, params, cfg = _model(dev)
    step, full = _mixed_case(dev, model)
    with torch.no_grad():
        logits = model.forward_mixed(max_decode_len=40, **step)
    assert tuple(logits.shape) == (5, 512)
    for row, seq in enumerate(full):
        ref = do.decoder_forward(params, seq.numpy()[None], cfg=cfg)[0, -1]
        err = _rel(_np(logits[row]), ref)
        assert err < REL_TOL, f"sequence {row}: {err}"


@pytest.mark.parametrize("q_rank", [60, 544])
def test_mixed_step_with_mla_ranks_outside_the_norm_kernel(q_rank):
    """A q rank that is not a multiple of 8 (60), and one whose q and kv
    latents together exceed the 512 columns one wave normalises (544 + 32):
    the step keeps torch's norms and latent-cache writes and every sequence
    still matches the oracle."""
    dev = _dev()
    model, params, cfg = _model(dev, mla_q_rank=q_rank)
    step, full = _mixed_case(dev, model)
    with torch.no_grad():
        logits = model.forward_mixed(max_decode_len=40, **step)
    for row, seq in enumerate(full):
        ref = do.decoder_forward(params, seq.numpy()[None], cfg=cfg)[0, -1]
        err = _rel(_np(logits[row]), ref)
        print(f"q rank {q_rank}, sequence {row}: rel err {err:.2e}", flush=True)
        assert err < REL_TOL, f"sequence {row}: {err}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_padded_prompt_and_cached_decode_match_the_unpadded_sequence(dtype):
    """The whole decoder with a left-padded row (set_pad_mask on its KDA and
    MLA layers, attention.py:660-670): the padded row's logits at its real
    positions, and those of two cached decode steps after it, equal those of
    the same tokens run alone without padding (KDA pad steps are identities,
    the MLA keys of pad positions are masked, and the position-free attention
    does not see the shift); and cached decode steps of the unpadded sequence
    equal its one-pass logits.  bf16 runs the unpadded cached steps through the
    HIP causal kernel (queries after cached keys) and the masked ones through
    fp32 attention scores."""
    from sophia_amd.kda import set_pad_mask
    dev = _dev()
    model, _, _ = _model(dev, seed=8)
    if dtype == torch.bfloat16:
        model.cast_weights_(torch.bfloat16)
    gen = torch.Generator().manual_seed(9)
    real, pad = 45, 7
    seq = torch.randint(0, 512, (1, real + 2), generator=gen)
    batch = torch.cat([torch.cat([torch.zeros(1, pad, dtype=torch.long), seq[:, :real]], 1),
                       torch.randint(0, 512, (1, real + pad), generator=gen)], 0).to(dev)
    mask = torch.ones(2, real + pad, dtype=torch.bool, device=dev)
    mask[0, :pad] = False
    nxt = torch.cat([seq[:, real:], torch.randint(0, 512, (1, 2), generator=gen)], 0).to(dev)   # [2, 2]
    with torch.no_grad():
        model.reset_runtime_cache()
        set_pad_mask(model, mask)
        padded = model(batch, start_pos=0)
        steps = [model(nxt[:, t:t + 1], start_pos=real + pad + t) for t in range(2)]
        set_pad_mask(model, None)
        model.reset_runtime_cache()
        alone = model(seq.to(dev), start_pos=0)          # all real + 2 tokens in one pass
        model.reset_runtime_cache()
        model(seq[:, :real].to(dev), start_pos=0)
        cached = [model(seq[:, real + t:real + t + 1].to(dev), start_pos=real + t) for t in range(2)]
    tol = 1e-2 if dtype == torch.float32 else 3e-2
    err = _rel(_np(padded[0, pad:]), _np(alone[0, :real]))
    err_steps = max(_rel(_np(steps[t][0, 0]), _np(alone[0, real + t])) for t in range(2))
    err_cached = max(_rel(_np(cached[t][0, 0]), _np(alone[0, real + t])) for t in range(2))
    print(f"{dtype}: padded prompt vs alone {err:.2e}, its cached steps {err_steps:.2e}, "
          f"unpadded cached steps vs one pass {err_cached:.2e}", flush=True)
    assert torch.isfinite(padded.float()).all()
    assert err < tol and err_steps < tol and err_cached < tol


def test_mixed_step_graph_replays_match_eager():
    from sophia_amd.decoder import MixedStepGraph
    dev = _dev()
    model, _, _ = _model(dev)
    step, _ = _mixed_case(dev, model)
    start = _snapshot(model)
    with torch.no_grad():
        eager = model.forward_mixed(max_decode_len=40, **step).clone()
        after = _snapshot(model)
    _restore(model, start)
    graph = MixedStepGraph(model, 2, 30, 3, 40, example=step)
    for replay in range(3):
        _restore(model, start)
        torch.cuda.synchronize()
        out = graph.run(**step)
        torch.cuda.synchronize()
        assert torch.allclose(out, eager, rtol=1e-4, atol=1e-4), f"replay {replay}"
        for a, b in zip(_snapshot(model), after):
            for x, y in zip(a, b):
                assert torch.allclose(x, y, rtol=1e-4, atol=1e-5), f"replay {replay} caches"
        with torch.no_grad():  # eager work between replays
            model(torch.zeros(1, 3, dtype=torch.long, device=dev), start_pos=0)


FULL_DIMS = dict(vocab_size=1024, n_layers=4, ffn_hidden=3968, mla_q_rank=384, mla_kv_rank=128,
                 dim=1536, num_heads=16, max_seq_len=256, max_batch_size=4)


def test_decoder_at_production_widths_matches_oracle():
    """Every width of the benchmark decoder (dim 1536, 16 heads x 128, SiTU-GLU
    3968, MLA ranks 384/128; 4 layers, vocab 1,024) in fp32 against the float64
    oracle (<= 2e-2 of max |logit|), then the same weights in bf16 through the
    mixed step (HIP causal attention, bf16 kernels throughout) against the same
    oracle: <= 6e-2 of max |logit| (bf16 activations through four layers)."""
    from sophia_amd.config import ModelArgs
    from sophia_amd.decoder import Transformer
    dev = _dev()
    torch.manual_seed(5)
    args = ModelArgs(**FULL_DIMS)
    model = Transformer(args)
    with torch.no_grad():
        for m in model.modules():
            if m.__class__.__name__ == "AttentionResidualMixer":
                m.query.weight.normal_(0.0, 0.05)
    model = model.to(dev)
    params = {k: _np(v).astype(np.float64) for k, v in model.state_dict().items()}
    cfg = dict(n_layers=4, num_heads=16, norm_eps=1e-5, attn_res_block_size=4, situ_gate_softcap=4.0,
               situ_up_softcap=25.0, mla_kv_rank=128, short_conv_kernel=4)
    ids = torch.randint(0, 1024, (2, 80), generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        logits = model(ids.to(dev), start_pos=0)
    ref = do.decoder_forward(params, ids.numpy(), cfg=cfg)
    err = _rel(_np(logits), ref)
    print(f"fp32 production-width logits rel err {err:.2e}")
    assert err < REL_TOL

    model.cast_weights_(torch.bfloat16)
    model.reset_runtime_cache()
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=dev)
    with torch.no_grad():
        last = model.forward_mixed(ids.to(dev), torch.empty(0, dtype=torch.long, device=dev),
                                   prefill_slots=i32([0, 1]), decode_slots=i32([]),
                                   decode_pos=torch.empty(0, dtype=torch.long, device=dev),
                                   max_decode_len=1)
    err16 = _rel(_np(last.float()), ref[:, -1])
    print(f"bf16 mixed-step last-token logits rel err {err16:.2e}")
    assert err16 < 6e-2


def test_decoder_with_trained_parameter_values_matches_oracle():
    """The small decoder with every A_log, dt_bias and norm weight (attn/ffn
    norms, depth-mix norms, MLA q/kv norms, KDA output norms, final norm)
    drawn away from its init value, against the float64 oracle."""
    from trained_params import perturb_like_trained
    dev = _dev()
    model, _, cfg = _model(dev, seed=3)
    touched = perturb_like_trained(model, seed=4)
    assert any(t.endswith("q_norm.weight") for t in touched)
    assert any(t.endswith("attn.A_log") for t in touched)
    params = {k: _np(v).astype(np.float64) for k, v in model.state_dict().items()}
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        logits = model(ids.to(dev), start_pos=0)
    ref = do.decoder_forward(params, ids.numpy(), cfg=cfg)
    err = _rel(_np(logits), ref)
    print(f"trained-value decoder logits rel err {err:.2e}")
    assert err < REL_TOL
