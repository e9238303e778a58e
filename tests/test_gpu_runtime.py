"""The continuous-batching runtime on the GPU: prefills that continue across
steps, ragged prefills in one step, the model-level cache API, batch-capacity
growth, the slot allocator and the functional cached decode.

References: the single-start_pos limit this removes (transformer.py:146-160);
cache_dump / cache_load (ml/runtime/model/runtime_host.py:179-212); batch
growth (tests/tests/test_dynamic_batch_capacity.py:29-51,120-141);
forward_cached_decode (ml/modeling/cache_decode.py:79-143).  Logits are
checked against the float64 oracle at max|y - y_ref| / max|y_ref| <= 2e-2
(fp32 model), bf16 against the fp32 model at <= 6e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decoder_oracle as do

pytestmark = pytest.mark.gpu

REL_TOL = 2e-2
SMALL = dict(vocab_size=512, n_layers=4, ffn_hidden=320, mla_q_rank=64, mla_kv_rank=32, dim=256,
             num_heads=2, max_seq_len=2600, max_batch_size=6)
CFG = dict(n_layers=4, num_heads=2, norm_eps=1e-5, attn_res_block_size=4, situ_gate_softcap=4.0,
           situ_up_softcap=25.0, mla_kv_rank=32, short_conv_kernel=4)


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
    model = Transformer(ModelArgs(**{**SMALL, **over}))
    with torch.no_grad():
        for m in model.modules():
            if m.__class__.__name__ == "AttentionResidualMixer":
                m.query.weight.normal_(0.0, 0.05)
    model = model.to(dev).eval()
    params = {k: _np(v).astype(np.float64) for k, v in model.state_dict().items()}
    return model, params


def _i32(xs, dev):
    return torch.tensor(xs, dtype=torch.int32, device=dev)


def _i64(xs, dev):
    return torch.tensor(xs, dtype=torch.long, device=dev)


def _oracle_last(params, seq) -> np.ndarray:
    return do.decoder_forward(params, np.asarray(seq)[None], cfg=CFG)[0, -1]


def test_long_prompt_prefilled_over_three_steps_while_others_decode():
    """A 2,500-token prompt prefilled in pieces of 900, 900 and 700 tokens over
    three steps (the second and third continue from the cached KDA state,
    conv history and MLA latents), while two other sequences decode one token
    per step; the last-token logits equal the oracle's one-shot run of the
    whole prompt."""
    dev = _dev()
    model, params = _model(dev)
    gen = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, 512, (2500,), generator=gen)
    b_hist = torch.randint(0, 512, (40,), generator=gen)
    c_hist = torch.randint(0, 512, (7,), generator=gen)
    dec = torch.randint(0, 512, (2, 2), generator=gen)
    slot_a, slot_b, slot_c = 4, 1, 3
    with torch.no_grad():
        # step 0: three new ragged prefills (A's first piece, B, C)
        ids0 = torch.cat([prompt[:900], b_hist, c_hist]).to(dev)
        out0 = model.forward_step(prefill_ids=ids0, prefill_lens=[900, 40, 7],
                                  prefill_slots=_i32([slot_a, slot_b, slot_c], dev))
        outs = [out0]
        for s, (a, b) in enumerate(((900, 1800), (1800, 2500))):
            outs.append(model.forward_step(
                prefill_ids=prompt[a:b].to(dev), prefill_lens=[b - a], prefill_pos=[a],
                prefill_slots=_i32([slot_a], dev), decode_ids=dec[:, s].to(dev),
                decode_slots=_i32([slot_b, slot_c], dev), decode_pos=_i64([40 + s, 7 + s], dev),
                max_decode_len=64))
    assert tuple(outs[0].shape) == (3, 512) and tuple(outs[-1].shape) == (3, 512)
    err_a = _rel(_np(outs[-1][0]), _oracle_last(params, prompt.numpy()))
    full_b = torch.cat([b_hist, dec[0]]).numpy()
    full_c = torch.cat([c_hist, dec[1]]).numpy()
    err_b = _rel(_np(outs[-1][1]), _oracle_last(params, full_b))
    err_c = _rel(_np(outs[-1][2]), _oracle_last(params, full_c))
    err_a0 = _rel(_np(outs[0][0]), _oracle_last(params, prompt[:900].numpy()))
    print(f"prompt over 3 steps: {err_a:.2e} (first piece {err_a0:.2e}); decodes {err_b:.2e}, {err_c:.2e}")
    assert max(err_a, err_a0, err_b, err_c) < REL_TOL


def test_ragged_prefills_in_one_step_equal_per_sequence_runs():
    """One step with three ragged new prefills (70, 5 and 131 tokens) and two
    decode rows equals each sequence run alone (and the oracle); in bf16 (HIP
    causal kernel for every packing) packed and lone runs agree to 1e-2 (they
    came out bit-identical on MI355X)."""
    dev = _dev()
    model, params = _model(dev, seed=2)
    gen = torch.Generator().manual_seed(3)
    lens = [70, 5, 131]
    seqs = [torch.randint(0, 512, (n,), generator=gen) for n in lens]
    hist = [torch.randint(0, 512, (n,), generator=gen) for n in (20, 33)]
    nxt = torch.randint(0, 512, (2,), generator=gen)
    with torch.no_grad():
        model.forward_step(prefill_ids=torch.cat(hist).to(dev), prefill_lens=[20, 33],
                           prefill_slots=_i32([0, 1], dev))
        packed = model.forward_step(prefill_ids=torch.cat(seqs).to(dev), prefill_lens=lens,
                                    prefill_slots=_i32([2, 3, 4], dev), decode_ids=nxt.to(dev),
                                    decode_slots=_i32([0, 1], dev), decode_pos=_i64([20, 33], dev),
                                    max_decode_len=40)
        alone = [model.forward_step(prefill_ids=s.to(dev), prefill_lens=[len(s)],
                                    prefill_slots=_i32([5], dev))[0] for s in seqs]
    # The packed step runs the fp32 MLA prefill as one masked SDPA per sequence,
    # the lone run as one is_causal SDPA (another backend), and the fp32 KDA
    # path rounds its MFMA operands to bf16, so the two agree to ~1e-3, not
    # bit for bit; both are checked against the oracle too.
    for i, s in enumerate(seqs):
        d_alone = _rel(_np(packed[i]), _np(alone[i]))
        d_ref = _rel(_np(packed[i]), _oracle_last(params, s.numpy()))
        print(f"sequence {i} ({len(s)} tokens): packed vs alone {d_alone:.2e}, vs oracle {d_ref:.2e}")
        assert d_alone < 5e-3, f"sequence {i} packed vs alone"
        assert d_ref < REL_TOL
    for j, h in enumerate(hist):
        full = torch.cat([h, nxt[j:j + 1]]).numpy()
        assert _rel(_np(packed[3 + j]), _oracle_last(params, full)) < REL_TOL
    model.cast_weights_(torch.bfloat16)
    with torch.no_grad():
        packed = model.forward_step(prefill_ids=torch.cat(seqs).to(dev), prefill_lens=lens,
                                    prefill_slots=_i32([2, 3, 4], dev))
        for i, s in enumerate(seqs):
            alone = model.forward_step(prefill_ids=s.to(dev), prefill_lens=[len(s)],
                                       prefill_slots=_i32([5], dev))[0]
            d = _rel(_np(packed[i]), _np(alone))
            print(f"bf16 sequence {i}: packed vs alone {d:.2e}")
            assert d < 1e-2


def _caches(model):
    out = []
    for layer in model.layers:
        a = layer.attn
        out += [a.recurrent_state.clone(), a.conv_state.clone()] if layer.layer_type == "kda" \
            else [a.latent_cache.clone()]
    return out


def test_cache_dump_reset_load_roundtrip_is_exact():
    """cache_dump -> reset -> cache_load restores every cache bit for bit, and
    decoding on from the restored caches gives the same logits; dumping
    chosen slots and loading them into other slots copies exactly those."""
    dev = _dev()
    model, _ = _model(dev, seed=4)
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 512, (3 * 30,), generator=gen).to(dev)
    nxt = torch.randint(0, 512, (3,), generator=gen).to(dev)
    with torch.no_grad():
        model.forward_step(prefill_ids=ids, prefill_lens=[30, 30, 30], prefill_slots=_i32([0, 1, 2], dev))
        before = _caches(model)
        snap = model.cache_dump(device="cpu")
        model.reset_runtime_cache()
        assert all(float(t.abs().max()) == 0.0 for t in _caches(model))
        model.cache_load(snap)
        for a, b in zip(_caches(model), before):
            assert torch.equal(a, b)
        step = dict(decode_ids=nxt, decode_slots=_i32([0, 1, 2], dev), decode_pos=_i64([30, 30, 30], dev),
                    max_decode_len=31)
        ref = model.forward_step(**step)
        model.cache_load(snap)
        again = model.forward_step(**step)
        assert torch.equal(ref, again)
        # slot-level: slots [2, 0] -> slots [5, 4]; the others keep their contents
        model.cache_load(snap)
        part = model.cache_dump(device="cpu", cache_pos=30, slots=_i32([2, 0], dev))
        model.cache_load(part, slots=_i32([5, 4], dev))
        for layer in model.layers:
            a = layer.attn
            if layer.layer_type == "kda":
                assert torch.equal(a.recurrent_state[5], a.recurrent_state[2])
                assert torch.equal(a.recurrent_state[4], a.recurrent_state[0])
                assert torch.equal(a.conv_state[5], a.conv_state[2])
            else:
                assert torch.equal(a.latent_cache[5, :30], a.latent_cache[2, :30])
                assert torch.equal(a.latent_cache[4, :30], a.latent_cache[0, :30])
        with pytest.raises(ValueError):
            model.cache_load(part, slots=_i32([5], dev))


def test_batch_capacity_grows_and_warm_growth_roundtrips():
    """The reference's growth tests on the GPU model: a batch of 3 on a model
    built for 1 grows every cache; growth after a small batch keeps it; a
    3-row cache dump loads into a fresh model and decodes the same next token
    (test_dynamic_batch_capacity.py:29-51,120-141)."""
    dev = _dev()
    model, _ = _model(dev, seed=6, max_batch_size=1, max_seq_len=64)
    gen = torch.Generator().manual_seed(7)
    small = torch.randint(0, 512, (1, 12), generator=gen).to(dev)
    large = torch.randint(0, 512, (3, 12), generator=gen).to(dev)
    with torch.no_grad():
        model(small, start_pos=0)
        logits = model(large, start_pos=0)
    assert tuple(logits.shape) == (3, 12, 512)
    assert int(model.args.max_batch_size) >= 3 and model.runtime_batch_capacity() >= 3
    cache = model.cache_dump(device="cpu", cache_pos=12, batch_size=3)
    restored, _ = _model(dev, seed=8, max_batch_size=1, max_seq_len=64)
    restored.load_state_dict(model.state_dict(), strict=True)
    restored.cache_load(cache)
    nxt = torch.randint(0, 512, (3, 1), generator=gen).to(dev)
    with torch.no_grad():
        a = model(nxt, start_pos=12)
        b = restored(nxt, start_pos=12)
    assert tuple(b.shape) == (3, 1, 512)
    assert torch.equal(a, b)


def test_slot_allocator_grows_zeroes_and_reuses():
    from sophia_amd.runtime import SlotAllocator
    dev = _dev()
    model, _ = _model(dev, seed=9, max_batch_size=2, max_seq_len=64)
    alloc = SlotAllocator(model)
    assert alloc.capacity == 2
    first = alloc.allocate(2)
    assert first.tolist() == [0, 1]
    for layer in model.layers:
        if layer.layer_type == "kda":
            layer.attn.recurrent_state.fill_(3.0)
    more = alloc.allocate(3)                    # grows the model's caches
    assert more.tolist() == [2, 3, 4] and alloc.capacity >= 5 and model.runtime_batch_capacity() >= 5
    alloc.release(first[:1])
    again = alloc.allocate(1)
    assert again.tolist() == [0]
    for layer in model.layers:
        if layer.layer_type == "kda":
            st = layer.attn.recurrent_state
            assert float(st[0].abs().max()) == 0.0      # handed out again: zeroed
            assert float(st[1].min()) == 3.0            # held: untouched
    with pytest.raises(ValueError):
        alloc.release([7])
    with pytest.raises(ValueError):
        alloc.release([3, 3])                   # the same slot twice: nothing released
    assert alloc.in_use == 5


def test_forward_cached_decode_matches_oracle():
    """forward_cached_decode (cache_decode.py:79-143): a 12-token prefill from
    no state, a one-token step and a 5-token step continuing from the
    returned state; every step's logits against the oracle's full run."""
    from sophia_amd.runtime import forward_cached_decode
    dev = _dev()
    model, params = _model(dev, seed=10, max_seq_len=64)
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(0, 512, (2, 18), generator=gen)
    ref = do.decoder_forward(params, ids.numpy(), cfg=CFG)
    with torch.no_grad():
        l0, st = forward_cached_decode(model=model, input_ids=ids[:, :12], cache_state=None, start_pos=0,
                                       logits_to_keep=None)
        l1, st = forward_cached_decode(model=model, input_ids=ids[:, 12:13], cache_state=st, start_pos=12,
                                       logits_to_keep=1)
        l2, st = forward_cached_decode(model=model, input_ids=ids[:, 13:18], cache_state=st, start_pos=13,
                                       logits_to_keep=None)
    assert tuple(l0.shape) == (2, 12, 512) and tuple(l1.shape) == (2, 1, 512) and tuple(l2.shape) == (2, 5, 512)
    assert st.cache_pos == 18 and st.batch_size == 2
    assert _rel(_np(l0), ref[:, :12]) < REL_TOL
    assert _rel(_np(l1), ref[:, 12:13]) < REL_TOL
    assert _rel(_np(l2), ref[:, 13:18]) < REL_TOL
    with pytest.raises(ValueError):
        forward_cached_decode(model=model, input_ids=ids[:, :1], cache_state=st, start_pos=3,
                              logits_to_keep=None)
    with pytest.raises(ValueError):
        forward_cached_decode(model=model, input_ids=ids[:, :1], cache_state=None, start_pos=3,
                              logits_to_keep=None)


def test_bf16_continued_prefill_matches_fp32_model():
    """bf16 weights and activations (the HIP causal kernel reading cached
    latents as keys): a 600-token prompt over three steps of 250, 250 and 100
    tokens, against the same weights in fp32 run in one shot."""
    dev = _dev()
    model, params = _model(dev, seed=12, max_seq_len=1024)
    gen = torch.Generator().manual_seed(13)
    prompt = torch.randint(0, 512, (600,), generator=gen).to(dev)
    with torch.no_grad():
        ref = model.forward_step(prefill_ids=prompt, prefill_lens=[600], prefill_slots=_i32([0], dev))[0]
        model.cast_weights_(torch.bfloat16)
        model.reset_runtime_cache()
        for a, b in ((0, 250), (250, 500), (500, 600)):
            out = model.forward_step(prefill_ids=prompt[a:b], prefill_lens=[b - a], prefill_pos=[a],
                                     prefill_slots=_i32([2], dev))
    err = _rel(_np(out[0]), _np(ref))
    print(f"bf16 continued prefill vs fp32 one shot: {err:.2e}")
    assert err < 6e-2
