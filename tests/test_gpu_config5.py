"""The benchmark decoder at its own shape: the whole 28-layer hybrid decoder
([KDA, KDA, KDA, MLA] x 7, dim 1536, 16 heads x 128, SiTU-GLU 3968, MLA ranks
384 / 128, vocab 65,536, tied; ModelArgs() defaults, random init, bf16) in one
continuous-batching step of 16 new sequences x 1,024 tokens packed with one
decode token for each of 240 running sequences (cached lengths U[1, 1023]),
captured in a HIP graph (the reference's decoder step, transformer.py:169-207,
captured as in sm120_graph_runner.py:318-371).

Checked here, at that shape:
  * every graph replay equals the eager step: the logits and every cache
    (21 KDA recurrent and conv states, 7 MLA latent caches), replays
    bit-identical to each other, eager work between replays;
  * sampled sequences of the packed step (2 of the 16 prefills, 3 of the 240
    decodes) against the same sequence run alone from the same caches: the
    last-token logits within 2e-2 of max |logit| and, for decodes, the
    sequence's recurrent state in every KDA layer.  The lone runs take other
    GEMM shapes (M = 1,024 or 1 instead of 16,624), so bf16 rounding differs
    between the two through 28 layers; the bound is the task's 2e-2.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

P, T, D, L = 16, 1024, 240, 1024
LOGIT_TOL = 2e-2


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float() - b.float()).abs().max()) / max(float(b.float().abs().max()), 1e-30)


@pytest.fixture(scope="module")
def bench_decoder():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from sophia_amd.config import ModelArgs
    from sophia_amd.decoder import Transformer

    dev = torch.device("cuda:0")
    args = ModelArgs(max_batch_size=P + D, max_seq_len=2048)
    assert (args.n_layers, args.dim, args.num_heads, args.vocab_size) == (28, 1536, 16, 65536)
    torch.manual_seed(4)
    with torch.device(dev):
        model = Transformer(args)
    model.cast_weights_(torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(4)
    decode = slice(P, P + D)
    for layer in model.layers:
        if layer.layer_type == "mla":
            layer.attn.latent_cache.normal_(generator=gen)
        else:
            # running sequences carry state: N(0, 0.02) recurrent states, conv history
            layer.attn.recurrent_state[decode].normal_(0.0, 0.02, generator=gen)
            layer.attn.conv_state[decode].normal_(0.0, 0.5, generator=gen)
    cpu = torch.Generator().manual_seed(4)
    step = dict(
        prefill_ids=torch.randint(0, args.vocab_size, (P, T), generator=cpu).to(dev),
        decode_ids=torch.randint(0, args.vocab_size, (D,), generator=cpu).to(dev),
        prefill_slots=torch.arange(P, dtype=torch.int32).to(dev),
        decode_slots=torch.arange(P, P + D, dtype=torch.int32).to(dev),
        decode_pos=torch.randint(1, L, (D,), generator=cpu).to(dev))
    start = _snapshot(model)
    with torch.no_grad():
        eager = model.forward_mixed(max_decode_len=L, **step).clone()
    torch.cuda.synchronize()
    after = _snapshot(model)
    print(f"packed step {P} x {T} + {D}: logits {tuple(eager.shape)}, max |logit| "
          f"{float(eager.float().abs().max()):.3f}", flush=True)
    yield model, step, start, after, eager
    del start, after


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


def test_config5_step_is_finite_and_advances_the_named_slots(bench_decoder):
    model, step, start, after, eager = bench_decoder
    assert tuple(eager.shape) == (P + D, 65536) and eager.dtype == torch.bfloat16
    assert bool(torch.isfinite(eager.float()).all())
    kda = [i for i, layer in enumerate(model.layers) if layer.layer_type == "kda"]
    assert len(kda) == 21
    for i in kda:
        s0, s1 = start[i][0], after[i][0]
        # prefill slots start from zero, decode slots moved on, the rest untouched
        assert bool(s1[:P + D].abs().amax(dim=(1, 2, 3)).gt(0).all())
        assert torch.equal(s0[P + D:], s1[P + D:])


def test_config5_graph_replays_equal_the_eager_step(bench_decoder):
    """Three replays of MixedStepGraph, each from the step's starting caches,
    with eager work on the same stream between them: every replay gives the
    eager step's logits and caches (to rounding; printed whether bitwise), and
    the replays are bit-identical to one another."""
    from sophia_amd.decoder import MixedStepGraph

    model, step, start, after, eager = bench_decoder
    dev = eager.device
    _restore(model, start)
    graph = MixedStepGraph(model, P, T, D, L, warmup=2, example=step)
    first = None
    for replay in range(3):
        _restore(model, start)
        torch.cuda.synchronize()
        out = graph.run(**step).clone()
        torch.cuda.synchronize()
        err = _rel(out, eager)
        print(f"replay {replay}: logits rel diff {err:.2e} (bitwise equal: {torch.equal(out, eager)})", flush=True)
        assert err <= 1e-3, f"replay {replay} logits"
        worst = 0.0
        for a, b in zip(_snapshot(model), after):
            for x, y in zip(a, b):
                worst = max(worst, _rel(x, y))
        print(f"replay {replay}: caches max rel diff {worst:.2e}", flush=True)
        assert worst <= 1e-4, f"replay {replay} caches"
        if first is None:
            first = out
        else:
            assert torch.equal(out, first), f"replay {replay} differs from replay 0"
        with torch.no_grad():   # eager work between replays
            model(torch.zeros(1, 3, dtype=torch.long, device=dev), start_pos=0)
    del graph


@pytest.mark.parametrize("kind,index", [("prefill", 3), ("prefill", 12), ("decode", 0), ("decode", 101),
                                        ("decode", 239)])
def test_config5_packed_row_equals_the_sequence_run_alone(bench_decoder, kind, index):
    model, step, start, after, eager = bench_decoder
    _restore(model, start)
    with torch.no_grad():
        if kind == "prefill":
            alone = model.forward_step(prefill_ids=step["prefill_ids"][index], prefill_lens=[T],
                                       prefill_slots=step["prefill_slots"][index:index + 1])
            row = index
        else:
            j = slice(index, index + 1)
            alone = model.forward_step(decode_ids=step["decode_ids"][j], decode_slots=step["decode_slots"][j],
                                       decode_pos=step["decode_pos"][j], max_decode_len=L)
            row = P + index
    torch.cuda.synchronize()
    err = _rel(alone[0], eager[row])
    print(f"{kind} {index}: last-token logits rel diff {err:.2e}", flush=True)
    assert err <= LOGIT_TOL
    slot = int(step["prefill_slots"][index]) if kind == "prefill" else int(step["decode_slots"][index])
    worst = 0.0
    for i, layer in enumerate(model.layers):
        if layer.layer_type == "kda":
            worst = max(worst, _rel(layer.attn.recurrent_state[slot], after[i][0][slot]))
    print(f"{kind} {index}: recurrent states (21 layers) max rel diff {worst:.2e}", flush=True)
    assert worst <= LOGIT_TOL
