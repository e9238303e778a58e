"""GPU parity of the decoder-side HIP kernels (sophia_decoder.h) through the
C ABI: the attention-residual depth mixer (blocks.py:38-48, optionally with
the RMSNorm that consumes it), the SiTU-GLU activation (blocks.py:23-27) and
the gated per-head outputs of the KDA and MLA mixers (attention.py:411-420,
655-656).

References are computed in float64 on the host from the same (rounded)
inputs: the module's formulas written with torch ops, and, for the mixer, the
oracle's restatement (oracle/decoder_oracle.attn_res_mix).

Tolerances (written per case): fp32 inputs, max|y - y_ref| <= 2e-5 max|y_ref|
(fp32 sums over at most 4096 x 16 terms); bf16 inputs, the kernel rounds its
fp32 result once, so |y - y_ref| <= 2^-8 |y_ref| + 1e-6 element-wise (half a
bf16 ulp is 2^-9; the extra factor covers the fp32 arithmetic before the
rounding).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decoder_oracle as do

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _mix_ref(partial, completed, w, q, eps, wo=None, out_eps=1e-6):
    """blocks.py:38-48 (then ops.py:49-64 RMSNorm when wo is given) in float64."""
    values = torch.cat((completed, partial.unsqueeze(-2)), dim=-2).double().cpu()
    w, q = w.double().cpu(), q.double().cpu()
    keys = values * torch.rsqrt(values.pow(2).mean(-1, keepdim=True) + eps) * w
    p = torch.softmax(keys @ q, dim=-1)
    y = (p.unsqueeze(-1) * values).sum(-2)
    if wo is not None:
        y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + out_eps) * wo.double().cpu()
    return y


def _check(y, ref, dtype):
    y = y.double().cpu()
    if dtype == torch.float32:
        err = float((y - ref).abs().max()) / max(float(ref.abs().max()), 1e-30)
        assert err <= 2e-5, err
    else:
        bad = (y - ref).abs() > ref.abs() * 2.0 ** -8 + 1e-6
        assert not bool(bad.any()), float((y - ref).abs().max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,n_blocks,dim", [(1, 0, 8), (5, 1, 24), (300, 3, 256),
                                               (257, 7, 1536), (64, 15, 1536), (33, 2, 4096),
                                               (17, 4, 2056)])
@pytest.mark.parametrize("normed", [False, True])
def test_attn_res_mix_matches_fp64_reference(dtype, rows, n_blocks, dim, normed):
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(rows * 131 + n_blocks * 7 + dim)
    partial = torch.randn(rows, dim, generator=g).to(dev, dtype)
    completed = (torch.randn(rows, n_blocks, dim, generator=g) * 2).to(dev, dtype)
    w = (1 + 0.2 * torch.randn(dim, generator=g)).to(dev)
    # queries large enough that the softmax is far from uniform
    q = (torch.randn(dim, generator=g) * 3 / dim ** 0.5).to(dev)
    wo = (1 + 0.2 * torch.randn(dim, generator=g)).to(dev) if normed else None
    y = ops.attn_res_mix(partial, completed, w, q, 1e-5, out_norm_weight=wo, out_eps=1e-5)
    torch.cuda.synchronize()
    assert y.shape == partial.shape and y.dtype == dtype
    _check(y, _mix_ref(partial, completed, w, q, 1e-5, wo, 1e-5), dtype)


def test_attn_res_mix_matches_oracle_on_strided_store_views():
    """Leading dims [B, S], completed a narrow view of a wider depth store and
    partial a strided slice, as the decoder passes them; checked against the
    oracle's restatement."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(5)
    B, S, D, nb = 3, 37, 256, 5
    store = torch.randn(B, S, 8, D, generator=g).to(dev)
    completed = store.narrow(-2, 0, nb)
    wide = torch.randn(B, S, 2 * D, generator=g).to(dev)
    partial = wide[..., D:]
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev)
    q = (0.2 * torch.randn(1, D, generator=g)).to(dev)
    y = ops.attn_res_mix(partial, completed, w, q, 1e-5)
    torch.cuda.synchronize()
    params = {"m.norm.weight": w.double().cpu().numpy(), "m.query.weight": q.double().cpu().numpy()}
    ref = do.attn_res_mix(params, "m", partial.double().cpu().numpy(),
                          completed.double().cpu().numpy(), norm_eps=1e-5)
    err = np.max(np.abs(y.double().cpu().numpy() - ref)) / np.max(np.abs(ref))
    assert err <= 2e-5, err


def test_attn_res_mix_bf16_query_weight_is_upcast():
    """A bf16 query weight (after a bf16 weight cast) is used at its bf16 value."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(9)
    partial = torch.randn(40, 512, generator=g).to(dev, torch.bfloat16)
    completed = torch.randn(40, 3, 512, generator=g).to(dev, torch.bfloat16)
    w = torch.ones(512, device=dev)
    q = (0.1 * torch.randn(1, 512, generator=g)).to(dev, torch.bfloat16)
    y = ops.attn_res_mix(partial, completed, w, q, 1e-5)
    torch.cuda.synchronize()
    _check(y, _mix_ref(partial, completed, w, q.float().reshape(-1), 1e-5), torch.bfloat16)


def _situ_ref(gu, cg=4.0, cu=25.0):
    gu = gu.double().cpu()
    gate, up = gu.chunk(2, dim=-1)
    return cg * torch.tanh(gate / cg) * torch.sigmoid(gate) * (cu * torch.tanh(up / cu))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden", [(1, 8), (3, 24), (1000, 3968), (129, 320)])
@pytest.mark.parametrize("u_sigma", [40.0, 0.5])
def test_situ_glu_matches_fp64_reference(dtype, rows, hidden, u_sigma):
    """u_sigma 40 spreads the up values over the soft cap's saturation region;
    0.5 keeps every |u| / 25 below 1/8 (the wavefronts' series-only path for
    the up side) except one planted value, whose wavefront takes the full
    path."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(rows + hidden)
    # spread over both soft caps' saturation regions and sigmoid's tails
    gu = torch.randn(rows, 2 * hidden, generator=g) * torch.tensor([6.0, u_sigma]).repeat_interleave(hidden)
    gu[0, :4] = torch.tensor([-90.0, 90.0, 0.0, -1e-3])
    if u_sigma < 1.0:
        gu[rows // 2, hidden + hidden // 2] = 30.0
    gu = gu.to(dev, dtype)
    y = ops.situ_glu(gu, 4.0, 25.0)
    torch.cuda.synchronize()
    assert y.shape == (rows, hidden) and y.dtype == dtype
    ref = _situ_ref(gu)
    yd = y.double().cpu()
    if dtype == torch.float32:
        # tanh and sigmoid from fp32 exponentials: a few ulp of the 100-sized output
        assert float((yd - ref).abs().max()) <= 2e-5 * max(float(ref.abs().max()), 1.0)
    else:
        assert not bool(((yd - ref).abs() > ref.abs() * 2.0 ** -8 + 1e-5).any())


def test_situ_glu_strided_input_and_leading_dims():
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(2)
    big = (torch.randn(2, 7, 3 * 64, generator=g) * 5).to(dev)
    gu = big[..., :128]  # rows of 128 values spaced 192 apart
    y = ops.situ_glu(gu, 4.0, 25.0)
    torch.cuda.synchronize()
    assert y.shape == (2, 7, 64)
    ref = _situ_ref(gu)
    assert float((y.double().cpu() - ref).abs().max()) <= 2e-5 * float(ref.abs().max())


def test_feed_forward_and_mixer_modules_match_reference_formulas():
    """FeedForward and AttentionResidualMixer (with and without the consuming
    norm) on the kernels against the reference modules' torch formulas."""
    from sophia_amd.config import ModelArgs
    from sophia_amd.decoder import AttentionResidualMixer, FeedForward
    from sophia_amd.kda import RMSNorm
    dev = _dev()
    torch.manual_seed(0)
    args = ModelArgs(dim=256, ffn_hidden=320)
    ffn = FeedForward(args).to(dev)
    mixer = AttentionResidualMixer(args).to(dev)
    norm = RMSNorm(256, 1e-5).to(dev)
    with torch.no_grad():
        for lin in (ffn.gate_up_proj, ffn.down_proj):
            lin.weight.normal_(0, 0.1)
        mixer.query.weight.normal_(0, 0.2)
        mixer.norm.weight.normal_(1, 0.1)
        norm.weight.normal_(1, 0.1)
        x = torch.randn(2, 9, 256, device=dev)
        completed = torch.randn(2, 9, 3, 256, device=dev)
        y = ffn(x)
        gate, up = (x @ ffn.gate_up_proj.weight.t()).split(320, dim=-1)
        h = 4.0 * torch.tanh(gate / 4.0) * torch.sigmoid(gate) * 25.0 * torch.tanh(up / 25.0)
        ref = h @ ffn.down_proj.weight.t()
        assert float((y - ref).abs().max()) <= 1e-4 * float(ref.abs().max())
        m = mixer(x, completed)
        ref = _mix_ref(x, completed, mixer.norm.weight, mixer.query.weight.reshape(-1), 1e-5)
        _check(m, ref, torch.float32)
        mn = mixer(x, completed, norm)
        ref = _mix_ref(x, completed, mixer.norm.weight, mixer.query.weight.reshape(-1), 1e-5,
                       norm.weight, 1e-5)
        _check(mn, ref, torch.float32)


def _gated_ref(o, gate, heads, head_dim, w=None, eps=1e-6):
    """attention.py:411-420 (with w) / 655-656 (without) in float64, o first
    rounded to the gate's dtype as the reference casts it."""
    rows = gate.reshape(-1, heads * head_dim).size(0)
    o = o.to(gate.dtype).double().cpu().reshape(rows, heads, head_dim)
    g = gate.double().cpu().reshape(rows, heads, head_dim)
    if w is not None:
        o = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + eps) * w.double().cpu()
    return (o * torch.sigmoid(g)).reshape(rows, heads * head_dim)


@pytest.mark.parametrize("dtype,o_dtype", [(torch.float32, torch.float32),
                                           (torch.bfloat16, torch.bfloat16),
                                           (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows,heads,head_dim", [(1, 16, 128), (300, 16, 128), (7, 3, 8),
                                                 (33, 2, 512), (64, 5, 64)])
@pytest.mark.parametrize("normed", [True, False])
def test_gated_head_norm_matches_fp64_reference(dtype, o_dtype, rows, heads, head_dim, normed):
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(rows * 3 + heads * 5 + head_dim)
    width = heads * head_dim
    o = (torch.randn(rows, heads, head_dim, generator=g) * 3).to(dev, o_dtype)
    # gate logits as a column slice of a wider fused projection (row stride > width)
    fused = (torch.randn(rows, width + 24, generator=g) * 4).to(dev, dtype)
    gate = fused[:, 16:16 + width]
    w = (1 + 0.3 * torch.randn(head_dim, generator=g)).to(dev) if normed else None
    y = ops.gated_head_norm(o, gate, heads, head_dim, norm_weight=w, eps=1e-5)
    torch.cuda.synchronize()
    assert y.shape == (rows, width) and y.dtype == dtype
    _check(y, _gated_ref(o, gate, heads, head_dim, w, 1e-5), dtype)


def test_gated_head_norm_rejects_misaligned_and_bad_shapes():
    from sophia_amd import ops
    dev = _dev()
    o = torch.zeros(4, 2 * 128, device=dev)
    fused = torch.zeros(4, 2 * 128 + 8, device=dev)
    with pytest.raises(RuntimeError, match="aligned"):
        ops.gated_head_norm(o, fused[:, 2:2 + 256], 2, 128)
    with pytest.raises(RuntimeError, match="head_dim"):
        ops.gated_head_norm(torch.zeros(4, 2 * 96, device=dev), torch.zeros(4, 2 * 96, device=dev), 2, 96)


def _mla_ref(qa, cache, slots, pos, scale):
    """Latent-space decode attention (the decode rows of attention.py:609-657
    with W_k / W_v folded out) in float64 from bf16-rounded qa and latents,
    as the reference casts both to the activation dtype."""
    qa = qa.to(torch.bfloat16).double().cpu()
    lat = cache.to(torch.bfloat16).double().cpu()
    rows, heads, rank = qa.shape
    out = torch.zeros(rows, heads, rank, dtype=torch.float64)
    for b in range(rows):
        s = int(slots[b])
        if not 0 <= s < cache.size(0):
            continue
        n = min(int(pos[b]) + 1, cache.size(1))
        if n <= 0:
            continue
        keys = lat[s, :n]                                   # [n, rank]
        p = torch.softmax(scale * qa[b] @ keys.t(), dim=-1)  # [heads, n]
        out[b] = p @ keys
    return out


@pytest.mark.parametrize("rank,heads,rows,splits", [(32, 2, 5, 1), (64, 3, 9, 2), (128, 16, 240, None),
                                                    (128, 16, 3, 7), (256, 16, 17, 3), (128, 1, 1, 1)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mla_decode_attn_matches_fp64_reference(rank, heads, rows, splits, dtype):
    """Positions from a single key to the whole cache (including lengths that
    end mid-tile), permuted slots, more splits than tiles, a slot outside the
    cache (zeros), against the float64 latent-space reference.  Tolerance: the
    probabilities are rounded to bf16 before the value sum (as the reference
    rounds them to the activation dtype), so max|y - ref| <= 1e-2 max|ref|."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(rank + heads * 7 + rows)
    n_slots, max_seq = rows + 3, 300
    cache = torch.randn(n_slots, max_seq, rank, generator=g).to(dev)
    qa = (torch.randn(rows, heads, rank, generator=g) * 0.3).to(dev, dtype)
    slots = torch.randperm(n_slots, generator=g)[:rows].to(torch.int32)
    pos = torch.randint(0, max_seq, (rows,), generator=g)
    pos[0] = 0
    if rows > 2:
        pos[1] = max_seq - 1
        pos[2] = 16 * 5 + 6
    if rows > 4:
        slots[3] = -1       # not a cache slot: zero output
        pos[4] = max_seq + 40  # clamped to the cache length
    scale = 128 ** -0.5
    y = ops.mla_decode_attn(qa, cache, slots.to(dev), pos.to(dev), scale, max_len=max_seq,
                            splits=splits)
    torch.cuda.synchronize()
    assert y.shape == (rows, heads, rank) and y.dtype == dtype
    ref = _mla_ref(qa, cache, slots, pos, scale)
    err = float((y.double().cpu() - ref).abs().max()) / float(ref.abs().max())
    assert err <= 1e-2, err
    if rows > 4:
        assert float(y[3].abs().max()) == 0.0


def _causal_ref(q, k, v, cu, scale):
    """Causal softmax attention per packed sequence, float32 on the host from
    the same bf16 inputs (scaled_dot_product_attention(is_causal=True) per
    sequence, attention.py:630-639)."""
    q, k, v = (t.float().cpu() for t in (q, k, v))
    out = torch.zeros_like(q)
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        n = b - a
        if n == 0:
            continue
        s = torch.einsum("thd,shd->hts", q[a:b], k[a:b]) * scale
        s = s.masked_fill(torch.ones(n, n, dtype=torch.bool).triu(1), float("-inf"))
        out[a:b] = torch.einsum("hts,shd->thd", torch.softmax(s, dim=-1), v[a:b])
    return out


@pytest.mark.parametrize("lengths,heads", [((1,), 1), ((77, 300, 128, 129, 0, 5), 3),
                                           ((1024, 1024), 16), ((1000,), 2)])
def test_causal_attention_matches_reference(lengths, heads):
    """Ragged packed sequences (an empty one, lengths at and around the 64-key
    and 128-query block edges), row-strided q (a slice of a fused projection)
    and an output view, against the float32 reference.  Tolerance: the
    probabilities enter the value product as bf16, so
    max|y - ref| <= 1e-2 max|ref|."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(sum(lengths) + heads)
    total = sum(lengths)
    cu = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32)
    width = heads * 128
    fused = (torch.randn(total, 3 * width + 64, generator=g)).to(dev, torch.bfloat16)
    q = fused[:, 64:64 + width].view(total, heads, 128)
    k = fused[:, 64 + width:64 + 2 * width].view(total, heads, 128)
    v = (torch.randn(total, heads, 128, generator=g)).to(dev, torch.bfloat16)
    big = torch.full((total, heads + 1, 128), 7.0, dtype=torch.bfloat16, device=dev)
    out = big[:, 1:]
    scale = 128 ** -0.5
    y = ops.causal_attention(q, k, v, cu.to(dev), max(lengths), scale=scale, out=out)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr()
    ref = _causal_ref(q, k, v, cu, scale)
    err = float((y.float().cpu() - ref).abs().max()) / float(ref.abs().max())
    assert err <= 1e-2, err
    assert bool((big[:, 0].float() == 7.0).all()), "wrote outside the output view"


@pytest.mark.parametrize("queries,keys,heads", [((1, 77, 200, 64, 5), (1, 300, 200, 1000, 70), 2),
                                                 ((1024, 3), (1024, 2051), 16), ((0, 128), (40, 129), 1)])
def test_causal_attention_after_cached_keys_matches_reference(queries, keys, heads):
    """Queries that continue after cached keys (cu_seqlens_k): sequence s has
    queries[s] query rows and keys[s] >= queries[s] key rows, and query i sits
    at position i + keys[s] - queries[s] (the tril(klen - seqlen) mask of
    ml/runtime/model/attention.py:641-654), against a float32 reference
    computed per sequence.  Same tolerance as above (bf16 probabilities)."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(sum(keys) + heads)
    tq, tk = sum(queries), sum(keys)
    cu = torch.tensor([0] + list(np.cumsum(queries)), dtype=torch.int32)
    cuk = torch.tensor([0] + list(np.cumsum(keys)), dtype=torch.int32)
    q = torch.randn(tq, heads, 128, generator=g).to(dev, torch.bfloat16)
    k = torch.randn(tk, heads, 128, generator=g).to(dev, torch.bfloat16)
    v = torch.randn(tk, heads, 128, generator=g).to(dev, torch.bfloat16)
    scale = 128 ** -0.5
    y = ops.causal_attention(q, k, v, cu.to(dev), max(queries), scale=scale, cu_seqlens_k=cuk.to(dev))
    torch.cuda.synchronize()
    qf, kf, vf = (t.float().cpu() for t in (q, k, v))
    ref = torch.zeros(tq, heads, 128)
    for s in range(len(queries)):
        a, b, ka, kb = int(cu[s]), int(cu[s + 1]), int(cuk[s]), int(cuk[s + 1])
        nq, nk = b - a, kb - ka
        if nq == 0:
            continue
        sc = torch.einsum("thd,shd->hts", qf[a:b], kf[ka:kb]) * scale
        allow = torch.ones(nq, nk, dtype=torch.bool).tril(nk - nq)
        sc = sc.masked_fill(~allow, float("-inf"))
        ref[a:b] = torch.einsum("hts,shd->thd", torch.softmax(sc, dim=-1), vf[ka:kb])
    err = float((y.float().cpu() - ref).abs().max()) / float(ref.abs().max())
    assert err <= 1e-2, err


def test_causal_attention_with_fewer_keys_than_queries():
    """A sequence with fewer keys than queries (0 keys, or 3 keys for 200
    queries) has no causal alignment: with device offsets only, the kernel
    writes zeros for its rows (never leaves them unwritten) and the other
    sequences are unaffected; with the host offsets the call is rejected
    before any launch."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(91)
    queries, keys, heads = (5, 200, 70, 9), (9, 3, 70, 0), 2
    tq, tk = sum(queries), sum(keys)
    cu = torch.tensor([0] + list(np.cumsum(queries)), dtype=torch.int32)
    cuk = torch.tensor([0] + list(np.cumsum(keys)), dtype=torch.int32)
    q = torch.randn(tq, heads, 128, generator=g).to(dev, torch.bfloat16)
    k = torch.randn(tk, heads, 128, generator=g).to(dev, torch.bfloat16)
    v = torch.randn(tk, heads, 128, generator=g).to(dev, torch.bfloat16)
    out = torch.full((tq, heads, 128), 7.0, dtype=torch.bfloat16, device=dev)
    scale = 128 ** -0.5
    y = ops.causal_attention(q, k, v, cu.to(dev), max(queries), scale=scale, cu_seqlens_k=cuk.to(dev), out=out)
    torch.cuda.synchronize()
    yc = y.float().cpu()
    for s in (1, 3):
        assert bool((yc[int(cu[s]):int(cu[s + 1])] == 0).all()), f"sequence {s} rows not zero"
    qf, kf, vf = (t.float().cpu() for t in (q, k, v))
    for s in (0, 2):
        a, b, ka, kb = int(cu[s]), int(cu[s + 1]), int(cuk[s]), int(cuk[s + 1])
        nq, nk = b - a, kb - ka
        sc = torch.einsum("thd,shd->hts", qf[a:b], kf[ka:kb]) * scale
        sc = sc.masked_fill(~torch.ones(nq, nk, dtype=torch.bool).tril(nk - nq), float("-inf"))
        ref = torch.einsum("hts,shd->thd", torch.softmax(sc, dim=-1), vf[ka:kb])
        assert float((yc[a:b] - ref).abs().max()) <= 1e-2 * float(ref.abs().max())
    with pytest.raises(RuntimeError, match="at least as many keys"):
        ops.causal_attention(q, k, v, cu.to(dev), max(queries), scale=scale, cu_seqlens_k=cuk.to(dev),
                             cu_seqlens_host=cu, cu_seqlens_k_host=cuk)


def test_mla_prefill_bf16_kernel_matches_sdpa_path():
    """SophiaMLA.forward in bf16 (HIP causal kernel) against the same module in
    fp32 (torch SDPA) on the same weights and input."""
    from sophia_amd.config import ModelArgs
    from sophia_amd.decoder import SophiaMLA
    dev = _dev()
    torch.manual_seed(3)
    args = ModelArgs(dim=256, num_heads=2, mla_q_rank=64, mla_kv_rank=32, max_seq_len=512,
                     max_batch_size=2)
    m32 = SophiaMLA(args).to(dev).eval()
    m32.use_cache = False
    with torch.no_grad():  # scores of order one, so that the softmax is far from uniform
        m32.q_up.weight.mul_(12.0)
        m32.k_up.weight.mul_(12.0)
    m16 = SophiaMLA(args).to(dev).eval()
    m16.load_state_dict(m32.state_dict())
    m16.use_cache = False
    for mod in m16.modules():
        if mod.__class__.__name__ == "RuntimeLinear":
            mod.weight.data = mod.weight.data.to(torch.bfloat16)
    x = torch.randn(2, 300, 256, device=dev)
    with torch.no_grad():
        y32 = m32(x)
        y16 = m16(x.to(torch.bfloat16))
    torch.cuda.synchronize()
    err = float((y16.float() - y32).abs().max()) / float(y32.abs().max())
    assert err <= 3e-2, err


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,n_blocks,dim", [(3, 0, 8), (300, 3, 256), (257, 7, 1536), (33, 2, 4096)])
def test_attn_res_mix_with_residual_add(dtype, rows, n_blocks, dim):
    """The residual add folded into the mix: the new partial block equals
    torch's partial + residual in the activation dtype bit for bit, and the
    mix (with the consuming norm) is taken over it."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(rows + 5 * n_blocks + dim)
    partial = torch.randn(rows, dim, generator=g).to(dev, dtype)
    residual = (torch.randn(rows, dim, generator=g) * 0.5).to(dev, dtype)
    completed = (torch.randn(rows, n_blocks, dim, generator=g) * 2).to(dev, dtype)
    w = (1 + 0.2 * torch.randn(dim, generator=g)).to(dev)
    q = (torch.randn(dim, generator=g) * 3 / dim ** 0.5).to(dev)
    wo = (1 + 0.2 * torch.randn(dim, generator=g)).to(dev)
    new_partial, y = ops.attn_res_mix(partial, completed, w, q, 1e-5, out_norm_weight=wo,
                                      out_eps=1e-5, residual=residual)
    torch.cuda.synchronize()
    summed = partial + residual
    assert torch.equal(new_partial, summed)
    _check(y, _mix_ref(summed, completed, w, q, 1e-5, wo, 1e-5), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attn_res_mix_writes_the_sum_into_a_depth_store_slot(dtype):
    """partial_out: the sum partial + residual written into the next slot of a
    depth store (strided rows) while the mix reads the store's earlier
    blocks: the slot holds the same bits as the default call's new partial
    block, the mix is bitwise the same, and the store's other slots are
    untouched."""
    from sophia_amd import ops
    dev = _dev()
    rows, n_blocks, n_max, dim = 300, 3, 5, 1536
    g = torch.Generator(device="cpu").manual_seed(91)
    partial = torch.randn(rows, dim, generator=g).to(dev, dtype)
    residual = (torch.randn(rows, dim, generator=g) * 0.5).to(dev, dtype)
    store = (torch.randn(rows, n_max, dim, generator=g) * 2).to(dev, dtype)
    before = store.clone()
    w = (1 + 0.2 * torch.randn(dim, generator=g)).to(dev)
    q = (torch.randn(dim, generator=g) * 3 / dim ** 0.5).to(dev)
    completed = store[:, :n_blocks]
    want_partial, want_y = ops.attn_res_mix(partial, completed, w, q, 1e-5, residual=residual)
    slot = store[:, n_blocks]
    got_partial, got_y = ops.attn_res_mix(partial, completed, w, q, 1e-5, residual=residual, partial_out=slot)
    torch.cuda.synchronize()
    assert got_partial.data_ptr() == slot.data_ptr()
    assert torch.equal(store[:, n_blocks], want_partial)
    assert torch.equal(got_y, want_y)
    for b in range(n_max):
        if b != n_blocks:
            assert torch.equal(store[:, b], before[:, b]), b
    with pytest.raises(RuntimeError, match="residual"):
        ops.attn_res_mix(partial, completed, w, q, 1e-5, partial_out=slot)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["rectangular", "ragged"])
def test_mla_latent_norms_and_cache_rows(dtype, mode):
    """sophia_mla_latent_norms: q_norm and kv_norm in place against torch's
    rms_norm with the weight cast to the activation dtype (RMSNorm.forward),
    within one rounding of that dtype; every latent row lands in its cache
    slot and position exactly as the kernel's own output (fp32 of the rounded
    value), slots or positions out of range write nothing, and every other
    cache entry is untouched.  Prefill rows mapped per sequence (equal-length
    prompts) or per row, then decode rows."""
    from sophia_amd import ops
    dev = _dev()
    g = torch.Generator(device="cpu").manual_seed(7 if mode == "rectangular" else 8)
    q_rank, kv_rank, n_slots, max_len, eps = 384, 128, 6, 12, 1e-6
    if mode == "rectangular":
        P, T = 3, 5
        n_pre = P * T
        seq_slots = torch.tensor([4, 0, 2], dtype=torch.int32, device=dev)
        want_pre = [(int(seq_slots[i // T]), i % T) for i in range(n_pre)]
        kw = dict(prefill_seq_slots=seq_slots, prefill_seq_len=T)
    else:
        want_pre = [(1, 3), (1, 4), (5, 0), (3, 11), (7, 2), (2, 12)]   # the last two: slot / position out of range
        n_pre = len(want_pre)
        kw = dict(prefill_row_slots=torch.tensor([s for s, _ in want_pre], device=dev),
                  prefill_row_pos=torch.tensor([p for _, p in want_pre], device=dev))
    want_dec = [(0, 7), (3, 0), (5, 11), (-1, 3)]                        # the last: out of range
    rows = n_pre + len(want_dec)
    q_lat = (torch.randn(rows, q_rank, generator=g) * 2).to(dev, dtype)
    kv_lat = (torch.randn(rows, kv_rank, generator=g) * 0.5).to(dev, dtype)
    qw = (1 + 0.3 * torch.randn(q_rank, generator=g)).to(dev)
    kvw = (1 + 0.3 * torch.randn(kv_rank, generator=g)).to(dev)
    cache = torch.randn(n_slots, max_len, kv_rank, generator=g).to(dev)
    before = cache.clone()
    want_q = torch.nn.functional.rms_norm(q_lat, (q_rank,), qw.to(dtype), eps)
    want_kv = torch.nn.functional.rms_norm(kv_lat, (kv_rank,), kvw.to(dtype), eps)
    ops.mla_latent_norms(q_lat, kv_lat, qw, eps, kvw, eps, latent_cache=cache, n_prefill=n_pre,
                         decode_slots=torch.tensor([s for s, _ in want_dec], dtype=torch.int32, device=dev),
                         decode_pos=torch.tensor([p for _, p in want_dec], device=dev), **kw)
    torch.cuda.synchronize()
    rtol = 2.0 ** -7 if dtype == torch.bfloat16 else 2e-6
    for got, want, name in ((q_lat, want_q, "q"), (kv_lat, want_kv, "kv")):
        err = float(((got.float() - want.float()).abs() / (want.float().abs() + 1e-6)).max())
        print(f"{name}_norm {dtype}: max rel diff to torch {err:.2e}", flush=True)
        assert err <= rtol, (name, err)
    written = torch.zeros(n_slots, max_len, dtype=torch.bool, device=dev)
    for i, (s, p) in enumerate(want_pre + want_dec):
        if 0 <= s < n_slots and 0 <= p < max_len:
            assert torch.equal(cache[s, p], kv_lat[i].float()), (i, s, p)
            written[s, p] = True
    assert torch.equal(cache[~written], before[~written])
