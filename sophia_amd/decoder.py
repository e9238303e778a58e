"""The Sophia hybrid decoder around the MI355X KDA mixer, and its captured
continuous-batching step.

Modules keep the reference's names, parameter shapes and semantics
(ml/runtime/model/attention.py:423-657 ``SophiaMLA``; blocks.py:12-87
``FeedForward`` / ``AttentionResidualMixer`` / ``SophiaBlock``;
transformer.py:17-207 and transformer_setup.py:33-79 ``Transformer``), so a
reference state_dict loads as is.  Layer i is MLA iff i % 4 == 3, the rest are
``sophia_amd.kda.SophiaKDA`` (gfx950 kernels).  The SiTU-GLU activation and
each attention-residual depth mix, with the RMSNorm that consumes it, run as
single HIP kernels (``ops.situ_glu``, ``ops.attn_res_mix``); depth blocks are
appended in place into one store per forward.  The projections of MLA and the
FFN run on library GEMMs and attention (hipBLASLt / SDPA through torch).

Besides the reference-shaped ``Transformer.forward(input_ids, attention_mask,
start_pos)`` (and ``forward_full``),
``Transformer.forward_mixed`` runs one continuous-batching step that the
reference cannot express (it has one start_pos per batch,
transformer.py:146-160): new sequences prefilled in a rectangular group,
packed with one decode token for each of many running sequences, every
sequence in its own cache slot.  ``MixedStepGraph`` captures that step in a
HIP graph after a warm-up on a side stream (the capture pattern of
ml/training/pretrain/engine/sm120_graph_runner.py:318-371) and replays it.
"""

from __future__ import annotations

import itertools
import math

import torch
import torch.nn.functional as F
from torch import nn

from .config import ModelArgs
from . import ops
from .kda import RMSNorm, RuntimeLinear, SophiaKDA, _require_gpu
from .state import LayerCacheSnapshot, RuntimeCacheSnapshot


class SophiaMLA(nn.Module):
    """NoPE multi-head latent attention with a full-rank output gate
    (attention.py:423-657)."""

    def __init__(self, args: ModelArgs) -> None:
        super().__init__()
        self.dim = int(args.dim)
        self.num_heads = int(args.num_heads)
        self.head_dim = int(args.head_dim)
        self.inner_dim = self.num_heads * self.head_dim
        self.q_rank = int(args.mla_q_rank)
        self.kv_rank = int(args.mla_kv_rank)
        self.use_cache = bool(args.use_cache)
        self.q_down = RuntimeLinear(self.dim, self.q_rank)
        self.q_norm = RMSNorm(self.q_rank, args.norm_eps)
        self.q_up = RuntimeLinear(self.q_rank, self.inner_dim)
        self.kv_down = RuntimeLinear(self.dim, self.kv_rank)
        self.kv_norm = RMSNorm(self.kv_rank, args.norm_eps)
        self.k_up = RuntimeLinear(self.kv_rank, self.inner_dim)
        self.v_up = RuntimeLinear(self.kv_rank, self.inner_dim)
        self.output_gate = RuntimeLinear(self.dim, self.inner_dim)
        self.o_proj = RuntimeLinear(self.inner_dim, self.dim)
        self.register_buffer("latent_cache", torch.zeros(
            int(args.max_batch_size), int(args.max_seq_len), self.kv_rank), persistent=False)
        self._v_t = None
        self._v_t_key = None
        self._in_w = None
        self._in_w_key = None

    def _input_weight(self, dtype: torch.dtype) -> torch.Tensor:
        """q_down, kv_down and output_gate stacked [q_rank + kv_rank + inner,
        dim]: the three projections of x in one GEMM (the packed step), kept
        until a weight changes."""
        params = (self.q_down.weight, self.kv_down.weight, self.output_gate.weight)
        if torch.is_grad_enabled() and any(p.requires_grad for p in params):
            return torch.cat(params, 0).to(dtype)
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in params) + (dtype,)
        if self._in_w_key != key:
            with torch.no_grad():
                self._in_w = torch.cat([p.detach() for p in params], 0).to(dtype).contiguous()
            self._in_w_key = key
        return self._in_w

    def _v_up_t(self, dtype: torch.dtype) -> torch.Tensor:
        """v_up's weight as [heads, kv_rank, head_dim] (the per-head blocks
        transposed, as the decode rows' value product takes them), kept until
        the weight changes so that no copy runs per step."""
        w = self.v_up.weight
        h, d, r = self.num_heads, self.head_dim, self.kv_rank
        if torch.is_grad_enabled() and w.requires_grad:
            return w.view(h, d, r).to(dtype).transpose(1, 2).contiguous()
        key = (w.data_ptr(), w._version, w.dtype, dtype)
        if self._v_t_key != key:
            self._v_t = w.detach().view(h, d, r).to(dtype).transpose(1, 2).contiguous()
            self._v_t_key = key
        return self._v_t

    # ------------------------------------------------------------- caches
    def ensure_batch_capacity(self, batch_size: int) -> None:
        required = int(batch_size)
        if required <= int(self.latent_cache.size(0)):
            return
        grown = self.latent_cache.new_zeros(required, int(self.latent_cache.size(1)), self.kv_rank)
        grown[: self.latent_cache.size(0)].copy_(self.latent_cache)
        self.latent_cache = grown

    def ensure_sequence_capacity(self, max_seq_len: int) -> None:
        required = int(max_seq_len)
        if required <= int(self.latent_cache.size(1)):
            return
        grown = self.latent_cache.new_zeros(int(self.latent_cache.size(0)), required, self.kv_rank)
        grown[:, : self.latent_cache.size(1)].copy_(self.latent_cache)
        self.latent_cache = grown

    def reset(self) -> None:
        if self.latent_cache.is_inference():
            self.latent_cache = torch.zeros_like(self.latent_cache)
        else:
            self.latent_cache.zero_()

    def cache_snapshot(self, *, device: str, batch_size: int, cache_pos: int | None,
                       slots: torch.Tensor | None = None):
        """Copies of latents [:cache_pos] of rows [:batch_size] (attention.py:
        570-575), or of the cache slots ``slots`` in that order."""
        end = int(self.latent_cache.size(1) if cache_pos is None else cache_pos)
        if slots is not None:
            idx = slots.to(device=self.latent_cache.device, dtype=torch.long)
            return LayerCacheSnapshot(latent=self.latent_cache[:, :end].index_select(0, idx).to(device))
        return LayerCacheSnapshot(latent=self.latent_cache[:batch_size, :end].to(device).clone())

    def validate_cache_snapshot(self, snapshot: LayerCacheSnapshot) -> None:
        if snapshot.recurrent is not None or snapshot.conv is not None:
            raise ValueError("MLA cache cannot contain KDA state")
        if snapshot.latent is not None and int(snapshot.latent.size(-1)) != self.kv_rank:
            raise ValueError("MLA latent cache shape mismatch")

    def load_cache_snapshot(self, snapshot: LayerCacheSnapshot, *,
                            slots: torch.Tensor | None = None) -> None:
        """attention.py:577-583; with ``slots``, row i of the snapshot goes to
        cache slot slots[i] (positions past the snapshot's length untouched)."""
        self.validate_cache_snapshot(snapshot)
        if snapshot.latent is None:
            return
        batch, length = int(snapshot.latent.size(0)), int(snapshot.latent.size(1))
        if slots is not None:
            self.ensure_sequence_capacity(length)
            idx = slots.to(device=self.latent_cache.device, dtype=torch.long)
            self.latent_cache[idx, :length] = snapshot.latent.to(self.latent_cache.device,
                                                                  dtype=self.latent_cache.dtype)
            return
        self.ensure_batch_capacity(batch)
        self.ensure_sequence_capacity(length)
        self.latent_cache[:batch, :length].copy_(
            snapshot.latent.to(self.latent_cache.device, dtype=self.latent_cache.dtype))

    # ------------------------------------------------------------- forward
    def _gate_out(self, x: torch.Tensor, out: torch.Tensor, gate: torch.Tensor | None = None) -> torch.Tensor:
        """attention.py:655-657: o_proj((o.float() * sigmoid(gate).float()).to(dtype)),
        the gate as one HIP kernel (ops.gated_head_norm without a norm);
        ``gate``: output_gate(x) when already projected."""
        if gate is None:
            gate = self.output_gate(x)
        gated = ops.gated_head_norm(out.to(x.dtype), gate, self.num_heads, self.head_dim)
        return self.o_proj(gated.view(*x.shape[:-1], self.inner_dim))

    def _causal(self, q, k, v, cu, max_len: int, out, *, cu_k=None, cu_host=None, cu_k_host=None):
        """Causal attention within each packed sequence, into ``out``.  Query
        rows are delimited by ``cu``, key/value rows by ``cu_k`` (default: the
        query rows); a sequence with more keys than queries continues after
        cached tokens (its queries are the last key positions, the
        tril(klen - seqlen) mask of attention.py:641-654).  The HIP kernel
        (``ops.causal_attention``) runs for bf16 activations; fp32 ones use
        torch SDPA, per sequence (host offsets ``cu_host`` / ``cu_k_host``)
        unless the sequences are equal-length and start from empty caches."""
        if q.dtype == torch.bfloat16:
            ops.causal_attention(q, k, v, cu, max_len, scale=self.head_dim ** -0.5, cu_seqlens_k=cu_k,
                                 out=out, cu_seqlens_host=cu_host, cu_seqlens_k_host=cu_k_host)
            return
        if cu_host is None:
            n = int(q.size(0)) // max_len
            o = F.scaled_dot_product_attention(*(t.reshape(n, max_len, self.num_heads, self.head_dim)
                                                 .transpose(1, 2) for t in (q, k, v)), is_causal=True)
            out.copy_(o.transpose(1, 2).reshape_as(out))
            return
        qo = [int(c) for c in cu_host.tolist()]
        ko = qo if cu_k_host is None else [int(c) for c in cu_k_host.tolist()]
        for s in range(len(qo) - 1):
            a, b, ka, kb = qo[s], qo[s + 1], ko[s], ko[s + 1]
            if b == a:
                continue
            allow = torch.ones((b - a, kb - ka), dtype=torch.bool, device=q.device).tril(kb - ka - (b - a))
            o = F.scaled_dot_product_attention(q[a:b].transpose(0, 1), k[ka:kb].transpose(0, 1),
                                               v[ka:kb].transpose(0, 1), attn_mask=allow)
            out[a:b] = o.transpose(0, 1)

    def forward(self, x: torch.Tensor, *, start_pos: int = 0) -> torch.Tensor:
        """attention.py:609-657 (pad-mask path: attention.py:585-600,635-654)."""
        bsz, seqlen, _ = x.shape
        q = self.q_up(self.q_norm(self.q_down(x))).view(bsz, seqlen, self.num_heads, self.head_dim)
        latent = self.kv_norm(self.kv_down(x))
        if self.use_cache:
            end = int(start_pos) + int(seqlen)
            self.ensure_batch_capacity(int(bsz))
            self.ensure_sequence_capacity(end)
            with torch.no_grad():
                self.latent_cache[:bsz, int(start_pos):end].copy_(latent.detach())
            latent_full = self.latent_cache[:bsz, :end].to(x.dtype)
        else:
            latent_full = latent
        klen = int(latent_full.size(1))
        k = self.k_up(latent_full).view(bsz, klen, self.num_heads, self.head_dim)
        v = self.v_up(latent_full).view_as(k)
        q_t, k_t, v_t = (t.transpose(1, 2) for t in (q, k, v))
        key_pad = self._key_mask(int(start_pos), bsz, klen, x.device)
        if key_pad is None and int(start_pos) == 0 and seqlen == klen:
            rows = bsz * seqlen
            cu = torch.arange(0, rows + 1, seqlen, dtype=torch.int32, device=x.device)
            out = torch.empty((rows, self.num_heads, self.head_dim), dtype=x.dtype, device=x.device)
            self._causal(q.reshape(rows, self.num_heads, self.head_dim),
                         k.reshape(rows, self.num_heads, self.head_dim),
                         v.reshape(rows, self.num_heads, self.head_dim), cu, seqlen, out)
            return self._gate_out(x, out.view(bsz, seqlen, self.num_heads, self.head_dim))
        if key_pad is None and x.dtype == torch.bfloat16 and self.head_dim == 128:
            # after cached keys, no padding: the HIP kernel, each row's queries
            # being the last seqlen of its klen key positions
            rows, h, d = bsz * seqlen, self.num_heads, self.head_dim
            cu = torch.arange(0, rows + 1, seqlen, dtype=torch.int32, device=x.device)
            cu_k = torch.arange(0, bsz * klen + 1, klen, dtype=torch.int32, device=x.device)
            out = torch.empty((rows, h, d), dtype=x.dtype, device=x.device)
            self._causal(q.reshape(rows, h, d), k.reshape(bsz * klen, h, d), v.reshape(bsz * klen, h, d), cu,
                         seqlen, out, cu_k=cu_k)
            return self._gate_out(x, out.view(bsz, seqlen, h, d))
        allow = torch.ones((seqlen, klen), dtype=torch.bool, device=x.device).tril(klen - seqlen)
        allow = allow[None, None].expand(bsz, 1, seqlen, klen)
        if key_pad is not None:
            allow = allow & key_pad[:, None, None, :]
        # fp32 scores for bf16 activations too: torch's batched bf16 products
        # on the transposed key views of the math path are avoided
        ct = torch.float32 if x.dtype == torch.bfloat16 else q_t.dtype
        mask = torch.zeros((bsz, 1, seqlen, klen), dtype=ct, device=x.device)
        mask = mask.masked_fill(~allow, float("-inf"))
        out = F.scaled_dot_product_attention(q_t.to(ct), k_t.to(ct), v_t.to(ct), attn_mask=mask)
        # a query with no key allowed (a pad position of a left-padded prompt)
        # gets zeros, as torch's math path gives, whichever backend ran
        out = out.masked_fill(~allow.any(-1, keepdim=True), 0.0).to(x.dtype)
        return self._gate_out(x, out.transpose(1, 2))

    def _key_mask(self, start_pos: int, bsz: int, k_len: int, device):
        """Which of the ``k_len`` key positions of each row are real tokens, or
        None when all are (the behaviour of attention.py:585-600).

        The rule: a prompt (start_pos 0) takes the pad mask set on the module
        before it ran (``set_pad_mask``); that mask is remembered, and keys
        at later positions (tokens generated after the prompt) are real.  A
        mask longer than ``k_len`` is cut to it.
        """
        if int(start_pos) == 0:
            given = getattr(self, "_pad_mask", None)
            self._prompt_mask = None if given is None else given[:bsz].to(device=device, dtype=torch.bool)
        prompt = getattr(self, "_prompt_mask", None)
        if prompt is None:
            return None
        known = prompt[:bsz, :k_len]
        missing = int(k_len) - int(known.size(1))
        return F.pad(known, (0, missing), value=True) if missing > 0 else known

    def forward_mixed(self, x: torch.Tensor, step: dict) -> torch.Tensor:
        """Packed continuous-batching step (``step`` from Transformer.forward_step).

        Rows [0, R) are prefill tokens of the sequences delimited by
        ``step["cu_prefill"]``; each writes its latent into its slot at its
        position and attends causally over the latents of its own sequence:
        its new tokens, plus the cached ones before them when the sequence
        continues (``step["reads_cache"]``: keys are gathered from the cache).
        The remaining rows are one token each for running sequences at
        positions ``decode_pos`` (int64, device) of slots ``decode_slots``,
        attending to their cached latents 0..pos.

        The decode part attends in latent space: with NoPE, q . (W_k,h c) =
        (W_k,h^T q) . c, so scores and the value sum are taken directly over
        the cached latents c and W_v,h is applied after the sum -- the same
        result as expanding K and V, without recomputing them every step.
        The softmax over the cached latents and their weighted sum run as one
        HIP kernel (``ops.mla_decode_attn``) that reads the fp32 cache in
        place.  ``max_decode_len`` (host int) bounds pos + 1 for every decode
        row; it sizes the kernel's key splits.
        """
        n = int(x.size(0))
        npre = int(step["n_prefill_rows"])
        nd = n - npre
        h, d, r = self.num_heads, self.head_dim, self.kv_rank
        cache = self.latent_cache
        # q_down, kv_down and output_gate in one GEMM; q_norm, kv_norm and the
        # latent-cache writes of every row in one kernel
        y = F.linear(x, self._input_weight(x.dtype))
        q_lat, latent, gate = y[:, :self.q_rank], y[:, self.q_rank:self.q_rank + r], y[:, self.q_rank + r:]
        rect = npre > 0 and bool(step["rectangular"])
        if (self.q_rank % 8 == 0 and r % 8 == 0 and self.q_rank + r <= 512 and int(y.stride(0)) % 8 == 0
                and x.dtype in (torch.float32, torch.bfloat16)):
            ops.mla_latent_norms(
                q_lat, latent, self.q_norm.weight, self.q_norm.eps, self.kv_norm.weight, self.kv_norm.eps,
                latent_cache=cache, n_prefill=npre,
                prefill_seq_slots=step["prefill_slots"] if rect else None,
                prefill_seq_len=int(step["max_prefill_len"]) if rect else 0,
                prefill_row_slots=step["row_slot"] if npre > 0 and not rect else None,
                prefill_row_pos=step["row_pos"] if npre > 0 and not rect else None,
                decode_slots=step["decode_slots"] if nd > 0 else None,
                decode_pos=step["decode_pos"] if nd > 0 else None)
        else:
            # ranks the kernel does not take: the norms and cache writes as torch
            # ops, and the gate copied to dense rows (its columns may start off a
            # 16-byte boundary, which the gate kernel requires)
            q_lat, latent, gate = self.q_norm(q_lat), self.kv_norm(latent), gate.contiguous()
            if npre > 0:
                if rect:
                    T = int(step["max_prefill_len"])
                    cache[step["prefill_slots"].long(), :T] = latent[:npre].view(-1, T, r).to(cache.dtype)
                else:
                    cache[step["row_slot"], step["row_pos"]] = latent[:npre].to(cache.dtype)
            if nd > 0:
                cache[step["decode_slots"].long(), step["decode_pos"]] = latent[npre:].to(cache.dtype)
        q = self.q_up(q_lat).view(n, h, d)
        out = torch.empty((n, h, d), dtype=x.dtype, device=x.device)
        if npre > 0:
            lat_p = latent[:npre]
            cu_k = cu_k_host = None
            lat_k = lat_p
            if not rect:
                if step["reads_cache"]:
                    lat_k = cache[step["key_slot"], step["key_pos"]].to(x.dtype)
                    cu_k, cu_k_host = step["cu_keys"], step["cu_keys_host"]
            k = self.k_up(lat_k).view(-1, h, d)
            v = self.v_up(lat_k).view(-1, h, d)
            self._causal(q[:npre], k, v, step["cu_prefill"], int(step["max_prefill_len"]), out[:npre],
                         cu_k=cu_k, cu_host=step["cu_prefill_host"], cu_k_host=cu_k_host)
        if nd > 0:
            w_k = self.k_up.weight.view(h, d, r).to(x.dtype)
            qa = torch.bmm(q[npre:].transpose(0, 1).contiguous(), w_k).transpose(0, 1)   # [D, h, r]
            # softmax over cached latents 0..pos and their weighted sum, one kernel
            ctx = ops.mla_decode_attn(qa.contiguous(), cache, step["decode_slots"], step["decode_pos"],
                                      d ** -0.5, max_len=int(step["max_decode_len"]))   # [D, h, r]
            o = torch.bmm(ctx.transpose(0, 1).contiguous(), self._v_up_t(x.dtype))
            out[npre:] = o.transpose(0, 1)
        return self._gate_out(x, out, gate)


class FeedForward(nn.Module):
    """SiTU-GLU (blocks.py:12-27)."""

    def __init__(self, args: ModelArgs) -> None:
        super().__init__()
        self.hidden = int(args.ffn_hidden)
        self.gate_softcap = float(args.situ_gate_softcap)
        self.up_softcap = float(args.situ_up_softcap)
        self.gate_up_proj = RuntimeLinear(int(args.dim), 2 * self.hidden)
        self.down_proj = RuntimeLinear(self.hidden, int(args.dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # gate_softcap tanh(g / gate_softcap) sigmoid(g) * up_softcap tanh(u / up_softcap)
        # as one HIP kernel over the fused [gate | up] projection.
        hidden = ops.situ_glu(self.gate_up_proj(x), self.gate_softcap, self.up_softcap)
        return self.down_proj(hidden)


class AttentionResidualMixer(nn.Module):
    """Content-dependent mixing over completed depth blocks and a partial
    block (blocks.py:30-48), as one HIP kernel (ops.attn_res_mix).  Works on
    any leading shape: partial [..., dim], completed [..., blocks, dim]."""

    def __init__(self, args: ModelArgs) -> None:
        super().__init__()
        self.norm = RMSNorm(args.dim, args.norm_eps)
        self.query = RuntimeLinear(args.dim, 1)
        self._query_f32 = None
        self._query_key = None

    def _query(self) -> torch.Tensor:
        """The query as fp32 [dim] (the reference upcasts it per call); kept
        until the weight changes, so that no cast runs per step."""
        w = self.query.weight
        key = (w.data_ptr(), w.dtype, w._version)
        if self._query_key != key:
            self._query_f32 = w.detach().reshape(-1).float().contiguous()
            self._query_key = key
        return self._query_f32

    def forward(self, partial_block: torch.Tensor, completed_blocks: torch.Tensor,
                out_norm: RMSNorm | None = None, *, residual: torch.Tensor | None = None,
                partial_out: torch.Tensor | None = None):
        """The mix; with ``out_norm``, ``out_norm(mix)`` from the same kernel.
        With ``residual``, the partial block is partial_block + residual (added
        in the same kernel) and ``(partial_block + residual, mix)`` is returned,
        the sum written into ``partial_out`` when given."""
        return ops.attn_res_mix(
            partial_block, completed_blocks, self.norm.weight, self._query(), self.norm.eps,
            out_norm_weight=None if out_norm is None else out_norm.weight,
            out_eps=1e-6 if out_norm is None else out_norm.eps, residual=residual,
            partial_out=partial_out)


def _store_slot(completed: torch.Tensor):
    """(completed enlarged by one block, that block's slot) when ``completed``
    is a view of a depth store with room for one more block (rows spaced at
    least one block apart and the storage long enough), else (None, None)."""
    n, dim = int(completed.size(-2)), int(completed.size(-1))
    strides = completed.stride()
    sizes = list(completed.shape)
    sizes[-2] = n + 1
    rows_ok = all(strides[i] >= (n + 1) * dim for i in range(completed.dim() - 2) if sizes[i] > 1)
    if completed.dim() >= 3 and strides[-1] == 1 and strides[-2] == dim and rows_ok:
        extent = completed.storage_offset() + 1 + sum((sz - 1) * st for sz, st in zip(sizes, strides))
        if all(sz > 0 for sz in sizes) and extent * completed.element_size() <= \
                completed.untyped_storage().nbytes():
            grown = completed.as_strided(sizes, strides, completed.storage_offset())
            return grown, grown.select(-2, n)
    return None, None


def _append_block(completed: torch.Tensor, partial: torch.Tensor) -> torch.Tensor:
    """torch.cat((completed, partial.unsqueeze(-2)), dim=-2) (blocks.py:73-76).
    In a depth store with room for one more block the block is written in
    place and the enlarged view returned, so that the earlier blocks are not
    copied again."""
    grown, slot = _store_slot(completed)
    if slot is not None:
        slot.copy_(partial)
        return grown
    return torch.cat((completed, partial.unsqueeze(-2)), dim=-2)


def depth_store(hidden: torch.Tensor, n_layers: int, block_size: int) -> torch.Tensor:
    """An empty ``completed`` view [..., 0, dim] over storage for every depth
    block the layers will append (one per ``block_size`` layers)."""
    n_max = max(1, -(-int(n_layers) // int(block_size)))
    store = hidden.new_empty(*hidden.shape[:-1], n_max, int(hidden.size(-1)))
    return store.narrow(-2, 0, 0)


class SophiaBlock(nn.Module):
    """blocks.py:51-87."""

    def __init__(self, args: ModelArgs, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = int(layer_idx)
        self.layer_type = args.layer_type(self.layer_idx)
        self.attn_norm = RMSNorm(args.dim, args.norm_eps)
        self.attn = SophiaMLA(args) if self.layer_type == "mla" else SophiaKDA(args)
        self.ffn_norm = RMSNorm(args.dim, args.norm_eps)
        self.ffn = FeedForward(args)
        self.attn_res_block_size = int(args.attn_res_block_size)
        self.attn_residual = AttentionResidualMixer(args)
        self.ffn_residual = AttentionResidualMixer(args)

    def _mix(self, partial_block, completed_blocks, attn, pending=None, defer=False):
        """blocks.py:66-87.  ``pending``: an FFN output of the previous layer
        not yet added to ``partial_block``; the add runs inside this layer's
        first depth mix.  With ``defer``, this layer's own FFN output is
        returned unadded as a third value, for the next layer (or the final
        mix) to add the same way.  attn_norm(attn_residual(...)) and
        ffn_norm(ffn_residual(...)) each run as one kernel: the mixes feed
        nothing but these norms."""
        boundary = self.layer_idx % self.attn_res_block_size == 0
        grown = slot = None
        if boundary and pending is not None:
            # the sum partial + pending completes a depth block: the mix
            # writes it straight into the store's next slot
            grown, slot = _store_slot(completed_blocks)
        if pending is None:
            attn_input = self.attn_residual(partial_block, completed_blocks, self.attn_norm)
        else:
            partial_block, attn_input = self.attn_residual(partial_block, completed_blocks,
                                                           self.attn_norm, residual=pending,
                                                           partial_out=slot)
        if boundary:
            completed_blocks = grown if slot is not None else _append_block(completed_blocks, partial_block)
            partial_block = attn(attn_input)
            ffn_input = self.ffn_residual(partial_block, completed_blocks, self.ffn_norm)
        else:
            partial_block, ffn_input = self.ffn_residual(partial_block, completed_blocks,
                                                         self.ffn_norm, residual=attn(attn_input))
        ffn_out = self.ffn(ffn_input)
        if defer:
            return partial_block, completed_blocks, ffn_out
        return partial_block + ffn_out, completed_blocks

    def forward(self, partial_block, completed_blocks, *, start_pos: int = 0, pending=None,
                defer: bool = False):
        return self._mix(partial_block, completed_blocks,
                         lambda y: self.attn(y, start_pos=int(start_pos)), pending, defer)

    def forward_mixed(self, partial_block, completed_blocks, step: dict, *, pending=None,
                      defer: bool = False):
        if self.layer_type == "mla":
            attn = lambda y: self.attn.forward_mixed(y, step)
        else:
            attn = lambda y: self.attn.forward_mixed(
                y, step["n_prefill_rows"], step["cu_prefill"], step["prefill_slots"],
                step["decode_slots"], prefill_reads_cache=step["reads_cache"],
                cu_prefill_host=step["cu_prefill_host"])
        return self._mix(partial_block, completed_blocks, attn, pending, defer)


def init_weights(model: nn.Module, args: ModelArgs) -> None:
    """transformer_setup.py:39-64: N(0, 0.02) for every linear, embedding and
    conv weight; residual-branch outputs at 0.02 / sqrt(2 n_layers); attention
    residual queries zero."""
    base_std = float(args.initializer_range)
    residual_std = base_std / math.sqrt(2.0 * max(int(args.n_layers), 1))
    from .kda import CausalDepthwiseConv1d
    for module in model.modules():
        if isinstance(module, (nn.Linear, RuntimeLinear)):
            nn.init.normal_(module.weight, mean=0.0, std=base_std)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=base_std)
        elif isinstance(module, CausalDepthwiseConv1d):
            nn.init.normal_(module.weight, mean=0.0, std=base_std)
    for layer in getattr(model, "layers", ()):
        nn.init.normal_(layer.attn.o_proj.weight, mean=0.0, std=residual_std)
        nn.init.normal_(layer.ffn.down_proj.weight, mean=0.0, std=residual_std)
        nn.init.zeros_(layer.attn_residual.query.weight)
        nn.init.zeros_(layer.ffn_residual.query.weight)
    nn.init.zeros_(model.output_attn_residual.query.weight)


class Transformer(nn.Module):
    """The [KDA, KDA, KDA, MLA] x (n_layers / 4) hybrid decoder
    (transformer.py:17-207, transformer_setup.py:67-79), tied embedding."""

    def __init__(self, args: ModelArgs) -> None:
        super().__init__()
        self.args = args
        self.tok_embeddings = nn.Embedding(args.vocab_size, args.dim)
        self.layers = nn.ModuleList([SophiaBlock(args, i) for i in range(args.n_layers)])
        self.norm = RMSNorm(args.dim, args.norm_eps)
        self.output_attn_residual = AttentionResidualMixer(args)
        self.output = RuntimeLinear(args.dim, args.vocab_size)
        self.output.weight = self.tok_embeddings.weight  # tie_word_embeddings
        init_weights(self, args)

    def reset_runtime_cache(self) -> None:
        for layer in self.layers:
            layer.attn.reset()

    def cast_weights_(self, dtype: torch.dtype) -> "Transformer":
        """Cast the GEMM weights (every RuntimeLinear and the tied embedding)
        to ``dtype`` in place.  Norm weights, A_log, dt_bias, conv taps and the
        recurrent, conv and latent caches stay fp32, as the reference keeps
        them (attention.py:98-180,469-476)."""
        for module in self.modules():
            if isinstance(module, (RuntimeLinear, nn.Embedding)):
                for param in module.parameters(recurse=False):
                    param.data = param.data.to(dtype)
        return self

    def _validate(self, input_ids: torch.Tensor, start_pos: int) -> None:
        """transformer.py:146-160."""
        if input_ids.dim() != 2:
            raise ValueError("input_ids must be [B, S]")
        if int(start_pos) < 0:
            raise ValueError(f"start_pos must be >= 0, got {start_pos}")
        if int(start_pos) > 0 and int(input_ids.size(1)) > 1:
            raise ValueError("incremental forward accepts one token when start_pos > 0")
        if int(start_pos) + int(input_ids.size(1)) > int(self.args.max_seq_len):
            raise ValueError("sequence exceeds max_seq_len")

    def forward(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
                start_pos: int = 0) -> torch.Tensor:
        """transformer.py:169-207: logits [B, S, vocab].  ``attention_mask`` is
        taken and type-checked as the reference's forward does, and, as there,
        not used: padding reaches the mixers through ``set_pad_mask``."""
        if attention_mask is not None and not torch.is_tensor(attention_mask):
            raise TypeError("attention_mask must be a tensor or None")
        _require_gpu(input_ids)
        self._validate(input_ids, start_pos)
        if self.args.use_cache:
            self.ensure_batch_capacity(int(input_ids.size(0)))
        hidden = self.tok_embeddings(input_ids)
        completed = depth_store(hidden, self.args.n_layers, self.args.attn_res_block_size)
        pending = None  # each layer's FFN output is added inside the next depth mix
        for layer in self.layers:
            hidden, completed, pending = layer(hidden, completed, start_pos=start_pos,
                                               pending=pending, defer=True)
        return self.output(self._final_mix(hidden, completed, pending))

    def forward_full(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
                     start_pos: int = 0) -> torch.Tensor:
        """transformer.py:212-218: the same as ``forward``."""
        return self.forward(input_ids, attention_mask=attention_mask, start_pos=start_pos)

    def _forward_hidden(self, input_ids: torch.Tensor, start_pos: int) -> torch.Tensor:
        """The final depth mix before the output norm (transformer.py:169-199)."""
        _require_gpu(input_ids)
        self._validate(input_ids, start_pos)
        if self.args.use_cache:
            self.ensure_batch_capacity(int(input_ids.size(0)))
        hidden = self.tok_embeddings(input_ids)
        completed = depth_store(hidden, self.args.n_layers, self.args.attn_res_block_size)
        pending = None
        for layer in self.layers:
            hidden, completed, pending = layer(hidden, completed, start_pos=start_pos,
                                               pending=pending, defer=True)
        if pending is None:
            return self.output_attn_residual(hidden, completed)
        return self.output_attn_residual(hidden, completed, residual=pending)[1]

    def forward_with_last_hidden(self, input_ids: torch.Tensor, start_pos: int = 0,
                                 return_all_logits: bool = True):
        """runtime_host.py:115-143: (logits, the last position's final mix
        [B, dim]); logits [B, S, vocab], or [B, vocab] of the last position
        when ``return_all_logits`` is False."""
        mix = self._forward_hidden(input_ids, int(start_pos))
        last_hidden = mix[:, -1, :]
        head = mix if return_all_logits else mix[:, -1:, :]
        logits = self.output(self.norm(head))
        return (logits if return_all_logits else logits[:, 0, :]), last_hidden

    def replay_with_cache(self, input_ids: torch.Tensor, start_pos: int = 0,
                          return_all_logits: bool = True):
        """runtime_host.py:146-170: a prompt (start_pos 0) or one token in one
        pass; several tokens after cached ones one at a time (the incremental
        forward takes one token), their logits concatenated."""
        if int(input_ids.size(1)) <= 1 or int(start_pos) == 0:
            return self.forward_with_last_hidden(input_ids, int(start_pos), return_all_logits)
        outputs, last_hidden = [], None
        for offset in range(int(input_ids.size(1))):
            logits, last_hidden = self.forward_with_last_hidden(input_ids[:, offset:offset + 1],
                                                                int(start_pos) + offset, True)
            outputs.append(logits)
        combined = torch.cat(outputs, dim=1)
        return (combined if return_all_logits else combined[:, -1, :]), last_hidden

    def _final_mix(self, hidden, completed, pending):
        """norm(output_attn_residual(hidden + pending, completed)) as one kernel."""
        if pending is None:
            return self.output_attn_residual(hidden, completed, self.norm)
        return self.output_attn_residual(hidden, completed, self.norm, residual=pending)[1]

    # ------------------------------------------------------------- runtime caches
    def runtime_batch_capacity(self) -> int:
        """Cache slots every layer holds."""
        return min(int(layer.attn.recurrent_state.size(0)) if layer.layer_type == "kda"
                   else int(layer.attn.latent_cache.size(0)) for layer in self.layers)

    def ensure_batch_capacity(self, batch_size: int) -> None:
        """Grow every layer's caches to at least ``batch_size`` slots, keeping
        the cached rows (the reference grows them on demand,
        test_dynamic_batch_capacity.py:29-51)."""
        required = self.args.ensure_runtime_batch_capacity(int(batch_size))
        for layer in self.layers:
            layer.attn.ensure_batch_capacity(required)

    def reset_slots(self, slots: torch.Tensor) -> None:
        """Zero the KDA recurrent state and conv history of cache slots
        ``slots`` in every layer (new sequences; MLA latents need no reset:
        attention never reads past a sequence's own length)."""
        for layer in self.layers:
            if layer.layer_type == "kda":
                layer.attn.reset_slots(slots)

    def cache_dump(self, *, device: str = "cpu", cache_pos: int | None = None,
                   batch_size: int | None = None,
                   slots: torch.Tensor | None = None) -> RuntimeCacheSnapshot:
        """Copies of every layer's caches (runtime_host.py:179-194): rows
        [:batch_size] (default: every slot), or the cache slots ``slots`` in
        that order; MLA latents up to ``cache_pos``."""
        if slots is None:
            active = self.runtime_batch_capacity() if batch_size is None else int(batch_size)
            if active <= 0:
                raise ValueError(f"batch_size must be >= 1, got {active}")
            self.ensure_batch_capacity(active)
        else:
            active = int(slots.numel())
        return RuntimeCacheSnapshot(layers=tuple(
            layer.attn.cache_snapshot(device=device, batch_size=active, cache_pos=cache_pos, slots=slots)
            for layer in self.layers))

    def cache_load(self, cache_snapshot: RuntimeCacheSnapshot, *,
                   slots: torch.Tensor | None = None) -> None:
        """Load a snapshot (runtime_host.py:196-212): every layer's snapshot is
        validated first, then all caches are reset and loaded into rows
        [:batch].  With ``slots``, snapshot row i goes to cache slot slots[i]
        and every other slot keeps its contents (no reset)."""
        if not isinstance(cache_snapshot, RuntimeCacheSnapshot):
            raise TypeError("cache snapshot must be a RuntimeCacheSnapshot")
        if len(cache_snapshot.layers) > len(self.layers):
            raise ValueError("cache snapshot has more layers than the model")
        if slots is not None and int(slots.numel()) != cache_snapshot.batch_size():
            raise ValueError(f"{int(slots.numel())} slots for a snapshot of "
                             f"{cache_snapshot.batch_size()} rows")
        required = cache_snapshot.batch_size() if slots is None else \
            (int(slots.max()) + 1 if slots.numel() else 0)
        if required:
            self.ensure_batch_capacity(required)
        for index, snapshot in enumerate(cache_snapshot.layers):
            if snapshot is not None:
                self.layers[index].attn.validate_cache_snapshot(snapshot)
        if slots is None:
            self.reset_runtime_cache()
        for index, snapshot in enumerate(cache_snapshot.layers):
            if snapshot is not None:
                self.layers[index].attn.load_cache_snapshot(snapshot, slots=slots)

    # ------------------------------------------------------------- packed steps
    def forward_step(self, *, prefill_ids: torch.Tensor | None = None, prefill_lens=(),
                     prefill_pos=None, prefill_slots: torch.Tensor | None = None,
                     decode_ids: torch.Tensor | None = None,
                     decode_slots: torch.Tensor | None = None,
                     decode_pos: torch.Tensor | None = None,
                     max_decode_len: int = 0, all_logits: bool = False) -> torch.Tensor:
        """One continuous-batching step over packed rows, which the reference
        cannot express (one start_pos per batch there, T > 1 only at
        start_pos 0, transformer.py:146-160).

        Prefill part: ``prefill_ids`` [sum(prefill_lens)] int64 holds the new
        tokens of len(prefill_lens) sequences back to back (any lengths >= 1),
        sequence i in cache slot ``prefill_slots[i]`` (int32, device) with
        ``prefill_pos[i]`` tokens already cached (host ints; 0 = a new
        sequence, whose KDA caches are zeroed here; > 0 = a prefill that
        continues, reading its slot's caches: a long prompt is prefilled in
        pieces across steps).  Decode part: ``decode_ids`` [D] one token for
        each running sequence, slots ``decode_slots`` [D] int32, positions
        ``decode_pos`` [D] int64 (tokens already cached, on the device), and
        ``max_decode_len`` (host int) bounding pos + 1.

        Returns the logits of each sequence's last token, [N + D, vocab]
        (prefill sequences first); with ``all_logits``, of every row,
        [sum(prefill_lens) + D, vocab].  With equal lengths and no continuation
        nothing is copied from the host, so the step is capturable
        (MixedStepGraph); otherwise small index tensors are built on the host.
        """
        dev = self.tok_embeddings.weight.device
        lens = [int(t) for t in prefill_lens]
        n_p = len(lens)
        pos = [0] * n_p if prefill_pos is None else [int(p) for p in prefill_pos]
        if len(pos) != n_p:
            raise ValueError("prefill_pos needs one entry per prefill sequence")
        if any(t < 1 for t in lens) or any(p < 0 for p in pos):
            raise ValueError("prefill lengths must be >= 1 and positions >= 0")
        if any(p + t > int(self.args.max_seq_len) for p, t in zip(pos, lens)):
            raise ValueError("a prefill sequence exceeds max_seq_len")
        rows = sum(lens)
        if n_p and (prefill_ids is None or int(prefill_ids.numel()) != rows or prefill_slots is None
                    or int(prefill_slots.numel()) != n_p):
            raise ValueError("prefill_ids must hold sum(prefill_lens) tokens and prefill_slots one "
                             "slot per sequence")
        D = 0 if decode_ids is None else int(decode_ids.numel())
        if D and (decode_slots is None or decode_pos is None or int(decode_slots.numel()) != D
                  or int(decode_pos.numel()) != D):
            raise ValueError("decode_slots and decode_pos need one entry per decode token")
        if n_p + D == 0:
            raise ValueError("empty step")
        if D and not 1 <= int(max_decode_len) <= int(self.args.max_seq_len):
            # decode rows write their latent at pos < max_decode_len: checked
            # here, before any launch (transformer.py:155-160 raises the same)
            raise ValueError("sequence exceeds max_seq_len" if int(max_decode_len) > 0
                             else "max_decode_len must bound pos + 1 of every decode row")
        _require_gpu(prefill_ids if n_p else decode_ids)
        reads = any(p > 0 for p in pos)
        rect = n_p > 0 and not reads and min(lens) == max(lens)
        step = dict(n_prefill_rows=rows, n_prefill_seqs=n_p, max_prefill_len=max(lens, default=0),
                    prefill_slots=prefill_slots, reads_cache=reads, rectangular=rect,
                    decode_slots=decode_slots, decode_pos=decode_pos,
                    max_decode_len=int(max_decode_len), cu_prefill=None, cu_prefill_host=None)
        if n_p and rect:
            T = lens[0]
            step["cu_prefill"] = torch.arange(0, (n_p + 1) * T, T, dtype=torch.int32, device=dev)
            last_pre = torch.arange(T - 1, n_p * T, T, device=dev)
        elif n_p:
            cu_host = torch.tensor([0] + list(itertools.accumulate(lens)), dtype=torch.int32)
            step["cu_prefill_host"] = cu_host
            step["cu_prefill"] = cu_host.to(dev)
            seq_of_row = torch.repeat_interleave(torch.arange(n_p), torch.tensor(lens)).to(dev)
            step["row_slot"] = prefill_slots.long()[seq_of_row]
            step["row_pos"] = torch.cat([torch.arange(p, p + t) for p, t in zip(pos, lens)]).to(dev)
            if reads:
                klens = [p + t for p, t in zip(pos, lens)]
                cuk_host = torch.tensor([0] + list(itertools.accumulate(klens)), dtype=torch.int32)
                step["cu_keys_host"] = cuk_host
                step["cu_keys"] = cuk_host.to(dev)
                seq_of_key = torch.repeat_interleave(torch.arange(n_p), torch.tensor(klens)).to(dev)
                step["key_slot"] = prefill_slots.long()[seq_of_key]
                step["key_pos"] = torch.cat([torch.arange(kl) for kl in klens]).to(dev)
                new = [i for i in range(n_p) if pos[i] == 0]
                if new:
                    self.reset_slots(prefill_slots.long()[torch.tensor(new, device=dev)])
            last_pre = (cu_host[1:].long() - 1).to(dev)
        ids = []
        if n_p:
            ids.append(prefill_ids.reshape(-1))
        if D:
            ids.append(decode_ids.reshape(-1))
        ids = torch.cat(ids) if len(ids) > 1 else ids[0]
        hidden = self.tok_embeddings(ids)
        completed = depth_store(hidden, self.args.n_layers, self.args.attn_res_block_size)
        pending = None
        for layer in self.layers:
            hidden, completed, pending = layer.forward_mixed(hidden, completed, step,
                                                             pending=pending, defer=True)
        if all_logits:
            return self.output(self._final_mix(hidden, completed, pending))
        parts = []
        if n_p:
            parts.append(last_pre)
        if D:
            parts.append(torch.arange(rows, rows + D, device=hidden.device))
        last = torch.cat(parts) if len(parts) > 1 else parts[0]
        return self.output(self._final_mix(hidden[last], completed[last],
                                           None if pending is None else pending[last]))

    def forward_mixed(self, prefill_ids: torch.Tensor, decode_ids: torch.Tensor, *,
                      prefill_slots: torch.Tensor, decode_slots: torch.Tensor,
                      decode_pos: torch.Tensor, max_decode_len: int,
                      cu_prefill: torch.Tensor | None = None) -> torch.Tensor:
        """``forward_step`` for ``prefill_ids`` [P, Tp]: P new sequences of Tp
        tokens each (cache slots ``prefill_slots`` [P] int32), plus
        ``decode_ids`` [D] as in forward_step.  Nothing is read back on the
        host, so the step is capturable (MixedStepGraph).  ``cu_prefill`` is
        accepted for compatibility and must be the offsets of that rectangle.
        Returns [P + D, vocab]."""
        del cu_prefill
        P, T = int(prefill_ids.size(0)), int(prefill_ids.size(1))
        return self.forward_step(prefill_ids=prefill_ids if P else None, prefill_lens=[T] * P,
                                 prefill_slots=prefill_slots, decode_ids=decode_ids,
                                 decode_slots=decode_slots, decode_pos=decode_pos,
                                 max_decode_len=max_decode_len)


class MixedStepGraph:
    """A captured ``Transformer.forward_mixed`` step with static inputs.

    Warm-up runs on a side stream, then one capture (the pattern of
    sm120_graph_runner.py:318-371); ``run`` copies the step's inputs into the
    static buffers and replays.  Every call advances the caches of the
    sequences it names, like the eager step.
    """

    def __init__(self, model: Transformer, n_prefill_seqs: int, prefill_len: int,
                 n_decode: int, max_decode_len: int, *, warmup: int = 2,
                 example: dict | None = None) -> None:
        dev = model.tok_embeddings.weight.device
        self.model = model
        self.max_decode_len = int(max_decode_len)
        P, T, D = int(n_prefill_seqs), int(prefill_len), int(n_decode)
        self.prefill_ids = torch.zeros((P, T), dtype=torch.long, device=dev)
        self.decode_ids = torch.zeros((D,), dtype=torch.long, device=dev)
        self.prefill_slots = torch.zeros((P,), dtype=torch.int32, device=dev)
        self.decode_slots = torch.zeros((D,), dtype=torch.int32, device=dev)
        self.decode_pos = torch.zeros((D,), dtype=torch.long, device=dev)
        self.cu_prefill = torch.arange(0, (P + 1) * T, T, dtype=torch.int32, device=dev)
        if example is not None:
            self._load(example)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(int(warmup)):
                self._step()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.logits = self._step()

    def _step(self) -> torch.Tensor:
        return self.model.forward_mixed(
            self.prefill_ids, self.decode_ids, prefill_slots=self.prefill_slots,
            decode_slots=self.decode_slots, decode_pos=self.decode_pos,
            max_decode_len=self.max_decode_len, cu_prefill=self.cu_prefill)

    def _load(self, inputs: dict) -> None:
        for name in ("prefill_ids", "decode_ids", "prefill_slots", "decode_slots", "decode_pos"):
            if name in inputs:
                getattr(self, name).copy_(inputs[name], non_blocking=True)

    def run(self, **inputs) -> torch.Tensor:
        """Copy the given inputs (same names and shapes as the buffers) and
        replay; returns the static logits buffer [P + D, vocab]."""
        self._load(inputs)
        self.graph.replay()
        return self.logits


__all__ = ["AttentionResidualMixer", "FeedForward", "MixedStepGraph", "SophiaBlock",
           "SophiaMLA", "Transformer", "init_weights"]
