"""The KDA token mixer on MI355X: a drop-in for the reference's ``SophiaKDA``.

Same parameter names, shapes and initialisation order as
ml/runtime/model/attention.py:66-143 (so a reference state_dict loads as is
and seeded initialisation draws the same stream), the same cache buffers and
cache/snapshot methods (attention.py:145-224), and the same
``forward(x, *, start_pos)`` semantics including the pad mask
(attention.py:373-420, 660-670).  ``forward_packed`` adds the packed ragged
entry (cu_seqlens + cache slots) used for continuous batching.

Compute: the input projections run as one fused GEMM (q|k|v|decay_down|beta|
output_gate, hipBLASLt through torch), the ShortConv and the KDA core run in
the gfx950 HIP kernels of ``sophia_amd/csrc`` (chunk-64 prefill, in-place
decode step), then RMSNorm * sigmoid(gate) and o_proj.  Tensors on the CPU are
rejected: the per-token reference recurrence is not part of this package.
"""

from __future__ import annotations

import functools
import math

import torch
import torch.nn.functional as F
from torch import nn

from . import ops, torch_ops
from .config import ModelArgs
from .state import LayerCacheSnapshot

PAD_LOGIT = -1.0e4  # attention.py:17
# Rows of the fused input projection are padded to a multiple of this many
# output columns (64 bf16 = one 128-byte line).
_PROJ_ROWS = 64


def _inverse_softplus(value: torch.Tensor) -> torch.Tensor:
    """attention.py:20-21."""
    return value + torch.log(-torch.expm1(-value))


def _require_gpu(x: torch.Tensor) -> None:
    if x.device.type != "cuda":
        raise RuntimeError(
            "sophia_amd KDA runs on a ROCm GPU only; move the module and inputs to 'cuda' "
            "(the per-token CPU recurrence is the test oracle, not a product path)")


class RuntimeLinear(nn.Module):
    """Bias-free linear with N(0, 0.02) init (ml/runtime/model/runtime_linear.py:10-33)."""

    def __init__(self, in_features: int, out_features: int, *, bias: bool = False) -> None:
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.weight = nn.Parameter(torch.empty(self.out_features, self.in_features))
        self.bias = nn.Parameter(torch.empty(self.out_features)) if bias else None
        nn.init.normal_(self.weight, mean=0.0, std=0.02)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.weight, self.bias)


class RMSNorm(nn.Module):
    """ops.py:49-64: functional.rms_norm over the last dim, fp32 weight."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.float32))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (int(x.size(-1)),), self.weight.to(x.dtype), float(self.eps))


def _needs_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def conv_forward(weight: torch.Tensor, kernel_size: int, x: torch.Tensor,
                 history: torch.Tensor | None = None):
    """CausalDepthwiseConv1d.forward (attention.py:32-60) on the HIP ShortConv:
    x [B, T, C], history [B, C, K-1] or None -> (silu(conv) [B, T, C],
    next_history [B, C, K-1] in x.dtype).  When x or the weight requires grad,
    it runs the functional ``sophia::short_conv`` (autograd: dx and dweight
    by sophia_short_conv_bwd) and next_history is the slice of cat(history, x)
    the reference returns (differentiable in x; the history itself gets no
    gradient); otherwise one launch writes next_history too."""
    _require_gpu(x)
    bsz, seqlen, channels = x.shape
    hist_len = int(kernel_size) - 1
    flat = x.reshape(bsz * seqlen, channels)
    cu = ops.cu_for_batch(bsz, seqlen, x.device)
    if _needs_grad(x, weight):
        hist = None
        if hist_len > 0 and history is not None:
            hist = history.detach().to(dtype=x.dtype).float().contiguous()
        y = torch_ops.short_conv(flat, weight, cu, hist, None, hist is not None, False)
        if hist_len > 0:
            prev = hist.to(x.dtype) if hist is not None else x.new_zeros((bsz, channels, hist_len))
            nxt = torch.cat((prev, x.transpose(1, 2)[..., -hist_len:]), dim=-1)[..., -hist_len:]
        else:
            nxt = x.new_zeros((bsz, channels, 0))
        return y.view(bsz, seqlen, channels), nxt
    state = None
    if hist_len > 0:
        state = torch.zeros((bsz, channels, hist_len), dtype=torch.float32, device=x.device)
        if history is not None:
            state.copy_(history.to(dtype=x.dtype).float())
    y = torch_ops.short_conv_fwd(flat, weight.detach(), cu, state, None,
                                 history is not None and hist_len > 0, hist_len > 0, False)
    next_history = (state.to(x.dtype) if state is not None
                    else x.new_zeros((bsz, channels, 0)))
    return y.view(bsz, seqlen, channels), next_history


class CausalDepthwiseConv1d(nn.Module):
    """attention.py:24-60 on the HIP ShortConv kernel."""

    def __init__(self, channels: int, kernel_size: int) -> None:
        super().__init__()
        self.channels = int(channels)
        self.kernel_size = int(kernel_size)
        self.weight = nn.Parameter(torch.empty(self.channels, self.kernel_size))
        nn.init.normal_(self.weight, mean=0.0, std=0.02)

    def forward(self, x: torch.Tensor, *, history: torch.Tensor | None = None):
        """x: [B, T, C]; history: [B, C, K-1] or None.  Returns
        (silu(conv) [B, T, C], next_history [B, C, K-1] in x.dtype);
        differentiable in x and the weight (``conv_forward``)."""
        return conv_forward(self.weight, self.kernel_size, x, history)


class SophiaKDA(nn.Module):
    """Kimi Delta Attention mixer (attention.py:63-420) on gfx950 kernels."""

    def __init__(self, args: ModelArgs) -> None:
        super().__init__()
        self.dim = int(args.dim)
        self.num_heads = int(args.num_heads)
        self.head_dim = int(args.head_dim)
        self.inner_dim = self.num_heads * self.head_dim
        self.decay_rank = int(args.kda_decay_rank)
        self.output_gate_rank = int(args.kda_output_gate_rank)
        self.output_gate_full_rank = bool(args.kda_output_gate_full_rank)
        self.lower_bound = float(args.kda_decay_lower_bound)
        self.dt_min = float(args.kda_dt_min)
        self.dt_max = float(args.kda_dt_max)
        self.dt_floor = float(args.kda_dt_floor)
        self.backend = str(args.kda_backend)
        self.use_cache = bool(args.use_cache)
        self.conv_kernel = int(args.short_conv_kernel)
        self.norm_eps = float(args.norm_eps)

        # Parameter creation order = the reference's RNG draw order.
        self.q_proj = RuntimeLinear(self.dim, self.inner_dim)
        self.k_proj = RuntimeLinear(self.dim, self.inner_dim)
        self.v_proj = RuntimeLinear(self.dim, self.inner_dim)
        self.q_conv = CausalDepthwiseConv1d(self.inner_dim, self.conv_kernel)
        self.k_conv = CausalDepthwiseConv1d(self.inner_dim, self.conv_kernel)
        self.v_conv = CausalDepthwiseConv1d(self.inner_dim, self.conv_kernel)
        self.decay_down = RuntimeLinear(self.dim, self.decay_rank)
        self.decay_up = RuntimeLinear(self.decay_rank, self.inner_dim)
        self.beta_proj = RuntimeLinear(self.dim, self.num_heads)
        self.A_log = nn.Parameter(torch.full((self.num_heads,), float(args.kda_a_log_init),
                                             dtype=torch.float32))
        dt = torch.exp(torch.rand(self.inner_dim, dtype=torch.float32)
                       * (math.log(self.dt_max) - math.log(self.dt_min))
                       + math.log(self.dt_min)).clamp_min(self.dt_floor)
        self.dt_bias = nn.Parameter(_inverse_softplus(dt))
        self.A_log._no_weight_decay = True  # type: ignore[attr-defined]
        self.dt_bias._no_weight_decay = True  # type: ignore[attr-defined]
        if self.output_gate_full_rank:
            self.output_gate = RuntimeLinear(self.dim, self.inner_dim)
        else:
            self.output_gate_down = RuntimeLinear(self.dim, self.output_gate_rank)
            self.output_gate_up = RuntimeLinear(self.output_gate_rank, self.inner_dim)
        self.output_norm = RMSNorm(self.head_dim, args.norm_eps)
        self.o_proj = RuntimeLinear(self.inner_dim, self.dim)

        self.register_buffer("recurrent_state", torch.zeros(
            int(args.max_batch_size), self.num_heads, self.head_dim, self.head_dim,
            dtype=torch.float32), persistent=False)
        self.register_buffer("conv_state", torch.zeros(
            int(args.max_batch_size), 3, self.inner_dim, self.conv_kernel - 1,
            dtype=torch.float32), persistent=False)
        self._fused_cache: dict[str, tuple[tuple, torch.Tensor]] = {}

    # ------------------------------------------------------------- caches
    def ensure_batch_capacity(self, batch_size: int) -> None:
        """attention.py:145-158."""
        required = int(batch_size)
        if required <= int(self.recurrent_state.size(0)):
            return
        recurrent = self.recurrent_state.new_zeros(required, self.num_heads, self.head_dim,
                                                   self.head_dim)
        recurrent[: self.recurrent_state.size(0)].copy_(self.recurrent_state)
        conv = self.conv_state.new_zeros(required, 3, self.inner_dim, self.conv_kernel - 1)
        conv[: self.conv_state.size(0)].copy_(self.conv_state)
        self.recurrent_state = recurrent
        self.conv_state = conv

    def ensure_sequence_capacity(self, max_seq_len: int) -> None:
        del max_seq_len  # the recurrent state does not grow with length

    def rebuild_runtime_buffers(self, max_seq_len: int) -> None:
        del max_seq_len
        device = self.q_proj.weight.device
        self.recurrent_state = torch.zeros(int(self.recurrent_state.size(0)), self.num_heads,
                                           self.head_dim, self.head_dim, device=device,
                                           dtype=torch.float32)
        self.conv_state = torch.zeros(int(self.conv_state.size(0)), 3, self.inner_dim,
                                      self.conv_kernel - 1, device=device, dtype=torch.float32)

    def reset(self) -> None:
        if self.recurrent_state.is_inference() or self.conv_state.is_inference():
            self.recurrent_state = torch.zeros_like(self.recurrent_state)
            self.conv_state = torch.zeros_like(self.conv_state)
        else:
            self.recurrent_state.zero_()
            self.conv_state.zero_()

    def refresh_state_buffers(self) -> None:
        self.rebuild_runtime_buffers(0)

    def reset_slots(self, slots: torch.Tensor) -> None:
        """Zero the recurrent and conv caches of the given slots (new sequences)."""
        idx = slots.to(device=self.recurrent_state.device, dtype=torch.long)
        self.recurrent_state.index_fill_(0, idx, 0.0)
        self.conv_state.index_fill_(0, idx, 0.0)

    def cache_snapshot(self, *, device: str, batch_size: int, cache_pos: int | None,
                       slots: torch.Tensor | None = None):
        """Copies of the caches of rows [:batch_size] (attention.py:212-216), or
        of the cache slots ``slots`` in that order."""
        del cache_pos
        if slots is not None:
            idx = slots.to(device=self.recurrent_state.device, dtype=torch.long)
            return LayerCacheSnapshot(recurrent=self.recurrent_state.index_select(0, idx).to(device),
                                      conv=self.conv_state.index_select(0, idx).to(device))
        return LayerCacheSnapshot(recurrent=self.recurrent_state[:batch_size].to(device).clone(),
                                  conv=self.conv_state[:batch_size].to(device).clone())

    def validate_cache_snapshot(self, snapshot: LayerCacheSnapshot) -> None:
        if snapshot.latent is not None:
            raise ValueError("KDA cache cannot contain MLA latent state")
        if (snapshot.recurrent is not None
                and tuple(snapshot.recurrent.shape[1:]) != tuple(self.recurrent_state.shape[1:])):
            raise ValueError("KDA recurrent cache shape mismatch")
        if (snapshot.conv is not None
                and tuple(snapshot.conv.shape[1:]) != tuple(self.conv_state.shape[1:])):
            raise ValueError("KDA convolution cache shape mismatch")

    def load_cache_snapshot(self, snapshot: LayerCacheSnapshot, *,
                            slots: torch.Tensor | None = None) -> None:
        """attention.py:218-224; with ``slots``, row i of the snapshot goes to
        cache slot slots[i] and the other slots are left as they are."""
        self.validate_cache_snapshot(snapshot)
        if slots is not None:
            idx = slots.to(device=self.recurrent_state.device, dtype=torch.long)
            if snapshot.recurrent is not None:
                self.recurrent_state.index_copy_(
                    0, idx, snapshot.recurrent.to(self.recurrent_state.device, dtype=torch.float32))
            if snapshot.conv is not None:
                self.conv_state.index_copy_(
                    0, idx, snapshot.conv.to(self.conv_state.device, dtype=torch.float32))
            return
        required = snapshot.batch_size()
        self.ensure_batch_capacity(required)
        if snapshot.recurrent is not None:
            self.recurrent_state[:required].copy_(
                snapshot.recurrent.to(self.recurrent_state.device, dtype=torch.float32))
        if snapshot.conv is not None:
            self.conv_state[:required].copy_(
                snapshot.conv.to(self.conv_state.device, dtype=torch.float32))

    # ------------------------------------------------------------- fused weights
    def _cached(self, key: str, params: tuple[torch.Tensor, ...], build, dtype: torch.dtype):
        if torch.compiler.is_compiling():
            # Traced graphs rebuild the fused weight (no identity stamps there).
            with torch.no_grad():
                return build().to(dtype).contiguous()
        stamp = tuple((p.data_ptr(), p._version) for p in params) + (dtype,)
        hit = self._fused_cache.get(key)
        if hit is not None and hit[0] == stamp:
            return hit[1]
        with torch.no_grad():
            value = build().to(dtype).contiguous()
        self._fused_cache[key] = (stamp, value)
        return value

    def _input_weight(self, dtype: torch.dtype) -> torch.Tensor:
        """[3*inner + (inner | gate_rank) + decay_rank + heads, dim], padded
        with zero rows to a multiple of _PROJ_ROWS: every projection of x in
        one GEMM, whose bf16 output rows then start on 128-byte boundaries, so
        that a head's 256 bytes of q, k or v are two whole cache lines for the
        kernels that copy them (the fused-conv prefill).  The q|k|v and gate
        columns come first, at multiples of 64 columns, because the ShortConv
        and gated-norm kernels read them with 16-byte vector loads."""
        mods = [self.q_proj, self.k_proj, self.v_proj,
                self.output_gate if self.output_gate_full_rank else self.output_gate_down,
                self.decay_down, self.beta_proj]
        params = tuple(m.weight for m in mods)

        def build(parts):
            w = torch.cat(parts, 0)
            pad = (-int(w.size(0))) % _PROJ_ROWS
            return torch.cat([w, w.new_zeros(pad, w.size(1))], 0) if pad else w

        if _needs_grad(*params):   # training: the fused weight is rebuilt each call, with autograd
            return build(params).to(dtype)
        return self._cached("in", params, lambda: build([p.detach() for p in params]), dtype)

    def _conv_weight(self, dtype: torch.dtype) -> torch.Tensor:
        """The q|k|v conv taps [3*inner, K] rounded to the activation dtype and
        held as fp32 (what the ShortConv kernels take), rebuilt only when a
        weight changes."""
        params = (self.q_conv.weight, self.k_conv.weight, self.v_conv.weight)
        if _needs_grad(*params):
            return torch.cat(params, 0).to(dtype).float().contiguous()
        return self._cached(f"conv_{dtype}", params,
                            lambda: torch.cat([p.detach() for p in params], 0).to(dtype),
                            torch.float32)

    def _project(self, x2: torch.Tensor):
        """x2: [N, dim] -> views (qkv [N, 3*inner], decay_down, beta, gate_logits)."""
        y = F.linear(x2, self._input_weight(x2.dtype))
        i, r, h = self.inner_dim, self.decay_rank, self.num_heads
        g = i if self.output_gate_full_rank else self.output_gate_rank
        qkv = y[:, : 3 * i]
        gate = y[:, 3 * i: 3 * i + g]
        dd = y[:, 3 * i + g: 3 * i + g + r]
        beta = y[:, 3 * i + g + r: 3 * i + g + r + h]
        if not self.output_gate_full_rank:
            gate = self.output_gate_up(gate)
        return qkv, dd, beta, gate

    # ------------------------------------------------------------- kernel seam
    @staticmethod
    def _fla_chunk_kda():
        """Chunk prefill callable (seam of attention.py:305-312)."""
        return ops.chunk_kda

    @staticmethod
    def _fla_fused_recurrent_kda():
        """One-token recurrent step (seam of attention.py:296-303); updates the
        cached state in place, the mixer's copy-back then has nothing to do."""
        return functools.partial(ops.fused_recurrent_kda, inplace_state=True)

    def _run_kda(self, q, k, v, decay_logits, beta_logits, initial_state):
        """attention.py:314-371 with the HIP kernels behind the same seam."""
        if self.backend == "reference":
            raise RuntimeError("kda_backend='reference' selects the per-token CPU recurrence, "
                               "which sophia_amd does not ship (it is the test oracle)")
        _require_gpu(q)
        if int(q.size(1)) == 1 and initial_state is not None:
            return self._fla_fused_recurrent_kda()(
                q=q, k=k, v=v, g=decay_logits, beta=beta_logits, A_log=self.A_log,
                dt_bias=self.dt_bias, initial_state=initial_state, output_final_state=True,
                use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                use_beta_sigmoid_in_kernel=True, lower_bound=self.lower_bound)
        output, final_state = self._fla_chunk_kda()(
            q=q, k=k, v=v, g=decay_logits, beta=beta_logits, initial_state=initial_state,
            output_final_state=bool(self.use_cache), use_qk_l2norm_in_kernel=True,
            use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, safe_gate=True,
            lower_bound=self.lower_bound, A_log=self.A_log, dt_bias=self.dt_bias)
        if final_state is None:
            final_state = q.new_zeros(int(q.size(0)), self.num_heads, self.head_dim,
                                      self.head_dim, dtype=torch.float32)
        return output, final_state

    # ------------------------------------------------------------- forward
    def _short_convolution_flat(self, qkv: torch.Tensor, cu: torch.Tensor, slots, *,
                                read: bool, write: bool, step: bool) -> torch.Tensor:
        """All three ShortConvs (q|k|v channels) in one launch; conv_state[:, i]
        is the history of projection i (attention.py:226-258)."""
        state = self.conv_state.view(self.conv_state.size(0), 3 * self.inner_dim,
                                     self.conv_kernel - 1) if self.conv_kernel > 1 else None
        conv_w = self._conv_weight(qkv.dtype)
        if _needs_grad(qkv, conv_w):
            # Training: the functional conv (autograd), reading a copy of the
            # history it convolves; the cache is then updated without grad.
            hist = state.clone() if (read and state is not None) else None
            y = torch_ops.short_conv(qkv, conv_w, cu, hist, slots, hist is not None, True)
            if write and state is not None:
                with torch.no_grad():
                    if step:
                        torch_ops.short_conv_step(qkv.detach(), conv_w.detach(), state, slots, read, True)
                    else:
                        torch_ops.short_conv_fwd(qkv.detach(), conv_w.detach(), cu, state, slots, read, True,
                                                 True)
            return y
        if step:
            return torch_ops.short_conv_step(qkv, conv_w, state, slots, read, True)
        return torch_ops.short_conv_fwd(qkv, conv_w, cu, state, slots, read, write, True)

    def _output(self, o: torch.Tensor, gate_logits: torch.Tensor, dtype) -> torch.Tensor:
        """attention.py:411-420: o_proj(RMSNorm(o) * sigmoid(gate)), the gated
        per-head norm as one HIP kernel (ops.gated_head_norm)."""
        if gate_logits.dtype != dtype:
            gate_logits = gate_logits.to(dtype)
        out = torch_ops.gated_head_norm(o, gate_logits, self.output_norm.weight,
                                        self.num_heads, self.head_dim, float(self.output_norm.eps))
        return self.o_proj(out)

    def forward(self, x: torch.Tensor, *, start_pos: int = 0) -> torch.Tensor:
        """attention.py:373-420."""
        _require_gpu(x)
        bsz, seqlen, _ = x.shape
        if self.use_cache:
            self.ensure_batch_capacity(int(bsz))
        pad_mask = getattr(self, "_pad_mask", None) if int(start_pos) == 0 else None
        if pad_mask is not None:
            keep = pad_mask[:, :seqlen].to(device=x.device, dtype=x.dtype).unsqueeze(-1)
            x = x * keep
        n = bsz * seqlen
        x2 = x.reshape(n, self.dim)
        qkv, dd, beta_logits, gate_logits = self._project(x2)
        cached = self.use_cache and int(start_pos) > 0
        cu = ops.cu_for_batch(bsz, seqlen, x.device)
        qkv = self._short_convolution_flat(qkv, cu, None, read=cached, write=self.use_cache,
                                           step=(seqlen == 1 and cached and self.use_cache))
        i = self.inner_dim
        shape4 = (bsz, seqlen, self.num_heads, self.head_dim)
        # Strided views of the conv output (no copies): the kernels take row strides.
        q = qkv[:, :i].view(shape4)
        k = qkv[:, i: 2 * i].view(shape4)
        v = qkv[:, 2 * i:].view(shape4)
        decay = self.decay_up(dd).view(shape4)
        beta_logits = beta_logits.reshape(bsz, seqlen, self.num_heads)
        if pad_mask is not None:
            drop = ~pad_mask[:, :seqlen].to(device=x.device).bool()
            decay = decay.masked_fill(drop[:, :, None, None], PAD_LOGIT)
            beta_logits = beta_logits.masked_fill(drop[:, :, None], PAD_LOGIT)
        initial_state = self.recurrent_state[:bsz] if cached else None
        output, final_state = self._run_kda(q, k, v, decay, beta_logits, initial_state)
        if self.use_cache and final_state is not initial_state:
            with torch.no_grad():
                self.recurrent_state[:bsz].copy_(final_state.detach().to(dtype=torch.float32))
        out = self._output(output.reshape(n, self.num_heads, self.head_dim), gate_logits, x.dtype)
        return out.view(bsz, seqlen, self.dim)

    def forward_packed(self, x: torch.Tensor, cu_seqlens: torch.Tensor, *,
                       state_slots: torch.Tensor | None = None, use_state: bool = True,
                       max_seqlen: int | None = None) -> torch.Tensor:
        """Packed ragged batch: x [total, dim] (or [1, total, dim]) holding the
        sequences delimited by int32 ``cu_seqlens`` [N+1].  Sequence s reads
        (when ``use_state``) and writes (when ``use_cache``) cache slot
        ``state_slots[s]`` (default s) of ``recurrent_state`` / ``conv_state``;
        zero a slot with ``reset_slots`` before a new sequence uses it.
        ``max_seqlen == 1`` (decode only) selects the one-step kernels.
        Returns [total, dim] (or [1, total, dim])."""
        _require_gpu(x)
        squeeze = x.dim() == 3
        x2 = x.reshape(-1, self.dim)
        n = int(x2.size(0))
        cu = cu_seqlens.to(device=x.device, dtype=torch.int32).contiguous()
        nseq = int(cu.numel()) - 1
        slots = None if state_slots is None else state_slots.to(
            device=x.device, dtype=torch.int32).contiguous()
        if self.use_cache and slots is None:
            self.ensure_batch_capacity(nseq)  # with explicit slots the caller sizes the caches
        qkv, dd, beta_logits, gate_logits = self._project(x2)
        read = bool(use_state) and self.use_cache
        step = max_seqlen == 1 and n == nseq and read
        qkv = self._short_convolution_flat(qkv, cu, slots, read=read, write=self.use_cache,
                                           step=step)
        i, h, d = self.inner_dim, self.num_heads, self.head_dim
        q = qkv[:, :i].unflatten(1, (h, d))
        k = qkv[:, i: 2 * i].unflatten(1, (h, d))
        v = qkv[:, 2 * i:].unflatten(1, (h, d))
        decay = self.decay_up(dd).view(n, h, d)
        state = self.recurrent_state if self.use_cache else None
        if step:
            o = ops.kda_decode_step(q, k, v, decay, beta_logits, state, A_log=self.A_log,
                                    dt_bias=self.dt_bias, lower_bound=self.lower_bound,
                                    state_slots=slots, read_state=True)
        else:
            o = ops.kda_chunk_fwd(q, k, v, decay, beta_logits, cu, A_log=self.A_log,
                                  dt_bias=self.dt_bias, lower_bound=self.lower_bound,
                                  initial_state=state if read else None, final_state=state,
                                  state_slots=slots,
                                  cu_seqlens_cpu=None if cu_seqlens.is_cuda else cu_seqlens)
        out = self._output(o, gate_logits, x.dtype)
        return out.view(1, n, self.dim) if squeeze else out


    def forward_mixed(self, x: torch.Tensor, n_prefill: int, cu_prefill: torch.Tensor,
                      prefill_slots: torch.Tensor | None, decode_slots: torch.Tensor | None, *,
                      prefill_reads_cache: bool = False,
                      cu_prefill_host: torch.Tensor | None = None) -> torch.Tensor:
        """One continuous-batching step over packed rows x [N, dim].

        Rows [0, n_prefill) hold prefill sequences delimited by int32
        ``cu_prefill`` (device, offsets from row 0, any lengths).  Without
        ``prefill_reads_cache`` they start from empty caches; with it each
        continues from the recurrent state and conv history in its slot of
        ``prefill_slots`` (a new sequence's slot must have been zeroed, e.g.
        with ``reset_slots``).  Either way they leave their final state and
        history in those slots.  Rows [n_prefill, N) are one decode token each
        for the sequences in ``decode_slots``, whose caches are read and
        advanced in place (decode kernels).  One fused projection GEMM and one
        output epilogue cover all rows.  ``cu_prefill_host``: host copy of
        ``cu_prefill`` (plans the prefill scan).  Returns [N, dim].
        """
        _require_gpu(x)
        x2 = x.reshape(-1, self.dim)
        n = int(x2.size(0))
        n_prefill = int(n_prefill)
        n_decode = n - n_prefill
        if not self.use_cache:
            raise RuntimeError("forward_mixed needs use_cache=True (it writes cache slots)")
        qkv, dd, beta_logits, gate_logits = self._project(x2)
        i, h, d = self.inner_dim, self.num_heads, self.head_dim
        hist = self.conv_kernel - 1
        conv_state = (self.conv_state.view(self.conv_state.size(0), 3 * i, hist)
                      if hist > 0 else None)
        conv_w = self._conv_weight(qkv.dtype)
        # The prefill rows' ShortConv runs inside the chunk prefill when the
        # rows before the conv are bf16 whole lines (the fused projection's).
        fused_prefill = (n_prefill > 0 and hist == 3 and qkv.dtype == torch.bfloat16
                         and qkv.stride(1) == 1 and qkv.stride(0) % 8 == 0 and qkv.data_ptr() % 16 == 0)
        fused_decode = n_decode > 0 and hist == 3
        conv_out = None
        if not (fused_prefill or n_prefill == 0) or not (fused_decode or n_decode == 0):
            conv_out = torch.empty((n, 3 * i), dtype=qkv.dtype, device=qkv.device)
        if n_prefill > 0 and not fused_prefill:
            ops.short_conv_fwd(qkv[:n_prefill], conv_w, cu_prefill, conv_state=conv_state,
                               state_slots=prefill_slots,
                               read_history=bool(prefill_reads_cache) and hist > 0,
                               write_history=hist > 0, out=conv_out[:n_prefill],
                               weight_rounded=True)
        if n_decode > 0 and not fused_decode:
            ops.short_conv_step(qkv[n_prefill:], conv_w, conv_state, state_slots=decode_slots,
                                read_history=True, out=conv_out[n_prefill:], weight_rounded=True)
        decay = self.decay_up(dd).view(n, h, d)
        o = torch.empty((n, h, d), dtype=x2.dtype, device=x2.device)
        gate_args = dict(A_log=self.A_log, dt_bias=self.dt_bias, lower_bound=self.lower_bound)
        states = dict(initial_state=self.recurrent_state if prefill_reads_cache else None,
                      final_state=self.recurrent_state, state_slots=prefill_slots,
                      cu_seqlens_cpu=cu_prefill_host)
        if fused_prefill:
            ops.kda_conv_chunk_fwd(qkv[:n_prefill], conv_w, conv_state, decay[:n_prefill],
                                   beta_logits[:n_prefill], cu_prefill,
                                   read_history=bool(prefill_reads_cache), out=o[:n_prefill],
                                   **states, **gate_args)
        elif n_prefill > 0:
            q = conv_out[:n_prefill, :i].unflatten(1, (h, d))
            k = conv_out[:n_prefill, i: 2 * i].unflatten(1, (h, d))
            v = conv_out[:n_prefill, 2 * i:].unflatten(1, (h, d))
            ops.kda_chunk_fwd(q, k, v, decay[:n_prefill], beta_logits[:n_prefill], cu_prefill,
                              out=o[:n_prefill], **states, **gate_args)
        if fused_decode:
            # ShortConv step and recurrent step of the decode rows in one launch.
            ops.kda_decode_conv_step(qkv[n_prefill:], conv_w, conv_state, decay[n_prefill:],
                                     beta_logits[n_prefill:], self.recurrent_state,
                                     state_slots=decode_slots, out=o[n_prefill:], **gate_args)
        elif n_decode > 0:
            q = conv_out[n_prefill:, :i].unflatten(1, (h, d))
            k = conv_out[n_prefill:, i: 2 * i].unflatten(1, (h, d))
            v = conv_out[n_prefill:, 2 * i:].unflatten(1, (h, d))
            ops.kda_decode_step(q, k, v, decay[n_prefill:],
                                beta_logits[n_prefill:], self.recurrent_state,
                                state_slots=decode_slots, read_state=True, out=o[n_prefill:],
                                **gate_args)
        return self._output(o, gate_logits, x2.dtype)


def set_pad_mask(model: nn.Module, mask: torch.Tensor | None) -> None:
    """attention.py:660-670: hang a [B, T] bool mask (True = real token) on
    every token mixer (KDA and, in the hybrid decoder, MLA), or clear it.
    Clearing also forgets the prompt mask an MLA layer keeps for the keys of
    later steps, so that an unpadded batch after a padded one sees none."""
    from .decoder import SophiaMLA   # the decoder module imports this one
    for module in model.modules():
        if isinstance(module, (SophiaKDA, SophiaMLA)):
            module._pad_mask = mask
            if mask is None and isinstance(module, SophiaMLA):
                module._prompt_mask = None


__all__ = ["CausalDepthwiseConv1d", "PAD_LOGIT", "RMSNorm", "RuntimeLinear", "SophiaKDA",
           "set_pad_mask"]
