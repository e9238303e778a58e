"""The HIP kernels as ``torch.library`` custom ops in the ``sophia::`` namespace.

The reference registers its own kernels the same way
(ml/training/pretrain/engine/sm120_concurrent_ffn.py:62-104): a CUDA/ROCm
implementation plus a fake (meta) implementation for shape inference, so that
``torch.compile`` traces a call as one opaque node instead of breaking the
graph at a foreign-function call.  Tensors a kernel updates in place (the
recurrent state, the conv history) are declared in ``mutates_args``.

Ops (each implementation is the eager wrapper of ``sophia_amd.ops``, which
checks every argument and launches through the C ABI on the current stream):
  sophia::short_conv_fwd    (x, weight, cu_seqlens, conv_state!, ...) -> y
  sophia::short_conv_step   (x, weight, conv_state!, ...) -> y
  sophia::kda_chunk_fwd     (q, k, v, g, beta, cu_seqlens, ..., final_state!, ...) -> o
  sophia::kda_chunk_bwd     (q, k, v, g, beta, cu_seqlens, d_out, ...) -> (dq, dk, dv, dg,
                            dbeta, dh0, dA_log, ddt_bias)
  sophia::kda_decode_step   (q, k, v, g, beta, state!, ...) -> o
  sophia::gated_head_norm   (o, gate, norm_weight, ...) -> y
  sophia::short_conv        (x, weight, cu_seqlens, history, ...) -> y   (functional: the
                            history is only read; the form training differentiates)
  sophia::short_conv_bwd    (dy, x, weight, ...) -> (dx, dweight)
  sophia::gated_head_norm_bwd (d_out, o, gate, norm_weight, ...) -> (d_o, d_gate, d_norm_weight)

Autograd is registered for ``sophia::short_conv`` and ``sophia::gated_head_norm``
(backward = the two ``*_bwd`` ops), so the mixer trains through them; the
reference's training plugin installs a differentiable conv the same way
(ml/training/pretrain/engine/sm120_concurrent_ffn.py:199-207,425-428).
"""

from typing import Optional

import torch

from . import ops

_LIB = "sophia"


@torch.library.custom_op(f"{_LIB}::short_conv_fwd", mutates_args=("conv_state",),
                         device_types="cuda")
def short_conv_fwd(x: torch.Tensor, weight: torch.Tensor, cu_seqlens: torch.Tensor,
                   conv_state: Optional[torch.Tensor], state_slots: Optional[torch.Tensor],
                   read_history: bool, write_history: bool, weight_rounded: bool) -> torch.Tensor:
    return ops.short_conv_fwd(x, weight, cu_seqlens, conv_state=conv_state, state_slots=state_slots,
                              read_history=read_history, write_history=write_history,
                              weight_rounded=weight_rounded)


@short_conv_fwd.register_fake
def _(x, weight, cu_seqlens, conv_state, state_slots, read_history, write_history, weight_rounded):
    return x.new_empty((x.shape[0], x.shape[1]))


@torch.library.custom_op(f"{_LIB}::short_conv_step", mutates_args=("conv_state",),
                         device_types="cuda")
def short_conv_step(x: torch.Tensor, weight: torch.Tensor, conv_state: torch.Tensor,
                    state_slots: Optional[torch.Tensor], read_history: bool,
                    weight_rounded: bool) -> torch.Tensor:
    return ops.short_conv_step(x, weight, conv_state, state_slots=state_slots,
                               read_history=read_history, weight_rounded=weight_rounded)


@short_conv_step.register_fake
def _(x, weight, conv_state, state_slots, read_history, weight_rounded):
    return x.new_empty((x.shape[0], x.shape[1]))


@torch.library.custom_op(f"{_LIB}::kda_chunk_fwd", mutates_args=("final_state",),
                         device_types="cuda")
def kda_chunk_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, cu_seqlens: torch.Tensor, A_log: Optional[torch.Tensor],
                  dt_bias: Optional[torch.Tensor], scale: float, lower_bound: float,
                  use_qk_l2norm: bool, use_gate: bool, use_beta_sigmoid: bool,
                  initial_state: Optional[torch.Tensor], final_state: Optional[torch.Tensor],
                  read_final_state: bool, state_slots: Optional[torch.Tensor],
                  cu_seqlens_cpu: Optional[torch.Tensor]) -> torch.Tensor:
    """Chunk prefill.  ``read_final_state``: the initial state is read from
    ``final_state`` itself (updated in place, the cached-prefill form); else
    from ``initial_state`` (read only, must not alias ``final_state``)."""
    h0 = final_state if read_final_state else initial_state
    return ops.kda_chunk_fwd(q, k, v, g, beta, cu_seqlens, A_log=A_log, dt_bias=dt_bias,
                             scale=scale, lower_bound=lower_bound, use_qk_l2norm=use_qk_l2norm,
                             use_gate=use_gate, use_beta_sigmoid=use_beta_sigmoid,
                             initial_state=h0, final_state=final_state, state_slots=state_slots,
                             cu_seqlens_cpu=cu_seqlens_cpu)


@kda_chunk_fwd.register_fake
def _(q, k, v, g, beta, cu_seqlens, A_log, dt_bias, scale, lower_bound, use_qk_l2norm, use_gate,
      use_beta_sigmoid, initial_state, final_state, read_final_state, state_slots, cu_seqlens_cpu):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2]))


@torch.library.custom_op(f"{_LIB}::kda_chunk_bwd", mutates_args=(), device_types="cuda")
def kda_chunk_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, cu_seqlens: torch.Tensor, d_out: torch.Tensor,
                  A_log: Optional[torch.Tensor], dt_bias: Optional[torch.Tensor], scale: float,
                  lower_bound: float, use_qk_l2norm: bool, use_gate: bool, use_beta_sigmoid: bool,
                  initial_state: Optional[torch.Tensor], d_final_state: Optional[torch.Tensor],
                  cu_seqlens_cpu: Optional[torch.Tensor], recurrent: bool = False,
                  grad_bf16: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                             torch.Tensor, torch.Tensor, torch.Tensor]:
    """Prefill backward: fp32 gradients of every input (dA_log / ddt_bias empty
    without the in-kernel gate; dq, dk, dv bf16 with ``grad_bf16``); the chunk
    form, or the fp32 recurrence with ``recurrent``."""
    return ops.kda_chunk_bwd(q, k, v, g, beta, cu_seqlens, d_out, A_log=A_log, dt_bias=dt_bias,
                             scale=scale, lower_bound=lower_bound, use_qk_l2norm=use_qk_l2norm,
                             use_gate=use_gate, use_beta_sigmoid=use_beta_sigmoid,
                             initial_state=initial_state, d_final_state=d_final_state,
                             cu_seqlens_cpu=cu_seqlens_cpu, recurrent=recurrent,
                             grad_dtype=torch.bfloat16 if grad_bf16 else torch.float32)


@kda_chunk_bwd.register_fake
def _(q, k, v, g, beta, cu_seqlens, d_out, A_log, dt_bias, scale, lower_bound, use_qk_l2norm,
      use_gate, use_beta_sigmoid, initial_state, d_final_state, cu_seqlens_cpu, recurrent=False,
      grad_bf16=False):
    total, heads, dim = q.shape
    n = cu_seqlens.shape[0] - 1
    f32 = dict(dtype=torch.float32)
    gqkv = dict(dtype=torch.bfloat16 if grad_bf16 else torch.float32)
    return (q.new_empty((total, heads, dim), **gqkv), q.new_empty((total, heads, dim), **gqkv),
            q.new_empty((total, heads, dim), **gqkv), q.new_empty((total, heads, dim), **f32),
            q.new_empty((total, heads), **f32), q.new_empty((n, heads, dim, dim), **f32),
            q.new_empty((heads if use_gate else 0,), **f32),
            q.new_empty((heads * dim if use_gate else 0,), **f32))


@torch.library.custom_op(f"{_LIB}::kda_decode_step", mutates_args=("state",), device_types="cuda")
def kda_decode_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                    beta: torch.Tensor, state: torch.Tensor, A_log: Optional[torch.Tensor],
                    dt_bias: Optional[torch.Tensor], scale: float, lower_bound: float,
                    use_qk_l2norm: bool, use_gate: bool, use_beta_sigmoid: bool,
                    state_slots: Optional[torch.Tensor], read_state: bool) -> torch.Tensor:
    return ops.kda_decode_step(q, k, v, g, beta, state, A_log=A_log, dt_bias=dt_bias, scale=scale,
                               lower_bound=lower_bound, use_qk_l2norm=use_qk_l2norm,
                               use_gate=use_gate, use_beta_sigmoid=use_beta_sigmoid,
                               state_slots=state_slots, read_state=read_state)


@kda_decode_step.register_fake
def _(q, k, v, g, beta, state, A_log, dt_bias, scale, lower_bound, use_qk_l2norm, use_gate,
      use_beta_sigmoid, state_slots, read_state):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2]))


@torch.library.custom_op(f"{_LIB}::gated_head_norm", mutates_args=(), device_types="cuda")
def gated_head_norm(o: torch.Tensor, gate: torch.Tensor, norm_weight: Optional[torch.Tensor],
                    heads: int, head_dim: int, eps: float) -> torch.Tensor:
    return ops.gated_head_norm(o, gate, heads, head_dim, norm_weight=norm_weight, eps=eps)


@gated_head_norm.register_fake
def _(o, gate, norm_weight, heads, head_dim, eps):
    rows = gate.numel() // (heads * head_dim)
    return gate.new_empty((rows, heads * head_dim))


# ---- training: functional ShortConv and the two backward ops, with autograd
@torch.library.custom_op(f"{_LIB}::short_conv", mutates_args=(), device_types="cuda")
def short_conv(x: torch.Tensor, weight: torch.Tensor, cu_seqlens: torch.Tensor,
               history: Optional[torch.Tensor], state_slots: Optional[torch.Tensor], read_history: bool,
               weight_rounded: bool) -> torch.Tensor:
    """ShortConv over a packed batch with the history (fp32 [slots, C, K-1])
    only read, never written."""
    return ops.short_conv_fwd(x, weight, cu_seqlens, conv_state=history, state_slots=state_slots,
                              read_history=read_history, write_history=False, weight_rounded=weight_rounded)


@short_conv.register_fake
def _(x, weight, cu_seqlens, history, state_slots, read_history, weight_rounded):
    return x.new_empty((x.shape[0], x.shape[1]))


@torch.library.custom_op(f"{_LIB}::short_conv_bwd", mutates_args=(), device_types="cuda")
def short_conv_bwd(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, cu_seqlens: torch.Tensor,
                   history: Optional[torch.Tensor], state_slots: Optional[torch.Tensor], read_history: bool,
                   weight_rounded: bool) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.short_conv_bwd(dy, x, weight, cu_seqlens, conv_state=history, state_slots=state_slots,
                              read_history=read_history, weight_rounded=weight_rounded)


@short_conv_bwd.register_fake
def _(dy, x, weight, cu_seqlens, history, state_slots, read_history, weight_rounded):
    return (x.new_empty((x.shape[0], x.shape[1])),
            x.new_empty((weight.shape[0], weight.shape[1]), dtype=torch.float32))


def _short_conv_setup(ctx, inputs, output):
    x, weight, cu_seqlens, history, state_slots, read_history, weight_rounded = inputs
    ctx.save_for_backward(x, weight, cu_seqlens, history, state_slots)
    ctx.flags = (bool(read_history), bool(weight_rounded))


def _short_conv_backward(ctx, dy):
    x, weight, cu_seqlens, history, state_slots = ctx.saved_tensors
    dx, dw = short_conv_bwd(dy.contiguous(), x, weight, cu_seqlens, history, state_slots, *ctx.flags)
    return dx, dw.to(weight.dtype), None, None, None, None, None


torch.library.register_autograd(f"{_LIB}::short_conv", _short_conv_backward, setup_context=_short_conv_setup)


@torch.library.custom_op(f"{_LIB}::gated_head_norm_bwd", mutates_args=(), device_types="cuda")
def gated_head_norm_bwd(d_out: torch.Tensor, o: torch.Tensor, gate: torch.Tensor,
                        norm_weight: Optional[torch.Tensor], heads: int, head_dim: int,
                        eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (d_o, d_gate, d_norm_weight); d_norm_weight is empty without the norm."""
    d_o, d_g, d_w = ops.gated_head_norm_bwd(d_out, o, gate, heads, head_dim, norm_weight=norm_weight, eps=eps)
    if d_w is None:
        d_w = gate.new_empty((0,), dtype=torch.float32)
    return d_o, d_g, d_w


@gated_head_norm_bwd.register_fake
def _(d_out, o, gate, norm_weight, heads, head_dim, eps):
    return (o.new_empty(o.shape), gate.new_empty(gate.shape),
            gate.new_empty((head_dim if norm_weight is not None else 0,), dtype=torch.float32))


def _gated_head_norm_setup(ctx, inputs, output):
    o, gate, norm_weight, heads, head_dim, eps = inputs
    ctx.save_for_backward(o, gate, norm_weight)
    ctx.args = (int(heads), int(head_dim), float(eps))


def _gated_head_norm_backward(ctx, d_out):
    o, gate, norm_weight = ctx.saved_tensors
    d_o, d_g, d_w = gated_head_norm_bwd(d_out.contiguous(), o, gate, norm_weight, *ctx.args)
    d_norm = None if norm_weight is None else d_w.reshape(norm_weight.shape).to(norm_weight.dtype)
    return d_o, d_g, d_norm, None, None, None


torch.library.register_autograd(f"{_LIB}::gated_head_norm", _gated_head_norm_backward,
                                setup_context=_gated_head_norm_setup)


__all__ = ["gated_head_norm", "gated_head_norm_bwd", "kda_chunk_bwd", "kda_chunk_fwd", "kda_decode_step",
           "short_conv", "short_conv_bwd", "short_conv_fwd", "short_conv_step"]
