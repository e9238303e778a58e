"""Plugging the HIP kernels into a reference-shaped model at its kernel seam.

The reference mixer selects its KDA kernels through two per-instance
callables, ``_fla_chunk_kda()`` for prefill and ``_fla_fused_recurrent_kda()``
for the one-token step (ml/runtime/model/attention.py:296-371), and its
plugins replace them together with ``CausalDepthwiseConv1d.forward``
(ml/training/pretrain/engine/sm120_concurrent_ffn.py:189-207,425-430).
``install_mi355x_kda`` does the same with this package's kernels:

* conv modules (``forward(x, *, history=None) -> (silu(conv), next_history)``,
  attention.py:32-60) get a forward that runs ``sophia::short_conv_fwd``, or,
  when x or the weight requires grad, the differentiable ``sophia::short_conv``
  (backward on the HIP kernel ``sophia_short_conv_bwd``);
* mixers get ``ops.chunk_kda`` and an in-place ``ops.fused_recurrent_kda``
  (the reference copies the final state back into the very buffer it passed
  as the initial state, attention.py:398-410, so updating it in place gives
  the same result without the copy).

Both callables run through ``sophia::`` custom ops, so a model compiled with
``torch.compile`` traces them without a graph break.
"""

from __future__ import annotations

import functools
from types import MethodType

import torch
from torch import nn

from . import ops
from .kda import conv_forward


def _conv_forward(self, x: torch.Tensor, *, history: torch.Tensor | None = None):
    """CausalDepthwiseConv1d.forward (attention.py:32-60) on the HIP kernel:
    x [B, T, C], history [B, C, K-1] or None -> (y [B, T, C], next_history in
    x.dtype), differentiable in x and the weight as the training plugin's
    causal_conv1d_fn is (sm120_concurrent_ffn.py:199-207)."""
    return conv_forward(self.weight, int(self.kernel_size), x, history)


def _chunk_kda():
    return ops.chunk_kda


def _fused_recurrent_kda():
    return functools.partial(ops.fused_recurrent_kda, inplace_state=True)


def _is_conv(module: nn.Module, conv_type) -> bool:
    if conv_type is not None:
        return isinstance(module, conv_type)
    return (type(module).__name__ == "CausalDepthwiseConv1d" and hasattr(module, "weight")
            and hasattr(module, "kernel_size"))


def _is_mixer(module: nn.Module, mixer_type) -> bool:
    if mixer_type is not None:
        return isinstance(module, mixer_type)
    return hasattr(module, "_fla_chunk_kda") and hasattr(module, "_fla_fused_recurrent_kda")


def install_mi355x_kda(model: nn.Module, *, conv_type=None, mixer_type=None) -> dict[str, int]:
    """Replace the KDA kernel seam and the ShortConv forward of every matching
    submodule of ``model`` (the reference's classes by default, matched by
    name and attributes; pass ``conv_type`` / ``mixer_type`` to match by
    class).  Returns how many modules of each kind were patched."""
    patched = {"conv": 0, "mixer": 0}
    for module in model.modules():
        if _is_conv(module, conv_type):
            module.forward = MethodType(_conv_forward, module)
            patched["conv"] += 1
        elif _is_mixer(module, mixer_type):
            module._fla_chunk_kda = _chunk_kda
            module._fla_fused_recurrent_kda = _fused_recurrent_kda
            patched["mixer"] += 1
    return patched


__all__ = ["install_mi355x_kda"]
