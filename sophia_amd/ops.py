"""Torch-facing entry points of the HIP kernels.

Each function checks devices, dtypes and shapes (raising ``RuntimeError`` the
way the reference's custom ops do, ml/training/pretrain/engine/
sm120_concurrent_ffn.py:49-59), allocates outputs and scratch from torch's
caching allocator, and launches the C ABI of ``include/sophia_kda.h`` on the
current stream.  Nothing here synchronises the device or reads device data on
the host, so every call can be captured in a HIP graph.

``chunk_kda`` and ``fused_recurrent_kda`` keep the signatures of the
flash-linear-attention functions that the reference mixer calls
(ml/runtime/model/attention.py:330-365) plus the varlen arguments of the
FlashKDA seam (sm120_concurrent_ffn.py:375-423), so they drop into
``SophiaKDA._fla_chunk_kda`` / ``_fla_fused_recurrent_kda``.
"""

from __future__ import annotations

import torch

from . import _native as nat

HEAD_DIM = 128
CHUNK_SIZE = 64


def _gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a tensor on a ROCm GPU (sophia_amd has no CPU path)")


def _rows(t: torch.Tensor, name: str, width: int) -> int:
    """Row stride (elements) of a [N, width] view whose rows are dense."""
    if t.dim() != 2 or t.size(1) != width:
        raise RuntimeError(f"{name} must be [N, {width}], got {tuple(t.shape)}")
    if t.size(1) > 1 and t.stride(1) != 1:
        raise RuntimeError(f"{name} rows must be contiguous")
    return int(t.stride(0)) if t.size(0) > 1 else width


def _heads_rows(t: torch.Tensor, name: str, heads: int, dim: int) -> int:
    """Row stride of a [N, H, D] view with dense [H, D] rows."""
    if t.dim() != 3 or t.size(1) != heads or t.size(2) != dim:
        raise RuntimeError(f"{name} must be [N, {heads}, {dim}], got {tuple(t.shape)}")
    if (heads > 1 and t.stride(1) != dim) or t.stride(2) != 1:
        raise RuntimeError(f"{name} must have dense [heads, dim] rows")
    return int(t.stride(0)) if t.size(0) > 1 else heads * dim


def _int32(t: torch.Tensor | None, name: str, device) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.int32 or t.device != device or not t.is_contiguous():
        raise RuntimeError(f"{name} must be a contiguous int32 tensor on {device}")
    return t


def _nrows(t: torch.Tensor, name: str, expect: int) -> None:
    """Leading (row) dimension check: a mis-sized tensor must raise here, not
    let a kernel index past its end."""
    if int(t.size(0)) != int(expect):
        raise RuntimeError(f"{name} has {int(t.size(0))} rows, expected {int(expect)}")


def _slot_count(slots: torch.Tensor | None, expect: int) -> None:
    if slots is not None and int(slots.numel()) != int(expect):
        raise RuntimeError(f"state_slots must hold {int(expect)} entries, got {int(slots.numel())}")


def _workspace(nbytes: int, device) -> tuple[torch.Tensor, int, int]:
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    addr = buf.data_ptr()
    pad = (-addr) % 256
    return buf, addr + pad, nbytes


# ------------------------------------------------------------------ ShortConv
def _conv_taps(weight: torch.Tensor, x: torch.Tensor, rounded: bool) -> torch.Tensor:
    """The conv taps as the kernels take them: fp32 [C, K] holding the weight
    rounded to x.dtype (the reference casts the weight to x's dtype)."""
    if not rounded:
        return weight.detach().to(device=x.device, dtype=x.dtype).float().contiguous()
    if weight.dtype != torch.float32 or not weight.is_contiguous() or weight.device != x.device:
        raise RuntimeError("a rounded conv weight must be contiguous fp32 on x's device")
    return weight


def short_conv_fwd(x: torch.Tensor, weight: torch.Tensor, cu_seqlens: torch.Tensor, *,
                   conv_state: torch.Tensor | None = None,
                   state_slots: torch.Tensor | None = None, read_history: bool = False,
                   write_history: bool = False, out: torch.Tensor | None = None,
                   weight_rounded: bool = False) -> torch.Tensor:
    """Causal depthwise conv + SiLU over a packed batch (CausalDepthwiseConv1d.forward,
    attention.py:32-60, applied per sequence of ``cu_seqlens``).

    x: [total, C] (rows may be strided); weight: [C, K] (cast to x.dtype then
    fp32, as the reference casts the weight to x's dtype); conv_state:
    [slots, C, K-1] fp32, read when ``read_history`` and written when
    ``write_history``.  ``weight_rounded``: weight is already the contiguous
    fp32 [C, K] copy of its x.dtype rounding (no cast is launched).
    Returns y [total, C] in x.dtype.
    """
    _gpu(x, "x")
    channels = int(x.size(1))
    xs = _rows(x, "x", channels)
    kernel = int(weight.size(1))
    if weight.dim() != 2 or int(weight.size(0)) != channels:
        raise RuntimeError(f"weight must be [{channels}, K], got {tuple(weight.shape)}")
    w = _conv_taps(weight, x, weight_rounded)
    cu = _int32(cu_seqlens, "cu_seqlens", x.device)
    n = int(cu.numel()) - 1
    if conv_state is not None:
        _gpu(conv_state, "conv_state")
        if (conv_state.dtype != torch.float32 or not conv_state.is_contiguous()
                or tuple(conv_state.shape[1:]) != (channels, kernel - 1)):
            raise RuntimeError(f"conv_state must be contiguous fp32 [slots, {channels}, "
                               f"{kernel - 1}], got {tuple(conv_state.shape)}")
    slots = _int32(state_slots, "state_slots", x.device)
    _slot_count(slots, n)
    y = out if out is not None else torch.empty((x.size(0), channels), dtype=x.dtype,
                                                device=x.device)
    ys = _rows(y, "out", channels)
    _nrows(y, "out", int(x.size(0)))
    if y.dtype != x.dtype:
        raise RuntimeError("out must have x's dtype")
    rc = nat.lib().sophia_short_conv_fwd(
        nat.ptr(x), xs, nat.ptr(y), ys, nat.dtype_code(x.dtype), nat.ptr(w), nat.ptr(conv_state),
        0 if conv_state is None else int(conv_state.size(0)),
        nat.ptr(slots), nat.ptr(cu), n, int(x.size(0)), channels, kernel, int(bool(read_history)),
        int(bool(write_history)), nat.stream_handle(x.device))
    nat.check(rc, "sophia_short_conv_fwd")
    return y


def short_conv_bwd(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, cu_seqlens: torch.Tensor, *,
                   conv_state: torch.Tensor | None = None, state_slots: torch.Tensor | None = None,
                   read_history: bool = False,
                   weight_rounded: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Backward of ``short_conv_fwd`` (sophia_short_conv_bwd): the gradients of
    x and of the taps for the output gradient ``dy``, with the forward's
    arguments (``conv_state`` is only read: the history samples the forward
    convolved; the history gets no gradient).  Returns (dx [total, C] in
    x.dtype, zero on rows outside every sequence; dweight [C, K] fp32, with
    respect to the taps the forward used -- the weight rounded to x.dtype)."""
    _gpu(x, "x")
    _gpu(dy, "dy")
    channels = int(x.size(1))
    total = int(x.size(0))
    xs = _rows(x, "x", channels)
    if dy.dtype != x.dtype or tuple(dy.shape) != (total, channels):
        raise RuntimeError(f"dy must be {x.dtype} [{total}, {channels}], got {dy.dtype} {tuple(dy.shape)}")
    dys = _rows(dy, "dy", channels)
    if weight.dim() != 2 or int(weight.size(0)) != channels:
        raise RuntimeError(f"weight must be [{channels}, K], got {tuple(weight.shape)}")
    kernel = int(weight.size(1))
    w = _conv_taps(weight, x, weight_rounded)
    cu = _int32(cu_seqlens, "cu_seqlens", x.device)
    n = int(cu.numel()) - 1
    if conv_state is not None:
        _gpu(conv_state, "conv_state")
        if (conv_state.dtype != torch.float32 or not conv_state.is_contiguous()
                or tuple(conv_state.shape[1:]) != (channels, kernel - 1)):
            raise RuntimeError(f"conv_state must be contiguous fp32 [slots, {channels}, {kernel - 1}]")
    slots = _int32(state_slots, "state_slots", x.device)
    _slot_count(slots, n)
    dx = torch.empty((total, channels), dtype=x.dtype, device=x.device)
    dw = torch.empty((channels, kernel), dtype=torch.float32, device=x.device)
    lib = nat.lib()
    need = int(lib.sophia_short_conv_bwd_workspace_size(total, channels, kernel))
    buf, ws_addr, ws_bytes = _workspace(need, x.device)
    rc = lib.sophia_short_conv_bwd(
        nat.ptr(x), xs, nat.ptr(dy), dys, nat.ptr(dx), channels, nat.dtype_code(x.dtype), nat.ptr(w),
        nat.ptr(conv_state), 0 if conv_state is None else int(conv_state.size(0)), nat.ptr(slots),
        nat.ptr(cu), n, total, channels, kernel, int(bool(read_history) and conv_state is not None),
        nat.ptr(dw), ws_addr, ws_bytes, nat.stream_handle(x.device))
    nat.check(rc, "sophia_short_conv_bwd")
    del buf
    return dx, dw


def short_conv_step(x: torch.Tensor, weight: torch.Tensor, conv_state: torch.Tensor, *,
                    state_slots: torch.Tensor | None = None, read_history: bool = True,
                    out: torch.Tensor | None = None, weight_rounded: bool = False) -> torch.Tensor:
    """One-token conv step for a batch of sequences (decode), history updated in place.
    x: [B, C]; conv_state: [slots, C, K-1] fp32."""
    _gpu(x, "x")
    _gpu(conv_state, "conv_state")
    channels = int(x.size(1))
    xs = _rows(x, "x", channels)
    kernel = int(weight.size(1))
    if (conv_state.dtype != torch.float32 or not conv_state.is_contiguous()
            or tuple(conv_state.shape[1:]) != (channels, kernel - 1)):
        raise RuntimeError("conv_state must be contiguous fp32 [slots, C, K-1]")
    w = _conv_taps(weight, x, weight_rounded)
    slots = _int32(state_slots, "state_slots", x.device)
    _slot_count(slots, int(x.size(0)))
    if slots is None and int(conv_state.size(0)) < int(x.size(0)):
        raise RuntimeError("conv_state has fewer slots than the batch")
    y = out if out is not None else torch.empty_like(x, memory_format=torch.contiguous_format)
    ys = _rows(y, "out", channels)
    _nrows(y, "out", int(x.size(0)))
    if y.dtype != x.dtype:
        raise RuntimeError("out must have x's dtype")
    rc = nat.lib().sophia_short_conv_step(
        nat.ptr(x), xs, nat.ptr(y), ys, nat.dtype_code(x.dtype), nat.ptr(w), nat.ptr(conv_state),
        int(conv_state.size(0)), nat.ptr(slots), int(x.size(0)), channels, kernel,
        int(bool(read_history)),
        nat.stream_handle(x.device))
    nat.check(rc, "sophia_short_conv_step")
    return y


# ------------------------------------------------------------------ KDA core
def _flags(use_qk_l2norm: bool, use_gate: bool, use_beta_sigmoid: bool) -> int:
    return ((nat.QK_L2NORM if use_qk_l2norm else 0) | (nat.GATE_IN_KERNEL if use_gate else 0)
            | (nat.BETA_SIGMOID if use_beta_sigmoid else 0))


def _gate_params(use_gate, A_log, dt_bias, heads, device):
    if not use_gate:
        return None, None
    if A_log is None or dt_bias is None:
        raise RuntimeError("use_gate_in_kernel needs A_log and dt_bias")
    a = A_log.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    b = dt_bias.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if a.numel() != heads or b.numel() != heads * HEAD_DIM:
        raise RuntimeError(f"A_log must have {heads} and dt_bias {heads * HEAD_DIM} elements")
    return a, b


def _state(t: torch.Tensor | None, name: str, heads: int, device) -> None:
    if t is None:
        return
    _gpu(t, name)
    if (t.dtype != torch.float32 or not t.is_contiguous() or t.dim() != 4
            or tuple(t.shape[1:]) != (heads, HEAD_DIM, HEAD_DIM) or t.device != device):
        raise RuntimeError(f"{name} must be contiguous fp32 [slots, {heads}, 128, 128]")


def kda_chunk_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, cu_seqlens: torch.Tensor, *, A_log=None, dt_bias=None,
                  scale: float | None = None, lower_bound: float = -5.0,
                  use_qk_l2norm: bool = True, use_gate: bool = True,
                  use_beta_sigmoid: bool = True, initial_state: torch.Tensor | None = None,
                  final_state: torch.Tensor | None = None,
                  state_slots: torch.Tensor | None = None,
                  out: torch.Tensor | None = None,
                  cu_seqlens_cpu: torch.Tensor | None = None,
                  scan_segments: bool = True) -> torch.Tensor:
    """Chunk-64 KDA prefill over a packed batch.

    q, k, v, g: [total, H, 128] (rows may be strided views of a wider
    buffer); beta: [total, H]; cu_seqlens: int32 [N+1] (copied to the device
    if needed).  initial_state / final_state: fp32 [slots, H, 128, 128] or
    None, indexed by ``state_slots`` (default: sequence index); they may be
    the same tensor.  ``cu_seqlens_cpu`` (FlashKDA's name; default: cu_seqlens
    itself when it lives on the host) lets the launch be planned from the
    sequence lengths; results are the same without it, but that a few long
    sequences are then scanned in segments (rounding differences only;
    ``scan_segments=False`` keeps one chain per sequence).
    Returns o [total, H, 128] in q.dtype.
    """
    return _prefill(q, k, v, g, beta, cu_seqlens, A_log, dt_bias, scale, lower_bound, use_qk_l2norm,
                    use_gate, use_beta_sigmoid, initial_state, final_state, state_slots, out,
                    cu_seqlens_cpu, scan_segments, None)


def kda_conv_chunk_fwd(x_qkv: torch.Tensor, conv_weight: torch.Tensor,
                       conv_state: torch.Tensor | None, g: torch.Tensor, beta: torch.Tensor,
                       cu_seqlens: torch.Tensor, *, read_history: bool = False, A_log=None,
                       dt_bias=None, scale: float | None = None, lower_bound: float = -5.0,
                       use_qk_l2norm: bool = True, use_gate: bool = True,
                       use_beta_sigmoid: bool = True, initial_state: torch.Tensor | None = None,
                       final_state: torch.Tensor | None = None,
                       state_slots: torch.Tensor | None = None, out: torch.Tensor | None = None,
                       cu_seqlens_cpu: torch.Tensor | None = None,
                       scan_segments: bool = True) -> torch.Tensor:
    """The prefill of a KDA layer with its ShortConv fused into the chunk
    prefill (sophia_kda_conv_chunk_fwd): ``short_conv_fwd`` of the q | k | v
    channels (write_history=True) followed by ``kda_chunk_fwd``, bitwise, with
    the conv outputs never written (attention.py:226-258, 349-365).

    x_qkv: bf16 [total, 3 * H * 128] rows before the conv (16-byte aligned,
    row stride a multiple of 8); conv_weight: contiguous fp32 [3 * H * 128, 4]
    taps already rounded to bf16; conv_state: contiguous fp32 [slots,
    3 * H * 128, 3] or None, the slot of each sequence read when
    ``read_history`` and replaced by its last 3 rows; it shares ``state_slots``
    (and the slot count) with initial_state / final_state.  Other arguments
    as ``kda_chunk_fwd``.  Returns o [total, H, 128] (bf16)."""
    _gpu(x_qkv, "x_qkv")
    _gpu(g, "g")
    device = x_qkv.device
    heads = int(g.size(1)) if g.dim() == 3 else 0
    inner = heads * HEAD_DIM
    _rows(x_qkv, "x_qkv", 3 * inner)
    if x_qkv.dtype != torch.bfloat16:
        raise RuntimeError("x_qkv must be bf16")
    if (conv_weight.dtype != torch.float32 or not conv_weight.is_contiguous()
            or tuple(conv_weight.shape) != (3 * inner, 4) or conv_weight.device != device):
        raise RuntimeError(f"conv_weight must be contiguous fp32 [{3 * inner}, 4] on {device}")
    if conv_state is not None:
        _gpu(conv_state, "conv_state")
        if (conv_state.dtype != torch.float32 or not conv_state.is_contiguous()
                or conv_state.dim() != 3 or tuple(conv_state.shape[1:]) != (3 * inner, 3)):
            raise RuntimeError(f"conv_state must be contiguous fp32 [slots, {3 * inner}, 3]")
    q = x_qkv[:, :inner].unflatten(1, (heads, HEAD_DIM))
    k = x_qkv[:, inner: 2 * inner].unflatten(1, (heads, HEAD_DIM))
    v = x_qkv[:, 2 * inner: 3 * inner].unflatten(1, (heads, HEAD_DIM))
    return _prefill(q, k, v, g, beta, cu_seqlens, A_log, dt_bias, scale, lower_bound, use_qk_l2norm,
                    use_gate, use_beta_sigmoid, initial_state, final_state, state_slots, out,
                    cu_seqlens_cpu, scan_segments, (conv_weight, conv_state, bool(read_history)))


def _prefill(q, k, v, g, beta, cu_seqlens, A_log, dt_bias, scale, lower_bound, use_qk_l2norm,
             use_gate, use_beta_sigmoid, initial_state, final_state, state_slots, out,
             cu_seqlens_cpu, scan_segments, conv):
    """kda_chunk_fwd, or with ``conv`` = (taps, histories or None,
    read_history) the fused-conv prefill on pre-conv q, k, v views."""
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (g, "g"), (beta, "beta")):
        _gpu(t, name)
    device = q.device
    total, heads = int(q.size(0)), int(q.size(1))
    qs = _heads_rows(q, "q", heads, HEAD_DIM)
    if k.stride() != q.stride() or v.stride() != q.stride():
        raise RuntimeError("q, k and v must share one row layout")
    _heads_rows(k, "k", heads, HEAD_DIM)
    _heads_rows(v, "v", heads, HEAD_DIM)
    if not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError("q, k and v must share one dtype")
    if int(k.size(0)) != total or int(v.size(0)) != total or int(g.size(0)) != total:
        raise RuntimeError("q, k, v and g must have the same number of tokens")
    gs = _heads_rows(g, "g", heads, HEAD_DIM)
    bs = _rows(beta, "beta", heads)
    _nrows(beta, "beta", total)
    if not isinstance(cu_seqlens, torch.Tensor):
        raise RuntimeError("cu_seqlens must be a tensor")
    if not cu_seqlens.is_cuda:
        # A host cu_seqlens is also the host copy that plans the launch.
        if cu_seqlens_cpu is None:
            cu_seqlens_cpu = cu_seqlens
        cu_seqlens = cu_seqlens.to(device=device, dtype=torch.int32).contiguous()
    cu = _int32(cu_seqlens, "cu_seqlens", device)
    n = int(cu.numel()) - 1
    if n < 1:
        raise RuntimeError("cu_seqlens must hold at least one sequence")
    cu_host = None
    if cu_seqlens_cpu is not None:
        cu_host = torch.as_tensor(cu_seqlens_cpu).to(dtype=torch.int32).contiguous()
        if cu_host.is_cuda or int(cu_host.numel()) != n + 1:
            raise RuntimeError("cu_seqlens_cpu must be a host copy of cu_seqlens")
    _state(initial_state, "initial_state", heads, device)
    _state(final_state, "final_state", heads, device)
    n_slots = [int(t.size(0)) for t in (initial_state, final_state) if t is not None]
    if len(n_slots) == 2 and n_slots[0] != n_slots[1]:
        raise RuntimeError("initial_state and final_state must have the same number of slots")
    n_slots = n_slots[0] if n_slots else 0
    if conv is not None and conv[1] is not None:
        conv_slots = int(conv[1].size(0))
        if n_slots and conv_slots != n_slots:
            raise RuntimeError("conv_state and the state tensors must have the same number of slots")
        n_slots = conv_slots
    if state_slots is None and n_slots and n_slots < n:
        raise RuntimeError("state tensors have fewer slots than sequences")
    slots = _int32(state_slots, "state_slots", device)
    _slot_count(slots, n)
    a_log, dtb = _gate_params(use_gate, A_log, dt_bias, heads, device)
    if scale is None:
        scale = HEAD_DIM ** -0.5
    o = out if out is not None else torch.empty((total, heads, HEAD_DIM), dtype=q.dtype,
                                                device=device)
    os_ = _heads_rows(o, "out", heads, HEAD_DIM)
    _nrows(o, "out", total)
    if o.dtype != q.dtype:
        raise RuntimeError("out must have q's dtype")
    lib = nat.lib()
    need = int(lib.sophia_kda_chunk_workspace_size(total, n, heads, HEAD_DIM))
    buf, ws_addr, ws_bytes = _workspace(need, device)
    common = (nat.ptr(g), gs, nat.dtype_code(g.dtype), nat.ptr(beta), bs, nat.dtype_code(beta.dtype),
              nat.ptr(a_log), nat.ptr(dtb), float(scale), float(lower_bound),
              _flags(use_qk_l2norm, use_gate, use_beta_sigmoid)
              | (0 if scan_segments else nat.SCAN_NO_SEGMENTS), nat.ptr(cu),
              None if cu_host is None else cu_host.data_ptr(), n, total, heads, HEAD_DIM,
              nat.ptr(initial_state), nat.ptr(final_state), n_slots, nat.ptr(slots), nat.ptr(o), os_,
              ws_addr, ws_bytes, nat.stream_handle(device))
    if conv is None:
        rc = lib.sophia_kda_chunk_fwd(nat.ptr(q), nat.ptr(k), nat.ptr(v), qs, nat.dtype_code(q.dtype),
                                      *common)
        nat.check(rc, "sophia_kda_chunk_fwd")
    else:
        rc = lib.sophia_kda_conv_chunk_fwd(nat.ptr(q), nat.ptr(k), nat.ptr(v), qs, nat.dtype_code(q.dtype),
                                           nat.ptr(conv[0]), nat.ptr(conv[1]), 4, int(conv[2]), *common)
        nat.check(rc, "sophia_kda_conv_chunk_fwd")
    del buf  # stream-ordered reuse by the caching allocator is safe
    return o


def kda_chunk_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, cu_seqlens: torch.Tensor, d_out: torch.Tensor, *,
                  A_log=None, dt_bias=None, scale: float | None = None,
                  lower_bound: float = -5.0, use_qk_l2norm: bool = True, use_gate: bool = True,
                  use_beta_sigmoid: bool = True, initial_state: torch.Tensor | None = None,
                  d_final_state: torch.Tensor | None = None,
                  cu_seqlens_cpu: torch.Tensor | None = None, recurrent: bool = False,
                  grad_dtype: torch.dtype = torch.float32):
    """Gradients of ``kda_chunk_fwd`` (no cache slots: one state per sequence).

    The HIP counterpart of FlashKDA's chunk_kda_train_bwd plus l2norm_bwd and
    fused_beta_sigmoid_bwd (sm120_concurrent_ffn.py:301-373).  Inputs as for
    kda_chunk_fwd; d_out: [total, H, 128] gradient of o; d_final_state: fp32
    [N, H, 128, 128] or None.  Returns fp32 (dq, dk, dv, dg, dbeta, dh0,
    dA_log, ddt_bias): dg with respect to the g input as passed, dh0
    [N, H, 128, 128], dA_log [H] and ddt_bias [H * 128] (empty without the
    in-kernel gate); ``grad_dtype=torch.bfloat16`` writes dq, dk and dv as
    bf16 instead (the fp32 gradients rounded to nearest even), the element
    type a bf16 forward's q, k, v carry.  A host ``cu_seqlens`` (or ``cu_seqlens_cpu``) is checked
    to rise from 0 to the token count.  The chunk form runs by default (bf16
    MFMA operands, fp32 accumulation and state, the forward's arithmetic);
    ``recurrent=True`` runs the per-token recurrence in fp32 instead.
    """
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (g, "g"), (beta, "beta"), (d_out, "d_out")):
        _gpu(t, name)
    device = q.device
    total, heads = int(q.size(0)), int(q.size(1))
    qs = _heads_rows(q, "q", heads, HEAD_DIM)
    if k.stride() != q.stride() or v.stride() != q.stride():
        raise RuntimeError("q, k and v must share one row layout")
    _heads_rows(k, "k", heads, HEAD_DIM)
    _heads_rows(v, "v", heads, HEAD_DIM)
    if not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError("q, k and v must share one dtype")
    for t, name in ((k, "k"), (v, "v"), (g, "g"), (beta, "beta"), (d_out, "d_out")):
        _nrows(t, name, total)
    gs = _heads_rows(g, "g", heads, HEAD_DIM)
    bs = _rows(beta, "beta", heads)
    ds = _heads_rows(d_out, "d_out", heads, HEAD_DIM)
    if not isinstance(cu_seqlens, torch.Tensor):
        raise RuntimeError("cu_seqlens must be a tensor")
    if cu_seqlens_cpu is None and not cu_seqlens.is_cuda:
        cu_seqlens_cpu = cu_seqlens
    cu_host = None if cu_seqlens_cpu is None else torch.as_tensor(cu_seqlens_cpu).to("cpu", torch.int64)
    cu = _int32(cu_seqlens.to(device=device, dtype=torch.int32).contiguous(), "cu_seqlens", device)
    n = int(cu.numel()) - 1
    if n < 1:
        raise RuntimeError("cu_seqlens must hold at least one sequence")
    if cu_host is not None and (int(cu_host.numel()) != n + 1 or int(cu_host[0]) != 0
                                or int(cu_host[-1]) != total
                                or bool((cu_host[1:] < cu_host[:-1]).any())):
        raise RuntimeError("cu_seqlens must rise from 0 to the token count")
    _state(initial_state, "initial_state", heads, device)
    _state(d_final_state, "d_final_state", heads, device)
    for t, name in ((initial_state, "initial_state"), (d_final_state, "d_final_state")):
        if t is not None:
            _nrows(t, name, n)
    a_log, dtb = _gate_params(use_gate, A_log, dt_bias, heads, device)
    if grad_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError("grad_dtype must be torch.float32 or torch.bfloat16")
    if scale is None:
        scale = HEAD_DIM ** -0.5
    f32 = dict(dtype=torch.float32, device=device)
    dq = torch.empty((total, heads, HEAD_DIM), dtype=grad_dtype, device=device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    dg = torch.empty((total, heads, HEAD_DIM), **f32)
    dbeta = torch.empty((total, heads), **f32)
    dh0 = torch.empty((n, heads, HEAD_DIM, HEAD_DIM), **f32)
    da = torch.empty((heads if use_gate else 0,), **f32)
    dbias = torch.empty((heads * HEAD_DIM if use_gate else 0,), **f32)
    lib = nat.lib()
    need = int(lib.sophia_kda_chunk_bwd_workspace_size(total, n, heads, HEAD_DIM))
    buf, ws_addr, ws_bytes = _workspace(need, device)
    rc = lib.sophia_kda_chunk_bwd(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), qs, nat.dtype_code(q.dtype), nat.ptr(g), gs,
        nat.dtype_code(g.dtype), nat.ptr(beta), bs, nat.dtype_code(beta.dtype), nat.ptr(a_log),
        nat.ptr(dtb), float(scale), float(lower_bound),
        _flags(use_qk_l2norm, use_gate, use_beta_sigmoid) | (nat.BWD_RECURRENT if recurrent else 0)
        | (nat.BWD_GRAD_BF16 if grad_dtype == torch.bfloat16 else 0),
        nat.ptr(cu), n, total, heads, HEAD_DIM,
        nat.ptr(initial_state), nat.ptr(d_out), ds, nat.dtype_code(d_out.dtype),
        nat.ptr(d_final_state), nat.ptr(dq), nat.ptr(dk), nat.ptr(dv), nat.ptr(dg),
        nat.ptr(dbeta), nat.ptr(dh0), nat.ptr(da) if use_gate else None,
        nat.ptr(dbias) if use_gate else None, ws_addr, ws_bytes, nat.stream_handle(device))
    nat.check(rc, "sophia_kda_chunk_bwd")
    del buf
    return dq, dk, dv, dg, dbeta, dh0, da, dbias


def kda_decode_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                    beta: torch.Tensor, state: torch.Tensor, *, A_log=None, dt_bias=None,
                    scale: float | None = None, lower_bound: float = -5.0,
                    use_qk_l2norm: bool = True, use_gate: bool = True,
                    use_beta_sigmoid: bool = True, state_slots: torch.Tensor | None = None,
                    read_state: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
    """One recurrent step for B sequences; ``state`` is updated in place.
    q, k, v, g: [B, H, 128]; beta: [B, H]; state: fp32 [slots, H, 128, 128]."""
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (g, "g"), (beta, "beta")):
        _gpu(t, name)
    device = q.device
    batch, heads = int(q.size(0)), int(q.size(1))
    qs = _heads_rows(q, "q", heads, HEAD_DIM)
    if k.stride() != q.stride() or v.stride() != q.stride() or not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError("q, k and v must share one row layout and dtype")
    _heads_rows(k, "k", heads, HEAD_DIM)
    _heads_rows(v, "v", heads, HEAD_DIM)
    gs = _heads_rows(g, "g", heads, HEAD_DIM)
    bs = _rows(beta, "beta", heads)
    for t, name in ((k, "k"), (v, "v"), (g, "g"), (beta, "beta")):
        _nrows(t, name, batch)
    _state(state, "state", heads, device)
    slots = _int32(state_slots, "state_slots", device)
    _slot_count(slots, batch)
    if slots is None and int(state.size(0)) < batch:
        raise RuntimeError("state has fewer slots than the batch")
    a_log, dtb = _gate_params(use_gate, A_log, dt_bias, heads, device)
    if scale is None:
        scale = HEAD_DIM ** -0.5
    o = out if out is not None else torch.empty((batch, heads, HEAD_DIM), dtype=q.dtype,
                                                device=device)
    os_ = _heads_rows(o, "out", heads, HEAD_DIM)
    _nrows(o, "out", batch)
    if o.dtype != q.dtype:
        raise RuntimeError("out must have q's dtype")
    rc = nat.lib().sophia_kda_decode_step(
        nat.ptr(q), nat.ptr(k), nat.ptr(v), qs, nat.dtype_code(q.dtype), nat.ptr(g), gs,
        nat.dtype_code(g.dtype), nat.ptr(beta), bs, nat.dtype_code(beta.dtype), nat.ptr(a_log),
        nat.ptr(dtb), float(scale), float(lower_bound),
        _flags(use_qk_l2norm, use_gate, use_beta_sigmoid), nat.ptr(state), int(state.size(0)),
        nat.ptr(slots),
        int(bool(read_state)), batch, heads, HEAD_DIM, nat.ptr(o), os_,
        nat.stream_handle(device))
    nat.check(rc, "sophia_kda_decode_step")
    return o


def kda_decode_conv_step(x_qkv: torch.Tensor, conv_weight: torch.Tensor, conv_state: torch.Tensor,
                         g: torch.Tensor, beta: torch.Tensor, state: torch.Tensor, *, A_log=None,
                         dt_bias=None, scale: float | None = None, lower_bound: float = -5.0,
                         use_qk_l2norm: bool = True, use_gate: bool = True,
                         use_beta_sigmoid: bool = True, state_slots: torch.Tensor | None = None,
                         read_state: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step of a KDA layer with its ShortConv in one launch:
    ``short_conv_step`` of the q | k | v channels followed by
    ``kda_decode_step`` (attention.py:236-257, 330-348).

    x_qkv: [B, 3 * H * 128] pre-conv projection rows (dense rows, row stride
    free); conv_weight: [3 * H * 128, 4] fp32 taps already rounded to
    x_qkv.dtype (contiguous); conv_state: fp32 [slots, 3 * H * 128, 3], each
    row's slot shifted in place; g: [B, H, 128]; beta: [B, H]; state: fp32
    [slots, H, 128, 128] updated in place.  Returns o [B, H, 128] in
    x_qkv.dtype."""
    for t, name in ((x_qkv, "x_qkv"), (g, "g"), (beta, "beta")):
        _gpu(t, name)
    device = x_qkv.device
    batch = int(x_qkv.size(0))
    heads = int(g.size(1)) if g.dim() == 3 else 0
    inner = heads * HEAD_DIM
    xs = _rows(x_qkv, "x_qkv", 3 * inner)
    gs = _heads_rows(g, "g", heads, HEAD_DIM)
    bs = _rows(beta, "beta", heads)
    for t, name in ((g, "g"), (beta, "beta")):
        _nrows(t, name, batch)
    if (conv_weight.dtype != torch.float32 or not conv_weight.is_contiguous()
            or tuple(conv_weight.shape) != (3 * inner, 4) or conv_weight.device != device):
        raise RuntimeError(f"conv_weight must be contiguous fp32 [{3 * inner}, 4] on {device}")
    _gpu(conv_state, "conv_state")
    if (conv_state.dtype != torch.float32 or not conv_state.is_contiguous()
            or tuple(conv_state.shape[1:]) != (3 * inner, 3)):
        raise RuntimeError(f"conv_state must be contiguous fp32 [slots, {3 * inner}, 3]")
    _state(state, "state", heads, device)
    if int(conv_state.size(0)) != int(state.size(0)):
        raise RuntimeError("conv_state and state must have the same number of slots")
    slots = _int32(state_slots, "state_slots", device)
    _slot_count(slots, batch)
    if slots is None and int(state.size(0)) < batch:
        raise RuntimeError("state has fewer slots than the batch")
    a_log, dtb = _gate_params(use_gate, A_log, dt_bias, heads, device)
    if scale is None:
        scale = HEAD_DIM ** -0.5
    o = out if out is not None else torch.empty((batch, heads, HEAD_DIM), dtype=x_qkv.dtype,
                                                device=device)
    os_ = _heads_rows(o, "out", heads, HEAD_DIM)
    _nrows(o, "out", batch)
    if o.dtype != x_qkv.dtype:
        raise RuntimeError("out must have x_qkv's dtype")
    base = x_qkv.data_ptr()
    esz = x_qkv.element_size()
    rc = nat.lib().sophia_kda_decode_conv_step(
        base, base + inner * esz, base + 2 * inner * esz, xs, nat.dtype_code(x_qkv.dtype),
        nat.ptr(conv_weight), nat.ptr(conv_state), 4, nat.ptr(g), gs, nat.dtype_code(g.dtype),
        nat.ptr(beta), bs, nat.dtype_code(beta.dtype), nat.ptr(a_log), nat.ptr(dtb), float(scale),
        float(lower_bound), _flags(use_qk_l2norm, use_gate, use_beta_sigmoid), nat.ptr(state),
        int(state.size(0)), nat.ptr(slots), int(bool(read_state)), batch, heads, HEAD_DIM,
        nat.ptr(o), os_, nat.stream_handle(device))
    nat.check(rc, "sophia_kda_decode_conv_step")
    return o


# -------------------------------------------- flash-linear-attention signatures
def _detached(t):
    """Gate parameters enter the kernels as values (the forward-only kernels
    take no gradient through them)."""
    return t.detach() if isinstance(t, torch.Tensor) else t


def cu_for_batch(bsz: int, seqlen: int, device) -> torch.Tensor:
    """cu_seqlens of a rectangular [bsz, seqlen] batch viewed as packed rows."""
    return torch.arange(0, (bsz + 1) * seqlen, seqlen, dtype=torch.int32, device=device)


def chunk_kda(q, k, v, g, beta, *, scale=None, initial_state=None, output_final_state=False,
              use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False,
              use_beta_sigmoid_in_kernel=False, safe_gate=False, lower_bound=None, A_log=None,
              dt_bias=None, cu_seqlens=None, cu_seqlens_cpu=None, chunk_size=64,
              allow_neg_eigval=False, state_v_first=False, **kwargs):
    """fla.ops.kda.chunk_kda as called at attention.py:349-365 (and FlashKDA's
    varlen form, sm120_concurrent_ffn.py:375-423).

    q, k, g: [B, T, H, 128]; v: [B, T, H, 128]; beta: [B, T, H].  With
    ``cu_seqlens`` B must be 1 and states are per sequence.  Returns
    (o [B, T, H, 128] in q.dtype, final_state fp32 [N, H, 128, 128] or None).
    The log-decay must stay in [-5, 0]: the gate computed in the kernel always
    does; a precomputed g needs ``safe_gate`` with ``lower_bound >= -5``.
    As in FlashKDAFunction.forward (sm120_concurrent_ffn.py:240-244),
    ``allow_neg_eigval`` makes the in-kernel beta sigmoid 2 sigmoid(beta)
    (beta in [0, 2]: the eigenvalues of I - beta k k^T reach -1) and does
    nothing without ``use_beta_sigmoid_in_kernel``; ``state_v_first`` takes and
    returns states as [N, H, V, K] (the transpose of the kernels' [K, V]).
    """
    if kwargs:
        raise TypeError(f"unexpected arguments: {sorted(kwargs)}")
    if int(chunk_size) != CHUNK_SIZE:
        raise RuntimeError("sophia_amd chunk_kda supports chunk_size=64 only")
    if allow_neg_eigval and use_beta_sigmoid_in_kernel:
        # 2 sigmoid(beta) on the device, ahead of the kernels (autograd carries
        # its derivative); the kernels then take beta as given.
        beta = 2.0 * torch.sigmoid(beta.float())
        use_beta_sigmoid_in_kernel = False
    if state_v_first:
        o, ht = chunk_kda(q, k, v, g, beta, scale=scale,
                          initial_state=None if initial_state is None else initial_state.transpose(-1, -2),
                          output_final_state=output_final_state,
                          use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                          use_gate_in_kernel=use_gate_in_kernel,
                          use_beta_sigmoid_in_kernel=use_beta_sigmoid_in_kernel, safe_gate=safe_gate,
                          lower_bound=lower_bound, A_log=A_log, dt_bias=dt_bias, cu_seqlens=cu_seqlens,
                          cu_seqlens_cpu=cu_seqlens_cpu, chunk_size=chunk_size)
        return o, (None if ht is None else ht.transpose(-1, -2))
    lb = -5.0 if lower_bound is None else float(lower_bound)
    if not use_gate_in_kernel and not safe_gate:
        raise RuntimeError("a precomputed gate needs safe_gate=True (log-decay in [lower_bound, 0])")
    if q.dim() != 4:
        raise RuntimeError(f"q must be [B, T, H, K], got {tuple(q.shape)}")
    bsz, seqlen, heads, _ = q.shape
    if cu_seqlens is not None:
        if bsz != 1:
            raise RuntimeError("varlen chunk_kda needs a packed batch of size 1")
        if cu_seqlens_cpu is None and not cu_seqlens.is_cuda:
            cu_seqlens_cpu = cu_seqlens
        cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    else:
        cu = cu_for_batch(bsz, seqlen, q.device)
    n = int(cu.numel()) - 1
    total = bsz * seqlen

    def flat(t, width):
        return t.reshape(total, heads, width) if t.dim() == 4 else t.reshape(total, heads)

    scale = float(HEAD_DIM ** -0.5 if scale is None else scale)
    if torch.is_grad_enabled() and any(
            isinstance(t, torch.Tensor) and t.requires_grad
            for t in (q, k, v, g, beta, A_log, dt_bias, initial_state)):
        o, ht = ChunkKDAFunction.apply(
            flat(q, HEAD_DIM), flat(k, HEAD_DIM), flat(v, HEAD_DIM), flat(g, HEAD_DIM),
            beta.reshape(total, heads), A_log, dt_bias, scale, initial_state,
            bool(output_final_state), bool(use_qk_l2norm_in_kernel), bool(use_gate_in_kernel),
            bool(use_beta_sigmoid_in_kernel), cu, cu_seqlens_cpu, lb)
        return o.view(bsz, seqlen, heads, HEAD_DIM), ht
    h0 = None
    if initial_state is not None:
        h0 = initial_state if (initial_state.dtype == torch.float32
                               and initial_state.is_contiguous()) else initial_state.float().contiguous()
    ht = torch.empty((n, heads, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=q.device) \
        if output_final_state else None
    # Through the sophia::kda_chunk_fwd custom op, so that torch.compile traces
    # the call as one node.
    o = torch_ops.kda_chunk_fwd(
        flat(q, HEAD_DIM), flat(k, HEAD_DIM), flat(v, HEAD_DIM), flat(g, HEAD_DIM),
        beta.reshape(total, heads), cu, _detached(A_log), _detached(dt_bias),
        scale, lb, bool(use_qk_l2norm_in_kernel),
        bool(use_gate_in_kernel), bool(use_beta_sigmoid_in_kernel), h0, ht, False, None,
        cu_seqlens_cpu)
    return o.view(bsz, seqlen, heads, HEAD_DIM), ht


def _meta(t):
    """(shape, dtype) of a tensor input, kept for its gradient; None otherwise."""
    return (t.shape, t.dtype) if isinstance(t, torch.Tensor) else None


def _grad_like(grad: torch.Tensor, meta):
    """A fp32 kernel gradient in the shape and dtype of the input it belongs to."""
    if meta is None:
        return None
    return grad.view(meta[0]).to(meta[1])


class ChunkKDAFunction(torch.autograd.Function):
    """FlashKDAFunction (ml/training/pretrain/engine/sm120_concurrent_ffn.py:
    209-373) over the HIP kernels: the forward is the chunk prefill
    (sophia::kda_chunk_fwd), the backward sophia::kda_chunk_bwd, which folds
    in the l2norm / beta-sigmoid backward the reference runs after
    chunk_kda_train_bwd.  Inputs are packed [total, H, 128] rows (beta
    [total, H]); returns (o, final_state or None).  The backward saves the
    inputs only and recomputes the states it needs."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, A_log, dt_bias, scale, initial_state, output_final_state,
                use_qk_l2norm, use_gate, use_beta_sigmoid, cu, cu_seqlens_cpu, lower_bound):
        total, heads = int(q.size(0)), int(q.size(1))
        n = int(cu.numel()) - 1
        h0 = None
        if initial_state is not None:
            h0 = initial_state.detach().float().reshape(n, heads, HEAD_DIM, HEAD_DIM).contiguous()
        a_log = None if A_log is None else A_log.detach()
        dtb = None if dt_bias is None else dt_bias.detach()
        ht = torch.empty((n, heads, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=q.device) \
            if output_final_state else None
        o = torch_ops.kda_chunk_fwd(q, k, v, g, beta, cu, a_log, dtb, scale, lower_bound,
                                    use_qk_l2norm, use_gate, use_beta_sigmoid, h0, ht, False, None,
                                    cu_seqlens_cpu)
        ctx.save_for_backward(q, k, v, g, beta, a_log, dtb, h0, cu)
        ctx.cu_cpu = cu_seqlens_cpu
        ctx.args = (float(scale), float(lower_bound), bool(use_qk_l2norm), bool(use_gate),
                    bool(use_beta_sigmoid))
        ctx.inputs = (_meta(A_log), _meta(dt_bias), _meta(initial_state))
        ctx.set_materialize_grads(False)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, beta, a_log, dtb, h0, cu = ctx.saved_tensors
        scale, lb, use_l2, use_gate, use_sig = ctx.args
        A_log, dt_bias, initial_state = ctx.inputs
        if do is None:
            do = torch.zeros((q.size(0), q.size(1), HEAD_DIM), dtype=torch.float32, device=q.device)
        dht = None if dht is None else dht.float().contiguous()
        # bf16 q, k, v take their gradients as bf16 from the kernel (no casts)
        dq, dk, dv, dg, db, dh0, da, dbias = torch_ops.kda_chunk_bwd(
            q, k, v, g, beta, cu, do.contiguous(), a_log, dtb, scale, lb, use_l2, use_gate,
            use_sig, h0, dht, ctx.cu_cpu, False, q.dtype == torch.bfloat16)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), db.to(beta.dtype),
                _grad_like(da, A_log) if use_gate else None,
                _grad_like(dbias, dt_bias) if use_gate else None, None,
                _grad_like(dh0, initial_state), None, None, None, None, None, None, None)


def flash_kda(q, k, v, g, beta, A_log, dt_bias, scale=None, initial_state=None,
              output_final_state=False, use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False,
              use_beta_sigmoid_in_kernel=False, allow_neg_eigval=False, state_v_first=False,
              cu_seqlens=None, cu_seqlens_cpu=None, safe_gate=False, lower_bound=None,
              chunk_size=64, **kwargs):
    """The reference's flash_kda training entry (sm120_concurrent_ffn.py:375-423):
    same arguments, differentiable in q, k, v, g, beta, A_log, dt_bias and
    initial_state.  Returns (o [B, T, H, 128], final_state or None)."""
    if kwargs:
        raise TypeError(sorted(kwargs))
    return chunk_kda(q, k, v, g, beta, scale=scale, initial_state=initial_state,
                     output_final_state=output_final_state,
                     use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                     use_gate_in_kernel=use_gate_in_kernel,
                     use_beta_sigmoid_in_kernel=use_beta_sigmoid_in_kernel, safe_gate=safe_gate,
                     lower_bound=lower_bound, A_log=A_log, dt_bias=dt_bias, cu_seqlens=cu_seqlens,
                     cu_seqlens_cpu=cu_seqlens_cpu, chunk_size=chunk_size,
                     allow_neg_eigval=allow_neg_eigval, state_v_first=state_v_first)


def fused_recurrent_kda(q, k, v, g, beta, *, A_log=None, dt_bias=None, scale=None,
                        initial_state=None, output_final_state=True,
                        use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False,
                        use_beta_sigmoid_in_kernel=False, lower_bound=None, inplace_state=False,
                        **kwargs):
    """fla.ops.kda.fused_recurrent_kda for one token (attention.py:330-348).

    q, k, v, g: [B, 1, H, 128]; beta: [B, 1, H]; initial_state fp32
    [B, H, 128, 128] or None.  With ``inplace_state`` the step updates
    ``initial_state`` itself and returns it as the final state (the mixer
    copies the final state back into that same buffer, attention.py:406-410).
    """
    if kwargs:
        raise TypeError(f"unexpected arguments: {sorted(kwargs)}")
    if q.dim() != 4 or int(q.size(1)) != 1:
        raise RuntimeError("sophia_amd fused_recurrent_kda advances one token: q must be [B, 1, H, K]")
    bsz, _, heads, _ = q.shape
    lb = -5.0 if lower_bound is None else float(lower_bound)
    if initial_state is None:
        state = torch.empty((bsz, heads, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=q.device)
        read = False
    elif inplace_state:
        state, read = initial_state, True
    else:
        state, read = initial_state.float().clone(memory_format=torch.contiguous_format), True
    o = torch_ops.kda_decode_step(
        q.reshape(bsz, heads, HEAD_DIM), k.reshape(bsz, heads, HEAD_DIM),
        v.reshape(bsz, heads, HEAD_DIM), g.reshape(bsz, heads, HEAD_DIM), beta.reshape(bsz, heads),
        state, _detached(A_log), _detached(dt_bias),
        float(HEAD_DIM ** -0.5 if scale is None else scale), lb, bool(use_qk_l2norm_in_kernel),
        bool(use_gate_in_kernel), bool(use_beta_sigmoid_in_kernel), None, read)
    return o.view(bsz, 1, heads, HEAD_DIM), (state if output_final_state else None)


# ------------------------------------------------------------------ decoder layers
def _aligned(t: torch.Tensor, name: str) -> None:
    if t.data_ptr() % 16:
        raise RuntimeError(f"{name} must be 16-byte aligned")


def attn_res_mix(partial: torch.Tensor, completed: torch.Tensor, norm_weight: torch.Tensor,
                 query_weight: torch.Tensor, eps: float, *,
                 out_norm_weight: torch.Tensor | None = None, out_eps: float = 1e-6,
                 residual: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, partial_out: torch.Tensor | None = None):
    """AttentionResidualMixer.forward (ml/runtime/model/blocks.py:38-48) in one
    kernel: softmax over the depth axis of [completed blocks..., partial] with
    scores RMSNorm(value) . query, then the weighted sum of the values; with
    ``out_norm_weight``, also the RMSNorm that consumes the mix (attn_norm /
    ffn_norm of blocks.py:72-87, the final norm of transformer.py:210).

    partial: [..., D]; completed: [..., n_blocks, D] with the same leading
    dims and dense rows; norm_weight, query_weight, out_norm_weight: [D] (or
    [1, D]), converted to fp32 as the reference upcasts the query.  Sums,
    scores, softmax and the output norm run in fp32 and the result is rounded
    once to partial.dtype (the reference rounds the softmax weights, the
    products and the mix to the activation dtype on the way).  Returns [..., D].

    ``residual`` ([..., D], same dtype): the partial block is first replaced
    by partial + residual (the residual add of SophiaBlock, blocks.py:78-86,
    rounded to the activation dtype as there); the call then returns
    ``(partial + residual, mix)``, the sum written into ``partial_out`` when
    given ([..., D] of partial's dtype; rows may be strided, e.g. the next
    slot of a depth store).
    """
    _gpu(partial, "partial")
    _gpu(completed, "completed")
    dim = int(partial.size(-1))
    lead = tuple(partial.shape[:-1])
    if completed.dim() != partial.dim() + 1 or tuple(completed.shape[:-2]) != lead \
            or int(completed.size(-1)) != dim:
        raise RuntimeError(f"completed must be [*{lead}, n_blocks, {dim}], got {tuple(completed.shape)}")
    if completed.dtype != partial.dtype:
        raise RuntimeError("partial and completed must share a dtype")
    n_blocks = int(completed.size(-2))
    p2 = partial.reshape(-1, dim)
    rows = int(p2.size(0))
    ps = _rows(p2, "partial", dim)
    c3 = completed.reshape(rows, n_blocks, dim)
    if n_blocks and dim > 1 and c3.stride(2) != 1:
        raise RuntimeError("completed rows must be contiguous")
    c_row = int(c3.stride(0)) if rows > 1 else n_blocks * dim
    c_blk = int(c3.stride(1)) if n_blocks > 1 else dim

    def f32(t: torch.Tensor, name: str) -> torch.Tensor:
        t = t.detach().reshape(-1).to(device=partial.device, dtype=torch.float32).contiguous()
        if int(t.numel()) != dim:
            raise RuntimeError(f"{name} must hold {dim} values")
        _aligned(t, name)
        return t

    w = f32(norm_weight, "norm_weight")
    q = f32(query_weight, "query_weight")
    wo = None if out_norm_weight is None else f32(out_norm_weight, "out_norm_weight")
    if out is not None and not out.is_contiguous():
        raise RuntimeError("out must be contiguous")
    y = out if out is not None else torch.empty((rows, dim), dtype=partial.dtype, device=partial.device)
    if y.dtype != partial.dtype or int(y.numel()) != rows * dim:
        raise RuntimeError(f"out must be {partial.dtype} with {rows * dim} elements")
    y2 = y.view(rows, dim)
    _aligned(p2, "partial")
    _aligned(y2, "out")
    if n_blocks:
        _aligned(c3, "completed")
    r2 = po = None
    rs = 0
    if residual is not None:
        _gpu(residual, "residual")
        if residual.dtype != partial.dtype or tuple(residual.shape) != tuple(partial.shape):
            raise RuntimeError("residual must match partial's shape and dtype")
        r2 = residual.reshape(-1, dim)
        rs = _rows(r2, "residual", dim)
        _aligned(r2, "residual")
        if partial_out is None:
            po = torch.empty((rows, dim), dtype=partial.dtype, device=partial.device)
        else:
            _gpu(partial_out, "partial_out")
            if partial_out.dtype != partial.dtype or tuple(partial_out.shape) != tuple(partial.shape):
                raise RuntimeError("partial_out must match partial's shape and dtype")
            po = partial_out.view(rows, dim)
            _aligned(po, "partial_out")
    elif partial_out is not None:
        raise RuntimeError("partial_out holds partial + residual: it needs a residual")
    pos_ = _rows(po, "partial_out", dim) if po is not None else dim
    rc = nat.lib().sophia_attn_res_mix(
        nat.ptr(p2), ps, nat.ptr(r2), rs, nat.ptr(po), pos_, nat.ptr(c3) if n_blocks else None, c_row,
        c_blk, n_blocks, nat.ptr(w), nat.ptr(q), float(eps), nat.ptr(wo), float(out_eps),
        nat.ptr(y2), dim, rows, dim, nat.dtype_code(partial.dtype), nat.stream_handle(partial.device))
    nat.check(rc, "sophia_attn_res_mix")
    if po is not None:
        return (partial_out if partial_out is not None else po.view(*lead, dim)), y2.view(*lead, dim)
    return y2.view(*lead, dim)


def situ_glu(gate_up: torch.Tensor, gate_softcap: float, up_softcap: float, *,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """The SiTU-GLU hidden of FeedForward.forward (ml/runtime/model/blocks.py:23-27)
    in one pass: with [gate | up] = gate_up,
    gate_softcap tanh(gate / gate_softcap) sigmoid(gate) * up_softcap tanh(up / up_softcap).
    gate_up: [..., 2H] with dense rows; returns [..., H] in gate_up.dtype,
    computed in fp32 and rounded once."""
    _gpu(gate_up, "gate_up")
    width = int(gate_up.size(-1))
    if width % 2:
        raise RuntimeError("gate_up must have an even last dimension")
    hidden = width // 2
    lead = tuple(gate_up.shape[:-1])
    g2 = gate_up.reshape(-1, width)
    rows = int(g2.size(0))
    gs = _rows(g2, "gate_up", width)
    if out is not None and not out.is_contiguous():
        raise RuntimeError("out must be contiguous")
    y = out if out is not None else torch.empty((rows, hidden), dtype=gate_up.dtype,
                                                device=gate_up.device)
    if y.dtype != gate_up.dtype or int(y.numel()) != rows * hidden:
        raise RuntimeError(f"out must be {gate_up.dtype} with {rows * hidden} elements")
    y2 = y.view(rows, hidden)
    _aligned(g2, "gate_up")
    _aligned(y2, "out")
    rc = nat.lib().sophia_situ_glu(nat.ptr(g2), gs, nat.ptr(y2), hidden, rows, hidden,
                                   float(gate_softcap), float(up_softcap),
                                   nat.dtype_code(gate_up.dtype), nat.stream_handle(gate_up.device))
    nat.check(rc, "sophia_situ_glu")
    return y2.view(*lead, hidden)


def mla_latent_norms(q_lat: torch.Tensor, kv_lat: torch.Tensor, q_norm_weight: torch.Tensor,
                     q_eps: float, kv_norm_weight: torch.Tensor, kv_eps: float, *,
                     latent_cache: torch.Tensor | None = None, n_prefill: int = 0,
                     prefill_seq_slots: torch.Tensor | None = None, prefill_seq_len: int = 0,
                     prefill_row_slots: torch.Tensor | None = None,
                     prefill_row_pos: torch.Tensor | None = None,
                     decode_slots: torch.Tensor | None = None,
                     decode_pos: torch.Tensor | None = None) -> None:
    """MLA's q_norm(q_down(x)) and kv_norm(kv_down(x)) in place (attention.py:
    611-614), and each normalised latent row written into ``latent_cache``
    ([slots, max_len, kv_rank] fp32) at its slot and position (attention.py:
    615-621): prefill rows [0, n_prefill) at (prefill_seq_slots[i //
    prefill_seq_len], i % prefill_seq_len) for equal-length prompts from
    position 0, else at (prefill_row_slots[i], prefill_row_pos[i]); the
    remaining rows at (decode_slots[j], decode_pos[j]).  q_lat [rows, q_rank]
    and kv_lat [rows, kv_rank] (dense rows, one dtype); the fp32 weights are
    rounded to that dtype as RMSNorm.forward casts them."""
    _gpu(q_lat, "q_lat")
    _gpu(kv_lat, "kv_lat")
    device = q_lat.device
    rows, q_rank = int(q_lat.size(0)), int(q_lat.size(1))
    kv_rank = int(kv_lat.size(1))
    if q_lat.dim() != 2 or kv_lat.dim() != 2 or int(kv_lat.size(0)) != rows or q_lat.dtype != kv_lat.dtype:
        raise RuntimeError("q_lat and kv_lat must be [rows, rank] of one dtype")
    qs = _rows(q_lat, "q_lat", q_rank)
    ks = _rows(kv_lat, "kv_lat", kv_rank)

    def f32(t, n, name):
        t = t.detach().reshape(-1).to(device=device, dtype=torch.float32).contiguous()
        if int(t.numel()) != n:
            raise RuntimeError(f"{name} must hold {n} values")
        return t

    qw = f32(q_norm_weight, q_rank, "q_norm_weight")
    kw = f32(kv_norm_weight, kv_rank, "kv_norm_weight")
    n_prefill = int(n_prefill)
    n_slots = max_len = 0
    if latent_cache is not None:
        _gpu(latent_cache, "latent_cache")
        if (latent_cache.dtype != torch.float32 or latent_cache.dim() != 3 or not latent_cache.is_contiguous()
                or int(latent_cache.size(2)) != kv_rank):
            raise RuntimeError(f"latent_cache must be contiguous fp32 [slots, max_len, {kv_rank}]")
        n_slots, max_len = int(latent_cache.size(0)), int(latent_cache.size(1))

    def idx(t, dtype, name, n):
        if t is None:
            return None
        _gpu(t, name)
        t = t.reshape(-1).to(dtype).contiguous()   # no copy when already so
        if int(t.numel()) < n:
            raise RuntimeError(f"{name} must hold at least {n} entries")
        return t

    seq_slots = idx(prefill_seq_slots, torch.int32, "prefill_seq_slots",
                    -(-n_prefill // max(int(prefill_seq_len), 1)) if prefill_seq_slots is not None else 0)
    row_slots = idx(prefill_row_slots, torch.int64, "prefill_row_slots", n_prefill)
    row_pos = idx(prefill_row_pos, torch.int64, "prefill_row_pos", n_prefill)
    dslots = idx(decode_slots, torch.int32, "decode_slots", rows - n_prefill)
    dpos = idx(decode_pos, torch.int64, "decode_pos", rows - n_prefill)
    rc = nat.lib().sophia_mla_latent_norms(
        nat.ptr(q_lat), qs, nat.ptr(kv_lat), ks, rows, q_rank, kv_rank, nat.dtype_code(q_lat.dtype),
        nat.ptr(qw), float(q_eps), nat.ptr(kw), float(kv_eps), nat.ptr(latent_cache), n_slots, max_len,
        n_prefill, nat.ptr(seq_slots), int(prefill_seq_len), nat.ptr(row_slots), nat.ptr(row_pos),
        nat.ptr(dslots), nat.ptr(dpos), nat.stream_handle(device))
    nat.check(rc, "sophia_mla_latent_norms")


def gated_head_norm(o: torch.Tensor, gate: torch.Tensor, heads: int, head_dim: int, *,
                    norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """The gated outputs of the token mixers in one pass over [rows, heads * head_dim]:
    with ``norm_weight``, KDA's output_norm(o.to(dtype)) * sigmoid(gate)
    (ml/runtime/model/attention.py:411-420, RMSNorm over each head); without,
    MLA's (o.float() * sigmoid(gate).float()).to(dtype) (attention.py:655-656).

    o: [..., heads * head_dim] (or [..., heads, head_dim]) in fp32 or gate's
    dtype; gate: [..., heads * head_dim] logits with dense rows (a column
    slice of a fused projection is fine).  Returns [rows, heads * head_dim] in
    gate.dtype, computed in fp32 and rounded once."""
    _gpu(o, "o")
    _gpu(gate, "gate")
    width = int(heads) * int(head_dim)
    o2 = o.reshape(-1, width)
    g2 = gate.reshape(-1, width)
    rows = int(g2.size(0))
    if int(o2.size(0)) != rows:
        raise RuntimeError(f"o has {int(o2.size(0))} rows, gate {rows}")
    os_ = _rows(o2, "o", width)
    gs = _rows(g2, "gate", width)
    if o.dtype not in (torch.float32, gate.dtype):
        raise RuntimeError("o must be float32 or gate's dtype")
    w = None
    if norm_weight is not None:
        w = norm_weight.detach().reshape(-1).to(device=gate.device, dtype=torch.float32).contiguous()
        if int(w.numel()) != int(head_dim):
            raise RuntimeError(f"norm_weight must hold {head_dim} values")
        _aligned(w, "norm_weight")
    if out is not None and not out.is_contiguous():
        raise RuntimeError("out must be contiguous")
    y = out if out is not None else torch.empty((rows, width), dtype=gate.dtype, device=gate.device)
    if y.dtype != gate.dtype or int(y.numel()) != rows * width:
        raise RuntimeError(f"out must be {gate.dtype} with {rows * width} elements")
    y2 = y.view(rows, width)
    for t, name in ((o2, "o"), (g2, "gate"), (y2, "out")):
        _aligned(t, name)
    rc = nat.lib().sophia_gated_head_norm(
        nat.ptr(o2), os_, nat.dtype_code(o.dtype), nat.ptr(g2), gs, nat.ptr(w), float(eps),
        nat.ptr(y2), width, rows, int(heads), int(head_dim), nat.dtype_code(gate.dtype),
        nat.stream_handle(gate.device))
    nat.check(rc, "sophia_gated_head_norm")
    return y2


def mla_decode_attn(qa: torch.Tensor, latent_cache: torch.Tensor, slots: torch.Tensor,
                    pos: torch.Tensor, scale: float, *, max_len: int | None = None,
                    splits: int | None = None, out_dtype: torch.dtype | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Absorbed MLA decode attention in latent space (the decode rows of
    SophiaMLA, ml/runtime/model/attention.py:609-657, with k = W_k c and
    v = W_v c folded out): for row b and head h,
    softmax_k(scale * qa[b, h] . latent[slots[b], k]) over k = 0..pos[b], then
    the probability-weighted sum of those latents.

    qa: [rows, heads, rank] (bf16 or fp32, heads <= 16, rank in 32/64/128/256);
    latent_cache: [n_slots, max_seq, rank] fp32 with dense rows; slots int32
    [rows]; pos int64 [rows].  ``max_len`` (host int, an upper bound on
    pos + 1) sizes the key splits; ``splits`` overrides them.  Returns
    [rows, heads, rank] in ``out_dtype`` (default qa.dtype)."""
    _gpu(qa, "qa")
    _gpu(latent_cache, "latent_cache")
    if qa.dim() != 3:
        raise RuntimeError(f"qa must be [rows, heads, rank], got {tuple(qa.shape)}")
    rows, heads, rank = (int(v) for v in qa.shape)
    if (latent_cache.dim() != 3 or latent_cache.dtype != torch.float32
            or int(latent_cache.size(2)) != rank or latent_cache.stride(2) != 1
            or latent_cache.stride(1) != rank):
        raise RuntimeError(f"latent_cache must be fp32 [slots, max_seq, {rank}] with dense rows")
    if qa.stride(2) != 1 or (heads > 1 and qa.stride(1) != rank):
        qa = qa.contiguous()
    qs = int(qa.stride(0)) if rows > 1 else heads * rank
    sl = _int32(slots, "slots", qa.device)
    if pos.dtype != torch.int64 or pos.device != qa.device or not pos.is_contiguous():
        raise RuntimeError("pos must be a contiguous int64 tensor on the device")
    if int(sl.numel()) != rows or int(pos.numel()) != rows:
        raise RuntimeError("slots and pos must hold one entry per row")
    n_slots, max_seq = int(latent_cache.size(0)), int(latent_cache.size(1))
    if splits is None:
        # One work-group per row once the rows fill the chip (the merge of
        # split partials costs more than it saves there); fewer rows split
        # their keys so that about 256 work-groups run.
        bound = max_seq if max_len is None else min(int(max_len), max_seq)
        splits = 1 if rows >= 128 else max(1, min(-(-256 // max(rows, 1)), -(-bound // 256)))
    dt = qa.dtype if out_dtype is None else out_dtype
    if out is not None and (not out.is_contiguous() or out.dtype != dt
                            or tuple(out.shape) != (rows, heads, rank)):
        raise RuntimeError(f"out must be contiguous {dt} [{rows}, {heads}, {rank}]")
    y = out if out is not None else torch.empty((rows, heads, rank), dtype=dt, device=qa.device)
    ws_bytes = int(nat.lib().sophia_mla_decode_workspace_size(rows, rank, int(splits)))
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=qa.device) if ws_bytes else None
    _aligned(qa, "qa")
    _aligned(latent_cache, "latent_cache")
    rc = nat.lib().sophia_mla_decode_attn(
        nat.ptr(qa), qs, nat.dtype_code(qa.dtype), nat.ptr(latent_cache),
        int(latent_cache.stride(0)) if n_slots > 1 else max_seq * rank, n_slots, max_seq,
        nat.ptr(sl), nat.ptr(pos), float(scale), nat.ptr(y), heads * rank, nat.dtype_code(dt), rows,
        heads, rank, int(splits), nat.ptr(ws), ws_bytes, nat.stream_handle(qa.device))
    nat.check(rc, "sophia_mla_decode_attn")
    return y


def gated_head_norm_bwd(d_out: torch.Tensor, o: torch.Tensor, gate: torch.Tensor, heads: int,
                        head_dim: int, *, norm_weight: torch.Tensor | None = None,
                        eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Backward of ``gated_head_norm`` (sophia_gated_head_norm_bwd): for the
    output gradient ``d_out`` [rows, heads * head_dim] (gate's dtype), returns
    (d_o in o's shape and dtype, d_gate in gate's shape and dtype, d_norm_weight
    [head_dim] fp32 or None without the norm)."""
    _gpu(o, "o")
    _gpu(gate, "gate")
    _gpu(d_out, "d_out")
    width = int(heads) * int(head_dim)
    o2 = o.reshape(-1, width)
    g2 = gate.reshape(-1, width)
    rows = int(g2.size(0))
    if int(o2.size(0)) != rows:
        raise RuntimeError(f"o has {int(o2.size(0))} rows, gate {rows}")
    d2 = d_out.reshape(-1, width)
    if d2.dtype != gate.dtype or int(d2.size(0)) != rows:
        raise RuntimeError(f"d_out must be {gate.dtype} with {rows} rows of {width}")
    os_ = _rows(o2, "o", width)
    gs = _rows(g2, "gate", width)
    ds = _rows(d2, "d_out", width)
    if o.dtype not in (torch.float32, gate.dtype):
        raise RuntimeError("o must be float32 or gate's dtype")
    w = None
    if norm_weight is not None:
        w = norm_weight.detach().reshape(-1).to(device=gate.device, dtype=torch.float32).contiguous()
        if int(w.numel()) != int(head_dim):
            raise RuntimeError(f"norm_weight must hold {head_dim} values")
        _aligned(w, "norm_weight")
    d_o = torch.empty((rows, width), dtype=o.dtype, device=o.device)
    d_g = torch.empty((rows, width), dtype=gate.dtype, device=gate.device)
    d_w = torch.empty((int(head_dim),), dtype=torch.float32, device=gate.device) if w is not None else None
    for t, name in ((o2, "o"), (g2, "gate"), (d2, "d_out")):
        _aligned(t, name)
    lib = nat.lib()
    need = int(lib.sophia_gated_head_norm_bwd_workspace_size(rows, int(heads), int(head_dim)))
    buf, ws_addr, ws_bytes = _workspace(need, gate.device)
    rc = lib.sophia_gated_head_norm_bwd(
        nat.ptr(d2), ds, nat.ptr(o2), os_, nat.dtype_code(o.dtype), nat.ptr(g2), gs, nat.ptr(w), float(eps),
        nat.ptr(d_o), width, nat.ptr(d_g), width, nat.ptr(d_w), rows, int(heads), int(head_dim),
        nat.dtype_code(gate.dtype), ws_addr, ws_bytes, nat.stream_handle(gate.device))
    nat.check(rc, "sophia_gated_head_norm_bwd")
    del buf
    return d_o.view(o.shape), d_g.view(gate.shape), d_w


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                     max_len: int, *, scale: float | None = None,
                     cu_seqlens_k: torch.Tensor | None = None,
                     out: torch.Tensor | None = None, cu_seqlens_host: torch.Tensor | None = None,
                     cu_seqlens_k_host: torch.Tensor | None = None) -> torch.Tensor:
    """Causal self-attention within each packed sequence (the prefill
    attention of SophiaMLA, ml/runtime/model/attention.py:630-654,
    ``scaled_dot_product_attention`` with a causal mask).

    q: [rows, heads, 128] bf16, the queries of the sequences delimited by
    ``cu_seqlens`` (int32, device); k, v: the keys and values, delimited by
    ``cu_seqlens_k`` (default: the same rows as q).  A sequence with more keys
    than queries continues after cached tokens: its queries are the last
    positions of its key range (the tril(keys - queries) mask).  ``max_len``
    (host int) must bound every sequence's query count.  Returns [rows, heads,
    128] bf16 (or writes ``out``, which may be a row-strided view).

    Every sequence needs at least as many keys as queries.  With the host
    copies of the offsets (``cu_seqlens_host``, ``cu_seqlens_k_host``) that is
    checked here (RuntimeError); without them the kernel writes zeros for the
    rows of a sequence that has fewer keys than queries."""
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _gpu(t, name)
        if t.dtype != torch.bfloat16:
            raise RuntimeError(f"{name} must be bfloat16")
    total, heads, hd = (int(x) for x in q.shape)
    if hd != 128:
        raise RuntimeError("causal_attention is built for head_dim 128")
    qs = _heads_rows(q, "q", heads, hd)
    ks = _heads_rows(k, "k", heads, hd)
    vs = _heads_rows(v, "v", heads, hd)
    total_k = int(k.size(0))
    if int(v.size(0)) != total_k:
        raise RuntimeError("k and v must have the same number of rows")
    cu = _int32(cu_seqlens, "cu_seqlens", q.device)
    cuk = _int32(cu_seqlens_k, "cu_seqlens_k", q.device)
    if cuk is None and total_k != total:
        raise RuntimeError("q, k and v must have the same number of rows without cu_seqlens_k")
    if cuk is not None and int(cuk.numel()) != int(cu.numel()):
        raise RuntimeError("cu_seqlens_k must have as many entries as cu_seqlens")
    if cu_seqlens_host is not None:
        qo = torch.as_tensor(cu_seqlens_host).to("cpu", torch.int64)
        ko = qo if cu_seqlens_k_host is None else torch.as_tensor(cu_seqlens_k_host).to("cpu", torch.int64)
        if int(qo.numel()) != int(cu.numel()) or int(ko.numel()) != int(cu.numel()):
            raise RuntimeError("host offsets must have as many entries as cu_seqlens")
        if bool(((ko[1:] - ko[:-1]) < (qo[1:] - qo[:-1])).any()):
            raise RuntimeError("every sequence needs at least as many keys as queries")
    y = out if out is not None else torch.empty((total, heads, hd), dtype=q.dtype, device=q.device)
    if y.dtype != torch.bfloat16 or tuple(y.shape) != (total, heads, hd):
        raise RuntimeError(f"out must be bfloat16 [{total}, {heads}, {hd}]")
    os_ = _heads_rows(y, "out", heads, hd)
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _aligned(t, name)
    rc = nat.lib().sophia_causal_attention(
        nat.ptr(q), qs, nat.ptr(k), ks, nat.ptr(v), vs, nat.ptr(y), os_, nat.ptr(cu), nat.ptr(cuk),
        int(cu.numel()) - 1, total, total_k, int(max_len), heads, hd,
        float(hd ** -0.5 if scale is None else scale), nat.DTYPE_BF16, nat.stream_handle(q.device))
    nat.check(rc, "sophia_causal_attention")
    return y


from . import torch_ops  # noqa: E402  (registers the sophia:: custom ops; imports this module)
