"""Model arguments of the Sophia hybrid decoder and its KDA mixer (the
reference's ``ModelArgs``, ml/runtime/model/config.py:8-45, with the value
checks of ml/core/spec/semantics/__init__.py:55-124 that concern them)."""

from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass
class ModelArgs:
    vocab_size: int = 65536
    n_layers: int = 28
    ffn_hidden: int = 3968
    mla_q_rank: int = 384
    mla_kv_rank: int = 128
    attn_res_block_size: int = 4
    situ_gate_softcap: float = 4.0
    situ_up_softcap: float = 25.0
    dropout: float = 0.0
    dim: int = 1536
    num_heads: int = 16
    head_dim: int = 128
    kda_decay_rank: int = 128
    kda_output_gate_rank: int = 128
    kda_output_gate_full_rank: bool = True
    kda_decay_lower_bound: float = -5.0
    kda_dt_min: float = 1e-3
    kda_dt_max: float = 1e-1
    kda_dt_floor: float = 1e-4
    kda_a_log_init: float = 0.0
    short_conv_kernel: int = 4
    norm_eps: float = 1e-5
    max_seq_len: int = 4096
    max_batch_size: int = 4
    initializer_range: float = 0.02
    kda_backend: str = "auto"
    use_cache: bool = True

    def __post_init__(self) -> None:
        for name in ("vocab_size", "n_layers", "ffn_hidden", "mla_q_rank", "mla_kv_rank",
                     "attn_res_block_size", "dim", "num_heads", "head_dim", "kda_decay_rank",
                     "kda_output_gate_rank", "short_conv_kernel", "max_seq_len", "max_batch_size"):
            value = int(getattr(self, name))
            if value <= 0:
                raise ValueError(f"{name} must be > 0, got {value}")
            setattr(self, name, value)
        lb = float(self.kda_decay_lower_bound)
        if not -5.0 <= lb < 0.0:
            raise ValueError(f"kda_decay_lower_bound must be in [-5, 0), got {lb}")
        for name in ("kda_dt_min", "kda_dt_max", "kda_dt_floor"):
            value = float(getattr(self, name))
            if not math.isfinite(value) or value <= 0.0:
                raise ValueError(f"{name} must be finite and > 0, got {value}")
        if self.kda_dt_min > self.kda_dt_max:
            raise ValueError(f"kda_dt_min must be <= kda_dt_max, got {self.kda_dt_min} > {self.kda_dt_max}")
        if self.kda_dt_floor > self.kda_dt_min:
            raise ValueError(f"kda_dt_floor must be <= kda_dt_min, got {self.kda_dt_floor} > {self.kda_dt_min}")
        if not math.isfinite(float(self.kda_a_log_init)):
            raise ValueError("kda_a_log_init must be finite")
        if not math.isfinite(float(self.norm_eps)) or float(self.norm_eps) <= 0.0:
            raise ValueError("norm_eps must be finite and > 0")
        if str(self.kda_backend) not in {"auto", "reference", "fla"}:
            raise ValueError(f"kda_backend must be one of auto/reference/fla, got {self.kda_backend!r}")
        if int(self.short_conv_kernel) > 4:
            raise ValueError("short_conv_kernel must be <= 4 (the HIP ShortConv kernels take at most 4 taps)")
        if int(self.head_dim) != 128:
            raise ValueError("the gfx950 KDA kernels are built for head_dim = 128")

    def layer_type(self, layer_idx: int) -> str:
        """config.py:51-52 of the reference: layer i is MLA iff i % 4 == 3."""
        return "mla" if int(layer_idx) % 4 == 3 else "kda"

    @property
    def attention_inner_dim(self) -> int:
        return int(self.num_heads) * int(self.head_dim)

    def ensure_runtime_batch_capacity(self, batch_size: int) -> int:
        required = int(batch_size)
        if required <= 0:
            raise ValueError(f"batch_size must be > 0, got {required}")
        self.max_batch_size = max(int(self.max_batch_size), required)
        return int(self.max_batch_size)


__all__ = ["ModelArgs"]
