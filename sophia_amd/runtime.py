"""Continuous-batching runtime around the hybrid decoder.

``SlotAllocator`` hands out and takes back the cache slots that
``Transformer.forward_step`` indexes (every KDA recurrent state, conv history
and MLA latent cache has one row per slot), growing the model's caches when
all slots are taken and zeroing a slot's KDA caches when it is handed out.

``RuntimeCacheState`` and ``forward_cached_decode`` are the functional cached
decode of the reference (ml/modeling/cache_decode.py:12-143): a step takes the
tokens and the cache state the previous step returned, loads that state,
advances it and returns the logits with the new state.  The reference runs
tokens after the first step one position at a time (its model takes T > 1
only at start_pos 0, runtime_host.py:146-170); here every step is one
``forward_step``, whatever its number of tokens.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .decoder import Transformer
from .state import RuntimeCacheSnapshot


class SlotAllocator:
    """Cache slots of ``model`` for continuous batching (host bookkeeping).

    ``allocate(n)`` returns n free slots (int32, on the model's device),
    lowest numbers first, with their KDA caches zeroed; when fewer than n are
    free the model's caches grow (``Transformer.ensure_batch_capacity``, at
    least doubling).  ``release(slots)`` returns them.  Slot numbers stay
    valid for as long as they are held."""

    def __init__(self, model: Transformer) -> None:
        self.model = model
        self._capacity = int(model.runtime_batch_capacity())
        self._free = list(range(self._capacity - 1, -1, -1))
        self._held: set[int] = set()

    @property
    def capacity(self) -> int:
        return self._capacity

    @property
    def in_use(self) -> int:
        return len(self._held)

    def held(self) -> list[int]:
        return sorted(self._held)

    def allocate(self, n: int) -> torch.Tensor:
        n = int(n)
        if n < 0:
            raise ValueError(f"cannot allocate {n} slots")
        if n > len(self._free):
            grown = max(2 * self._capacity, len(self._held) + n)
            self.model.ensure_batch_capacity(grown)
            self._free = list(range(grown - 1, self._capacity - 1, -1)) + self._free
            self._capacity = grown
        taken = [self._free.pop() for _ in range(n)]
        self._held.update(taken)
        dev = self.model.tok_embeddings.weight.device
        slots = torch.tensor(taken, dtype=torch.int32, device=dev)
        if n:
            self.model.reset_slots(slots)
        return slots

    def release(self, slots) -> None:
        values = [int(s) for s in (slots.tolist() if isinstance(slots, torch.Tensor) else slots)]
        if len(set(values)) != len(values):
            raise ValueError(f"slots released twice in one call: {sorted(values)}")
        for s in values:
            if s not in self._held:
                raise ValueError(f"slot {s} is not held")
        for s in values:
            self._held.remove(s)
            self._free.append(s)
        self._free.sort(reverse=True)


@dataclass
class RuntimeCacheState:
    """A decode's cache between steps (cache_decode.py:12-16)."""

    cache: RuntimeCacheSnapshot
    batch_size: int
    cache_pos: int

    def clone(self) -> "RuntimeCacheState":
        return RuntimeCacheState(cache=self.cache.clone(), batch_size=int(self.batch_size),
                                 cache_pos=int(self.cache_pos))


def forward_cached_decode(*, model: Transformer, input_ids: torch.Tensor,
                          cache_state: RuntimeCacheState | None, start_pos: int | None,
                          logits_to_keep: int | None) -> tuple[torch.Tensor, RuntimeCacheState]:
    """One cached decode step (cache_decode.py:79-143): ``input_ids`` [B, T]
    continue the sequences held by ``cache_state`` (None: a fresh prefill,
    which needs start_pos 0 or None).  Returns (logits [B, T', vocab] -- the
    last ``logits_to_keep`` positions, all of them when it is None or 0 --,
    the new state, dumped to the host).  The same errors as the reference
    for inconsistent positions and batch sizes (ValueError)."""
    if logits_to_keep is not None and int(logits_to_keep) < 0:
        raise ValueError(f"logits_to_keep must be >= 0 when provided, got {logits_to_keep}")
    if input_ids.dim() != 2 or int(input_ids.size(1)) <= 0:
        raise ValueError("input_ids must be [B, T] with T >= 1")
    bsz, seqlen = int(input_ids.size(0)), int(input_ids.size(1))
    # Every check runs before the caches are touched or anything is launched.
    cache_pos = 0 if cache_state is None else int(cache_state.cache_pos)
    if cache_pos + seqlen > int(model.args.max_seq_len):
        raise ValueError("sequence exceeds max_seq_len")
    if cache_state is None:
        if start_pos is not None and int(start_pos) != 0:
            raise ValueError("cache_state is required when start_pos > 0 for cached decode")
        model.ensure_batch_capacity(bsz)
        model.reset_runtime_cache()
    else:
        if cache_pos < 0:
            raise ValueError(f"cache cache_pos must be >= 0, got {cache_pos}")
        if start_pos is not None and int(start_pos) != cache_pos:
            raise ValueError(f"start_pos ({start_pos}) must match cache cache_pos ({cache_pos})")
        cache_state = cache_state.clone()
        batch = int(cache_state.batch_size or bsz)
        if batch <= 0:
            raise ValueError(f"cache batch_size must be > 0, got {batch}")
        if batch != bsz:
            raise ValueError(f"cache batch_size does not match input_ids: {batch} != {bsz}")
        model.cache_load(cache_state.cache)
    dev = model.tok_embeddings.weight.device
    slots = torch.arange(bsz, dtype=torch.int32, device=dev)
    keep = 0 if logits_to_keep is None else int(logits_to_keep)
    ids = input_ids.to(dev)
    if seqlen == 1 and cache_pos > 0:
        logits = model.forward_step(decode_ids=ids[:, 0], decode_slots=slots,
                                    decode_pos=torch.full((bsz,), cache_pos, dtype=torch.long, device=dev),
                                    max_decode_len=cache_pos + 1).unsqueeze(1)
    else:
        logits = model.forward_step(prefill_ids=ids.reshape(-1), prefill_lens=[seqlen] * bsz,
                                    prefill_pos=[cache_pos] * bsz, prefill_slots=slots,
                                    all_logits=keep != 1)
        logits = logits.view(bsz, seqlen if keep != 1 else 1, -1)
    if keep > 0:
        logits = logits[:, -keep:, :]
    next_pos = cache_pos + seqlen
    return logits, RuntimeCacheState(cache=model.cache_dump(device="cpu", cache_pos=next_pos, batch_size=bsz),
                                     batch_size=bsz, cache_pos=next_pos)


__all__ = ["RuntimeCacheState", "SlotAllocator", "forward_cached_decode"]
