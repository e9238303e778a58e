"""Host bookkeeping of the continuous-batching slot allocator (CPU, no kernel
launch): a stand-in model records the calls SlotAllocator makes to it."""

from __future__ import annotations

import types

import pytest
import torch

from sophia_amd.runtime import SlotAllocator


class _Model:
    """The four things SlotAllocator uses: the cache capacity, its growth, the
    zeroing of handed-out slots and the embedding's device."""

    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.grown: list[int] = []
        self.reset: list[list[int]] = []
        self.tok_embeddings = types.SimpleNamespace(weight=torch.empty(1))

    def runtime_batch_capacity(self) -> int:
        return self.capacity

    def ensure_batch_capacity(self, n: int) -> None:
        self.grown.append(n)
        self.capacity = max(self.capacity, n)

    def reset_slots(self, slots: torch.Tensor) -> None:
        self.reset.append(slots.tolist())


def test_allocate_lowest_first_grows_and_zeroes():
    model = _Model(2)
    alloc = SlotAllocator(model)
    assert alloc.allocate(2).tolist() == [0, 1]
    assert model.grown == [] and model.reset == [[0, 1]]
    # three more than the two free: the caches at least double
    more = alloc.allocate(3)
    assert more.dtype == torch.int32 and more.tolist() == [2, 3, 4]
    assert model.grown == [5] and alloc.capacity == 5 and alloc.in_use == 5
    alloc.release(torch.tensor([1, 3], dtype=torch.int32))
    assert alloc.held() == [0, 2, 4]
    # freed slots come back lowest first and are zeroed again
    assert alloc.allocate(1).tolist() == [1]
    assert model.reset[-1] == [1]
    assert alloc.allocate(0).numel() == 0 and model.reset[-1] == [1]


def test_release_rejects_foreign_and_repeated_slots():
    alloc = SlotAllocator(_Model(4))
    alloc.allocate(3)
    with pytest.raises(ValueError):
        alloc.release([3])          # never handed out
    with pytest.raises(ValueError):
        alloc.release([1, 1])       # the same slot twice in one call
    assert alloc.held() == [0, 1, 2]  # a rejected call releases nothing
    alloc.release([1])
    with pytest.raises(ValueError):
        alloc.release([1])          # already released
    with pytest.raises(ValueError):
        alloc.allocate(-1)
