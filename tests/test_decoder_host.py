"""Host logic of the decoder (CPU tensors, no kernel launch): the in-place
append of depth blocks that replaces torch.cat((completed, partial), dim=-2)
of blocks.py:73-76."""

from __future__ import annotations

import torch

from sophia_amd.decoder import _append_block, depth_store


def test_depth_store_appends_in_place_and_matches_cat():
    torch.manual_seed(0)
    hidden = torch.randn(2, 5, 16)
    completed = depth_store(hidden, n_layers=12, block_size=4)  # room for 3 blocks
    assert completed.shape == (2, 5, 0, 16)
    ref = hidden.new_empty(2, 5, 0, 16)
    base = completed.untyped_storage().data_ptr()
    for i in range(3):
        partial = torch.randn(2, 5, 16)
        completed = _append_block(completed, partial)
        ref = torch.cat((ref, partial.unsqueeze(-2)), dim=-2)
        assert completed.untyped_storage().data_ptr() == base, "block was not appended in place"
        assert torch.equal(completed, ref)
    # The store is full: the next append falls back to a concatenation.
    partial = torch.randn(2, 5, 16)
    grown = _append_block(completed, partial)
    assert grown.untyped_storage().data_ptr() != base
    assert torch.equal(grown, torch.cat((ref, partial.unsqueeze(-2)), dim=-2))
    # The earlier view is untouched by later appends.
    assert torch.equal(completed, ref)


def test_append_to_plain_tensor_concatenates():
    completed = torch.randn(4, 2, 8)  # dense: rows spaced by exactly two blocks
    partial = torch.randn(4, 8)
    out = _append_block(completed, partial)
    assert torch.equal(out, torch.cat((completed, partial.unsqueeze(-2)), dim=-2))
    assert out.untyped_storage().data_ptr() != completed.untyped_storage().data_ptr()
    empty = torch.empty(3, 0, 8)
    out = _append_block(empty, torch.ones(3, 8))
    assert torch.equal(out, torch.ones(3, 1, 8))


def test_append_with_flattened_token_rows():
    """The mixed step's [tokens, blocks, dim] layout, one token row."""
    hidden = torch.randn(1, 32)
    completed = depth_store(hidden, n_layers=8, block_size=4)
    a, b = torch.randn(1, 32), torch.randn(1, 32)
    completed = _append_block(_append_block(completed, a), b)
    assert torch.equal(completed, torch.stack((a, b), dim=-2))
