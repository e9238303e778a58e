"""Cache snapshot types at the mixer boundary (the reference's
ml/runtime/model/state.py:14-122): payload keys and round trips.  CPU only."""

from __future__ import annotations

import pytest
import torch

from sophia_amd.state import LayerCacheSnapshot, RuntimeCacheSnapshot


def test_payload_roundtrip_keeps_layer_indices_and_fields():
    rec = torch.randn(2, 16, 128, 128)
    conv = torch.randn(2, 3, 2048, 3)
    lat = torch.randn(2, 7, 128)
    snap = RuntimeCacheSnapshot(layers=(LayerCacheSnapshot(recurrent=rec, conv=conv), None,
                                        None, LayerCacheSnapshot(latent=lat)))
    payload = snap.to_payload()
    assert sorted(payload) == ["layer_0_conv", "layer_0_recurrent", "layer_3_latent"]
    back = RuntimeCacheSnapshot.from_payload(payload)
    assert len(back.layers) == 4 and back.layers[1] is None and back.layers[2] is None
    assert torch.equal(back.layers[0].recurrent, rec) and torch.equal(back.layers[0].conv, conv)
    assert torch.equal(back.layers[3].latent, lat)
    # the payload holds copies, not views of the live buffers
    payload["layer_0_recurrent"].zero_()
    assert torch.equal(back.layers[0].recurrent, rec)


def test_payload_rejects_unknown_keys_and_non_tensors():
    with pytest.raises(ValueError, match="does not end in"):
        RuntimeCacheSnapshot.from_payload({"layer_0_state": torch.zeros(1)})
    # a known field suffix on a prefix other than layer_<i> is skipped, as the
    # reference's parser skips it (state.py:107-113)
    assert RuntimeCacheSnapshot.from_payload({"block_0_conv": torch.zeros(1)}).layers == ()
    with pytest.raises(TypeError):
        LayerCacheSnapshot.from_field_map({"recurrent": [1, 2, 3]})
    assert RuntimeCacheSnapshot.from_payload({}).layers == ()


def test_layer_snapshot_batch_size_and_empty():
    assert LayerCacheSnapshot().is_empty()
    assert LayerCacheSnapshot().batch_size() == 0
    snap = LayerCacheSnapshot(recurrent=torch.zeros(3, 1, 1, 1), conv=torch.zeros(5, 1, 1))
    assert snap.batch_size() == 5
    assert LayerCacheSnapshot.from_field_map({"recurrent": None, "conv": None}) is None


def test_payload_key_grammar():
    from sophia_amd.state import parse_payload_key, payload_key

    assert payload_key(12, "latent") == "layer_12_latent"
    assert parse_payload_key("layer_12_latent") == (12, "latent")
    assert parse_payload_key("layer_007_conv") == (7, "conv")
    # a known field after a foreign prefix is skipped
    assert parse_payload_key("block_3_recurrent") is None
    assert parse_payload_key("_conv") is None
    for bad in ("layer_x_conv", "layer__conv", "layer_-1_conv", "layer_1_conv_recurrent"):
        with pytest.raises(ValueError):
            parse_payload_key(bad)
    for bad in ("conv", "layer_0_state", "layer_0_Conv", ""):
        with pytest.raises(ValueError):
            parse_payload_key(bad)
    with pytest.raises(ValueError):
        payload_key(0, "state")


def test_payload_skips_foreign_prefix_but_keeps_layers():
    t = torch.ones(2, 3)
    back = RuntimeCacheSnapshot.from_payload({"block_9_conv": t, "layer_1_latent": t})
    assert len(back.layers) == 2 and back.layers[0] is None
    assert torch.equal(back.layers[1].latent, t) and back.layers[1].latent is not t
