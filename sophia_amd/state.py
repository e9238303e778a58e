"""Cache snapshot types at the mixer boundary (the reference's
ml/runtime/model/state.py:14-122): per-layer ``recurrent`` / ``conv`` /
``latent`` tensors and the ``layer_{i}_{field}`` payload keys."""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass

import torch

_CACHE_SUFFIXES = (("_recurrent", "recurrent"), ("_conv", "conv"), ("_latent", "latent"))


def _clone(value: torch.Tensor | None) -> torch.Tensor | None:
    return None if value is None else value.detach().clone()


@dataclass(frozen=True)
class LayerCacheSnapshot:
    recurrent: torch.Tensor | None = None
    conv: torch.Tensor | None = None
    latent: torch.Tensor | None = None

    def clone(self) -> "LayerCacheSnapshot":
        return LayerCacheSnapshot(_clone(self.recurrent), _clone(self.conv), _clone(self.latent))

    def tensor_fields(self):
        return (("recurrent", self.recurrent), ("conv", self.conv), ("latent", self.latent))

    def is_empty(self) -> bool:
        return all(value is None for _, value in self.tensor_fields())

    def batch_size(self) -> int:
        return max((int(v.size(0)) for _, v in self.tensor_fields() if v is not None), default=0)

    def to_payload(self, *, prefix: str) -> dict[str, torch.Tensor]:
        return {f"{prefix}_{name}": v.detach().clone() for name, v in self.tensor_fields()
                if v is not None}

    @classmethod
    def from_field_map(cls, field_map: Mapping[str, object] | None):
        if field_map is None:
            return None
        values = {}
        for name in ("recurrent", "conv", "latent"):
            value = field_map.get(name)
            if value is not None and not torch.is_tensor(value):
                raise TypeError(f"layer cache field {name!r} must be a tensor or None")
            values[name] = _clone(value)
        snap = cls(**values)
        return None if snap.is_empty() else snap


@dataclass(frozen=True)
class RuntimeCacheSnapshot:
    layers: tuple = ()

    def to_payload(self) -> dict[str, torch.Tensor]:
        payload: dict[str, torch.Tensor] = {}
        for index, item in enumerate(self.layers):
            if item is not None and not item.is_empty():
                payload.update(item.to_payload(prefix=f"layer_{index}"))
        return payload

    @classmethod
    def from_payload(cls, payload: Mapping[str, object]) -> "RuntimeCacheSnapshot":
        by_layer: dict[int, dict[str, object]] = {}
        for raw_key, value in payload.items():
            key = str(raw_key)
            for suffix, field in _CACHE_SUFFIXES:
                if key.endswith(suffix):
                    prefix = key[: -len(suffix)]
                    if not prefix.startswith("layer_"):
                        break
                    by_layer.setdefault(int(prefix[len("layer_"):]), {})[field] = value
                    break
            else:
                raise ValueError(f"unrecognized runtime cache payload key: {key}")
        if not by_layer:
            return cls()
        layers = [None] * (max(by_layer) + 1)
        for index, fields in by_layer.items():
            layers[index] = LayerCacheSnapshot.from_field_map(fields)
        return cls(layers=tuple(layers))


__all__ = ["LayerCacheSnapshot", "RuntimeCacheSnapshot"]
