"""Cache snapshots of the token mixers and their flat payload form.

A layer's cache is up to three tensors: the KDA ``recurrent`` state
[B, H, 128, 128], the KDA ``conv`` history [B, 3, 2048, 3] and the MLA
``latent`` cache [B, T, rank].  A whole model's snapshot flattens to a
``{str: Tensor}`` payload keyed ``layer_<index>_<field>`` -- the format of the
reference's runtime caches (ml/runtime/model/state.py:14-122), kept so that
payloads move between the two unchanged.

Payload grammar (what ``RuntimeCacheSnapshot.from_payload`` accepts):
  key    := prefix "_" field
  field  := "recurrent" | "conv" | "latent"      (otherwise: ValueError)
  prefix := "layer_" index                       (another prefix: key ignored)
  index  := decimal digits                       (otherwise: ValueError)
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from dataclasses import dataclass, fields

import torch

FIELDS = ("recurrent", "conv", "latent")
LAYER_PREFIX = "layer_"


def payload_key(index: int, field: str) -> str:
    """The payload key of one cache tensor of layer ``index``."""
    if field not in FIELDS:
        raise ValueError(f"cache field must be one of {FIELDS}, got {field!r}")
    return f"{LAYER_PREFIX}{int(index)}_{field}"


def parse_payload_key(key: str) -> tuple[int, str] | None:
    """(layer index, field) of a payload key; None for a key whose field is
    known but whose prefix is not ``layer_<index>`` (such keys are skipped).
    Raises ValueError for a key that names no cache field or whose layer
    index is not a decimal number."""
    head, sep, field = key.rpartition("_")
    if not sep or field not in FIELDS:
        raise ValueError(f"payload key {key!r} does not end in _recurrent, _conv or _latent")
    if not head.startswith(LAYER_PREFIX):
        return None
    digits = head[len(LAYER_PREFIX):]
    if not digits.isdigit():
        raise ValueError(f"payload key {key!r}: layer index {digits!r} is not a number")
    return int(digits), field


def _copy(t: torch.Tensor | None) -> torch.Tensor | None:
    return t.detach().clone() if t is not None else None


@dataclass(frozen=True)
class LayerCacheSnapshot:
    """The cache tensors of one mixer layer (None where the layer has none)."""

    recurrent: torch.Tensor | None = None
    conv: torch.Tensor | None = None
    latent: torch.Tensor | None = None

    def items(self) -> Iterator[tuple[str, torch.Tensor]]:
        """(field, tensor) for each field that holds a tensor."""
        for f in fields(self):
            t = getattr(self, f.name)
            if t is not None:
                yield f.name, t

    def tensor_fields(self) -> tuple[tuple[str, torch.Tensor | None], ...]:
        return tuple((name, getattr(self, name)) for name in FIELDS)

    def clone(self) -> "LayerCacheSnapshot":
        return LayerCacheSnapshot(**{name: _copy(t) for name, t in self.tensor_fields()})

    def is_empty(self) -> bool:
        return next(self.items(), None) is None

    def batch_size(self) -> int:
        """Rows of the largest cache tensor (0 for an empty snapshot)."""
        return max((int(t.shape[0]) for _, t in self.items()), default=0)

    def to_payload(self, *, prefix: str) -> dict[str, torch.Tensor]:
        """``{prefix_field: copy}`` for the fields that hold a tensor."""
        return {f"{prefix}_{name}": t.detach().clone() for name, t in self.items()}

    @classmethod
    def from_field_map(cls, field_map: Mapping[str, object] | None) -> "LayerCacheSnapshot | None":
        """Snapshot holding copies of ``field_map``'s tensors; None when the map
        is None or names no tensor.  A field holding something other than a
        tensor (or None) raises TypeError."""
        if field_map is None:
            return None
        chosen: dict[str, torch.Tensor | None] = {}
        for name in FIELDS:
            value = field_map.get(name)
            if value is not None and not isinstance(value, torch.Tensor):
                raise TypeError(f"cache field {name!r} holds {type(value).__name__}, "
                                "expected a tensor or None")
            chosen[name] = _copy(value)
        snap = cls(**chosen)
        return snap if not snap.is_empty() else None


@dataclass(frozen=True)
class RuntimeCacheSnapshot:
    """Per-layer cache snapshots of a whole model, indexed by layer number
    (None for a layer without a cache)."""

    layers: tuple = ()

    def clone(self) -> "RuntimeCacheSnapshot":
        return RuntimeCacheSnapshot(layers=tuple(None if layer is None else layer.clone()
                                                 for layer in self.layers))

    def is_empty(self) -> bool:
        return all(layer is None or layer.is_empty() for layer in self.layers)

    def batch_size(self) -> int:
        """Rows of the largest cache tensor over all layers (0 when empty)."""
        return max((layer.batch_size() for layer in self.layers if layer is not None), default=0)

    def to_payload(self) -> dict[str, torch.Tensor]:
        payload: dict[str, torch.Tensor] = {}
        for index, layer in enumerate(self.layers):
            if layer is None:
                continue
            for name, t in layer.items():
                payload[payload_key(index, name)] = t.detach().clone()
        return payload

    @classmethod
    def from_payload(cls, payload: Mapping[str, object]) -> "RuntimeCacheSnapshot":
        """Inverse of ``to_payload`` under the grammar in the module docstring;
        layers that no key names are None."""
        grouped: dict[int, dict[str, object]] = {}
        for key, value in payload.items():
            parsed = parse_payload_key(str(key))
            if parsed is None:
                continue
            index, field = parsed
            grouped.setdefault(index, {})[field] = value
        if not grouped:
            return cls()
        layers: list[LayerCacheSnapshot | None] = [None] * (max(grouped) + 1)
        for index, field_map in grouped.items():
            layers[index] = LayerCacheSnapshot.from_field_map(field_map)
        return cls(layers=tuple(layers))


__all__ = ["FIELDS", "LayerCacheSnapshot", "RuntimeCacheSnapshot", "parse_payload_key",
           "payload_key"]
