"""Pre-stacked layer weights (``src/foldjax/models/_stacking.py``).

The reference stacks every layer's parameters on a leading layer axis once,
at load time, so that ``lax.scan`` receives the weights already stacked
instead of concatenating them inside the traced graph
(``_stacking.py:1-22``, ``stacked_or_stack`` :148). Here the same idea
applies to packed HIP weights: ``StackedLayers`` holds one ``[L, ...]`` device
tensor per weight kind, and each layer's packed weight object is a set of
views into those tensors (no copies, one allocation per kind). It reads like
the layer list it replaces: a length, iteration and indexing.
"""

from __future__ import annotations

import dataclasses
from collections.abc import Iterator, Sequence
from typing import Any

import torch


def _is_packed(obj) -> bool:
    return dataclasses.is_dataclass(obj) and not isinstance(obj, type)


def _stack_leaf(leaves: Sequence[Any]):
    first = leaves[0]
    if first is None:
        if any(leaf is not None for leaf in leaves):
            raise ValueError("cannot stack mixed None/non-None layer leaves")
        return None, [None] * len(leaves)
    if isinstance(first, torch.Tensor):
        shapes = {tuple(t.shape) for t in leaves}
        dtypes = {t.dtype for t in leaves}
        devices = {t.device for t in leaves}
        if len(shapes) != 1 or len(dtypes) != 1 or len(devices) != 1:
            raise ValueError(f"cannot stack layer leaves of differing shape, dtype or device: {shapes}, {dtypes}")
        buf = torch.stack(list(leaves), 0).contiguous()
        return buf, [buf[i] for i in range(len(leaves))]
    if _is_packed(first):
        if any(type(leaf) is not type(first) for leaf in leaves):
            raise ValueError("cannot stack layers of differing structure")
        bufs, views = {}, [dict() for _ in leaves]
        grouped = set()
        # field groups a packed layer keeps back to back in one buffer (e.g.
        # the single attention's q|k|v|g, run as one projection GEMM) stay
        # back to back: one [L, len(group) * rows, ...] buffer, each layer's
        # fields consecutive slices of its row
        for group in getattr(type(first), "STACK_GROUPS", ()):
            parts = [[getattr(leaf, name) for name in group] for leaf in leaves]
            flat = [t for p in parts for t in p]
            if any(t is None for t in flat) or len({(tuple(t.shape), t.dtype, t.device) for t in flat}) != 1:
                continue
            buf = torch.stack([torch.cat(p, 0) for p in parts], 0).contiguous()
            bufs["|".join(group)] = buf
            for i in range(len(leaves)):
                for name, x in zip(group, buf[i].chunk(len(group), 0)):
                    views[i][name] = x
            grouped.update(group)
        for f in dataclasses.fields(first):
            if f.name in grouped:
                continue
            b, v = _stack_leaf([getattr(leaf, f.name) for leaf in leaves])
            bufs[f.name] = b
            for i, x in enumerate(v):
                views[i][f.name] = x
        return bufs, [type(first)(**v) for v in views]
    raise TypeError(f"cannot stack a layer leaf of type {type(first).__name__}")


class StackedLayers:
    """A homogeneous list of packed layers whose tensors share one
    ``[L, ...]`` buffer per weight kind (``_stacking.py:59-126``)."""

    __slots__ = ("stacked", "layers")

    def __init__(self, layers: Sequence[Any]):
        layers = list(layers)
        if not layers:
            raise ValueError("StackedLayers requires at least one layer")
        if not all(_is_packed(layer) for layer in layers):
            raise TypeError("StackedLayers takes packed layer weights (e.g. PairformerLayerWeights)")
        self.stacked, self.layers = _stack_leaf(layers)

    def __len__(self) -> int:
        return len(self.layers)

    def __bool__(self) -> bool:
        return bool(self.layers)

    def __iter__(self) -> Iterator[Any]:
        return iter(self.layers)

    def __getitem__(self, index):
        return self.layers[index]

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return f"StackedLayers(length={len(self.layers)})"


def _signature(obj):
    if obj is None:
        return None
    if isinstance(obj, torch.Tensor):
        return (tuple(obj.shape), obj.dtype, obj.device)
    if _is_packed(obj):
        return (type(obj),) + tuple((f.name, _signature(getattr(obj, f.name))) for f in dataclasses.fields(obj))
    return (type(obj),)


def stackable(layers: Sequence[Any]) -> bool:
    """Whether ``layers`` are packed weights of one structure whose tensors
    match in shape, dtype and device (what ``StackedLayers`` needs)."""
    layers = list(layers)
    if not layers or not all(_is_packed(layer) for layer in layers):
        return False
    first = _signature(layers[0])
    return all(_signature(layer) == first for layer in layers[1:])


def stacked_or_stack(layers) -> StackedLayers:
    """``_stacking.py:148``: the stacked form of ``layers``, stacking only if
    needed (a ``StackedLayers`` is returned unchanged)."""
    if isinstance(layers, StackedLayers):
        return layers
    layers = list(layers)
    if not layers:
        raise ValueError("cannot stack an empty layer list")
    return StackedLayers(layers)
