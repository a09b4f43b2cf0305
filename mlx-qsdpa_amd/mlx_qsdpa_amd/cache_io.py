"""Saving and loading quantized caches through ``state`` / ``meta_state``.

A list of caches (one per layer) goes to one safetensors file: each
cache's ``state`` tensors under "<layer>.<name>" keys, its class name and
``meta_state`` strings in the file's metadata.  Loading rebuilds every
cache with ``Class.from_state(state, meta_state)`` -- the protocol of
mlx_qsdpa/cache.py:127-156, which the reference defines for
QuantizedSDPACache; the three other caches here gain the same pair.
Rotating caches save their windows in temporal order and come back with
the ring unrotated.  Only safetensors is read: nothing in a file executes.
"""

from __future__ import annotations

import json

import torch
from safetensors.torch import load_file, save_file

from . import cache as _cache

_CLASSES = {c.__name__: c for c in (_cache.QuantizedSDPACache, _cache.BatchQuantizedSDPACache,
                                   _cache.QuantizedRotatingSDPACache,
                                   _cache.BatchQuantizedRotatingSDPACache)}
_KV = ("keys", "values")
_PARTS = ("packed", "scales", "biases")


def save_cache(path, caches, metadata=None) -> None:
    """Write `caches` (a list) and optional string `metadata` to `path`."""
    tensors, layers = {}, []
    for i, c in enumerate(caches):
        name = type(c).__name__
        if name not in _CLASSES:
            raise TypeError(f"cannot save a {name}")
        st = c.state
        for j, kv in enumerate(_KV):
            if st[j] is not None:
                for part, t in zip(_PARTS, st[j]):
                    tensors[f"{i}.{kv}.{part}"] = t.contiguous()
        extra = [f"{i}.offset", f"{i}.left_padding"] if len(st) == 4 else []
        for key, t in zip(extra, st[2:]):
            tensors[key] = torch.as_tensor(t, dtype=torch.int64).contiguous()
        layers.append({"class": name, "meta_state": list(c.meta_state), "empty": st[0] is None})
    meta = {"qsdpa_caches": json.dumps(layers)}
    meta.update({str(k): str(v) for k, v in (metadata or {}).items()})
    save_file(tensors, str(path), metadata=meta)


def load_cache(path, device=None, return_metadata=False):
    """The caches written by save_cache, on `device` (default: as saved)."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt") as f:
        meta = dict(f.metadata() or {})
    tensors = load_file(str(path), device="cpu")
    layers = json.loads(meta.pop("qsdpa_caches"))
    caches = []
    for i, layer in enumerate(layers):
        cls = _CLASSES[layer["class"]]

        def get(key):
            t = tensors[f"{i}.{key}"]
            return t if device is None else t.to(device)

        kv = [None, None] if layer["empty"] else [tuple(get(f"{kv}.{p}") for p in _PARTS) for kv in _KV]
        if f"{i}.offset" in tensors:
            state = (kv[0], kv[1], tensors[f"{i}.offset"], tensors[f"{i}.left_padding"])
        else:
            state = (kv[0], kv[1])
        caches.append(cls.from_state(state, tuple(layer["meta_state"])))
    return (caches, meta) if return_metadata else caches
