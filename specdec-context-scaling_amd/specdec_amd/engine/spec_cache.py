"""Cache-length / trim / consistency API (mirror of specdec/engine/spec_cache.py:4-46).

Same signatures, semantics and errors as the reference, per the contract in
docs/design_g4_cache_api.md:13-28:

* ``cache_length(None) == 0``; otherwise ``cache[0]["k"].shape[2]``;
* ``trim_cache(None, 0) is None``; ``trim_cache(None, n > 0)`` raises ValueError;
  ``new_len`` must be an int (not bool) with ``0 < new_len <= length`` (ValueError);
  returns a NEW list of NEW dicts whose tensors are sliced ``[:, :, :new_len]`` (views) and
  whose other values (``"fmt"``, the page pool handle) are kept; the input is not mutated;
* ``check_consistent`` raises RuntimeError if any >=3-D tensor disagrees on dim 2 within a
  layer or across layers.

The paged v_fp8 cache satisfies this contract unchanged: its ``"k"``, ``"v"`` and
``"v_scale"`` entries are zero-storage tensors of the logical shapes (B,KV,T,D) / (B,KV,T,1)
(``expand`` of a single element), so slicing them trims the logical length while the pages
stay in the shared pool handle under ``"pages"``.  ``check_consistent`` additionally
verifies, for paged layers, that the pool has reserved slots for every logical token.
"""
from __future__ import annotations

import torch


def cache_length(cache) -> int:
    if cache is None:
        return 0
    return int(cache[0]["k"].shape[2])


def trim_cache(cache, new_len: int):
    if cache is None:
        if new_len == 0:
            return None
        raise ValueError("trim_cache(None, n > 0) is not a valid request")
    if not isinstance(new_len, int) or isinstance(new_len, bool):
        raise ValueError("new_len must be an int")
    cur = cache_length(cache)
    if new_len <= 0 or new_len > cur:
        raise ValueError(f"new_len {new_len} out of range (current {cur})")
    trimmed = []
    for layer in cache:
        trimmed.append({key: (val[:, :, :new_len] if isinstance(val, torch.Tensor) else val)
                        for key, val in layer.items()})
    return trimmed


def check_consistent(cache) -> None:
    if cache is None:
        return
    per_layer = []
    for i, layer in enumerate(cache):
        dims = [(key, int(val.shape[2])) for key, val in layer.items()
                if isinstance(val, torch.Tensor) and val.dim() >= 3]
        if len({d for _, d in dims}) != 1:
            raise RuntimeError(f"cache token dim mismatch at layer {i}: {dims}")
        per_layer.append(dims[0][1])
        pages = layer.get("pages")
        if pages is not None:
            have = pages.reserved_tokens()
            if have < dims[0][1]:
                raise RuntimeError(f"paged layer {i} covers {dims[0][1]} tokens but only {have} slots are reserved")
    if len(set(per_layer)) != 1:
        raise RuntimeError(f"cross-layer token length mismatch: {per_layer}")
