"""Paged FP8-V cache layout, restated in numpy (TEST INFRASTRUCTURE ONLY).

The reference keeps a contiguous per-layer cache ``{"k": (B,KV,T,D) bf16, "v": (B,KV,T,D)
fp8, "v_scale": (B,KV,T,1) fp32}`` grown by ``torch.cat`` (model_self.py:778-800,
docs/design_g4_cache_api.md:7-11).  This build stores the same bytes in pages of
``BLOCK = 16`` tokens per KV head, addressed through a block table:

* ``k_pages [num_blocks, KV, D/8, 16, 8]`` uint16 (BF16 bits): 8-dimension chunks, then
  tokens, then the 8 dimensions of the chunk;
* ``v_pages [num_blocks, KV, D, 16]``  uint8 (E4M3FN codes), dimension-major inside a page;
* ``v_scales[num_blocks, KV, 16]``     float32;
* a token's slot is ``block * 16 + offset``.

``write`` places per-token rows by slot mapping; ``gather`` rebuilds the contiguous cache of
one sequence from its block-table row.  Pinned by the write->gather round trip (closed
form: the contiguous input comes back bit for bit for any permutation of blocks).
"""
from __future__ import annotations

import numpy as np

BLOCK = 16


def alloc(num_blocks: int, kv_heads: int, head_dim: int):
    k_pages = np.zeros((num_blocks, kv_heads, head_dim // 8, BLOCK, 8), dtype=np.uint16)
    v_pages = np.zeros((num_blocks, kv_heads, head_dim, BLOCK), dtype=np.uint8)
    v_scales = np.zeros((num_blocks, kv_heads, BLOCK), dtype=np.float32)
    return k_pages, v_pages, v_scales


def write(k_pages, v_pages, v_scales, k_bits, v_payload, v_scale, slot_mapping) -> None:
    """k_bits (n,KV,D) uint16 or None; v_payload (n,KV,D) uint8; v_scale (n,KV) f32; slot < 0 skips."""
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = slots >= 0
    blk = slots[ok] // BLOCK
    off = slots[ok] % BLOCK
    if k_bits is not None:
        kb = np.asarray(k_bits)[ok]                         # (n, KV, D)
        k_pages[blk, :, :, off, :] = kb.reshape(kb.shape[0], kb.shape[1], -1, 8)
    v_pages[blk, :, :, off] = np.asarray(v_payload)[ok]
    v_scales[blk, :, off] = np.asarray(v_scale)[ok]


def gather(k_pages, v_pages, v_scales, block_row, seq_len: int):
    """-> k (KV,T,D) uint16, v (KV,T,D) uint8, s (KV,T) f32 for one sequence of length seq_len."""
    nb = -(-seq_len // BLOCK)
    blocks = np.asarray(block_row[:nb], dtype=np.int64)
    kv, d = k_pages.shape[1], k_pages.shape[2] * 8
    k = k_pages[blocks].transpose(1, 0, 3, 2, 4).reshape(kv, nb * BLOCK, d)[:, :seq_len]
    v = v_pages[blocks].transpose(1, 0, 3, 2).reshape(kv, nb * BLOCK, d)[:, :seq_len]
    s = v_scales[blocks].transpose(1, 0, 2).reshape(kv, nb * BLOCK)[:, :seq_len]
    return k, v, s


def slots_for(block_row, start: int, count: int) -> np.ndarray:
    """Slots of token positions start .. start+count-1 of a sequence with this block-table row."""
    pos = np.arange(start, start + count, dtype=np.int64)
    return np.asarray(block_row, dtype=np.int64)[pos // BLOCK] * BLOCK + pos % BLOCK
