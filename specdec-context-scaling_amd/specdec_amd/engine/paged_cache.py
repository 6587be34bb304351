"""Paged FP8-V KV cache: page pool, block allocator and block tables.

The reference keeps, per layer, ``{"fmt": "v_fp8", "k": BF16 (B,KV,T,D), "v": fp8 (B,KV,T,D),
"v_scale": fp32 (B,KV,T,1)}`` and grows it with ``torch.cat`` every step
(specdec/engine/model_self.py:778-800; docs/design_g4_cache_api.md:7-11).  This module
stores the same bytes in pages of 16 tokens per KV head so an append writes only the new
slots and attention reads pages in place:

    k_pages  (L, num_blocks, KV, D/8, 16, 8)  BF16 (8-dimension chunks x tokens x 8)
    v_pages  (L, num_blocks, KV, D, 16)  E4M3FN codes (uint8), dimension-major per page
    v_scales (L, num_blocks, KV, 16)     fp32

All L layers share one block table per sequence (a token occupies the same slot in every
layer).  The allocator hands out blocks from a free list; with ``seed`` the free list is a
seeded permutation, which scatters a sequence's blocks the way a long-running server's
fragmented pool does.  When the pool runs out it doubles (new page tensors, one copy).

Recording into a HIP graph: ``append_attend`` takes each new token's slot from the block
table on the device and, with equal lengths, passes no length array, and the pool owns its
attention workspace, so a decode or verify step copies nothing from the host and allocates
nothing.  What it cannot do inside a recording -- add blocks (a new block table is copied
from the host), grow the pool (new page tensors), grow the workspace -- raises instead;
``reserve_all`` and ``workspace`` before recording make room.

Ownership rule (the reference's trim returns views and its appends build new tensors, so an
untrimmed handle keeps its data; here appends write pages in place): after
``trim``/``set_length`` to n tokens, the next append overwrites slots n.. of that sequence,
so any handle that still covers those positions sees the new tokens.  The SpecDec loop
never reuses a pre-trim handle (specdec/engine/spec_dec.py:238,246).
"""
from __future__ import annotations

import random

import torch

from .._native import SdvError
from ..kernels import ops

BLOCK = ops.BLOCK


def _recording(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_current_stream_capturing()


def _no_recording(device: torch.device, what: str) -> None:
    if _recording(device):
        raise SdvError(f"{what} while a HIP graph is being recorded; reserve the tokens (reserve_all) and size the "
                       f"workspace before recording")


class BlockAllocator:
    """Free list of physical page blocks."""

    def __init__(self, num_blocks: int, seed: int | None = None):
        self.num_blocks = 0
        self.seed = seed
        self._rng = random.Random(seed) if seed is not None else None
        self.free: list[int] = []
        self.grow(num_blocks)

    def grow(self, new_total: int) -> None:
        fresh = list(range(self.num_blocks, new_total))
        if self._rng is not None:
            self._rng.shuffle(fresh)
        # pop() takes from the end: keep ascending order for the unseeded allocator
        self.free = fresh[::-1] + self.free
        self.num_blocks = new_total

    def alloc(self, n: int) -> list[int]:
        if n > len(self.free):
            raise RuntimeError(f"block pool exhausted: need {n}, {len(self.free)} free of {self.num_blocks}")
        return [self.free.pop() for _ in range(n)]

    def release(self, blocks) -> None:
        self.free.extend(reversed(list(blocks)))


class PagedKVCache:
    """Page pool for ``num_layers`` layers and ``batch`` sequences."""

    def __init__(self, kv_heads: int, head_dim: int, *, num_layers: int = 1, batch: int = 1,
                 num_blocks: int | None = None, capacity_tokens: int = 256, device="cuda",
                 seed: int | None = None, scale_mode: str = "div", growable: bool = True):
        if head_dim not in (64, 128):
            raise ValueError(f"head_dim must be 64 or 128 (got {head_dim})")
        self.kv_heads, self.head_dim = kv_heads, head_dim
        self.num_layers, self.batch = num_layers, batch
        self.device = torch.device(device)
        self.scale_mode = scale_mode
        self.growable = growable
        if num_blocks is None:
            num_blocks = batch * -(-capacity_tokens // BLOCK)
        self.alloc = BlockAllocator(num_blocks, seed)
        self.k_pages, self.v_pages, self.v_scales = self._new_pages(num_blocks)
        self.blocks: list[list[int]] = [[] for _ in range(batch)]
        self.lengths: list[int] = [0] * batch
        self._bt = None
        self._tiles = None  # (lengths, device tile table) of the last prefill
        self._ws = None     # attention workspace owned by the pool
        # replaced workspaces, kept alive for graphs that recorded them; each replacement is at
        # least twice the size of the one before, so they hold at most the current one's bytes
        self._retired = []
        self._q_heads, self._q_len = 0, 0  # the largest query shape append_attend has served

    # ------------------------------------------------------------------ storage
    def _new_pages(self, nb: int):
        L, KV, D = self.num_layers, self.kv_heads, self.head_dim
        k = torch.zeros((L, nb, KV, D // 8, BLOCK, 8), dtype=torch.bfloat16, device=self.device)
        v = torch.zeros((L, nb, KV, D, BLOCK), dtype=torch.uint8, device=self.device)
        s = torch.ones((L, nb, KV, BLOCK), dtype=torch.float32, device=self.device)
        return k, v, s

    def _grow(self, min_blocks: int) -> None:
        _no_recording(self.device, "the page pool would grow")
        old = self.alloc.num_blocks
        new = max(min_blocks, 2 * old)
        k, v, s = self._new_pages(new)
        k[:, :old].copy_(self.k_pages)
        v[:, :old].copy_(self.v_pages)
        s[:, :old].copy_(self.v_scales)
        self.k_pages, self.v_pages, self.v_scales = k, v, s
        self.alloc.grow(new)

    def layer(self, i: int):
        """(k_pages, v_pages, v_scales) of layer i (contiguous views)."""
        return self.k_pages[i], self.v_pages[i], self.v_scales[i]

    # ------------------------------------------------------------------ sequences
    def reserve(self, seq: int, n_tokens: int) -> None:
        """Make sure sequence `seq` has blocks for its first n_tokens positions."""
        need = -(-n_tokens // BLOCK) - len(self.blocks[seq])
        if need <= 0:
            return
        _no_recording(self.device, f"sequence {seq} needs {need} more page blocks")
        if need > len(self.alloc.free):
            if not self.growable:
                raise RuntimeError(f"block pool exhausted ({self.alloc.num_blocks} blocks) and growable=False")
            self._grow(self.alloc.num_blocks + need)
        self.blocks[seq].extend(self.alloc.alloc(need))
        self._bt = None

    def reserve_all(self, n_tokens: int, q_heads: int | None = None, q_len: int | None = None) -> None:
        """Everything a recorded step up to n_tokens positions needs, before recording it: page
        blocks for the first n_tokens positions of every sequence, the device block table, and
        the attention workspace append_attend needs at that length for q_heads query heads and
        q_len new tokens per call (default: the largest append_attend has served; with no call
        served and none given, the workspace is sized by the first call)."""
        for b in range(self.batch):
            self.reserve(b, n_tokens)
        self.block_table()
        heads = q_heads or self._q_heads
        rows = max(q_len or 0, self._q_len, 1)
        if heads:
            tmax = max(n_tokens, max(self.lengths))
            self.workspace(ops.attention_workspace_bytes(1, self.batch, heads, self.kv_heads, rows, self.head_dim,
                                                         tmax))

    def workspace(self, nbytes: int) -> torch.Tensor:
        """The pool's attention workspace, at least nbytes.  A larger one (at least twice the
        size) replaces it; the old one is kept alive, since a recorded graph may use it."""
        if self._ws is None or self._ws.numel() < nbytes:
            _no_recording(self.device, f"the attention workspace would grow to {nbytes} bytes")
            grow = 0
            if self._ws is not None:
                self._retired.append(self._ws)
                grow = 2 * self._ws.numel()
            self._ws = ops.new_workspace(self.device, max(nbytes, grow))
        return self._ws

    def set_length(self, seq: int, n: int) -> None:
        if n < 0 or n > len(self.blocks[seq]) * BLOCK:
            raise ValueError(f"length {n} outside the reserved {len(self.blocks[seq]) * BLOCK} slots")
        self.lengths[seq] = n

    def free_sequence(self, seq: int) -> None:
        self.alloc.release(self.blocks[seq])
        self.blocks[seq] = []
        self.lengths[seq] = 0
        self._bt = None

    def max_blocks(self) -> int:
        return max(1, max(len(b) for b in self.blocks))

    def block_table(self) -> torch.Tensor:
        """int32 (batch, max_blocks) on the device; unused entries are -1 (never read)."""
        if self._bt is None:
            _no_recording(self.device, "the block table would be rebuilt")
            mb = self.max_blocks()
            rows = [b + [-1] * (mb - len(b)) for b in self.blocks]
            self._bt = torch.tensor(rows, dtype=torch.int32).to(self.device)
        return self._bt

    def slot_mapping(self, starts: list[int], count: int) -> torch.Tensor:
        """int32 (batch * count,) slots of positions starts[b] .. starts[b]+count-1, token-major."""
        out = []
        for b in range(self.batch):
            blks = self.blocks[b]
            out.extend(blks[p // BLOCK] * BLOCK + p % BLOCK for p in range(starts[b], starts[b] + count))
        return torch.tensor(out, dtype=torch.int32).to(self.device)

    # ------------------------------------------------------------------ kernels
    def append(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, starts: list[int] | None = None):
        """Write S new tokens per sequence for one layer: k_new/v_new BF16 (B, S, KV, D).

        Positions start at ``starts`` (default: the current lengths); lengths become
        start + S.  Runs kernel 1 (quantize V, copy K) into the pages.
        """
        B, S = k_new.shape[0], k_new.shape[1]
        starts = list(self.lengths) if starts is None else list(starts)
        for b in range(B):
            self.reserve(b, starts[b] + S)
        slots = self.slot_mapping(starts, S)
        kp, vp, vs = self.layer(layer)
        ops.quant_append(v_new.reshape(B * S, self.kv_heads, self.head_dim), slots, kp, vp, vs,
                         k_new.reshape(B * S, self.kv_heads, self.head_dim), scale_mode=self.scale_mode)
        for b in range(B):
            self.lengths[b] = starts[b] + S

    def append_attend(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                      starts: list[int] | None = None, *, q_token_major: bool = False,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """append(layer, k_new, v_new, starts) then attend(layer, q) in one call
        (sdv_paged_attention_append): the same pages and output, one launch on the single-launch
        path.  k_new/v_new BF16 (B, S, KV, D); q (B, H, S, D) (or (B, S, H, D)).

        Each new token's slot comes from the block table on the device; with equal lengths no
        length array is passed either, and the workspace is the pool's own: such a call copies
        nothing from the host and can be recorded into a HIP graph."""
        B, S = k_new.shape[0], k_new.shape[1]
        starts = list(self.lengths) if starts is None else list(starts)
        for b in range(B):
            self.reserve(b, starts[b] + S)
        for b in range(B):
            self.lengths[b] = starts[b] + S
        kp, vp, vs = self.layer(layer)
        shp = (B * S, self.kv_heads, self.head_dim)
        tmax = max(self.lengths)
        uniform = all(n == tmax for n in self.lengths)
        H = q.shape[2] if q_token_major else q.shape[1]
        self._q_heads, self._q_len = max(self._q_heads, H), max(self._q_len, S)
        ws = self.workspace(ops.attention_workspace_bytes(1, B, H, self.kv_heads, S, self.head_dim, tmax))
        return ops.paged_attention(q, kp, vp, vs, self.block_table(), None if uniform else self.seq_lens_tensor(),
                                   tmax, q_token_major=q_token_major, out=out, workspace_tensor=ws,
                                   append=(k_new.reshape(shp), v_new.reshape(shp), None),
                                   scale_mode=self.scale_mode)

    def varlen_slots(self, lengths: list[int]) -> torch.Tensor:
        """int32 (sum(lengths),) slots of positions 0..lengths[b]-1 of each sequence in turn."""
        out = []
        for b, n in enumerate(lengths):
            pos = torch.arange(n, dtype=torch.int64)
            blk = torch.tensor(self.blocks[b][:-(-n // BLOCK)], dtype=torch.int64)
            out.append(blk[pos // BLOCK] * BLOCK + pos % BLOCK)
        return torch.cat(out).to(torch.int32).to(self.device)

    def prefill(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, lengths: list[int],
                slots: torch.Tensor | None = None) -> torch.Tensor:
        """Write whole prompts of different lengths into one layer (one kernel 1 launch).

        k_new/v_new BF16 (sum(lengths), KV, D), sequence after sequence (the varlen layout);
        lengths become ``lengths``.  Returns the slot mapping so that later layers can pass it.
        The launch takes a tile table that starts a tile at every sequence's first row (built
        once per set of lengths), so whole page blocks are written with 16-byte stores.
        """
        if len(lengths) != self.batch:
            raise ValueError(f"{len(lengths)} lengths for a batch of {self.batch}")
        for b, n in enumerate(lengths):
            self.reserve(b, n)
        if slots is None:
            slots = self.varlen_slots(lengths)
        key = tuple(lengths)
        if self._tiles is None or self._tiles[0] != key:
            t = torch.tensor(ops.varlen_tile_starts(list(lengths)), dtype=torch.int32).to(self.device)
            self._tiles = (key, t)
        kp, vp, vs = self.layer(layer)
        ops.quant_append(v_new, slots, kp, vp, vs, k_new, scale_mode=self.scale_mode,
                         tile_starts=self._tiles[1])
        for b, n in enumerate(lengths):
            self.lengths[b] = n
        return slots

    def seq_lens_tensor(self, lengths: list[int] | None = None) -> torch.Tensor:
        return torch.tensor(self.lengths if lengths is None else lengths, dtype=torch.int32).to(self.device)

    def attend(self, layer: int, q: torch.Tensor, *, q_token_major: bool = False, lengths=None,
               out: torch.Tensor | None = None) -> torch.Tensor:
        """Attention of q (B,H,S,D) (or (B,S,H,D)) over this layer's pages at the current lengths."""
        lengths = self.lengths if lengths is None else lengths
        kp, vp, vs = self.layer(layer)
        return ops.paged_attention(q, kp, vp, vs, self.block_table(), self.seq_lens_tensor(lengths),
                                   max(lengths), q_token_major=q_token_major, out=out)

    def gather(self, layer: int, seq: int, n: int | None = None):
        """Contiguous (k BF16 (KV,T,D), v payload float8_e4m3fn (KV,T,D), v_scale fp32 (KV,T,1))."""
        n = self.lengths[seq] if n is None else n
        nb = -(-n // BLOCK)
        idx = torch.tensor(self.blocks[seq][:nb], dtype=torch.long, device=self.device)
        kp, vp, vs = self.layer(layer)
        KV, D = self.kv_heads, self.head_dim
        k = kp[idx].permute(1, 0, 3, 2, 4).reshape(KV, nb * BLOCK, D)[:, :n]
        v = vp[idx].permute(1, 0, 3, 2).reshape(KV, nb * BLOCK, D)[:, :n]
        s = vs[idx].permute(1, 0, 2).reshape(KV, nb * BLOCK)[:, :n]
        return k, v.contiguous().view(torch.float8_e4m3fn), s.unsqueeze(-1)

    # ------------------------------------------------------------------ accounting
    def logical_bytes_per_token_layer(self) -> int:
        """K BF16 + V FP8 + fp32 scale per token per layer: 776 B for KV=2, D=128."""
        return self.kv_heads * (2 * self.head_dim + self.head_dim + 4)

    def footprint(self) -> dict:
        tok = sum(self.lengths)
        fp8 = tok * self.num_layers * self.logical_bytes_per_token_layer()
        bf16 = tok * self.num_layers * self.kv_heads * 4 * self.head_dim
        scales = tok * self.num_layers * self.kv_heads * 4
        return {"tokens": tok, "fp8v_bytes": fp8, "bf16_bytes": bf16, "saved_frac": 1 - fp8 / max(bf16, 1),
                "scale_frac_of_fp8v": scales / max(fp8, 1),
                "pool_bytes": self.k_pages.numel() * 2 + self.v_pages.numel() + self.v_scales.numel() * 4}


# ---------------------------------------------------------------------- engine layer dicts
_ANCHORS: dict = {}


def shape_carrier(shape, dtype, device) -> torch.Tensor:
    """A zero-storage tensor of the given logical shape (one element, expanded).

    The paged layer dict stores these under "k", "v" and "v_scale" so that code written for
    the reference's contiguous cache -- ``cache[0]["k"].shape[2]`` for the length
    (model_self.py:847-848, spec_cache.py:4-7), ``val[:, :, :n]`` to trim (spec_cache.py:
    23-28), ``cache[0]["k"].device`` for new token tensors (spec_dec.py:174,185) -- keeps
    working unchanged while the bytes live in the page pool.
    """
    dev = torch.device(device)
    key = (dtype, dev)
    anchor = _ANCHORS.get(key)
    if anchor is None:
        anchor = torch.zeros((), dtype=dtype, device=dev)
        _ANCHORS[key] = anchor
    return anchor.expand(*shape)


class LayerPages:
    """Handle of one engine layer's pages, carried in its cache dict under "pages"."""

    def __init__(self, pool: "PagedKVCache", layer: int = 0):
        self.pool = pool
        self.layer = layer

    def reserved_tokens(self) -> int:
        return min(len(b) for b in self.pool.blocks) * BLOCK

    def layer_dict(self, length: int) -> dict:
        """{"fmt", "k", "v", "v_scale", "pages"} for a logical length of `length` tokens."""
        p = self.pool
        B, KV, D, dev = p.batch, p.kv_heads, p.head_dim, p.device
        return {"fmt": "v_fp8",
                "k": shape_carrier((B, KV, length, D), torch.bfloat16, dev),
                "v": shape_carrier((B, KV, length, D), torch.float8_e4m3fn, dev),
                "v_scale": shape_carrier((B, KV, length, 1), torch.float32, dev),
                "pages": self}

    def materialize(self, length: int) -> dict:
        """Contiguous copies {"fmt", "k", "v", "v_scale"} in the reference's layout (for tools
        that read the cache tensors themselves)."""
        ks, vs, ss = zip(*(self.pool.gather(self.layer, b, length) for b in range(self.pool.batch)))
        return {"fmt": "v_fp8", "k": torch.stack(ks), "v": torch.stack(vs), "v_scale": torch.stack(ss)}
