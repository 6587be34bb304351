"""The persistent per-group kernel (csrc/sdv_attn.hip, group_kernel): calls with 256 or more
(layer, sequence, KV head) groups of one row tile -- config 4's 28 layers x 32 ragged
sequences is one -- take it instead of the three-launch path.  Each group is computed whole
by one workgroup, claimed longest sequence first from a counter that the last workgroup
resets.  Checked against the eager oracle (max-abs 2e-2, rel-L2 1e-3): ragged lengths from 1
token to a few blocks, verify rows (S=2, offset-causal mask), head_dim 64, a batch larger than
the length ordering covers (natural order), holes in the block table; and repeated calls
bitwise equal (the counter is back at zero after every call)."""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_close
from oracle import attention as oatt
from oracle import quant as oq
from specdec_amd import workloads as wl
from specdec_amd.engine.paged_cache import PagedKVCache
from specdec_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _cache(dev, layers, kv, d, lens, seed):
    g = wl.gen(seed, dev)
    cache = PagedKVCache(kv, d, num_layers=layers, batch=len(lens), num_blocks=sum(-(-t // 16) for t in lens) + 9,
                         device=dev, seed=seed, growable=False)
    slots = None
    for layer in range(layers):
        k = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        slots = cache.prefill(layer, k, v, lens, slots)
    return cache


def _run(dev, cache, h, s, seed, block_table=None):
    g = wl.gen(seed, dev)
    L, B = cache.num_layers, cache.batch
    q = torch.randn((L, B, h, s, cache.head_dim), generator=g, device=dev).to(torch.bfloat16)
    lens = list(cache.lengths)
    assert L * B * cache.kv_heads >= 1024 and ops.single_launch_workgroups(L, B, h, cache.kv_heads, s,
                                                                           cache.head_dim, max(lens)) == 0
    bt = cache.block_table() if block_table is None else block_table
    outs = [ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, bt, cache.seq_lens_tensor(),
                                max(lens)) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2]), "repeated calls differ"
    return q, outs[0]


def _check(cache, q, out, pairs, label, holes=None):
    for layer, b in pairs:
        k, v, sc = cache.gather(layer, b)
        v_hat = oq.dequantize_kv_fp8(v.cpu()[None], sc.cpu()[None], torch.bfloat16)
        kk = k.cpu()[None]
        if holes:  # a block whose id is invalid holds no tokens: its keys are masked out
            keep = torch.ones(kk.shape[2], dtype=torch.bool)
            for blk in holes.get(b, ()):
                keep[blk * 16:(blk + 1) * 16] = False
            kk, v_hat = kk[:, :, keep], v_hat[:, :, keep]
        want = oatt.eager_attention(q[layer, b:b + 1].cpu(), kk, v_hat)
        assert_close(out[layer, b:b + 1].cpu(), want, f"{label} layer {layer} seq {b} T={cache.lengths[b]}")


def test_group_ragged_decode(cuda_device):
    """16 layers x 32 sequences x 2 KV heads = 1024 groups, lengths 1 .. 700."""
    announce("group kernel decode 16x32, T=1..700")
    lens = [1, 2, 15, 16, 17, 700] + wl.ragged_lengths(26, 1, 700, seed=61)
    cache = _cache(cuda_device, 16, 2, 128, lens, seed=610)
    q, out = _run(cuda_device, cache, 12, 1, seed=611)
    _check(cache, q, out, [(0, 0), (0, 1), (3, 2), (7, 3), (15, 4), (15, 5), (9, 17), (12, 31)], "group decode")


def test_group_verify_rows(cuda_device):
    """S=2 (12 rows of the 12/2 head group): the offset-causal mask on the group kernel."""
    announce("group kernel verify S=2 16x32")
    lens = wl.ragged_lengths(32, 2, 500, seed=62)
    cache = _cache(cuda_device, 16, 2, 128, lens, seed=620)
    q, out = _run(cuda_device, cache, 12, 2, seed=621)
    _check(cache, q, out, [(0, 0), (5, 9), (15, 31)], "group verify")


def test_group_head_dim_64(cuda_device):
    """The 0.5B draft shape (14q/2kv, D=64): 24 layers x 24 sequences x 2 KV heads."""
    announce("group kernel D=64 24x24")
    lens = wl.ragged_lengths(24, 1, 400, seed=63)
    cache = _cache(cuda_device, 24, 2, 64, lens, seed=630)
    q, out = _run(cuda_device, cache, 14, 1, seed=631)
    _check(cache, q, out, [(0, 0), (11, 7), (23, 23)], "group d64")


def test_group_large_batch_natural_order(cuda_device):
    """1100 sequences (more than the length ordering covers): groups in natural order."""
    announce("group kernel B=1100, one layer")
    lens = wl.ragged_lengths(1100, 1, 64, seed=64)
    cache = _cache(cuda_device, 1, 1, 128, lens, seed=640)
    q, out = _run(cuda_device, cache, 6, 1, seed=641)
    _check(cache, q, out, [(0, 0), (0, 555), (0, 1099)], "group natural order")


def test_group_block_table_holes(cuda_device):
    """Invalid block ids (-1 and past the pool) hold no tokens."""
    announce("group kernel with block-table holes")
    lens = wl.ragged_lengths(32, 40, 300, seed=65)
    cache = _cache(cuda_device, 16, 2, 128, lens, seed=650)
    bt = cache.block_table().clone()
    holes = {0: (1,), 5: (0, 2), 9: (1,)}
    for b, blks in holes.items():
        for blk in blks:
            bt[b, blk] = -1 if blk % 2 == 0 else cache.k_pages.shape[1] + 3
    q, out = _run(cuda_device, cache, 12, 1, seed=651, block_table=bt)
    _check(cache, q, out, [(0, 0), (4, 5), (15, 9), (2, 3)], "group holes", holes=holes)
