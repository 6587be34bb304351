"""sdv_paged_attention_append: the append of the new tokens and the attention over them in one
call must leave the same bytes in the pages and give the same output as sdv_quant_append
followed by sdv_paged_attention (model_self.py:697-706 then 739-776, one layer forward).

Both sides run on the GPU from identical caches; the comparison is bitwise, for the single
launch (each workgroup writes the new tokens of its own page blocks) and for the calls whose
attention runs in other kernels (the append kernel runs first).  The attention itself is checked against the eager
oracle by tests/test_gpu_attention.py.
"""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from specdec_amd import workloads as wl
from specdec_amd.engine.paged_cache import PagedKVCache
from specdec_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _twin_caches(dev, kv, d, lens, seed):
    """Two identical paged caches (same fragmented pool, same contents)."""
    out = []
    for _ in range(2):
        g = wl.gen(seed, dev)
        c = PagedKVCache(kv, d, num_layers=1, batch=len(lens), num_blocks=sum(-(-t // 16) for t in lens) + 40,
                         device=dev, seed=seed, growable=False)
        k = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        c.prefill(0, k, v, lens)
        out.append(c)
    return out


def _same_pages(a, b):
    return (torch.equal(a.k_pages.view(torch.int16), b.k_pages.view(torch.int16))
            and torch.equal(a.v_pages, b.v_pages) and torch.equal(a.v_scales.view(torch.int32), b.v_scales.view(torch.int32)))


@pytest.mark.parametrize("h,kv,d,lens,s", [
    (12, 2, 128, [8191], 1),            # decode, 8K context: one launch, 32 items per group
    (12, 2, 128, [99], 1),              # short context
    (12, 2, 128, [2046], 5),            # verify: positions 2046..2050 straddle blocks 127 / 128
    (14, 2, 64, [4095], 1),             # draft shape (D=64, 16 wavefronts)
    (12, 2, 128, [700, 33, 2047], 1),   # ragged batch
    (12, 2, 128, [300, 1000], 16),      # 96 query rows: the prefill kernels, append kernel first
])
def test_append_attend_matches_append_then_attend(cuda_device, h, kv, d, lens, s):
    announce(f"append+attend h={h} kv={kv} d={d} lens={lens} s={s}")
    sep, fused = _twin_caches(cuda_device, kv, d, lens, seed=700 + s + d)
    g = wl.gen(701 + s, cuda_device)
    B = len(lens)
    k_new = torch.randn((B, s, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
    v_new = (3 * torch.randn((B, s, kv, d), generator=g, device=cuda_device)).to(torch.bfloat16)
    q = torch.randn((B, h, s, d), generator=g, device=cuda_device).to(torch.bfloat16)
    sep.append(0, k_new, v_new)
    want = sep.attend(0, q)
    got = fused.append_attend(0, q, k_new, v_new)
    torch.cuda.synchronize()
    assert fused.lengths == sep.lengths
    assert _same_pages(sep, fused), "pages differ"
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (got.float() - want.float()).abs().max()


def test_append_attend_multi_layer_and_token_major(cuda_device):
    """Four layers in one launch with layered new tokens, q in the projection layout."""
    announce("append+attend 4 layers, token-major q")
    L, kv, d, h, s, T0 = 4, 2, 128, 12, 1, 3000
    caches = []
    for _ in range(2):
        g = wl.gen(710, cuda_device)
        c = PagedKVCache(kv, d, num_layers=L, batch=1, num_blocks=200 + 4, device=cuda_device, seed=710,
                         growable=False)
        for layer in range(L):
            k = torch.randn((T0, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
            v = torch.randn((T0, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
            c.prefill(layer, k, v, [T0])
        caches.append(c)
    sep, fused = caches
    g = wl.gen(711, cuda_device)
    k_new = torch.randn((L, s, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
    v_new = torch.randn((L, s, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
    q = torch.randn((L, 1, s, h, d), generator=g, device=cuda_device).to(torch.bfloat16)
    slots = sep.slot_mapping([T0], s)
    for layer in range(L):
        kp, vp, vs = sep.layer(layer)
        ops.quant_append(v_new[layer], slots, kp, vp, vs, k_new[layer])
    sl = torch.tensor([T0 + s], dtype=torch.int32, device=cuda_device)
    for c in caches:
        c.reserve(0, T0 + s)
        c.lengths[0] = T0 + s
    want = ops.paged_attention(q, sep.k_pages, sep.v_pages, sep.v_scales, sep.block_table(), sl, T0 + s,
                               q_token_major=True)
    got = ops.paged_attention(q, fused.k_pages, fused.v_pages, fused.v_scales, fused.block_table(), sl, T0 + s,
                              q_token_major=True, append=(k_new, v_new, slots))
    torch.cuda.synchronize()
    assert ops.single_launch_workgroups(L, 1, h, kv, s, d, T0 + s) > 0
    assert _same_pages(sep, fused)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_append_attend_where_only_the_plain_call_fits_one_launch(cuda_device):
    """24 layers x 4 sequences of the draft shape (14/2/64) at T = 8000: one 500-block item per
    group.  The single launch holds that call with 8 wavefronts, but an appending call runs 16,
    whose LDS for the wavefronts' p.V slots no longer fits beside 500 blocks of scores (items of
    460-509 blocks are in that band for 7 query rows).  The append must then run as its own
    kernel before whichever path serves the attention, leaving the same pages and output as the
    two calls."""
    announce("append+attend 24 layers x 4 seqs 14/2/64 at T=8000 (appending launch does not fit)")
    L, B, kv, d, h, s, T0 = 24, 4, 2, 64, 14, 1, 7999
    assert ops.single_launch_workgroups(L, B, h, kv, s, d, T0 + s) > 0
    caches = []
    for _ in range(2):
        g = wl.gen(720, cuda_device)
        c = PagedKVCache(kv, d, num_layers=L, batch=B, num_blocks=B * 500 + 8, device=cuda_device, seed=720,
                         growable=False)
        slots = None
        for layer in range(L):
            k = torch.randn((B * T0, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
            v = torch.randn((B * T0, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
            slots = c.prefill(layer, k, v, [T0] * B, slots)
        caches.append(c)
    sep, fused = caches
    g = wl.gen(721, cuda_device)
    k_new = torch.randn((L, B * s, kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
    v_new = (3 * torch.randn((L, B * s, kv, d), generator=g, device=cuda_device)).to(torch.bfloat16)
    q = torch.randn((L, B, h, s, d), generator=g, device=cuda_device).to(torch.bfloat16)
    for c in caches:
        for b in range(B):
            c.reserve(b, T0 + s)
    slots = sep.slot_mapping([T0] * B, s)
    for layer in range(L):
        kp, vp, vs = sep.layer(layer)
        ops.quant_append(v_new[layer], slots, kp, vp, vs, k_new[layer])
    for c in caches:
        for b in range(B):
            c.lengths[b] = T0 + s
    sl = sep.seq_lens_tensor()
    want = ops.paged_attention(q, sep.k_pages, sep.v_pages, sep.v_scales, sep.block_table(), sl, T0 + s)
    got = ops.paged_attention(q, fused.k_pages, fused.v_pages, fused.v_scales, fused.block_table(), sl, T0 + s,
                              append=(k_new, v_new, None))
    torch.cuda.synchronize()
    assert _same_pages(sep, fused), "the new tokens were not written"
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_append_attend_rejects_bad_shapes(cuda_device):
    c = PagedKVCache(2, 128, num_layers=1, batch=1, num_blocks=8, device=cuda_device, seed=1, growable=False)
    kp, vp, vs = c.layer(0)
    q = torch.zeros((1, 12, 1, 128), dtype=torch.bfloat16, device=cuda_device)
    bt = torch.zeros((1, 8), dtype=torch.int32, device=cuda_device)
    sl = torch.ones((1,), dtype=torch.int32, device=cuda_device)
    kn = torch.zeros((2, 2, 128), dtype=torch.bfloat16, device=cuda_device)   # 2 tokens for B*S = 1
    slots = torch.zeros((1,), dtype=torch.int32, device=cuda_device)
    with pytest.raises(Exception):
        ops.paged_attention(q, kp, vp, vs, bt, sl, 16, append=(kn, kn, slots))
