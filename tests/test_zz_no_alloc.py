"""sdv_paged_attention_noalloc -- the entry point that allocates nothing -- through the C ABI.

It runs the same kernels as sdv_paged_attention with the library's per-GPU scratch array in
place of a caller's workspace, so its outputs must equal sdv_paged_attention's bit for bit:
checked on two calls in a row, the second with a smaller input (the scratch keeps the first
call's contents), and a call whose path needs more workspace than the scratch holds must be
rejected with SDV_ERR_WORKSPACE before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from specdec_amd import _native
from specdec_amd import workloads as wl
from specdec_amd.engine.paged_cache import PagedKVCache
from specdec_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _cache(dev, layers, kv, d, t, seed):
    g = wl.gen(seed, dev)
    cache = PagedKVCache(kv, d, num_layers=layers, num_blocks=t // 16 + 3, device=dev, seed=seed, growable=False)
    slots = None
    for layer in range(layers):
        k = torch.randn((t, kv, d), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((t, kv, d), generator=g, device=dev).to(torch.bfloat16)
        slots = cache.prefill(layer, k, v, [t], slots)
    return cache


def _noalloc(q, cache, t, out, sl=None):
    """One sdv_paged_attention_noalloc call (q (L, 1, H, S, D) or (1, H, S, D) for one layer);
    sl: the lengths tensor (made here when None, which cannot happen inside a graph recording)."""
    lib = _native.load()
    layered = q.dim() == 5
    L = q.shape[0] if layered else 1
    B, H, S, D = q.shape[-4:]
    kp, vp, vs = (cache.k_pages, cache.v_pages, cache.v_scales) if layered else cache.layer(0)
    per = (lambda x: x[0].numel()) if layered else (lambda x: 0)
    bt = cache.block_table()
    sl = cache.seq_lens_tensor() if sl is None else sl
    nb = kp.shape[-5]
    return lib.sdv_paged_attention_noalloc(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), vs.data_ptr(), nb,
                                           per(kp), per(vp), per(vs), bt.data_ptr(), bt.shape[1], sl.data_ptr(),
                                           L, B, H, cache.kv_heads, S, D, t, 0, out.data_ptr(),
                                           torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_workspace_entry_point(cuda_device):
    # call 1: the headline shape, 28 layers at 8K, one launch of the single-launch kernel
    announce("noalloc: 28 layers x 12/2/128 T=8192 decode")
    big = _cache(cuda_device, 28, 2, 128, 8192, seed=910)
    g = wl.gen(911, cuda_device)
    q1 = torch.randn((28, 1, 12, 1, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    out1 = torch.empty_like(q1)
    assert _noalloc(q1, big, 8192, out1) == _native.SDV_OK
    ref1 = ops.paged_attention(q1, big.k_pages, big.v_pages, big.v_scales, big.block_table(),
                               big.seq_lens_tensor(), 8192)
    torch.cuda.synchronize()
    assert torch.equal(out1, ref1), "noalloc call 1 differs from sdv_paged_attention"
    # call 2, smaller: one layer, verify S=5 at T=2048 (the scratch still holds call 1's area)
    announce("noalloc: 1 layer x 12/2/128 S=5 T=2048 verify")
    small = _cache(cuda_device, 1, 2, 128, 2048, seed=912)
    q2 = torch.randn((1, 12, 5, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    out2 = torch.empty_like(q2)
    assert _noalloc(q2, small, 2048, out2) == _native.SDV_OK
    kp, vp, vs = small.layer(0)
    ref2 = ops.paged_attention(q2, kp, vp, vs, small.block_table(), small.seq_lens_tensor(), 2048)
    torch.cuda.synchronize()
    assert torch.equal(out2, ref2), "noalloc call 2 differs from sdv_paged_attention"
    # and the first shape again, bitwise as before
    out3 = torch.empty_like(q1)
    assert _noalloc(q1, big, 8192, out3) == _native.SDV_OK
    torch.cuda.synchronize()
    assert torch.equal(out3, ref1)


@pytest.mark.parametrize("L,B,s,t,group", [(1, 160, 5, 4096, False), (32, 16, 1, 8000, True)])
def test_noalloc_rejects_what_the_scratch_cannot_hold(cuda_device, L, B, s, t, group):
    """Shapes whose path needs more workspace than the scratch holds are rejected on the host
    and write nothing: 320 groups of two row tiles (verify rows, more groups than the single
    launch holds: three launches, with scores, statistics and partials of every group) and
    1024 one-tile groups with 2^18 - 6144 tokens x KV heads per layer (too little work for one
    single launch per layer: the per-group kernel, 256 score rows per query row of the longest
    sequence)."""
    announce(f"noalloc: oversize shape L={L} B={B} S={s} T={t} rejected ({'per-group' if group else 'three-launch'})")
    assert L == 1 or B * 2 * t < 1 << 18, "one single launch per layer would serve this shape"
    lib = _native.load()
    h, kv, d = 12, 2, 128
    need = lib.sdv_attention_workspace_size(L, B, h, kv, s, d, t)
    assert lib.sdv_attention_single_launch(L, B, h, kv, s, d, t) == 0
    assert need > _native.NOALLOC_MAX_WORKSPACE
    if group:
        assert need == _native.SYNC_BYTES + 256 * (h // kv) * t * 2
    cache = PagedKVCache(kv, d, num_layers=L, batch=B, num_blocks=B * (t // 16) + 1, device=cuda_device,
                         growable=False)
    for b in range(B):
        cache.reserve(b, t)
        cache.set_length(b, t)
    q = torch.zeros((L, B, h, s, d), dtype=torch.bfloat16, device=cuda_device)
    if L == 1:
        q = q[0]
    out = torch.full_like(q, 7.0)
    assert _noalloc(q, cache, t, out) == _native.SDV_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a rejected call must not write its output"


def _batch_cache(dev, layers, kv, d, lens, seed):
    g = wl.gen(seed, dev)
    cache = PagedKVCache(kv, d, num_layers=layers, batch=len(lens), num_blocks=sum(-(-t // 16) for t in lens) + 5,
                         device=dev, seed=seed, growable=False)
    slots = None
    for layer in range(layers):
        k = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        slots = cache.prefill(layer, k, v, lens, slots)
    return cache


def test_noalloc_group_and_prefill_paths(cuda_device):
    """The per-group kernel (a claim counter that its last workgroup resets) and the head_dim 64
    prefill (a counter per row group that the last key part resets) through the scratch, in the
    order group -> prefill -> smaller group -> prefill again -> prefill whose pass-2 parts
    follow each row group's key count: every call equals sdv_paged_attention's output bit for
    bit."""
    lib = _native.load()
    g = wl.gen(920, cuda_device)

    def ref(q, cache, t):
        if q.dim() == 5:
            return ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                                       cache.seq_lens_tensor(), t)
        kp, vp, vs = cache.layer(0)
        return ops.paged_attention(q, kp, vp, vs, cache.block_table(), cache.seq_lens_tensor(), t)

    def both(q, cache, t, what):
        out = torch.empty_like(q)
        assert _noalloc(q, cache, t, out) == _native.SDV_OK, what
        want = ref(q, cache, t)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"{what}: noalloc differs from sdv_paged_attention"

    announce("noalloc: per-group kernel, 28 layers x 19 ragged sequences (1064 groups)")
    lens_a = wl.ragged_lengths(19, 200, 2048, seed=921)
    big = _batch_cache(cuda_device, 28, 2, 128, lens_a, seed=922)
    assert lib.sdv_attention_workspace_size(28, 19, 12, 2, 1, 128, max(lens_a)) <= _native.NOALLOC_MAX_WORKSPACE
    qa = torch.randn((28, 19, 12, 1, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    both(qa, big, max(lens_a), "group 28x19")

    announce("noalloc: prefill rows, 14/2/64, S=300 over T=3000 (key parts)")
    pf = _cache(cuda_device, 1, 2, 64, 3000, seed=923)
    qp = torch.randn((1, 14, 300, 64), generator=g, device=cuda_device).to(torch.bfloat16)
    both(qp, pf, 3000, "prefill 300x3000")

    announce("noalloc: per-group kernel, 16 layers x 32 sequences up to 700 tokens")
    lens_b = wl.ragged_lengths(32, 1, 700, seed=924)
    small = _batch_cache(cuda_device, 16, 2, 128, lens_b, seed=925)
    qb = torch.randn((16, 32, 12, 1, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    both(qb, small, max(lens_b), "group 16x32")

    announce("noalloc: prefill rows again")
    both(qp, pf, 3000, "prefill again")

    announce("noalloc: prefill rows, 14/2/64, S=256 over T=3000 (pass-2 parts by key count)")
    qk = torch.randn((1, 14, 256, 64), generator=g, device=cuda_device).to(torch.bfloat16)
    assert lib.sdv_attention_workspace_size(1, 1, 14, 2, 256, 64, 3000) <= _native.NOALLOC_MAX_WORKSPACE
    both(qk, pf, 3000, "prefill 256x3000")


def test_noalloc_serves_per_layer_launches(cuda_device):
    """8 layers x 32 sequences at 12K: more groups than one launch holds, but enough work per
    layer for one single launch per layer, which needs only the synchronisation area -- so the
    scratch serves it although the layout of the per-group kernel (sdv_attention_workspace_size:
    a 12K row of scores per query row for each of its 256 workgroups) would not fit; bitwise
    sdv_paged_attention's output."""
    announce("noalloc: 8 layers x 32 x 12/2/128 T=12288 (one single launch per layer)")
    lib = _native.load()
    L, B, t = 8, 32, 12288
    assert lib.sdv_attention_workspace_size(L, B, 12, 2, 1, 128, t) > _native.NOALLOC_MAX_WORKSPACE
    assert lib.sdv_attention_single_launch(L, B, 12, 2, 1, 128, t) == 0
    cache = _batch_cache(cuda_device, L, 2, 128, [t] * B, seed=930)
    g = wl.gen(931, cuda_device)
    q = torch.randn((L, B, 12, 1, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    out = torch.empty_like(q)
    assert _noalloc(q, cache, t, out) == _native.SDV_OK
    want = ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                               cache.seq_lens_tensor(), t)
    torch.cuda.synchronize()
    assert torch.equal(out, want), "noalloc per-layer launches differ from sdv_paged_attention"


@pytest.fixture()
def _restore_wait_limit():
    yield
    ops.set_wait_limit(0)


def test_noalloc_failure_state_is_readable_and_clearable(cuda_device, _restore_wait_limit):
    """A graph-recorded noalloc call whose waits give up (a host-set wait bound: every kernel
    still runs to its end) counts in, and poisons, the scratch; the status of the scratch (a
    NULL workspace) shows it, later recorded calls are refused (NaN) until the scratch is
    reset, and after the reset they are exact again."""
    announce("noalloc: recorded call whose waits give up, scratch status, reset")
    L, t = 4, 2048
    cache = _cache(cuda_device, L, 2, 128, t, seed=940)
    g = wl.gen(941, cuda_device)
    q = torch.randn((L, 1, 12, 1, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    out = torch.empty_like(q)
    sl = cache.seq_lens_tensor()
    cache.block_table()
    assert _noalloc(q, cache, t, out, sl) == _native.SDV_OK  # outside capture first: takes the scratch
    ref = ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                              cache.seq_lens_tensor(), t)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    ops.reset_workspace(None)
    assert ops.workspace_status(None) == (0, False)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    ops.set_wait_limit(0xFFFFFFFF)
    bad = torch.cuda.CUDAGraph()
    with torch.cuda.graph(bad, stream=side):
        rc_bad = _noalloc(q, cache, t, out, sl)
    ops.set_wait_limit(0)
    good = torch.cuda.CUDAGraph()
    with torch.cuda.graph(good, stream=side):
        rc_good = _noalloc(q, cache, t, out, sl)
    assert rc_bad == _native.SDV_OK and rc_good == _native.SDV_OK
    bad.replay()
    torch.cuda.synchronize()
    fails, poisoned = ops.workspace_status(None)
    print(f"recorded noalloc call whose waits give up: {fails} failures, poisoned={poisoned}")
    assert fails > 0 and poisoned
    with pytest.raises(ops.SdvError):
        ops.check_workspace(None)
    good.replay()                          # refused while poisoned: NaN everywhere, counted
    torch.cuda.synchronize()
    assert bool(torch.isnan(out.float()).all())
    assert ops.workspace_status(None)[0] > fails
    ops.reset_workspace(None)
    good.replay()
    torch.cuda.synchronize()
    assert ops.workspace_status(None) == (0, False)
    assert torch.equal(out, ref), "a recorded call after the reset differs"
