"""Paged prefill / chunked-prefill attention (many query rows) against the eager oracle.

Reference: the prefill chunk of model_self.py:637-648 (2048-token chunks) attends over the
cache plus the chunk with the offset-causal keep-mask of model_self.py:471-479 (row i sees keys
j <= T - S + i); its fused path (cuDNN SDPA, :491-504) exists to avoid the O(S*T) score tensor
of the eager path (docs/data_ledger.md:1145-1152: 74.1 MiB transient at 12q/2048q/8192kv).
Here the two prefill passes keep 64 bytes per query row in the workspace (a (max, sum) for
each of eight key parts); the numbers must still be the eager BF16 path's (max-abs 2e-2,
rel-L2 1e-3 per row block).  The oracle runs on the
CPU in row chunks (row i of a chunk of rows [i0, i1) sees keys j <= T - S + i0 + i, the same
mask), so its memory stays bounded.
"""
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


def _oracle_rows(q, k, v_hat, i0, i1, t):
    """Eager attention of rows [i0, i1) of an S-row block over T keys (all heads)."""
    s = q.shape[2]
    tk = t - s + i1
    return oatt.eager_attention(q[:, :, i0:i1], k[:, :, :tk], v_hat[:, :, :tk])


def _prefill_case(dev, h, kv, d, s, t, seed, chunk_rows=256, check_rows=None):
    g = wl.gen(seed, dev)
    cache = PagedKVCache(kv, d, num_blocks=t // 16 + 11, device=dev, seed=seed, growable=False)
    k = torch.randn((t, kv, d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((t, kv, d), generator=g, device=dev).to(torch.bfloat16)
    cache.prefill(0, k, v, [t])
    q = torch.randn((1, h, s, d), generator=g, device=dev).to(torch.bfloat16)
    kp, vp, vs = cache.layer(0)
    nbytes = ops.attention_workspace_bytes(1, 1, h, kv, s, d, t)
    ws = ops.new_workspace(dev, nbytes)
    out = ops.paged_attention(q, kp, vp, vs, cache.block_table(), cache.seq_lens_tensor(), t, workspace_tensor=ws)
    torch.cuda.synchronize()
    kc, vc, sc = cache.gather(0, 0)
    v_hat = oq.dequantize_kv_fp8(vc.cpu()[None], sc.cpu()[None], torch.bfloat16)
    qc, kcc = q.cpu(), kc.cpu()[None]
    rows = check_rows or [(i, min(s, i + chunk_rows)) for i in range(0, s, chunk_rows)]
    worst = (0.0, 0.0)
    for i0, i1 in rows:
        want = _oracle_rows(qc, kcc, v_hat, i0, i1, t)
        st = assert_close(out[:, :, i0:i1].cpu(), want, f"{h}/{kv}/{d} S={s} T={t} rows {i0}:{i1}")
        worst = (max(worst[0], st["max_abs"]), max(worst[1], st["rel_l2"]))
    return nbytes, worst


def test_prefill_chunk_target_2048x8192(cuda_device):
    """The reference's target prefill chunk: 12 query heads, 2048 query rows over 8192 keys."""
    announce("prefill 12/2/128 S=2048 T=8192")
    nbytes, worst = _prefill_case(cuda_device, 12, 2, 128, 2048, 8192, seed=700)
    print(f"workspace {nbytes / 2**20:.2f} MiB, worst max-abs {worst[0]:.3e} rel-L2 {worst[1]:.3e}")
    assert nbytes <= 100 * 2**20


def test_prefill_chunk_draft_2048x8192(cuda_device):
    """The draft's prefill chunk: 14 query heads, head_dim 64."""
    announce("prefill 14/2/64 S=2048 T=8192")
    nbytes, worst = _prefill_case(cuda_device, 14, 2, 64, 2048, 8192, seed=701)
    print(f"workspace {nbytes / 2**20:.2f} MiB, worst max-abs {worst[0]:.3e} rel-L2 {worst[1]:.3e}")
    assert nbytes <= 100 * 2**20


@pytest.mark.parametrize("h,d,s,t", [(12, 128, 2048, 2048), (12, 128, 300, 1000), (14, 64, 33, 77),
                                     (12, 128, 11, 40000), (12, 128, 1000, 1000), (14, 64, 11, 270000)])
def test_prefill_shapes(cuda_device, h, d, s, t):
    """A first chunk from an empty cache (T = S, triangular mask), odd sizes, short blocks over
    long contexts and S not a multiple of 16.  A workgroup stages 256 page ids in LDS at a time:
    at T = 270,000 (16,875 blocks) every pass-1 key part (of 64) spans two such windows and every
    pass-2 part (of 8) nine, so both passes cross windows with stages in flight."""
    announce(f"prefill {h}/2/{d} S={s} T={t}")
    _prefill_case(cuda_device, h, 2, d, s, t, seed=710 + s + t, chunk_rows=512)


@pytest.mark.parametrize("s,h,d", [(96, 12, 128), (256, 12, 128), (256, 14, 64)])
def test_prefill_ragged_batch_token_major(cuda_device, s, h, d):
    """Two sequences of different lengths in one call, q in the projection layout (B, S, H, D).
    With S a multiple of pass 2's 128 rows (S = 256) pass 2's parts follow each row group's key
    count, planned for the longest sequence: the shorter one's row groups leave parts empty."""
    announce(f"prefill ragged batch, token-major q, S={s} {h}/2/{d}")
    g = wl.gen(720 + s + d, cuda_device)
    lens, kv = [3000, 700], 2
    cache = PagedKVCache(kv, d, batch=2, num_blocks=sum(-(-x // 16) for x in lens) + 5, device=cuda_device,
                         seed=721, growable=False)
    k = torch.randn((sum(lens), kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
    v = torch.randn((sum(lens), kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
    cache.prefill(0, k, v, lens)
    q = torch.randn((2, s, h, d), generator=g, device=cuda_device).to(torch.bfloat16)
    kp, vp, vs = cache.layer(0)
    assert ops.single_launch_workgroups(1, 2, h, kv, s, d, max(lens)) == 0
    out = ops.paged_attention(q, kp, vp, vs, cache.block_table(), cache.seq_lens_tensor(), max(lens),
                              q_token_major=True)
    torch.cuda.synchronize()
    for b, t in enumerate(lens):
        kc, vc, sc = cache.gather(0, b)
        v_hat = oq.dequantize_kv_fp8(vc.cpu()[None], sc.cpu()[None], torch.bfloat16)
        want = oatt.eager_attention(q[b:b + 1].transpose(1, 2).cpu(), kc.cpu()[None], v_hat)
        assert_close(out[b:b + 1].transpose(1, 2).cpu(), want, f"ragged b={b} T={t}")


def test_prefill_multi_layer_call(cuda_device):
    """Two layers x two ragged sequences of 128 new rows in one call (q in the projection layout
    (L, B, S, H, D)): every (layer, sequence) pair has its own pass-1 statistics, dequantized V
    and pass-2 parts (by key count: S is a multiple of 128), and each output is within the bar
    of the eager reference."""
    announce("prefill 2 layers x 2 ragged sequences, S=128, one call")
    g = wl.gen(725, cuda_device)
    L, lens, s, h, kv, d = 2, [2500, 900], 128, 12, 2, 128
    cache = PagedKVCache(kv, d, num_layers=L, batch=2, num_blocks=sum(-(-x // 16) for x in lens) + 5,
                         device=cuda_device, seed=726, growable=False)
    slots = None
    for layer in range(L):
        k = torch.randn((sum(lens), kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
        v = torch.randn((sum(lens), kv, d), generator=g, device=cuda_device).to(torch.bfloat16)
        slots = cache.prefill(layer, k, v, lens, slots)
    q = torch.randn((L, 2, s, h, d), generator=g, device=cuda_device).to(torch.bfloat16)
    out = ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                              cache.seq_lens_tensor(), max(lens), q_token_major=True)
    torch.cuda.synchronize()
    for layer in range(L):
        for b, t in enumerate(lens):
            kc, vc, sc = cache.gather(layer, b)
            v_hat = oq.dequantize_kv_fp8(vc.cpu()[None], sc.cpu()[None], torch.bfloat16)
            want = oatt.eager_attention(q[layer, b:b + 1].transpose(1, 2).cpu(), kc.cpu()[None], v_hat)
            assert_close(out[layer, b:b + 1].transpose(1, 2).cpu(), want, f"layer {layer} b={b} T={t}")


def test_prefill_deterministic(cuda_device):
    """Repeated calls are bitwise identical (fixed-order reductions, no atomics)."""
    announce("prefill determinism")
    g = wl.gen(730, cuda_device)
    cache = PagedKVCache(2, 128, num_blocks=140, device=cuda_device, seed=731, growable=False)
    t = 2000
    cache.prefill(0, torch.randn((t, 2, 128), generator=g, device=cuda_device).to(torch.bfloat16),
                  torch.randn((t, 2, 128), generator=g, device=cuda_device).to(torch.bfloat16), [t])
    q = torch.randn((1, 12, 500, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    kp, vp, vs = cache.layer(0)
    outs = [ops.paged_attention(q, kp, vp, vs, cache.block_table(), cache.seq_lens_tensor(), t) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


@pytest.mark.parametrize("h,d,s", [(14, 64, 300), (12, 128, 300), (12, 128, 256)])
def test_prefill_key_parts_repeat_and_replay(cuda_device, h, d, s):
    """Pass 2 splits each row group's keys in parts, and the part that finishes last sums them
    (a per-row-group counter that it zeroes again): repeated eager calls and the replays of a
    recorded call -- which reuse one tag -- with eager calls between them are bitwise equal, on
    a batch of two sequences (two counters per KV head); S = 256 takes the parts by key count."""
    announce(f"prefill {h}/2/{d} S={s} key parts: repeats and graph replays")
    g = wl.gen(740 + d + s, cuda_device)
    lens, kv = [3000, 1200], 2
    cache = PagedKVCache(kv, d, batch=2, num_blocks=sum(-(-x // 16) for x in lens) + 5, device=cuda_device,
                         seed=741, growable=False)
    cache.prefill(0, torch.randn((sum(lens), kv, d), generator=g, device=cuda_device).to(torch.bfloat16),
                  torch.randn((sum(lens), kv, d), generator=g, device=cuda_device).to(torch.bfloat16), lens)
    q = torch.randn((2, s, h, d), generator=g, device=cuda_device).to(torch.bfloat16)
    kp, vp, vs = cache.layer(0)
    bt, sl = cache.block_table(), cache.seq_lens_tensor()
    ws = ops.new_workspace(cuda_device, ops.attention_workspace_bytes(1, 2, h, kv, s, d, max(lens)))

    def call(out=None):
        return ops.paged_attention(q, kp, vp, vs, bt, sl, max(lens), q_token_major=True, out=out, workspace_tensor=ws)

    eager = [call() for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(eager[0], eager[1]) and torch.equal(eager[1], eager[2])
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]), "a replay differs from the eager call"
        again = call()
        torch.cuda.synchronize()
        assert torch.equal(again, eager[0]), "an eager call after a replay differs"
    for b, t in enumerate(lens):  # and the numbers are the eager path's
        kc, vc, sc = cache.gather(0, b)
        v_hat = oq.dequantize_kv_fp8(vc.cpu()[None], sc.cpu()[None], torch.bfloat16)
        want = oatt.eager_attention(q[b:b + 1].transpose(1, 2).cpu(), kc.cpu()[None], v_hat)
        assert_close(eager[0][b:b + 1].transpose(1, 2).cpu(), want, f"key parts b={b} T={t}")
