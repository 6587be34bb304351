"""The single launch's failure path on the GPU, driven from the host.

The single launch's cross-workgroup waits are bounded (csrc/sdv_attn.hip, fused_kernel).  The
host sets the bound that makes every wait give up at its first check (sdv_attention_set_wait_limit
with UINT32_MAX; a bound of one poll gives up only at an entry not yet published, which depends
on timing), while every workgroup still runs to its end -- no kernel is made to fault or hang.  Checked: the failure is surfaced (NaN outputs where the call could not
complete, the workspace's failure count), outputs that did complete are exact, the next eager
call on the same workspace is exact, and a graph-recorded call that failed poisons the
workspace so that later graph replays are refused (NaN, counted) until the workspace is
reset.  Mirrors the reference's rule that errors are raised, never swallowed
(model_self.py:331-332).
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

L, KV, H, D, T = 28, 2, 12, 128, 2048
GIVE_UP = 0xFFFFFFFF  # wait bound: every wait gives up at its first check


def _cache(dev):
    g = wl.gen(880, dev)
    cache = PagedKVCache(KV, D, num_layers=L, num_blocks=T // 16 + 5, device=dev, seed=881, growable=False)
    slots = None
    for layer in range(L):
        k = torch.randn((T, KV, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((T, KV, D), generator=g, device=dev).to(torch.bfloat16)
        slots = cache.prefill(layer, k, v, [T], slots)
    return cache


def _want(cache, q, layer):
    k, v, sc = cache.gather(layer, 0)
    v_hat = oq.dequantize_kv_fp8(v.cpu()[None], sc.cpu()[None], torch.bfloat16)
    return oatt.eager_attention(q[layer].cpu(), k.cpu()[None], v_hat)


def _call(cache, q, ws, out):
    return ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                               cache.seq_lens_tensor(), T, out=out, workspace_tensor=ws)


def _check_partial(out, cache, q, layers=(0, 9, 27)):
    """Finite outputs are exact; returns the number of NaN outputs over all layers."""
    nans = int(torch.isnan(out.float()).sum())
    for layer in layers:
        got = out[layer].float().cpu()
        want = _want(cache, q, layer).float()
        ok = ~torch.isnan(got)
        if ok.any():
            assert float((got[ok] - want[ok]).abs().max()) <= 2e-2, f"layer {layer}: a finite output is wrong"
    return nans


@pytest.fixture()
def restore_wait_limit():
    yield
    ops.set_wait_limit(0)


def test_expired_waits_are_surfaced_and_the_next_call_is_exact(cuda_device, restore_wait_limit):
    announce("sync failure: eager call whose waits give up, then a normal call")
    assert ops.single_launch_workgroups(L, 1, H, KV, 1, D, T) > 0
    cache = _cache(cuda_device)
    g = wl.gen(882, cuda_device)
    q = torch.randn((L, 1, H, 1, D), generator=g, device=cuda_device).to(torch.bfloat16)
    ws = ops.new_workspace(cuda_device, ops.attention_workspace_bytes(L, 1, H, KV, 1, D, T))
    out = torch.empty_like(q)
    ops.set_wait_limit(GIVE_UP)
    _call(cache, q, ws, out)
    torch.cuda.synchronize()
    fails, poisoned = ops.workspace_status(ws)
    nans = _check_partial(out, cache, q)
    print(f"waits given up: {fails} failures, {nans} NaN outputs of {out.numel()}")
    assert fails > 0 and nans > 0, "expired waits were not surfaced"
    assert not poisoned, "an eager call must not poison the workspace"
    with pytest.raises(ops.SdvError):
        ops.check_workspace(ws)
    # the next eager call on the same workspace (words the failed call left behind carry its tag)
    ops.set_wait_limit(0)
    q2 = torch.randn((L, 1, H, 1, D), generator=g, device=cuda_device).to(torch.bfloat16)
    out2 = _call(cache, q2, ws, torch.empty_like(q2))
    torch.cuda.synchronize()
    assert ops.workspace_status(ws) == (fails, False), "the next call failed too"
    for layer in (0, 9, 27):
        assert_close(out2[layer].cpu(), _want(cache, q2, layer), f"next call layer {layer}")
    # and bitwise what a fresh workspace gives
    ref = _call(cache, q2, ops.new_workspace(cuda_device, ws.numel()), torch.empty_like(q2))
    torch.cuda.synchronize()
    assert torch.equal(out2, ref)


def test_graph_poison_refuses_replays_until_reset(cuda_device, restore_wait_limit):
    announce("sync failure: graph-recorded call whose waits give up, poison, reset")
    cache = _cache(cuda_device)
    g = wl.gen(883, cuda_device)
    q = torch.randn((L, 1, H, 1, D), generator=g, device=cuda_device).to(torch.bfloat16)
    ws = ops.new_workspace(cuda_device, ops.attention_workspace_bytes(L, 1, H, KV, 1, D, T))
    out = torch.empty_like(q)
    bt, sl = cache.block_table(), cache.seq_lens_tensor()

    def step():
        ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, bt, sl, T, out=out,
                            workspace_tensor=ws)

    step()                       # outside capture first (workspace ready, library loaded)
    torch.cuda.synchronize()
    good = torch.cuda.CUDAGraph()
    with torch.cuda.graph(good):
        step()
    for _ in range(3):           # normal replays with new inputs each time are exact
        q.copy_(torch.randn(q.shape, generator=g, device=cuda_device).to(torch.bfloat16))
        good.replay()
        torch.cuda.synchronize()
        for layer in (0, 27):
            assert_close(out[layer].cpu(), _want(cache, q, layer), f"replay layer {layer}")
    assert ops.workspace_status(ws) == (0, False)

    ops.set_wait_limit(GIVE_UP)
    bad = torch.cuda.CUDAGraph()
    with torch.cuda.graph(bad):
        step()
    ops.set_wait_limit(0)
    bad.replay()
    torch.cuda.synchronize()
    fails, poisoned = ops.workspace_status(ws)
    print(f"graph replay whose waits give up: {fails} failures, poisoned={poisoned}")
    assert fails > 0 and poisoned

    good.replay()                # refused: every output NaN, counted
    torch.cuda.synchronize()
    assert bool(torch.isnan(out.float()).all()), "a poisoned graph replay must write NaN everywhere"
    assert ops.workspace_status(ws)[0] > fails

    step()                       # eager calls are unaffected by the poison
    torch.cuda.synchronize()
    assert_close(out[5].cpu(), _want(cache, q, 5), "eager call on a poisoned workspace")

    ops.reset_workspace(ws)
    good.replay()
    torch.cuda.synchronize()
    assert ops.workspace_status(ws) == (0, False)
    for layer in (0, 27):
        assert_close(out[layer].cpu(), _want(cache, q, layer), f"replay after reset layer {layer}")
