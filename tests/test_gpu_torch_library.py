"""torch.ops.sdv.* on the GPU: torch.library.opcheck (schema, fake tensors, AOT dispatch) on
small real inputs, and torch.compile(fullgraph=True) of the reference-signature op
(kernels.ops.attention, specdec/kernels/ops.py:67-76) giving the eager op's output bit for
bit."""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from specdec_amd import workloads as wl
from specdec_amd.engine.paged_cache import PagedKVCache
from specdec_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _layer(dev, lens, seed, h=12, kv=2, d=128, s=5):
    g = wl.gen(seed, dev)
    cache = PagedKVCache(kv, d, batch=len(lens), num_blocks=sum(-(-t // 16) for t in lens) + 9, device=dev,
                         seed=seed, growable=False)
    k = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
    cache.prefill(0, k, v, lens)
    q = torch.randn((len(lens), h, s, d), generator=g, device=dev).to(torch.bfloat16)
    return cache, q


def test_opcheck_paged_attention(cuda_device):
    announce("opcheck sdv::paged_attention")
    cache, q = _layer(cuda_device, [300, 77], seed=900)
    kp, vp, vs = cache.layer(0)
    args = (q, kp, vp, vs, cache.block_table(), cache.seq_lens_tensor(), 300)
    torch.library.opcheck(torch.ops.sdv.paged_attention.default, args)
    torch.library.opcheck(torch.ops.sdv.paged_attention.default, args[:5] + (None, 300))


def test_opcheck_quant_append_and_append_attend(cuda_device):
    announce("opcheck sdv::quant_append, sdv::paged_attention_append")
    cache, q = _layer(cuda_device, [200], seed=901, s=1)
    kp, vp, vs = cache.layer(0)
    g = wl.gen(902, cuda_device)
    cache.reserve(0, 232)
    slots = cache.slot_mapping([200], 32)
    k_new = torch.randn((32, 2, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    v_new = torch.randn((32, 2, 128), generator=g, device=cuda_device).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.sdv.quant_append.default, (v_new, slots, kp, vp, vs, k_new, "rcp"))
    sl = torch.tensor([201], dtype=torch.int32, device=cuda_device)
    torch.library.opcheck(torch.ops.sdv.paged_attention_append.default,
                          (q, kp, vp, vs, cache.block_table(), sl, 201, k_new[:1], v_new[:1], None, "rcp"))


def test_compiled_reference_op_matches_eager(cuda_device):
    """ops.attention traced by dynamo in one graph (no breaks) and run through AOT autograd."""
    announce("torch.compile of ops.attention")
    g = wl.gen(903, cuda_device)
    B, H, KV, T, S, D = 1, 12, 2, 1000, 5, 128
    q = torch.randn((B, H, S, D), generator=g, device=cuda_device).to(torch.bfloat16)
    k = torch.randn((B, KV, T, D), generator=g, device=cuda_device).to(torch.bfloat16)
    payload = torch.randn((B, KV, T, D), generator=g, device=cuda_device).to(torch.float8_e4m3fn)
    scale = torch.rand((B, KV, T, 1), generator=g, device=cuda_device) * 0.01 + 1e-3
    eager = ops.attention(q, k, (payload, scale))
    compiled = torch.compile(lambda a, b, c, d: ops.attention(a, b, (c, d)), fullgraph=True, backend="aot_eager")
    got = compiled(q, k, payload, scale)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)
