"""The FP8-V pack recorded into HIP graphs: the draft proposal chain and the target verify block.

Reference: experiments/cuda_graph_local -- local_ops.capture (local_ops.py:19-39: warm-up on a
side stream, then record), the draft chain A3 (draft_graph.py: s=1 steps with the cache advancing
inside the chain) and the M=5 block verify B2 (verify_graph.py:11-27), all at a fixed history
length with the tokens in a static device tensor.  There the recorded steps concatenate new cache
tensors, so the graph holds them in its memory pool (2.0 / 0.89 GiB, README.md:113-115); here a
recorded step writes the new tokens into the paged cache in place: slots come from the block
table on the device, the lengths are the call's scalars and the workspace is the pool's own, so
a recorded step copies nothing from the host and allocates nothing but activations.

Checks: a replay gives the logits of the same steps run eagerly through the pack, bit for bit;
after new tokens are copied into the static tensor, a replay gives the eager logits of the new
tokens; the greedy tokens equal the unpatched eager engine's (up to near ties, as in
tests/test_gpu_engine.py); and recording a step that would have to copy from the host (blocks
not reserved) raises instead of recording a stale copy.
"""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from oracle import engine as oeng
from specdec_amd import SdvError
from specdec_amd.kernels import patch

pytestmark = pytest.mark.gpu

TIE_FRAC = 0.02


def _prefill(model, prompt, use_pack=True):
    if use_pack:
        patch.install("fp8v", oeng, scale_mode="rcp", capacity_tokens=64, seed=5)
    else:
        patch.restore()
    model.set_kv_format("v_fp8")
    dev = model.embed_tokens.weight.device
    with torch.no_grad(), oeng.attention_phase("prefill"):
        lg, cache = model._run(model.embed_tokens(torch.tensor([prompt], device=dev)), None)
    return lg, cache


def _view(cache):
    """Shallow copies of the layer dicts: a chain advances the view's dicts, not the original's."""
    return [dict(layer) for layer in cache]


def _chain(model, toks, cache, phase):
    """len(toks) s=1 steps (draft proposal) or one block of all tokens (verify); logits per token."""
    out = []
    with torch.no_grad(), oeng.attention_phase(phase):
        if phase == "verify":
            lg, cache = model._run(model.embed_tokens(toks), cache)
            return lg, cache
        for i in range(toks.shape[1]):
            lg, cache = model._run(model.embed_tokens(toks[:, i:i + 1]), cache)
            out.append(lg)
    return torch.cat(out, 1), cache


def _record(fn):
    """local_ops.capture: warm up on a side stream, then record one call; returns (graph, outputs)."""
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    torch.cuda.synchronize()
    return graph, outs


def _argmax_match(got, want, what):
    """Greedy tokens of two logit blocks agree except at near ties of the eager logits."""
    g, w = got.float()[0], want.float()[0]
    for j in range(w.shape[0]):
        a, b = int(g[j].argmax()), int(w[j].argmax())
        if a != b:
            top = w[j].topk(2).values
            assert float(top[0] - top[1]) < TIE_FRAC * float(w[j].std()), f"{what}: token {j} differs clearly"


@pytest.mark.parametrize("case", ["draft_chain", "target_verify"])
def test_pack_steps_replay_from_a_graph(cuda_device, case):
    announce(f"graph-recorded pack: {case}")
    if case == "draft_chain":   # 0.5B-shaped attention (14/2/64), 5 proposal steps
        model = oeng.tiny_model(12, heads=14, kv_heads=2, head_dim=64, layers=3, device=cuda_device)
        phase = "propose"
    else:                       # 1.5B-shaped attention (12/2/128), one 5-row verify block
        model = oeng.tiny_model(11, layers=3, device=cuda_device)
        phase = "verify"
    gen = torch.Generator().manual_seed(23)
    prompt = torch.randint(0, 512, (90,), generator=gen).tolist()
    toks = torch.randint(0, 512, (1, 5), generator=gen).to(cuda_device)
    try:
        _, cache = _prefill(model, prompt)
        patch.reserve(cache, len(prompt) + 5)
        want, _ = _chain(model, toks, _view(cache), phase)          # eager, through the pack
        graph, (got, _) = _record(lambda: _chain(model, toks, _view(cache), phase))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), "a replay differs from the eager steps"
        # the same graph with new tokens in the static tensor
        toks.copy_(torch.randint(0, 512, (1, 5), generator=gen).to(cuda_device))
        graph.replay()
        torch.cuda.synchronize()
        got2 = got.clone()
        want2, _ = _chain(model, toks, _view(cache), phase)
        torch.cuda.synchronize()
        assert torch.equal(got2, want2), "a replay with new tokens differs from the eager steps"
        new_toks = toks[0].tolist()
    finally:
        patch.restore()
    # the unpatched eager engine (contiguous v_fp8 cache, eager attention) on the same tokens
    _, ecache = _prefill(model, prompt, use_pack=False)
    eager, _ = _chain(model, torch.tensor([new_toks], device=cuda_device), ecache, phase)
    rel = float((got2.float() - eager.float()).norm() / eager.float().norm())
    print(f"{case}: replay vs unpatched engine logits rel-L2 {rel:.2e}")
    assert rel <= 1e-2
    _argmax_match(got2, eager, case)


def test_recording_without_reserved_blocks_raises(cuda_device):
    """A step that needs a new page block would copy a new block table from the host: inside a
    recording that raises (the graph would replay a stale table), and reserving first fixes it."""
    announce("graph-recorded pack: unreserved blocks raise")
    model = oeng.tiny_model(11, layers=2, device=cuda_device)
    prompt = list(range(1, 65))                      # 64 tokens: the next token opens a new block
    toks = torch.tensor([[7]], device=cuda_device)
    try:
        _, cache = _prefill(model, prompt)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(SdvError):
            with torch.cuda.graph(graph):
                _chain(model, toks, _view(cache), "propose")
        torch.cuda.synchronize()
        patch.reserve(cache, len(prompt) + 1)       # outside the recording: now it records
        graph, (got, _) = _record(lambda: _chain(model, toks, _view(cache), "propose"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
    finally:
        patch.restore()
