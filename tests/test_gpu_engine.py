"""The FP8-V pack inside an engine: prefill, decode, block verify, trim + repair, SpecDec.

The engine is the restated reference engine (oracle.engine, after model_self.py and
spec_dec.py); the pack replaces its SelfAttention.forward for the v_fp8 format
(specdec/kernels/patch.py:55-136 is the reference's counterpart).  Checks:

* layer 0's cache after prefill / decode / verify / trim / repair equals the eager engine's
  cache byte for byte (BF16 K, E4M3FN V payload, fp32 scales): layer 0's K and V depend on
  the embeddings only, so both engines quantize identical inputs;
* every call's logits agree with the eager engine's (teacher forced, same tokens);
* greedy SpecDec under the pack emits the eager engine's tokens up to the first position
  whose eager top-2 logit margin is a near tie (the only place BF16 rounding differences
  between two correct attention implementations may flip an argmax).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from helpers import bits16
from oracle import engine as oeng
from specdec_amd.engine import spec_cache as sc
from specdec_amd.kernels import patch

pytestmark = pytest.mark.gpu

LOGIT_REL_L2 = 1e-2      # whole-model logits, two layers, vs the eager engine
TIE_FRAC = 0.02          # near tie: top-2 margin below 2% of the logits' standard deviation


def _call_seq(model, prompt, use_pack: bool):
    """prefill(77) -> decode 1 -> verify 5 -> trim to pre+2 -> repair step -> decode 1."""
    if use_pack:
        patch.install("fp8v", oeng, scale_mode="rcp", capacity_tokens=48, seed=7)
    else:
        patch.restore()
    model.set_kv_format("v_fp8")
    dev = model.embed_tokens.weight.device
    emb = lambda ids: model.embed_tokens(torch.tensor([ids], device=dev))   # noqa: E731
    logits = []
    with torch.inference_mode():
        lg, cache = model._run(emb(prompt), None)
        logits.append(lg)
        lg, cache = model._run(emb([17]), cache)
        logits.append(lg)
        pre = sc.cache_length(cache)
        lg, cache = model._run(emb([3, 141, 59, 26, 5]), cache)
        logits.append(lg)
        cache = sc.trim_cache(cache, pre + 2)
        lg, cache = model._run(emb([358]), cache)
        logits.append(lg)
        lg, cache = model._run(emb([97]), cache)
        logits.append(lg)
    patch.restore()
    return logits, cache


def test_engine_cache_bytes_and_logits(cuda_device):
    announce("engine teacher-forced prefill/decode/verify/trim/repair")
    model = oeng.tiny_model(11, device=cuda_device)
    prompt = torch.randint(0, 512, (77,), generator=torch.Generator().manual_seed(3)).tolist()
    want_lg, want_cache = _call_seq(model, prompt, use_pack=False)
    got_lg, got_cache = _call_seq(model, prompt, use_pack=True)
    T = sc.cache_length(want_cache)
    assert T == 77 + 1 + 2 + 1 + 1 and sc.cache_length(got_cache) == T
    sc.check_consistent(got_cache)
    assert all("pages" in layer for layer in got_cache)
    for i, (g, w) in enumerate(zip(got_lg, want_lg)):
        g, w = g.float().cpu(), w.float().cpu()
        assert g.shape == w.shape and torch.isfinite(g).all()
        rel = float((g - w).norm() / w.norm())
        print(f"call {i}: logits rel_l2={rel:.2e}")
        assert rel <= LOGIT_REL_L2, f"call {i}: rel_l2 {rel:.3e}"
    got0 = got_cache[0]["pages"].materialize(T)
    w0 = want_cache[0]
    assert np.array_equal(bits16(got0["k"]), bits16(w0["k"]))
    assert torch.equal(got0["v"].view(torch.uint8).cpu(), w0["v"].view(torch.uint8).cpu())
    assert torch.equal(got0["v_scale"].cpu().view(torch.int32), w0["v_scale"].cpu().view(torch.int32))


def _first_divergence(a, b):
    for j, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return j
    return None


def _near_tie(target, ids_prefix) -> tuple[bool, float]:
    """Eager, uncached target logits for the next token after ids_prefix; (is near tie, margin)."""
    patch.restore()
    target.set_kv_format("v_fp8")
    dev = target.embed_tokens.weight.device
    with torch.inference_mode():
        lg, _ = target._run(target.embed_tokens(torch.tensor([ids_prefix], device=dev)), None)
    row = lg[0, -1].float()
    top = row.topk(2).values
    margin = float(top[0] - top[1])
    return margin < TIE_FRAC * float(row.std()), margin


@pytest.mark.parametrize("case", ["copy_draft", "d64_draft"])
def test_specdec_tokens_match_eager(cuda_device, case):
    """SpecDec (k=4) with the target on the paged FP8-V pack vs the same loop on the eager engine."""
    announce(f"engine specdec {case}")
    target = oeng.tiny_model(11, device=cuda_device)
    if case == "copy_draft":
        draft = oeng.tiny_model(11, device=cuda_device)            # same weights: long accepted runs
        draft_kv = "base_bf16"
    else:
        draft = oeng.tiny_model(12, heads=14, kv_heads=2, head_dim=64, layers=1, device=cuda_device)
        draft_kv = "v_fp8"                                           # D=64 draft on the pack as well
    prompt = torch.randint(0, 512, (1, 60), generator=torch.Generator().manual_seed(5))
    kw = dict(k=4, target_kv="v_fp8", draft_kv=draft_kv)
    patch.restore()
    want = oeng.spec_decode_greedy(target, draft, prompt, 40, **kw)
    oeng.CALLS.clear()
    patch.install("fp8v", oeng, scale_mode="rcp", capacity_tokens=48, seed=9)
    try:
        got = oeng.spec_decode_greedy(target, draft, prompt, 40, **kw)
    finally:
        patch.restore()
    assert all("pages" in layer for layer in got["target_cache"])
    assert {c[1] for c in oeng.CALLS} >= {"prefill", "propose", "verify"}
    st = got["stats"]
    print(case, "eager", want["stats"], "pack", st)
    assert st["rounds"] > 0 and st["accepted"] <= st["proposed"] and len(got["gen"]) >= 40
    if case == "copy_draft":
        assert st["accepted"] >= st["proposed"] // 2
    else:
        assert st["mismatch_rounds"] > 0                            # trim + repair exercised
    j = _first_divergence(got["ids"], want["ids"])
    if j is not None:
        tie, margin = _near_tie(target, got["ids"][:j])
        assert tie, f"tokens diverge at {j} with a clear eager margin {margin:.3f}"
        print(f"diverged at {j} on a near tie (margin {margin:.3f})")
