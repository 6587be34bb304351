"""Pins for the restated engine (oracle.engine) on the CPU.

* cached decode == full forward (the reference's own gate, specdec/engine/test_cache_equiv.py:
  13-40: |delta| < 1e-3 on the last row and the same argmax), for the BF16-K/V format and for
  v_fp8 (whose per-token quantization is independent of how the prompt is split);
* SpecDec is lossless: greedy spec_decode_greedy emits target.generate's tokens (spec_dec.py's
  purpose; the reference's g4_b6_correctness.py checks the same), with a copy draft (every
  round accepted) and an unrelated draft (mismatch, trim and repair every round);
* RoPE is a rotation (pair norms kept, identity at position 0); RMSNorm output has unit RMS;
* the v_fp8 cache holds exactly quantize_kv_fp8 of the projected V, one group per head.
"""
from __future__ import annotations

import torch

from oracle import engine as oeng
from oracle import quant as oq


def _model(seed, **kw):
    return oeng.tiny_model(seed, vocab=300, hidden=64, heads=8, kv_heads=2, head_dim=64, inter=128,
                           dtype=torch.float32, **kw)


def test_cached_decode_equals_full_forward():
    for fmt in ("fp16", "v_fp8"):
        m = _model(0)
        m.set_kv_format(fmt)
        ids = torch.randint(0, 300, (1, 10), generator=torch.Generator().manual_seed(1))
        with torch.no_grad():
            full = m(ids)
            _, c = m._run(m.embed_tokens(ids[:, :9]), None)
            step, c = m._run(m.embed_tokens(ids[:, 9:]), c)
        assert (full[:, -1] - step[:, -1]).abs().max() < 1e-3, fmt
        assert torch.equal(full[:, -1].argmax(-1), step[:, -1].argmax(-1))
        assert c[0]["k"].shape[2] == 10


def test_specdec_is_lossless():
    target = _model(0)
    prompt = torch.randint(0, 300, (1, 12), generator=torch.Generator().manual_seed(2))
    target.set_kv_format("fp16")
    ar = target.generate(prompt, 24)[0].tolist()
    for draft, expect_all in ((_model(0), True), (_model(5, layers=1), False)):
        out = oeng.spec_decode_greedy(target, draft, prompt, 24, k=4)
        assert out["ids"][:len(ar)] == ar
        st = out["stats"]
        if expect_all:
            assert st["accepted"] == st["proposed"] and st["mismatch_rounds"] == 0
        else:
            assert st["mismatch_rounds"] > 0
        assert out["target_cache"][0]["k"].shape[2] == len(out["ids"])   # every emitted token is cached


def test_rope_and_rmsnorm():
    cos, sin = oeng.Build_Rope_cache(64, 7, 1e6, "cpu", torch.float32, start_pos=0)
    assert torch.equal(cos[0, 0, 0], torch.ones(64)) and torch.equal(sin[0, 0, 0], torch.zeros(64))
    x = torch.randn(1, 2, 7, 64, dtype=torch.float64)
    y = oeng.apply_rope(x, cos.double(), sin.double())
    pair = lambda t: (t[..., :32] ** 2 + t[..., 32:] ** 2)     # noqa: E731  (dims i and i+32 rotate together)
    assert torch.allclose(pair(x), pair(y))
    n = oeng.RMSNORM(64)(torch.randn(3, 64) * 7)
    assert torch.allclose(n.pow(2).mean(-1), torch.ones(3), atol=1e-4)


def test_vfp8_cache_is_quantized_projection():
    m = _model(3, layers=1)
    m.set_kv_format("v_fp8")
    ids = torch.randint(0, 300, (1, 9), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        _, c = m._run(m.embed_tokens(ids), None)
        a = m.layers[0].self_attn
        x = m.layers[0].input_layernorm(m.embed_tokens(ids))
        v = a.v_proj(x).view(1, 9, 2, 64).transpose(1, 2)
    q, s = oq.quantize_kv_fp8(v, 64, "div")
    assert torch.equal(c[0]["v"].view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(c[0]["v_scale"], s)
    assert c[0]["fmt"] == "v_fp8" and c[0]["k"].dtype == torch.float32
