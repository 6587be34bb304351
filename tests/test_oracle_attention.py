"""Pins oracle.attention (restatement of specdec/engine/model_self.py:739-776).

Checks chosen so that a plausible mistake fails one of them:
* agreement with the float64 truth within the BF16 noise bound at BASELINE shapes;
* closed forms: T = 1 gives exactly v_hat; identical keys give the mean of v_hat;
* the offset-causal mask: row i of an S=5 block equals S=1 attention over T-5+i+1 keys;
* planted mistakes (K transposed per head pair, 1/sqrt(D) dropped, mask off by one, V not
  dequantized) break those checks;
* the golden fixture (frozen oracle output) still matches bit for bit.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import attention as oatt
from oracle import quant as oq
from specdec_amd import workloads as wl

BOUND_TRUTH = 1.5e-2  # rel-L2 of eager BF16 vs fp64 truth (BF16 p and scores: ~5e-3 measured)


def _f64(t):
    return t.double().numpy()


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _vhat(v, d):
    q, s = oq.quantize_kv_fp8(v, d)
    return oq.dequantize_kv_fp8(q, s, torch.bfloat16)


@pytest.mark.parametrize("h,kv,d,t,s", [(12, 2, 128, 2048, 1), (12, 2, 128, 8192, 1),
                                        (12, 2, 128, 2048, 5), (14, 2, 64, 4096, 1)])
def test_eager_close_to_fp64_truth(h, kv, d, t, s):
    g = wl.gen(100 + t + s)
    q = wl.randn_bf16((1, h, s, d), g)
    k = wl.randn_bf16((1, kv, t, d), g)
    vh = _vhat(wl.randn_bf16((1, kv, t, d), g), d)
    o = oatt.eager_attention(q, k, vh)
    truth = oatt.attention_fp64(_f64(q), _f64(k), _f64(vh))
    assert oatt.rel_l2(_f64(o), truth) < BOUND_TRUTH
    o32 = oatt.attention_fp32(q, k, vh)
    assert oatt.rel_l2(_f64(o32), truth) < 5e-3


def test_single_key_returns_v_hat():
    g = wl.gen(7)
    q = wl.randn_bf16((1, 12, 1, 128), g)
    k = wl.randn_bf16((1, 2, 1, 128), g)
    vh = _vhat(wl.randn_bf16((1, 2, 1, 128), g), 128)
    o = oatt.eager_attention(q, k, vh)
    assert torch.equal(o, oatt.kv_repeat(vh, 6))


def test_identical_keys_give_mean_of_v_hat():
    g = wl.gen(8)
    t = 256
    q = wl.randn_bf16((1, 12, 1, 128), g)
    k = wl.randn_bf16((1, 2, 1, 128), g).expand(1, 2, t, 128).contiguous()
    vh = _vhat(wl.randn_bf16((1, 2, t, 128), g), 128)
    o = oatt.eager_attention(q, k, vh)
    mean = oatt.kv_repeat(vh, 6).double().mean(dim=2, keepdim=True)  # p = bf16(1/256) exact
    assert float((o.double() - mean).abs().max()) <= 2.0 ** -8 * float(mean.abs().max()) + 1e-6


def test_verify_rows_equal_truncated_decode():
    g = wl.gen(9)
    t, s = 300, 5
    q = wl.randn_bf16((1, 12, s, 128), g)
    k = wl.randn_bf16((1, 2, t, 128), g)
    vh = _vhat(wl.randn_bf16((1, 2, t, 128), g), 128)
    o = oatt.eager_attention(q, k, vh)
    for i in range(s):
        n = t - s + i + 1
        oi = oatt.eager_attention(q[:, :, i:i + 1], k[:, :, :n], vh[:, :, :n])
        assert oatt.rel_l2(_f64(o[:, :, i:i + 1]), _f64(oi)) < 1e-4, i


def test_planted_mistakes_fail():
    g = wl.gen(10)
    t, s = 512, 5
    q = wl.randn_bf16((1, 12, s, 128), g)
    k = wl.randn_bf16((1, 2, t, 128), g)
    v = wl.randn_bf16((1, 2, t, 128), g)
    vh = _vhat(v, 128)
    truth = oatt.attention_fp64(_f64(q), _f64(k), _f64(vh))
    good = oatt.rel_l2(_f64(oatt.eager_attention(q, k, vh)), truth)
    assert good < BOUND_TRUTH
    # K of the two KV heads swapped (a GQA head-index slip)
    bad = oatt.eager_attention(q, k.flip(1), vh)
    assert oatt.rel_l2(_f64(bad), truth) > 10 * good
    # scale 1/sqrt(D) dropped
    kr, vr = oatt.kv_repeat(k, 6), oatt.kv_repeat(vh, 6)
    sc = torch.matmul(q, kr.transpose(-2, -1)).masked_fill(~oatt.causal_keep(s, t), float("-inf"))
    bad = torch.matmul(torch.softmax(sc, -1, dtype=torch.float32).to(torch.bfloat16), vr)
    assert oatt.rel_l2(_f64(bad), truth) > 10 * good
    # mask off by one (row i sees T-S+i+1 keys -> T-S+i+2)
    sc = (torch.matmul(q, kr.transpose(-2, -1)) / 128 ** 0.5)
    j = torch.arange(t)[None]
    i = torch.arange(s)[:, None]
    sc = sc.masked_fill(~(j <= (t - s) + i + 1), float("-inf"))
    bad = torch.matmul(torch.softmax(sc, -1, dtype=torch.float32).to(torch.bfloat16), vr)
    n = t - s + 1  # row 0 must equal decode over the first T-S+1 keys (bound 1e-4 above)
    row0 = oatt.eager_attention(q[:, :, :1], k[:, :, :n], vh[:, :, :n])
    assert oatt.rel_l2(_f64(bad[:, :, :1]), _f64(row0)) > 1e-3
    # V payload used without its scale
    qv, _ = oq.quantize_kv_fp8(v, 128)
    bad = oatt.eager_attention(q, k, qv.to(torch.bfloat16))
    assert oatt.rel_l2(_f64(bad), truth) > 10 * good


def test_vfp8_step_matches_one_shot():
    """Appending in two steps (prefill, then S=1) equals attention over the whole cache."""
    g = wl.gen(12)
    t = 96
    q = wl.randn_bf16((1, 12, 1, 128), g)
    k = wl.randn_bf16((1, 2, t, 128), g)
    v = wl.randn_bf16((1, 2, t, 128), g)
    _, cache = oatt.vfp8_decode_step(None, wl.randn_bf16((1, 12, t - 1, 128), g), k[:, :, :-1], v[:, :, :-1])
    o, cache2 = oatt.vfp8_decode_step(cache, q, k[:, :, -1:], v[:, :, -1:])
    assert cache2["v"].shape[2] == t and cache2["v_scale"].shape == (1, 2, t, 1)
    assert torch.equal(o, oatt.eager_attention(q, k, _vhat(v, 128)))


def test_golden_attention_fixture():
    z = np.load(GOLDEN / "attn_eager.npz")
    q, k, v = wl.config0(seed=0)
    h = hashlib.sha256()
    for a in (_bits(q), _bits(k), _bits(v)):
        h.update(a.tobytes())
    assert h.hexdigest().encode() == z["cfg0_input_sha256"].tobytes(), "torch CPU RNG drifted"
    o = oatt.eager_attention(q, k, _vhat(v, 128))
    assert np.array_equal(_bits(o), z["cfg0_out"])
    for name, d in (("verify", 128), ("draft", 64)):
        qq, kk, vv = (torch.from_numpy(z[f"{name}_{x}"].view(np.int16)).view(torch.bfloat16) for x in "qkv")
        o = oatt.eager_attention(qq, kk, _vhat(vv, d))
        assert np.array_equal(_bits(o), z[f"{name}_out"]), name


@pytest.mark.parametrize("d", [128, 64])
def test_reciprocal_scale_equals_division_for_every_bf16(d):
    """The kernels compute bf16(s * RN(1/sqrt(D))) where eager computes bf16(s / sqrt(D))
    (model_self.py:754) on a BF16 s; both round to the same BF16 for all 65536 inputs."""
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    fin = torch.isfinite(x.float())
    eager = x / (d ** 0.5)                                          # the reference expression
    kern = (x.float() * torch.tensor(1.0 / d ** 0.5, dtype=torch.float32)).to(torch.bfloat16)
    assert torch.equal(eager.view(torch.int16)[fin], kern.view(torch.int16)[fin])
