"""Pins the rounding points of oracle.attention.eager_attention with a second derivation.

The eager path (model_self.py:739-776) rounds at fixed points: BF16 q.k^T (fp32 accumulate),
BF16 of the scaled score, fp32 softmax normalised by the global max and sum, probabilities
rounded to BF16, fp32-accumulated p.v_hat, BF16 output; v_hat = bf16(fp32(code) * scale)
(model_self.py:316-320).  ``derive`` below restates that sequence in numpy with an explicit
round-to-nearest-even BF16 (integer arithmetic on the fp32 bit pattern), independent of
torch's kernels; it must agree with the torch restatement to a few 1e-6 rel-L2 (the only
freedom left is the fp32 summation order inside the two products, which moves a score across
a BF16 rounding boundary now and then).  Each planted mistake -- the probabilities kept in
fp32, the scores kept in fp32, the scaled score not rounded (for D = 128: with D = 64 the
scale 1/8 is exact and only dropping both score roundings shows), an online (running-max)
normalisation -- moves the result by far more than that bound, so an oracle that made one of
them would fail here.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import quant as oq
from specdec_amd import workloads as wl

AGREE = 2e-5   # derivation vs torch restatement (rel-L2)
TEETH = 2e-4   # every planted mistake must move the result by at least this much


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest BF16 (ties to even), returned as fp32.  Inputs are finite or -inf."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32)
    return np.where(np.isinf(x), x, out)


def derive(q, k, v_hat, *, round_p=True, round_scores=True, round_scaled=True, online=False):
    """numpy restatement of the eager rounding sequence (q (B,H,S,D), k/v_hat (B,KV,T,D) fp32
    holding BF16 values) -> (B,H,S,D) fp32 holding BF16 values."""
    b_, h, s, d = q.shape
    kv, t = k.shape[1], k.shape[2]
    g = h // kv
    keep = oatt.causal_keep(s, t).numpy() if s > 1 else np.ones((1, t), dtype=bool)
    scale = np.float32(math.sqrt(d))
    out = np.empty(q.shape, dtype=np.float32)
    for bi in range(b_):
        for hi in range(h):
            kh, vh = k[bi, hi // g], v_hat[bi, hi // g]
            sc = (q[bi, hi].astype(np.float64) @ kh.astype(np.float64).T).astype(np.float32)
            if round_scores:
                sc = bf16_round(sc)
            sc = (sc / scale).astype(np.float32)
            if round_scaled:
                sc = bf16_round(sc)
            sc = np.where(keep, sc, np.float32(-np.inf))
            if online:   # one pass: BF16 p against each 64-key chunk's own max, rescaled partials
                o_acc = np.zeros((s, d), dtype=np.float64)
                l_acc = np.zeros(s, dtype=np.float64)
                m_run = np.full(s, -np.inf)
                for j0 in range(0, t, 64):
                    blk = sc[:, j0:j0 + 64]
                    mc = blk.max(axis=-1)
                    m_new = np.maximum(m_run, mc)
                    safe = np.where(np.isinf(m_new), 0.0, m_new)
                    pc = bf16_round(np.exp((blk - safe[:, None]).astype(np.float32)).astype(np.float32))
                    corr = np.where(np.isinf(m_run), 0.0, np.exp(m_run - safe))
                    o_acc = o_acc * corr[:, None] + pc.astype(np.float64) @ vh[j0:j0 + 64].astype(np.float64)
                    l_acc = l_acc * corr + pc.astype(np.float64).sum(axis=-1)
                    m_run = m_new
                out[bi, hi] = bf16_round((o_acc / l_acc[:, None]).astype(np.float32))
                continue
            mx = sc.max(axis=-1, keepdims=True)
            e = np.exp((sc - mx).astype(np.float32)).astype(np.float32)
            p = (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
            if round_p:
                p = bf16_round(p)
            o = (p.astype(np.float64) @ vh.astype(np.float64)).astype(np.float32)
            out[bi, hi] = bf16_round(o)
    return out


def _case(h, kv, d, t, s, seed):
    g = wl.gen(seed)
    q = wl.randn_bf16((1, h, s, d), g)
    k = wl.randn_bf16((1, kv, t, d), g)
    v = wl.randn_bf16((1, kv, t, d), g)
    pq, ps = oq.quantize_kv_fp8(v, d)
    v_hat = oq.dequantize_kv_fp8(pq, ps, torch.bfloat16)
    want = oatt.eager_attention(q, k, v_hat).float().numpy()
    return q.float().numpy(), k.float().numpy(), v_hat.float().numpy(), want


CASES = [(12, 2, 128, 2048, 1, 1), (12, 2, 128, 1024, 5, 2), (14, 2, 64, 1536, 1, 3), (12, 2, 128, 300, 16, 4)]


@pytest.mark.parametrize("h,kv,d,t,s,seed", CASES)
def test_eager_matches_numpy_derivation(h, kv, d, t, s, seed):
    q, k, v_hat, want = _case(h, kv, d, t, s, seed)
    got = derive(q, k, v_hat)
    rl = oatt.rel_l2(got, want)
    print(f"derivation vs eager h={h} d={d} t={t} s={s}: rel-L2 {rl:.2e}")
    assert rl <= AGREE


@pytest.mark.parametrize("mistake", ["p_fp32", "scores_fp32", "scaled_unrounded", "no_score_rounding", "online"])
@pytest.mark.parametrize("h,kv,d,t,s,seed", CASES[:3])
def test_planted_rounding_mistakes_fail(h, kv, d, t, s, seed, mistake):
    if mistake in ("scores_fp32", "scaled_unrounded") and d == 64:
        pytest.skip("1/sqrt(64) = 1/8 is exact: bf16(bf16(x)/8) = bf16(x/8) = bf16(x)/8, so either one of the "
                    "two score roundings alone gives the eager scores (dropping both is checked)")
    q, k, v_hat, want = _case(h, kv, d, t, s, seed)
    kw = {"p_fp32": dict(round_p=False), "scores_fp32": dict(round_scores=False),
          "scaled_unrounded": dict(round_scaled=False),
          "no_score_rounding": dict(round_scores=False, round_scaled=False), "online": dict(online=True)}[mistake]
    rl = oatt.rel_l2(derive(q, k, v_hat, **kw), want)
    print(f"planted {mistake} h={h} d={d} t={t} s={s}: rel-L2 {rl:.2e}")
    assert rl >= TEETH, f"{mistake} is not distinguishable from the eager rounding ({rl:.2e})"


def test_bf16_round_known_values():
    """Ties to even and carries into the exponent, checked against torch's BF16 cast."""
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, 3.0e38, -2.5, 1e-30, 0.0, -0.0,
                     1 + 2 ** -8, 1 + 3 * 2 ** -8, 65535.0, -np.inf], dtype=np.float32)
    rng = np.random.default_rng(0)
    vals = np.concatenate([vals, rng.standard_normal(100000).astype(np.float32) * 10])
    ref = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
    assert np.array_equal(bf16_round(vals).view(np.uint32), ref.view(np.uint32))
