"""Eager GQA attention and the v_fp8 decode step, restated in torch-CPU (TEST INFRASTRUCTURE ONLY).

* ``kv_repeat``          -- model_self.py:294-298 (and kernels/reference.py:33-37).
* ``eager_attention``    -- model_self.py:739-776 / kernels/reference.py:47-56: BF16 ``q @ k^T``
                            (fp32 accumulate, BF16 result), ``/ sqrt(D)`` (BF16 result), the
                            offset-causal mask ``triu(diagonal = T - S + 1)`` (model_self.py:
                            755-764, reference.py:40-44; empty for S == 1), fp32 softmax,
                            probabilities rounded to BF16, BF16 ``p @ v`` (fp32 accumulate).
* ``attention_fp32``     -- kernels/reference.py:59-70 (fp32 algorithm reference).
* ``attention_fp64``     -- numpy float64 ground truth on the same (rounded) inputs.
* ``vfp8_decode_step``   -- the v_fp8 branch of SelfAttention.forward with a cache
                            (model_self.py:689-706 quantize current V, :715-728 K cat and V
                            dequant+cat, :739-776 attention, :778-800 append payload + scale).

Pinned by (tests/test_oracle_attention.py): agreement with the fp64 truth within the BF16
noise bound at every BASELINE shape; T = 1 gives exactly v_hat; identical keys give the
mean of v_hat; the S = 5 rows equal S = 1 attention over the first T - 5 + i + 1 keys;
planted mistakes (transposed K, dropped 1/sqrt(D), mask off by one) fail those checks.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .quant import dequantize_kv_fp8, quantize_kv_fp8


def kv_repeat(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """(B, KV, T, D) -> (B, KV * n_rep, T, D), each KV head repeated n_rep times in place."""
    if n_rep == 1:
        return x
    b, kv, t, d = x.shape
    return x[:, :, None].expand(b, kv, n_rep, t, d).reshape(b, kv * n_rep, t, d)


def causal_keep(s: int, t: int) -> torch.Tensor:
    """Row i of an S-row block over T keys sees key j iff j <= (T - S) + i."""
    j = torch.arange(t)[None, :]
    i = torch.arange(s)[:, None]
    return j <= (t - s) + i


def eager_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """q (B,H,S,D), k/v (B,KV,T,D), all BF16 -> (B,H,S,D) BF16, eager rounding points."""
    n_rep = q.shape[1] // k.shape[1]
    kr = kv_repeat(k, n_rep)
    vr = kv_repeat(v, n_rep)
    scores = torch.matmul(q, kr.transpose(-2, -1)) / (q.shape[-1] ** 0.5)
    s, t = q.shape[-2], k.shape[-2]
    if s > 1:
        scores = scores.masked_fill(~causal_keep(s, t), float("-inf"))
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(probs, vr)


def attention_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """kernels/reference.py:59-70: same mask, fp32 scores/softmax/PV, output in q.dtype."""
    n_rep = q.shape[1] // k.shape[1]
    kr = kv_repeat(k, n_rep).float()
    vr = kv_repeat(v, n_rep).float()
    scores = torch.matmul(q.float(), kr.transpose(-2, -1)) * (q.shape[-1] ** -0.5)
    s, t = q.shape[-2], k.shape[-2]
    if s > 1:
        scores = scores.masked_fill(~causal_keep(s, t), float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), vr).to(q.dtype)


def attention_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """Float64 ground truth.  q (B,H,S,D), k/v (B,KV,T,D) as float arrays; returns float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, h, s, d = q.shape
    kv, t = k.shape[1], k.shape[2]
    g = h // kv
    out = np.empty((b, h, s, d), dtype=np.float64)
    keep = causal_keep(s, t).numpy()
    for bi in range(b):
        for hi in range(h):
            kh = k[bi, hi // g]
            vh = v[bi, hi // g]
            sc = q[bi, hi] @ kh.T / math.sqrt(d)
            sc = np.where(keep, sc, -np.inf)
            sc = sc - sc.max(axis=-1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(axis=-1, keepdims=True)
            out[bi, hi] = p @ vh
    return out


def vfp8_decode_step(cache: dict | None, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                     group_size: int | None = None, scale_mode: str = "div"):
    """One v_fp8 attention step on a contiguous cache dict (model_self.py:689-728, 739-800).

    cache: None or {"fmt": "v_fp8", "k": BF16 (B,KV,T0,D), "v": fp8 (B,KV,T0,D),
    "v_scale": fp32 (B,KV,T0,1)}.  q (B,H,S,D), k_new/v_new (B,KV,S,D) BF16 (post-RoPE).
    Returns (out (B,H,S,D) BF16, new cache dict).  The cache argument is not mutated.
    """
    gs = group_size if group_size is not None else v_new.shape[-1]
    qv, vs = quantize_kv_fp8(v_new, gs, scale_mode)
    v_cur = dequantize_kv_fp8(qv, vs, v_new.dtype)
    if cache is None:
        k_all, v_all = k_new, v_cur
        new = {"fmt": "v_fp8", "k": k_new, "v": qv, "v_scale": vs}
    else:
        k_all = torch.cat([cache["k"], k_new], dim=2)
        v_all = torch.cat([dequantize_kv_fp8(cache["v"], cache["v_scale"], v_new.dtype), v_cur], dim=2)
        new = {"fmt": "v_fp8", "k": k_all,
               "v": torch.cat([cache["v"], qv], dim=2),
               "v_scale": torch.cat([cache["v_scale"], vs], dim=2)}
    return eager_attention(q, k_all, v_all), new


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max()) if a.size else 0.0
