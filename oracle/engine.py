"""A small engine restated from the reference (TEST INFRASTRUCTURE ONLY).

The FP8-V pack (specdec_amd.kernels.patch) patches ``SelfAttention.forward`` of an engine
module the way the reference's kernels/patch.py patches specdec.engine.model_self.  The
reference module cannot be imported here, so the tests hand the pack this restatement of the
parts it touches, and compare the patched engine against the unpatched one:

* ``RMSNORM``, ``Embedding``, ``MLP``         -- model_self.py:225-270 (SiLU-gated MLP);
* ``Build_Rope_cache``, ``rotate_half``,
  ``apply_rope``, ``kv_repeat``              -- :272-298;
* ``quantize_kv_fp8`` / ``dequantize_kv_fp8`` -- :304-320 via oracle.quant, with the divisor
  evaluated the way torch evaluates ``m / 448`` on the tensor's device (IEEE division on the
  CPU, multiplication by RN(1/448) on a GPU);
* ``SelfAttention.forward``                   -- :668-809 for the "fp16" (BF16 K/V) and "v_fp8"
  (BF16 K, FP8 V with one scale per token and KV head) formats, eager attention only; the
  full-FP8 ablation ("fp8") and the diagnostic probes are out of scope;
* ``DecoderLayer``, ``QwenLM._run / generate / set_kv_format`` -- :811-900;
* phase tagging and call accounting          -- :413-536 reduced to what a pack calls:
  ``_ATTENTION_PHASE``, ``attention_phase``, ``decide_attention_path``, ``_record_attention_call``;
* ``spec_decode_greedy``                      -- spec_dec.py:189-263 (block verify mode).

Two deliberate departures, neither changing a value: matmul right operands that are
transposed views are made contiguous first (batched BF16 products on transposed views have
faulted this GPU pool), and ``set_kv_format("v_fp8")`` accepts head_dim 64 with one group
per head (the reference asserts head_dim % 128 == 0).
"""
from __future__ import annotations

import contextlib
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import quant as oq
from .attention import kv_repeat  # noqa: F401  (re-exported: part of the engine surface)

E4M3_MAX = oq.E4M3_MAX
GROUP_SIZE = 32
GROUP_V = 128


# --------------------------------------------------------------------------- accounting
_ATTENTION_PHASE = "other"
ATTENTION_STRATEGY = "eager"
CALLS: list = []


@contextlib.contextmanager
def attention_phase(name: str):
    global _ATTENTION_PHASE
    prev, _ATTENTION_PHASE = _ATTENTION_PHASE, name
    try:
        yield
    finally:
        _ATTENTION_PHASE = prev


def decide_attention_path(phase: str, s: int, strategy: str | None = None):
    strat = ATTENTION_STRATEGY if strategy is None else strategy
    if strat == "cudnn_prefill" and phase == "prefill" and s >= 2:
        return "fused", None
    return "eager", f"strategy={strat}" if strat != "cudnn_prefill" else f"phase={phase!r}"


def _record_attention_call(path, phase, s, T, reason, heads, kv_heads, head_dim) -> None:
    CALLS.append((path, phase, s, T))


# --------------------------------------------------------------------------- layers
class RMSNORM(nn.Module):
    def __init__(self, hidden: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * y.to(x.dtype)


class Embedding(nn.Module):
    def __init__(self, vocab: int, hidden: int):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(vocab, hidden))

    def forward(self, ids):
        return self.weight[ids]


class MLP(nn.Module):
    def __init__(self, hidden: int, inter: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden, inter, bias=False)
        self.up_proj = nn.Linear(hidden, inter, bias=False)
        self.down_proj = nn.Linear(inter, hidden, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


def Build_Rope_cache(head_dim, seq_len, theta, device, dtype, start_pos=0):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    pos = torch.arange(start_pos, start_pos + seq_len, device=device, dtype=torch.float32)
    ang = torch.outer(pos, inv)
    cos = torch.cat([ang.cos(), ang.cos()], -1)[None, None]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[None, None]
    return cos.to(dtype), sin.to(dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], -1)


def apply_rope(x, cos, sin):
    return x * cos + rotate_half(x) * sin


def quantize_kv_fp8(x, group_size=GROUP_SIZE):
    return oq.quantize_kv_fp8(x, group_size, "rcp" if x.is_cuda else "div")


def dequantize_kv_fp8(q, scale, dtype=torch.float16):
    return oq.dequantize_kv_fp8(q, scale, dtype)


def _eager(q, k_all, v_all, s, T, masked: bool):
    n_rep = q.shape[1] // k_all.shape[1]
    kr = kv_repeat(k_all, n_rep)
    vr = kv_repeat(v_all, n_rep).contiguous()
    scores = torch.matmul(q.contiguous(), kr.transpose(-2, -1).contiguous()) / (q.shape[-1] ** 0.5)
    if masked:
        drop = torch.triu(torch.ones(s, T, device=q.device, dtype=torch.bool), diagonal=T - s + 1)
        scores = scores.masked_fill(drop, float("-inf"))
    p = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(p, vr).to(q.dtype)


class SelfAttention(nn.Module):
    def __init__(self, hidden, heads, kv_heads, head_dim, attn_bias=False):
        super().__init__()
        self.q_proj = nn.Linear(hidden, heads * head_dim, bias=attn_bias)
        self.k_proj = nn.Linear(hidden, kv_heads * head_dim, bias=attn_bias)
        self.v_proj = nn.Linear(hidden, kv_heads * head_dim, bias=attn_bias)
        self.o_proj = nn.Linear(heads * head_dim, hidden, bias=False)
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.kv_format = "fp16"

    def forward(self, x, cos, sin, cache=None):
        b, s, _ = x.shape
        q = self.q_proj(x).view(b, s, self.heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(b, s, self.kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(b, s, self.kv_heads, self.head_dim).transpose(1, 2)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
        fmt = cache.get("fmt", self.kv_format) if cache is not None else self.kv_format
        if fmt not in ("fp16", "v_fp8"):
            raise ValueError(f"cache format {fmt!r} is not restated here")
        qv = vs = None
        if fmt == "v_fp8":
            qv, vs = quantize_kv_fp8(v, self.head_dim)          # one group per head
            v_cur = dequantize_kv_fp8(qv, vs, x.dtype)
        else:
            v_cur = v
        if cache is None:
            k_all, v_all = k, v_cur
        elif fmt == "fp16":
            k_all = torch.cat([cache["k"], k], 2)
            v_all = torch.cat([cache["v"], v], 2)
            cache["k"], cache["v"] = k_all, v_all
        else:
            k_all = torch.cat([cache["k"], k], 2)
            cache["k"] = k_all
            v_all = torch.cat([dequantize_kv_fp8(cache["v"], cache["v_scale"], x.dtype), v_cur], 2)
        T = k_all.shape[2] if cache is not None else s
        path, reason = decide_attention_path(_ATTENTION_PHASE, s)
        _record_attention_call(path, _ATTENTION_PHASE, s, T, reason, self.heads, self.kv_heads, self.head_dim)
        out = _eager(q, k_all, v_all, s, T, masked=(cache is None or s > 1))
        out = out.transpose(1, 2).contiguous().view(b, s, self.heads * self.head_dim)
        if cache is None:
            new = {"fmt": "v_fp8", "k": k_all, "v": qv, "v_scale": vs} if fmt == "v_fp8" else {"k": k_all, "v": v_all}
        elif fmt == "v_fp8":
            cache["v"] = torch.cat([cache["v"], qv], 2)
            cache["v_scale"] = torch.cat([cache["v_scale"], vs], 2)
            new = cache
        else:
            new = cache
        return self.o_proj(out), new


class DecoderLayer(nn.Module):
    def __init__(self, hidden, heads, kv_heads, head_dim, inter, attn_bias=False):
        super().__init__()
        self.self_attn = SelfAttention(hidden, heads, kv_heads, head_dim, attn_bias)
        self.mlp = MLP(hidden, inter)
        self.input_layernorm = RMSNORM(hidden)
        self.post_attention_layernorm = RMSNORM(hidden)

    def forward(self, x, cos, sin, cache=None):
        a, c = self.self_attn(self.input_layernorm(x), cos, sin, cache)
        x = x + a
        return x + self.mlp(self.post_attention_layernorm(x)), c


class QwenLM(nn.Module):
    def __init__(self, vocab, hidden, heads, kv_heads, head_dim, inter, num_layers, rope_theta=1_000_000.0,
                 attn_bias=False):
        super().__init__()
        self.embed_tokens = Embedding(vocab, hidden)
        self.layers = nn.ModuleList(DecoderLayer(hidden, heads, kv_heads, head_dim, inter, attn_bias)
                                    for _ in range(num_layers))
        self.norm = RMSNORM(hidden)
        self.head_dim, self.rope_theta, self.kv_format = head_dim, rope_theta, "fp16"

    def _run(self, x, cache_list=None, need_logits=True):
        start = cache_list[0]["k"].shape[2] if cache_list is not None and cache_list[0] is not None else 0
        cos, sin = Build_Rope_cache(self.head_dim, x.size(1), self.rope_theta, x.device, x.dtype, start)
        new = []
        for i, layer in enumerate(self.layers):
            x, c = layer(x, cos, sin, cache_list[i] if cache_list is not None else None)
            new.append(c)
        x = self.norm(x)
        return (x @ self.embed_tokens.weight.T if need_logits else None), new

    def forward(self, token_ids):
        return self._run(self.embed_tokens(token_ids))[0]

    def generate(self, prompt_ids, max_new_tokens, eos_id=None):
        gen = prompt_ids
        with torch.no_grad():
            lg, cache = self._run(self.embed_tokens(prompt_ids), None)
            for _ in range(max_new_tokens):
                nxt = lg[:, -1].argmax(-1)
                if eos_id is not None and (nxt == eos_id).all():
                    break
                gen = torch.cat([gen, nxt[:, None]], 1)
                lg, cache = self._run(self.embed_tokens(nxt[:, None]), cache)
        return gen

    def set_kv_format(self, fmt: str) -> None:
        if fmt not in ("fp16", "v_fp8"):
            raise ValueError(fmt)
        self.kv_format = fmt
        for layer in self.layers:
            layer.self_attn.kv_format = fmt


# --------------------------------------------------------------------------- SpecDec (spec_dec.py)
def _cache_length(cache):
    return 0 if cache is None else int(cache[0]["k"].shape[2])


def _trim(cache, n):
    return [{k: (v[:, :, :n] if isinstance(v, torch.Tensor) else v) for k, v in layer.items()} for layer in cache]


def _run_ids(model, ids, cache):
    dev = model.embed_tokens.weight.device
    with torch.inference_mode():
        return model._run(model.embed_tokens(torch.tensor([ids], device=dev)), cache, need_logits=True)


def spec_decode_greedy(target, draft, prompt_ids, max_new_tokens, *, k=4, eos_id=None,
                       target_kv="base_bf16", draft_kv="base_bf16", trim=None):
    """spec_dec.py:189-263: propose k draft tokens, verify them in one target block, accept the
    matching prefix, on a mismatch trim both caches and step the replacement token."""
    fmt = {"base_bf16": "fp16", "v_fp8": "v_fp8"}
    trim = trim or _trim
    target.set_kv_format(fmt[target_kv])
    draft.set_kv_format(fmt[draft_kv])
    ids = [int(t) for t in prompt_ids[0]]
    with attention_phase("prefill"):
        tgt_lg, tgt_cache = _run_ids(target, ids, None)
        drf_lg, drf_cache = _run_ids(draft, ids, None)
    saved_next, drf_lg = tgt_lg[:, -1:], drf_lg[:, -1:]
    gen: list = []
    st = dict(rounds=0, proposed=0, accepted=0, mismatch_rounds=0, all_accept_rounds=0)
    while len(gen) < max_new_tokens:
        k_eff = min(k, max_new_tokens - len(gen))
        pre = _cache_length(tgt_cache)
        cands, lg = [], drf_lg
        with attention_phase("propose"):
            for _ in range(k_eff):
                t = int(lg.reshape(-1, lg.shape[-1])[-1].argmax())
                cands.append(t)
                lg, drf_cache = _run_ids(draft, [t], drf_cache)
                if t == eos_id:
                    break
        prop_lg, kp = lg, len(cands)
        with attention_phase("verify"):
            blk_lg, tgt_blk = _run_ids(target, cands, tgt_cache)
        rows = blk_lg[0, -kp:]
        g = [int(x.argmax()) for x in [saved_next] + [rows[j] for j in range(kp - 1)]]
        m = 0
        while m < kp and g[m] == cands[m]:
            m += 1
        if m < kp:
            r = g[m]
            emitted = cands[:m] + [r]
            with attention_phase("repair"):
                lg_t, tgt_cache = _run_ids(target, [r], trim(tgt_blk, pre + m))
                saved_next = lg_t[:, -1:]
                drf_lg, drf_cache = _run_ids(draft, [r], trim(drf_cache, pre + m))
                drf_lg = drf_lg[:, -1:]
            st["mismatch_rounds"] += 1
        else:
            emitted = list(cands)
            tgt_cache = tgt_blk
            drf_cache = trim(drf_cache, pre + kp)
            saved_next, drf_lg = rows[kp - 1], prop_lg
            st["all_accept_rounds"] += 1
        gen += emitted
        st["accepted"] += m
        st["proposed"] += kp
        st["rounds"] += 1
        if emitted and emitted[-1] == eos_id:
            break
    return {"ids": ids + gen, "gen": gen, "stats": st, "target_cache": tgt_cache}


def tiny_model(seed: int, *, vocab=512, hidden=256, heads=12, kv_heads=2, head_dim=128, inter=512, layers=2,
               device="cpu", dtype=torch.bfloat16) -> QwenLM:
    """Random-init model with the target's GQA geometry (12 query heads over 2 KV heads).

    Embeddings are drawn small (std 0.05) so the layers, not the token's own embedding,
    dominate the residual stream; with the tied LM head (logits = x @ E^T) a random model
    whose residual is mostly its input embedding just repeats its last token.
    """
    torch.manual_seed(seed)
    m = QwenLM(vocab, hidden, heads, kv_heads, head_dim, inter, layers)
    with torch.no_grad():
        m.embed_tokens.weight.mul_(0.05)
        for p in m.parameters():
            if p.dim() == 2 and p is not m.embed_tokens.weight:
                nn.init.normal_(p, std=1.0 / math.sqrt(p.shape[1]))
    return m.to(device=device, dtype=dtype).eval()
