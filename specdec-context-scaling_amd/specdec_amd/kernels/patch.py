"""Engine packs: install the FP8-V paged path on a live engine (mirror of specdec/kernels/patch.py).

The reference swaps methods of its engine module ``specdec.engine.model_self`` in place:
``install(pack)`` captures the originals once (patch.py:26-33), restores them, then
assigns the pack's replacements (patch.py:139-157, ``SelfAttention.forward = _attn_forward``
at :155); ``restore()`` puts the originals back (:160-169); ``current_pack()`` names the
active pack (:172-173).  Unknown packs raise ValueError.

Packs here:

* ``"torch"`` -- the engine's own methods (nothing patched);
* ``"fp8v"``  -- ``SelfAttention.forward`` for the ``v_fp8`` cache format runs on libsdv:
  the projections and RoPE stay in torch as in the reference forward (model_self.py:
  668-685); the current K/V go through kernel 1 (quantize V to E4M3FN with the per-token,
  per-KV-head max-abs/448 scale, copy K, write both into page slots) and attention through
  kernels 2/3 over the pages (keys j <= T - s + i, the reference mask of :755-764), which
  replaces the dequantize + cat + kv_repeat + eager attention of :715-776 and the cat-based
  append of :778-800.  Appending first is exact: eager attends over dequant(quant(v_cur))
  for the current tokens (:703-704), which is what the kernel reads back.  Other cache
  formats ("fp16", "fp8") fall through to the engine's original forward.

The layer cache keeps the reference's dict contract ``{"fmt": "v_fp8", "k", "v", "v_scale"}``
(docs/design_g4_cache_api.md:7-11) with zero-storage shape carriers for the three tensors
and the page pool under ``"pages"``, so ``QwenLM._run`` (start_pos from ``cache[0]["k"].shape[2]``),
``spec_cache.cache_length / trim_cache / check_consistent`` and the SpecDec loop run
unchanged; a trim just shortens the carriers and the next append overwrites the rejected
slots.  Phase accounting goes through the engine's own ``decide_attention_path`` and
``_record_attention_call`` (as patch.py:104-106 does), or this package's mirror when the
engine has none.
"""
from __future__ import annotations

import importlib

import torch

from .._native import SdvError
from ..engine import accounting
from ..engine.paged_cache import LayerPages, PagedKVCache

_PACKS = ("torch", "fp8v")
_ORIG: dict = {}
_PACK = "torch"
_TARGET = None
_OPTS = {"scale_mode": "rcp", "capacity_tokens": 256, "seed": None}


def _default_module():
    return importlib.import_module("specdec.engine.model_self")


def install(pack: str, model_module=None, *, scale_mode: str = "rcp", capacity_tokens: int = 256,
            seed: int | None = None) -> str:
    """Activate a pack on `model_module` (default: the reference's specdec.engine.model_self).

    scale_mode: how max|v| / 448 is evaluated -- "rcp" (max * RN(1/448): what torch's device
    kernels compute, i.e. the reference engine running on a GPU) or "div" (IEEE division:
    torch on the CPU).  capacity_tokens: initial page capacity per layer (pools grow by
    doubling).  seed: shuffle the free block list (fragmented placement) when set.
    """
    global _PACK, _TARGET
    if pack not in _PACKS:
        raise ValueError(f"unknown pack {pack!r}; choose from {sorted(_PACKS)}")
    if scale_mode not in ("rcp", "div"):
        raise ValueError("scale_mode must be 'rcp' or 'div'")
    m = model_module if model_module is not None else (_TARGET or _default_module())
    if _TARGET is not None and m is not _TARGET:
        restore()
        _ORIG.clear()
    _TARGET = m
    if not _ORIG:
        _ORIG["attn"] = m.SelfAttention.forward
    restore()
    _OPTS.update(scale_mode=scale_mode, capacity_tokens=int(capacity_tokens), seed=seed)
    if pack == "fp8v":
        m.SelfAttention.forward = _fp8v_forward
    _PACK = pack
    return pack


def restore() -> None:
    global _PACK
    if _ORIG and _TARGET is not None:
        _TARGET.SelfAttention.forward = _ORIG["attn"]
    _PACK = "torch"


def current_pack() -> str:
    return _PACK


def enable_fp8v(model) -> None:
    """Put every attention layer of `model` on the v_fp8 cache format.

    The reference's set_kv_format("v_fp8") requires head_dim % 128 == 0 (one 128-wide group
    per head, model_self.py:889-890), which excludes the 0.5B draft (head_dim 64).  The paged
    path quantizes with one group per head for any head_dim in {64, 128}
    (quantize_kv_fp8(v, group_size=head_dim), model_self.py:304-314).
    """
    model.kv_format = "v_fp8"
    for layer in model.layers:
        layer.self_attn.kv_format = "v_fp8"


def reserve(cache_list, n_tokens: int, q_len: int | None = None) -> None:
    """Page blocks, device block tables and attention workspaces for n_tokens positions in
    every layer of an engine cache, so that steps up to that length can be recorded into a
    HIP graph: a recorded step then copies nothing from the host and allocates nothing (the
    reference's graph experiments record the draft chain and the verify block at a fixed
    history length, experiments/cuda_graph_local/draft_graph.py, verify_graph.py).  The
    workspaces are sized for q_len new tokens per step (default: the largest step each layer
    has run; PagedKVCache.reserve_all)."""
    for layer in cache_list:
        pages = layer.get("pages") if layer is not None else None
        if pages is None:
            continue
        pool = pages.pool
        pool.reserve_all(n_tokens, q_len=q_len)


def _accounting(m):
    if hasattr(m, "decide_attention_path") and hasattr(m, "_record_attention_call"):
        return m.decide_attention_path, m._record_attention_call, getattr(m, "_ATTENTION_PHASE", "other")
    return accounting.decide_attention_path, accounting.record_attention_call, accounting.current_attention_phase()


def _fp8v_forward(self, x, cos, sin, cache=None):
    m = _TARGET
    fmt = cache.get("fmt", self.kv_format) if cache is not None else self.kv_format
    if fmt != "v_fp8" or (cache is not None and "pages" not in cache):
        return _ORIG["attn"](self, x, cos, sin, cache)
    if x.device.type != "cuda":
        raise SdvError("the fp8v pack runs on a HIP device; move the model there or install('torch')")
    if x.dtype != torch.bfloat16:
        raise SdvError(f"the fp8v pack computes in bfloat16 (the model runs in {x.dtype})")
    b, s, _ = x.shape
    H, KV, D = self.heads, self.kv_heads, self.head_dim
    q = self.q_proj(x).view(b, s, H, D).transpose(1, 2)
    k = self.k_proj(x).view(b, s, KV, D).transpose(1, 2)
    v = self.v_proj(x).view(b, s, KV, D).transpose(1, 2)
    q = m.apply_rope(q, cos, sin)
    k = m.apply_rope(k, cos, sin)

    if cache is None:
        if torch.cuda.is_current_stream_capturing():
            raise SdvError("a prefill from an empty cache creates the page pool; run it before recording a graph")
        pool = PagedKVCache(KV, D, batch=b, capacity_tokens=max(_OPTS["capacity_tokens"], s), device=x.device,
                            seed=_OPTS["seed"], scale_mode=_OPTS["scale_mode"])
        pages = LayerPages(pool)
        t0 = 0
    else:
        pages = cache["pages"]
        pool = pages.pool
        t0 = int(cache["k"].shape[2])          # logical length (a trim may have shortened it)
        for i in range(b):
            pool.set_length(i, t0)
    T = t0 + s

    # the decision is recorded as the engine would record it; both paths run on libsdv
    decide, record, phase = _accounting(m)
    path, reason = decide(phase, s)
    record(path, phase, s, T, reason, H, KV, D)

    # append the s new tokens (quantized V, BF16 K) and attend over the context, one call
    out = pool.append_attend(0, q.transpose(1, 2).contiguous(), k.transpose(1, 2), v.transpose(1, 2),
                             starts=[t0] * b, q_token_major=True)   # (b, s, H, D)
    out = out.view(b, s, H * D)
    new = pages.layer_dict(T)
    if cache is None:
        cache = new
    else:
        cache.update(new)                      # _run advances the cache dict in place
    return self.o_proj(out), cache
