"""Attention-path decision and call accounting (mirror of specdec/engine/model_self.py:333-536).

The reference tags each forward with a phase (``prefill``, ``decode``, ``propose``,
``verify``, ``repair``, ``other``) through the ``attention_phase`` context manager, decides the
path with the pure function ``decide_attention_path(phase, s, strategy)`` -- only
``prefill`` blocks of at least ``PREFILL_FUSED_MIN_S`` rows may take the fused prefill path
under the ``cudnn_prefill`` strategy -- and records every call in module statistics
(``_record_attention_call``).  The FP8-V pack keeps that bookkeeping: when it patches a
reference engine module it calls that module's own functions; this module is the same
bookkeeping for engines that do not carry it.

Names, arguments, defaults and errors follow the reference; messages are in English.
"""
from __future__ import annotations

import contextlib
import copy

ATTENTION_STRATEGIES = ("eager", "cudnn_prefill")   # model_self.py:333
PREFILL_FUSED_MIN_S = 2                              # :334 (cuDNN SDPA has no seq_len == 1 kernel)
SHORT_BLOCK_POLICY = "eager_fallback"                # :335
FUSED_BACKEND_NAME = "CUDNN_ATTENTION"               # :336
PHASES = ("prefill", "decode", "propose", "verify", "repair", "other")
_MAX_FALLBACK_LOGGED = 32                            # :341

ATTENTION_STRATEGY = "eager"
_ATTENTION_PHASE = "other"
_ATTENTION_STATS: dict | None = None


def _fresh_stats() -> dict:
    return {"strategy": ATTENTION_STRATEGY, "requested_backend": FUSED_BACKEND_NAME,
            "calls": {"eager": 0, "fused": 0}, "by_phase": {}, "fused_by_phase": {}, "eager_by_phase": {},
            "s_max_by_phase": {}, "fused_s_max_by_phase": {}, "fallbacks": [], "fallback_count": 0,
            "eager_reason_kinds": {}, "phases_seen": [], "errors": []}


def _stats() -> dict:
    global _ATTENTION_STATS
    if _ATTENTION_STATS is None:
        _ATTENTION_STATS = _fresh_stats()
    return _ATTENTION_STATS


def set_attention_strategy(name: str) -> str:
    global ATTENTION_STRATEGY
    if name not in ATTENTION_STRATEGIES:
        raise ValueError(f"unknown attention strategy {name!r} (choose from {ATTENTION_STRATEGIES})")
    ATTENTION_STRATEGY = name
    _stats()["strategy"] = name
    return ATTENTION_STRATEGY


def attention_strategy() -> str:
    return ATTENTION_STRATEGY


@contextlib.contextmanager
def attention_phase(name: str):
    """Tag the enclosed forwards with a phase (model_self.py:413-429)."""
    global _ATTENTION_PHASE
    prev = _ATTENTION_PHASE
    _ATTENTION_PHASE = name
    st = _stats()
    if name not in st["phases_seen"]:
        st["phases_seen"].append(name)
    try:
        yield
    finally:
        _ATTENTION_PHASE = prev


def current_attention_phase() -> str:
    return _ATTENTION_PHASE


def reset_attention_stats() -> None:
    global _ATTENTION_STATS
    _ATTENTION_STATS = _fresh_stats()


def attention_stats() -> dict:
    st = copy.deepcopy(_stats())
    st["strategy"] = ATTENTION_STRATEGY
    return st


def decide_attention_path(phase: str, s: int, strategy: str | None = None) -> tuple[str, str | None]:
    """Pure decision (model_self.py:456-468): ("eager" | "fused", reason)."""
    strat = ATTENTION_STRATEGY if strategy is None else strategy
    if strat != "cudnn_prefill":
        return "eager", f"strategy={strat}"
    if phase != "prefill":
        return "eager", f"phase={phase!r} != 'prefill' (only prefill may fuse)"
    if s < PREFILL_FUSED_MIN_S:
        return "eager", f"s={s} < PREFILL_FUSED_MIN_S={PREFILL_FUSED_MIN_S} (no seq_len=1 fused kernel)"
    return "fused", None


def record_attention_call(path: str, phase: str, s: int, T: int, reason: str | None,
                          heads: int, kv_heads: int, head_dim: int) -> None:
    """Call accounting (model_self.py:507-536)."""
    st = _stats()
    st["calls"][path] += 1
    st["by_phase"][phase] = st["by_phase"].get(phase, 0) + 1
    key = "fused_by_phase" if path == "fused" else "eager_by_phase"
    st[key][phase] = st[key].get(phase, 0) + 1
    if s > st["s_max_by_phase"].get(phase, 0):
        st["s_max_by_phase"][phase] = s
    if path == "fused" and s > st["fused_s_max_by_phase"].get(phase, 0):
        st["fused_s_max_by_phase"][phase] = s
    if path == "eager" and ATTENTION_STRATEGY == "cudnn_prefill":
        st["fallback_count"] += 1
        kind = "other"
        if reason and "PREFILL_FUSED_MIN_S" in reason:
            kind = "short_block_seq_len_lt_min"
        elif reason and reason.startswith("phase="):
            kind = "phase_not_prefill"
        st["eager_reason_kinds"][kind] = st["eager_reason_kinds"].get(kind, 0) + 1
        if len(st["fallbacks"]) < _MAX_FALLBACK_LOGGED:
            st["fallbacks"].append(dict(phase=phase, s=s, T=T, reason=reason, kind=kind, heads=heads,
                                        kv_heads=kv_heads, head_dim=head_dim, policy=SHORT_BLOCK_POLICY))


# the reference's private name, so a pack can call either module the same way
_record_attention_call = record_attention_call
