"""Pack mechanics and engine bookkeeping on the CPU (no kernel launches).

Mirrors the reference's pack contract (specdec/kernels/patch.py:139-173: unknown pack ->
ValueError, install/restore swap SelfAttention.forward, current_pack) and the attention
accounting (specdec/engine/model_self.py:398-536), with the paged layer dicts run through
the reference cache API (spec_cache.py:4-46).
"""
from __future__ import annotations

import pytest
import torch

from oracle import engine as oeng
from specdec_amd import SdvError
from specdec_amd.engine import accounting as acc
from specdec_amd.engine import spec_cache as sc
from specdec_amd.engine.paged_cache import LayerPages, PagedKVCache, shape_carrier
from specdec_amd.kernels import patch


@pytest.fixture
def engine():
    orig = oeng.SelfAttention.forward
    yield oeng
    patch.restore()
    assert oeng.SelfAttention.forward is orig


def test_install_restore_and_unknown(engine):
    orig = engine.SelfAttention.forward
    assert patch.install("fp8v", engine) == "fp8v"
    assert patch.current_pack() == "fp8v"
    assert engine.SelfAttention.forward is patch._fp8v_forward
    assert patch.install("torch", engine) == "torch"
    assert engine.SelfAttention.forward is orig
    patch.install("fp8v", engine)
    patch.restore()
    assert patch.current_pack() == "torch" and engine.SelfAttention.forward is orig
    with pytest.raises(ValueError):
        patch.install("all", engine)
    with pytest.raises(ValueError):
        patch.install("fp8v", engine, scale_mode="nearest")
    assert engine.SelfAttention.forward is orig


def test_non_vfp8_formats_fall_through(engine):
    """The fp16 (BF16 K/V) format runs the engine's own forward under the pack, bit for bit."""
    model = engine.tiny_model(3, layers=1, dtype=torch.float32)
    ids = torch.tensor([[5, 9, 1, 7, 3]])
    want, _ = model._run(model.embed_tokens(ids), None)
    patch.install("fp8v", engine)
    got, cache = model._run(model.embed_tokens(ids), None)
    assert torch.equal(got, want)
    assert "pages" not in cache[0]


def test_vfp8_needs_device_and_bf16(engine):
    model = engine.tiny_model(3, layers=1, dtype=torch.float32)
    patch.enable_fp8v(model)
    patch.install("fp8v", engine)
    with pytest.raises(SdvError):
        model._run(model.embed_tokens(torch.tensor([[1, 2]])), None)


def test_paged_layer_dicts_follow_the_cache_api():
    """Carriers give length / trim / consistency exactly as contiguous tensors would."""
    pool = PagedKVCache(2, 128, batch=1, capacity_tokens=64, device="cpu")
    pool.reserve(0, 37)
    pool.set_length(0, 37)
    cache = [LayerPages(pool).layer_dict(37) for _ in range(3)]
    assert sc.cache_length(cache) == 37
    sc.check_consistent(cache)
    assert cache[0]["k"].shape == (1, 2, 37, 128) and cache[0]["v_scale"].shape == (1, 2, 37, 1)
    assert cache[0]["v"].dtype == torch.float8_e4m3fn
    assert cache[0]["k"].untyped_storage().nbytes() <= 8          # no per-token storage
    t = sc.trim_cache(cache, 30)
    assert sc.cache_length(t) == 30 and sc.cache_length(cache) == 37
    assert t[1]["pages"] is cache[1]["pages"] and t[0]["fmt"] == "v_fp8"
    sc.check_consistent(t)
    bad = [dict(cache[0]), LayerPages(pool).layer_dict(36)]
    with pytest.raises(RuntimeError):
        sc.check_consistent(bad)
    over = [LayerPages(pool).layer_dict(49)]                      # 48 slots reserved
    with pytest.raises(RuntimeError):
        sc.check_consistent(over)
    for badn in (0, 38, True):
        with pytest.raises(ValueError):
            sc.trim_cache(cache, badn)
    assert shape_carrier((4, 5), torch.float32, "cpu").sum() == 0


def test_accounting_mirror():
    acc.reset_attention_stats()
    acc.set_attention_strategy("eager")
    assert acc.decide_attention_path("prefill", 64) == ("eager", "strategy=eager")
    acc.set_attention_strategy("cudnn_prefill")
    try:
        assert acc.decide_attention_path("prefill", 64) == ("fused", None)
        path, why = acc.decide_attention_path("prefill", 1)
        assert path == "eager" and "PREFILL_FUSED_MIN_S" in why
        path, why = acc.decide_attention_path("verify", 5)
        assert path == "eager" and why.startswith("phase=")
        with acc.attention_phase("prefill"):
            assert acc.current_attention_phase() == "prefill"
            with acc.attention_phase("verify"):
                assert acc.current_attention_phase() == "verify"
            assert acc.current_attention_phase() == "prefill"
        assert acc.current_attention_phase() == "other"
        acc.record_attention_call("fused", "prefill", 64, 64, None, 12, 2, 128)
        acc.record_attention_call("eager", "prefill", 1, 65, "s=1 < PREFILL_FUSED_MIN_S=2 (x)", 12, 2, 128)
        acc.record_attention_call("eager", "verify", 5, 70, "phase='verify' != 'prefill'", 12, 2, 128)
        st = acc.attention_stats()
        assert st["calls"] == {"eager": 2, "fused": 1}
        assert st["by_phase"] == {"prefill": 2, "verify": 1}
        assert st["eager_reason_kinds"] == {"short_block_seq_len_lt_min": 1, "phase_not_prefill": 1}
        assert st["s_max_by_phase"] == {"prefill": 64, "verify": 5}
        assert st["phases_seen"] == ["prefill", "verify"]
        with pytest.raises(ValueError):
            acc.set_attention_strategy("flash")
    finally:
        acc.set_attention_strategy("eager")
        acc.reset_attention_stats()
