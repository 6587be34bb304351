"""Cache API contract (specdec/engine/spec_cache.py:4-46, docs/design_g4_cache_api.md:13-51).

Restates the reference's own self-test (spec_cache.py:49-65) and the B4 contract cases
(specdec/engine/g4_b4_cache_tests.py:89-130, 140-178) on CPU dict caches, and runs the
same cases on paged v_fp8 layer dicts (zero-storage shape carriers + a pool handle).
"""
from __future__ import annotations

import pytest
import torch

from specdec_amd.engine import spec_cache as sc
from specdec_amd.engine.paged_cache import BlockAllocator


def _dict_cache(layers=2, t=8, fp8=False):
    out = []
    for _ in range(layers):
        layer = {"k": torch.zeros(1, 2, t, 4), "v": torch.zeros(1, 2, t, 4)}
        if fp8:
            layer = {"fmt": "v_fp8", "k": torch.zeros(1, 2, t, 4, dtype=torch.bfloat16),
                     "v": torch.zeros(1, 2, t, 4, dtype=torch.float8_e4m3fn), "v_scale": torch.ones(1, 2, t, 1)}
        out.append(layer)
    return out


class _FakePages:
    def __init__(self, n):
        self.n = n

    def reserved_tokens(self):
        return self.n


def _carrier(shape, dtype):
    return torch.empty((), dtype=dtype).expand(*shape)


def _paged_cache(layers=2, t=8, reserved=16):
    pages = _FakePages(reserved)
    return [{"fmt": "v_fp8", "k": _carrier((1, 2, t, 4), torch.bfloat16),
             "v": _carrier((1, 2, t, 4), torch.float8_e4m3fn), "v_scale": _carrier((1, 2, t, 1), torch.float32),
             "pages": pages} for _ in range(layers)]


def test_reference_selftest_cases():
    fake = _dict_cache()
    assert sc.cache_length(fake) == 8 and sc.cache_length(None) == 0
    assert sc.trim_cache(None, 0) is None
    t = sc.trim_cache(fake, 3)
    sc.check_consistent(t)
    assert sc.cache_length(t) == 3 and fake[0]["k"].shape[2] == 8
    for bad in (-1, 9):
        with pytest.raises(ValueError):
            sc.trim_cache(fake, bad)
    badc = [{"k": torch.zeros(1, 2, 8, 4), "v": torch.zeros(1, 2, 7, 4)}]
    with pytest.raises(RuntimeError):
        sc.check_consistent(badc)


@pytest.mark.parametrize("make", [lambda: _dict_cache(fp8=True), _paged_cache])
def test_b4_contract(make):
    cache = make()
    L0 = sc.cache_length(cache)
    sc.check_consistent(cache)
    t1 = sc.trim_cache(cache, L0 - 1)
    t0 = sc.trim_cache(cache, 1)
    sc.check_consistent(t1)
    sc.check_consistent(t0)
    assert sc.cache_length(t1) == L0 - 1 and sc.cache_length(t0) == 1
    assert all(l["v_scale"].shape[2] == l["v"].shape[2] for l in t0)       # scale stays in sync
    assert all(l["fmt"] == "v_fp8" for l in t0)                           # fmt kept
    raises = 0
    for bad in (L0 + 5, -1, 0):
        try:
            sc.trim_cache(cache, bad)
        except ValueError:
            raises += 1
    assert raises == 3
    with pytest.raises(ValueError):
        sc.trim_cache(cache, True)                                        # bool is not an int here
    with pytest.raises(ValueError):
        sc.trim_cache(cache, 2.0)
    assert sc.cache_length(sc.trim_cache(cache, L0)) == L0                # idempotent
    assert sc.cache_length(cache) == L0                                   # input untouched
    assert t0 is not cache and t0[0] is not cache[0]
    for m in range(5):                                                    # mismatch m = 0..4
        r = sc.trim_cache(cache, 3 + m)
        sc.check_consistent(r)
        assert sc.cache_length(r) == 3 + m


def test_bad_cache_detection():
    cache = _dict_cache(layers=4, fp8=True)
    cache[3]["v"] = cache[3]["v"][:, :, :-1]
    with pytest.raises(RuntimeError):
        sc.check_consistent(cache)
    cache = _dict_cache(layers=3)
    cache[1] = {k: v[:, :, :5] for k, v in cache[1].items()}
    with pytest.raises(RuntimeError, match="cross-layer"):
        sc.check_consistent(cache)


def test_paged_reservation_is_checked():
    cache = _paged_cache(t=20, reserved=16)
    with pytest.raises(RuntimeError, match="reserved"):
        sc.check_consistent(cache)
    sc.check_consistent(sc.trim_cache(cache, 16))


def test_carriers_have_no_storage_and_trim_as_views():
    cache = _paged_cache(t=8192)
    k = cache[0]["k"]
    assert k.untyped_storage().nbytes() <= 4 and k.shape == (1, 2, 8192, 4)
    t = sc.trim_cache(cache, 100)
    assert t[0]["pages"] is cache[0]["pages"]


def test_block_allocator_seeded_fragmentation():
    a = BlockAllocator(64)
    assert a.alloc(4) == [0, 1, 2, 3]
    b = BlockAllocator(64, seed=7)
    got = b.alloc(8)
    assert got != sorted(got) and len(set(got)) == 8
    c = BlockAllocator(64, seed=7)
    assert c.alloc(8) == got                       # seeded: reproducible
    b.release(got)
    assert len(b.free) == 64
    with pytest.raises(RuntimeError, match="exhausted"):
        b.alloc(65)
    b.grow(80)
    assert len(b.alloc(70)) == 70


def test_varlen_tile_starts_cover_rows_and_follow_blocks():
    """The prefill tile table covers every packed row exactly once, never crosses a page block,
    and makes every whole page block one tile (so the kernel takes its 16-byte stores)."""
    import random
    from specdec_amd.kernels import ops
    rng = random.Random(11)
    for _ in range(200):
        nseq = rng.randint(1, 6)
        lengths = [rng.choice([0, 1, 5, 15, 16, 17, 31, 32, 33, rng.randint(0, 200)]) for _ in range(nseq)]
        starts = [rng.choice([0, 0, 3, 15, 16, rng.randint(0, 100)]) for _ in range(nseq)]
        t = ops.varlen_tile_starts(lengths, starts)
        assert t[-1] == sum(lengths) and t == sorted(t)
        assert all(0 < b - a <= 16 for a, b in zip(t, t[1:]))
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + n)
        tiles = set(zip(t, t[1:]))
        for b, (n, p0) in enumerate(zip(lengths, starts)):
            for a_, e in tiles:
                if cu[b] <= a_ < cu[b + 1]:
                    assert e <= cu[b + 1]                                 # no tile spans two sequences
                    first, last = p0 + a_ - cu[b], p0 + e - 1 - cu[b]
                    assert first // 16 == last // 16                      # one page block per tile
            for blk in range((p0 + 15) // 16, (p0 + n) // 16):            # whole blocks inside the run
                a_ = cu[b] + 16 * blk - p0
                assert (a_, a_ + 16) in tiles
    with pytest.raises(ValueError):
        ops.varlen_tile_starts([-1])
