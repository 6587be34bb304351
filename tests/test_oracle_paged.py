"""Pins oracle.paged: write by slot mapping then gather returns the contiguous cache bit for
bit, for scattered blocks, partial last blocks and skipped (negative) slots."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import paged as opaged


@pytest.mark.parametrize("d", [128, 64])
def test_write_gather_round_trip(d):
    rng = np.random.default_rng(3)
    kv, nb = 2, 40
    lens = [1, 16, 17, 100, 250]
    kp, vp, vs = opaged.alloc(nb, kv, d)
    order = rng.permutation(nb)
    rows, at = [], 0
    want = []
    for t in lens:
        n = -(-t // 16)
        rows.append(order[at:at + n])
        at += n
        k = rng.integers(0, 1 << 16, (t, kv, d), dtype=np.uint16)
        v = rng.integers(0, 256, (t, kv, d), dtype=np.uint8)
        s = rng.random((t, kv), dtype=np.float32)
        slots = opaged.slots_for(rows[-1], 0, t).copy()
        opaged.write(kp, vp, vs, k, v, s, slots)
        want.append((k, v, s))
    for row, t, (k, v, s) in zip(rows, lens, want):
        gk, gv, gs = opaged.gather(kp, vp, vs, row, t)
        assert np.array_equal(gk, k.transpose(1, 0, 2))
        assert np.array_equal(gv, v.transpose(1, 0, 2))
        assert np.array_equal(gs, s.T)


def test_layout_addresses_match_the_abi_formula():
    """K token t, dim d of a page at ((d/8)*16 + t)*8 + d%8; V at d*16 + t (include/sdv.h)."""
    kp, vp, vs = opaged.alloc(1, 1, 128)
    k = np.arange(16 * 128, dtype=np.uint16).reshape(16, 1, 128)
    v = (np.arange(16 * 128) % 251).astype(np.uint8).reshape(16, 1, 128)
    opaged.write(kp, vp, vs, k, v, np.ones((16, 1), np.float32), np.arange(16))
    flat_k, flat_v = kp[0, 0].ravel(), vp[0, 0].ravel()
    for t, dd in [(0, 0), (3, 7), (5, 8), (15, 127), (9, 64)]:
        assert flat_k[((dd // 8) * 16 + t) * 8 + dd % 8] == k[t, 0, dd]
        assert flat_v[dd * 16 + t] == v[t, 0, dd]


def test_skipped_slots_leave_pages_untouched():
    kp, vp, vs = opaged.alloc(2, 1, 64)
    opaged.write(kp, vp, vs, np.ones((3, 1, 64), np.uint16), np.ones((3, 1, 64), np.uint8),
                 np.ones((3, 1), np.float32), [-1, 17, -5])
    assert kp.sum() == 64 and vp.sum() == 64 and vs.sum() == 1
