"""Pins the oracle's from-spec E4M3FN codec (oracle/fp8_e4m3.c).

The reference reaches E4M3FN through torch's ``.to(torch.float8_e4m3fn)``
(specdec/engine/model_self.py:312) and back through ``.to(torch.float32)`` (:318).  The
codec is checked against torch's CPU cast over EVERY fp32 bit pattern, and against the OCP
spec's fixed points.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8


def test_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = fp8.decode(codes)
    th = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(th)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), th[~nan].view(np.uint32))  # -0.0 included


def test_spec_fixed_points():
    enc = lambda v: int(fp8.encode(np.array([v], dtype=np.float32))[0])  # noqa: E731
    assert enc(448.0) == 0x7E and enc(-448.0) == 0xFE
    assert enc(2.0 ** -9) == 0x01 and enc(2.0 ** -6) == 0x08
    assert enc(1.0) == 0x38 and enc(-0.0) == 0x80 and enc(0.0) == 0x00
    assert enc(464.0) == 0x7E            # tie between 448 (even mantissa) and 480 -> 448
    assert enc(np.nextafter(np.float32(464.0), np.float32(500.0))) == 0x7F   # rounds past 448 -> NaN
    assert enc(float("inf")) == 0x7F and enc(float("-inf")) == 0xFF and enc(float("nan")) == 0x7F
    assert enc(2.0 ** -10) == 0x00        # half of the smallest subnormal: tie -> even (0)
    assert enc(3 * 2.0 ** -10) == 0x02    # 1.5 subnormal steps: tie -> even (2)
    assert enc(2.0 ** -9 * 7.5) == 0x08   # 7.5 steps: tie -> 8 = 2^-6 normal
    assert enc(1.0 + 2.0 ** -4) == 0x38   # halfway 1.0 / 1.125: ties to even mantissa 0
    assert enc(1.0 + 3 * 2.0 ** -4) == 0x3A


@pytest.mark.parametrize("half", ["positive", "negative"])
def test_encode_exhaustive_against_torch(half):
    """Every fp32 bit pattern of one sign (2^31 values) encodes exactly as torch's cast."""
    chunk = 1 << 24
    base = 0 if half == "positive" else 1 << 31
    mismatches = 0
    first = None
    for lo in range(base, base + (1 << 31), chunk):
        ours = fp8.encode_range(lo, chunk)
        bits = np.arange(lo, lo + chunk, dtype=np.uint64).astype(np.uint32)
        th = torch.from_numpy(bits.view(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        bad = np.nonzero(ours != th)[0]
        if bad.size:
            mismatches += bad.size
            first = first or (hex(lo + int(bad[0])), int(ours[bad[0]]), int(th[bad[0]]))
    assert mismatches == 0, f"{mismatches} mismatches, first {first}"


def test_planted_encoder_mistake_is_caught():
    """A round-half-up encoder (a plausible slip) must differ from torch on some input."""
    x = np.float32(1.0 + 2.0 ** -4)  # exact tie
    th = int(torch.tensor([x]).to(torch.float8_e4m3fn).view(torch.uint8)[0])
    half_up = 0x39
    assert th != half_up and int(fp8.encode(np.array([x]))[0]) == th
