"""Pins oracle.quant (restatement of specdec/engine/model_self.py:300-320).

Independent checks, none of which retypes the formula under test:
* a second derivation (numpy fp32 arithmetic + the from-spec C encoder) must agree bitwise;
* the reference's own invariants (fp8_vonly_v1_roundtrip.py:91-102, fp8_kv_v1_roundtrip.py:
  41-93): all-zero row -> payload 0 and scale 1; each nonzero row's max maps to exactly
  +-448; max|q| <= 448 and finite; round trip error <= max/16; determinism; scale shape;
* the golden fixture (frozen oracle output) still matches.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import quant as oq
from specdec_amd import workloads as wl


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("mode", ["div", "rcp"])
@pytest.mark.parametrize("d", [128, 64])
def test_second_derivation_agrees(mode, d):
    v, _, _ = wl.config1(seed=5, tokens=256, layers=4, head_dim=d)
    q, s = oq.quantize_kv_fp8(v, d, mode)
    q2, s2 = oq.quantize_numpy(_bits(v), mode)
    assert np.array_equal(q.view(torch.uint8).numpy(), q2)
    assert np.array_equal(s.squeeze(-1).numpy().view(np.uint32), s2.view(np.uint32))


def test_scale_modes_differ_where_expected():
    """m/448 and m*RN(1/448) are different functions (pins that 'rcp' is not silently 'div')."""
    m = torch.rand(1 << 16, generator=wl.gen(3)) * 8
    div = m / 448.0
    rcp = m * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    frac = float((div != rcp).float().mean())
    assert 0.3 < frac < 0.7


def test_reference_invariants_config1_shape():
    v, _, _ = wl.config1(seed=1)  # (28, 2048, 2, 128), outliers and zero rows
    q, s = oq.quantize_kv_fp8(v, 128)
    assert q.dtype == torch.float8_e4m3fn and q.shape == v.shape
    assert s.dtype == torch.float32 and tuple(s.shape) == tuple(v.shape[:-1]) + (1,)
    qf = q.float()
    assert torch.isfinite(qf).all() and qf.abs().max() <= 448.0
    zero_rows = (v.float().abs().amax(-1) == 0)
    assert zero_rows.any()
    assert (s.squeeze(-1)[zero_rows] == 1.0).all() and (qf[zero_rows] == 0).all()
    rowmax = qf.abs().amax(-1)
    assert (rowmax[~zero_rows] == 448.0).all()
    hat = oq.dequantize_kv_fp8(q, s, torch.float32)
    err = (hat - v.float()).abs().amax(-1)
    assert (err <= v.float().abs().amax(-1) / 16).all()
    q2, s2 = oq.quantize_kv_fp8(v, 128)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)


def test_dequant_brute_force_all_codes():
    """fp32(code) * scale rounded once to BF16, for all 256 codes and assorted scales."""
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).reshape(1, 1, 1, 256)
    for sc in (1.0, 1 / 448, 3.7e-3, 0.0123, 7.0):
        s = torch.full((1, 1, 1, 2), sc, dtype=torch.float32)  # 2 groups of 128
        got = oq.dequantize_kv_fp8(codes, s, torch.bfloat16).float().numpy().ravel()
        dec = codes.view(torch.uint8).numpy().ravel()
        from oracle import fp8
        want = (fp8.decode(dec).astype(np.float64) * np.float32(sc)).astype(np.float32)
        want = torch.from_numpy(want).to(torch.bfloat16).float().numpy()
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan], want[~nan])


def test_golden_edge_fixture():
    z = np.load(GOLDEN / "quant_edge.npz")
    for d in (128, 64):
        v = torch.from_numpy(z[f"d{d}_v"].view(np.int16)).view(torch.bfloat16)
        for mode in ("div", "rcp"):
            q, s = oq.quantize_kv_fp8(v, d, mode)
            assert np.array_equal(q.view(torch.uint8).numpy(), z[f"d{d}_{mode}_q"]), (d, mode)
            assert np.array_equal(s.squeeze(-1).numpy().view(np.uint32), z[f"d{d}_{mode}_s"].view(np.uint32))
    # the edge rows exercise what they claim to
    q = z["d128_div_q"]
    assert (q[3] == 0).all() and (z["d128_div_s"][3] == 1.0).all()
    assert ((q[4, 0] == 0x80) | (q[4, 0] == 0)).all() and (q[4, 0] == 0x80).any()
    sub = ((q[9, 1] & 0x78) == 0) & ((q[9, 1] & 0x07) != 0)
    assert sub.any()                                 # E4M3 subnormal codes next to the 1e4 outlier
    assert (q[10, 0] & 0x7F == 0x7E).all()           # BF16-subnormal row: fp32 denormal scale, max -> 448


def test_planted_mistake_in_scale_is_caught():
    """Dropping the zero guard (s == 0 -> 1) must break the all-zero-row invariant."""
    v = torch.zeros((1, 2, 4, 128), dtype=torch.bfloat16)
    xf = v.float()
    s_bad = xf.abs().amax(-1, keepdim=True) / 448.0
    q_bad = (xf / s_bad).to(torch.float8_e4m3fn)
    assert torch.isnan(q_bad.float()).all()
    q, s = oq.quantize_kv_fp8(v, 128)
    assert (q.float() == 0).all() and (s == 1).all()
