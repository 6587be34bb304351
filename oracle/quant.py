"""V-only FP8 quantize / dequantize, restated in torch-CPU (TEST INFRASTRUCTURE ONLY).

Follows specdec/engine/model_self.py:300-320 (``E4M3_MAX``, ``GROUP_V``,
``quantize_kv_fp8``, ``dequantize_kv_fp8``): per group of ``group_size`` trailing
elements, ``m = max|x|`` in fp32, ``s = m / 448`` with ``s == 0 -> 1``, payload
``(x / s)`` cast to ``float8_e4m3fn``; dequant is ``fp32(q) * s`` rounded once to the
working dtype.  The v_fp8 format uses ``group_size = head_dim`` (one scale per token and
KV head, model_self.py:690,703).

``scale_mode`` selects how ``m / 448`` is evaluated, because torch itself evaluates
``tensor / python_scalar`` differently by device:

* ``"div"`` -- IEEE division, what torch does on the CPU (the golden fixtures' mode);
* ``"rcp"`` -- ``m * RN_f32(1/448)``, what torch's CUDA/ROCm kernels do for a scalar divisor
  (measured on the MI355X box: 100% of 4M random scales).

``x / s`` is a tensor/tensor division and is IEEE on both devices.

Pinned by: the from-spec codec (oracle.fp8) exhaustively against torch's cast; the
reference's own invariant checks restated as tests (all-zero row -> payload 0 and scale
1.0, fp8_vonly_v1_roundtrip.py:91-94 / fp8_kv_v1_roundtrip.py:50-54; per-row max maps to
exactly +-448, fp8_vonly_v1_roundtrip.py:99-102; max|q| <= 448 and finite,
fp8_kv_v1_roundtrip.py:41-47; round trip error <= max/16, :77-93; determinism); and an
independent numpy/C re-derivation (numpy division + C encoder) that must agree bitwise.
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0          # model_self.py:300
GROUP_V = 128             # model_self.py:302 (v_fp8 on the 1.5B target: one group per head)

_RCP_448 = torch.tensor(1.0 / E4M3_MAX, dtype=torch.float32)


def quantize_kv_fp8(x: torch.Tensor, group_size: int, scale_mode: str = "div"):
    """model_self.py:304-314.  Returns (payload float8_e4m3fn shaped like x, scale fp32 (..., g))."""
    d = x.shape[-1]
    if d % group_size:
        raise ValueError(f"head_dim {d} % group_size {group_size} != 0")
    groups = d // group_size
    xf = x.to(torch.float32).reshape(*x.shape[:-1], groups, group_size)
    amax = xf.abs().amax(dim=-1, keepdim=True)
    if scale_mode == "div":
        scale = amax / E4M3_MAX
    elif scale_mode == "rcp":
        scale = amax * _RCP_448
    else:
        raise ValueError(f"unknown scale_mode {scale_mode!r}")
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    payload = (xf / scale).to(torch.float8_e4m3fn).reshape(x.shape)
    return payload, scale.squeeze(-1)


def dequantize_kv_fp8(q: torch.Tensor, scale: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """model_self.py:316-320: fp32(q) * scale (one fp32 rounding), then one rounding to dtype."""
    groups = scale.shape[-1]
    qf = q.to(torch.float32).reshape(*q.shape[:-1], groups, q.shape[-1] // groups)
    return (qf * scale.unsqueeze(-1)).reshape(q.shape).to(dtype)


def quantize_numpy(x_bf16_bits: np.ndarray, scale_mode: str = "div"):
    """Independent re-derivation for one group per row: numpy fp32 arithmetic + the C codec.

    ``x_bf16_bits``: uint16 array (..., D) of bf16 bit patterns.  Returns (uint8 payload, f32
    scale (...,)).  Used only to cross-check ``quantize_kv_fp8`` (different code, same maths).
    """
    from . import fp8

    xf = (x_bf16_bits.astype(np.uint32) << 16).view(np.float32)
    amax = np.abs(xf).max(axis=-1)
    if scale_mode == "div":
        s = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    else:
        s = (amax * np.float32(1.0 / E4M3_MAX)).astype(np.float32)
    s = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        y = (xf / s[..., None]).astype(np.float32)
    return fp8.encode(y), s
