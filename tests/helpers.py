"""Test helpers: build paged caches from CPU data with the oracle, compare with tolerances."""
from __future__ import annotations

import numpy as np
import torch

from oracle import attention as oatt
from oracle import paged as opaged
from oracle import quant as oq

ATOL = 2e-2      # BASELINE: attention max-abs vs the eager BF16 path
REL_L2 = 1e-3    # BASELINE: attention rel-L2 vs the eager BF16 path


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def quantize_rows(v: torch.Tensor, mode: str = "div"):
    """v BF16 (..., D) -> (uint8 payload (..., D), f32 scale (...)) via the oracle."""
    q, s = oq.quantize_kv_fp8(v, v.shape[-1], mode)
    return q.view(torch.uint8).numpy(), s.squeeze(-1).numpy()


def build_pages(k_seqs, v_seqs, num_blocks: int, block_rows, mode: str = "div"):
    """Oracle-built pages for sequences: k_seqs/v_seqs lists of BF16 (KV, T_b, D) tensors.

    block_rows[b] lists the physical blocks of sequence b.  Returns numpy (k_pages,
    v_pages, v_scales) in the library's layout.
    """
    kv, d = k_seqs[0].shape[0], k_seqs[0].shape[2]
    kp, vp, vs = opaged.alloc(num_blocks, kv, d)
    for b, (k, v) in enumerate(zip(k_seqs, v_seqs)):
        t = k.shape[1]
        q, s = quantize_rows(v.transpose(0, 1).contiguous(), mode)       # (T, KV, D), (T, KV)
        slots = opaged.slots_for(block_rows[b], 0, t)
        opaged.write(kp, vp, vs, bits16(k.transpose(0, 1)), q, s, slots)
    return kp, vp, vs


def to_dev(a: np.ndarray, dev, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def eager_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, d: int, mode: str = "div") -> torch.Tensor:
    """Oracle eager attention with V quantized/dequantized as the reference does (CPU)."""
    pq, ps = oq.quantize_kv_fp8(v, d, mode)
    return oatt.eager_attention(q, k, oq.dequantize_kv_fp8(pq, ps, torch.bfloat16))


def assert_close(got: torch.Tensor, want: torch.Tensor, what: str = "") -> dict:
    g = got.detach().float().cpu().double().numpy()
    w = want.detach().float().cpu().double().numpy()
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    ma = oatt.max_abs(g, w)
    rl = oatt.rel_l2(g, w)
    assert ma <= ATOL and rl <= REL_L2, f"{what}: max_abs={ma:.3e} rel_l2={rl:.3e}"
    return {"max_abs": ma, "rel_l2": rl}
