"""Writes the golden fixtures under tests/golden/ from the CPU oracle (torch-CPU restatement).

    python tests/golden/make_golden.py

The reference repository commits no tensors for this path (its FP8 checks are invariant
tests, specdec/engine/fp8_vonly_v1_roundtrip.py, fp8_kv_v1_roundtrip.py), so the fixtures
are the oracle's outputs on seeded inputs, frozen so that a later change to the oracle or
to torch's CPU kernels is noticed.  Inputs that are cheap to regenerate (config 0) are
stored as a sha256 of their bytes; small cases store inputs in full.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "specdec-context-scaling_amd"))

from oracle import attention as oatt  # noqa: E402
from oracle import quant as oq  # noqa: E402
from specdec_amd import workloads as wl  # noqa: E402

OUT = Path(__file__).resolve().parent


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def quant_cases():
    """Edge-heavy small V rows for both head dims and both scale modes."""
    g = wl.gen(11)
    out = {}
    for d in (128, 64):
        n, kv = 48, 2
        v = torch.randn((n, kv, d), generator=g)
        v[3] = 0.0                                   # all-zero rows -> scale 1, payload 0
        v[4, 0] = -0.0                               # negative zeros keep their sign bit
        v[5] *= 1e-3                                 # small rows
        v[6, 1, :] = torch.randn(d, generator=g) * 1e-30   # codes in the E4M3 subnormal range
        v[7, :, 0] *= 20.0                           # outlier channel
        v[8, 0] = torch.linspace(-3, 3, d)           # exact max ties
        v[9, 1, 5] = 1e4                             # one huge element, rest -> subnormals/zeros
        v[10, 0, :] = 2.0 ** -130                    # BF16 subnormal inputs
        vb = v.to(torch.bfloat16)
        for mode in ("div", "rcp"):
            q, s = oq.quantize_kv_fp8(vb, d, mode)
            out[f"d{d}_{mode}_q"] = q.view(torch.uint8).numpy()
            out[f"d{d}_{mode}_s"] = s.squeeze(-1).numpy()
        out[f"d{d}_v"] = bits16(vb)
    np.savez_compressed(OUT / "quant_edge.npz", **out)


def attn_cases():
    out = {}
    # config 0: one layer, T = 2048, S = 1; inputs regenerated from seed 0 in the tests
    q, k, v = wl.config0(seed=0)
    out["cfg0_input_sha256"] = np.frombuffer(sha(bits16(q), bits16(k), bits16(v)).encode(), dtype=np.uint8)
    qv, vs = oq.quantize_kv_fp8(v, 128)
    vhat = oq.dequantize_kv_fp8(qv, vs, torch.bfloat16)
    o = oatt.eager_attention(q, k, vhat)
    out["cfg0_out"] = bits16(o)
    out["cfg0_vq_sha256"] = np.frombuffer(sha(qv.view(torch.uint8).numpy(), vs.numpy()).encode(), dtype=np.uint8)
    # small verify case (S = 5) and draft shape (D = 64, G = 7), inputs stored in full
    g = wl.gen(21)
    for name, (h, kvh, d, t, s) in {"verify": (12, 2, 128, 77, 5), "draft": (14, 2, 64, 50, 1)}.items():
        qq = wl.randn_bf16((1, h, s, d), g)
        kk = wl.randn_bf16((1, kvh, t, d), g)
        vv = wl.randn_bf16((1, kvh, t, d), g)
        pq, ps = oq.quantize_kv_fp8(vv, d)
        o = oatt.eager_attention(qq, kk, oq.dequantize_kv_fp8(pq, ps, torch.bfloat16))
        out[f"{name}_q"], out[f"{name}_k"], out[f"{name}_v"] = bits16(qq), bits16(kk), bits16(vv)
        out[f"{name}_out"] = bits16(o)
    np.savez_compressed(OUT / "attn_eager.npz", **out)


if __name__ == "__main__":
    torch.set_num_threads(8)
    quant_cases()
    attn_cases()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
