"""Seeded synthetic inputs of the BASELINE configurations (no weights, no datasets).

Shapes (Qwen2.5): 1.5B target H=12, KV=2, D=128, 28 layers; 0.5B draft H=14, KV=2, D=64,
24 layers.  Every generator takes a ``torch.Generator`` seed and a device, so a CPU run
(oracle) and a GPU run (kernels) can be fed the same values by generating on the CPU and
copying, or large benchmark caches can be generated on the device directly.

* config 0 -- one layer, decode (S=1), B=1, T=2048: q, k, v ~ N(0,1) cast to BF16.
* config 1 -- quantize+append of a 2048-token prefill chunk into 28 layers x 2 KV heads x
              128 dims: V ~ N(0,1) BF16, 1% of the (KV head, dim) channels of each layer
              scaled x20 (seeded), 0.1% of (token, layer) rows all zero, slots from a seeded
              permutation of the 128 blocks.
* config 2 -- decode over a 28-layer T=8192 cache, 512 blocks per sequence placed by a
              seeded permutation.
* config 3 -- verify S=5 at T in {2048, 4096, 8192} (target) and 5 sequential S=1 draft
              decodes (0.5B shape).
* config 4 -- B=32 ragged T_b ~ U{2048..32768}, fragmented allocator, 1% outlier channels.
"""
from __future__ import annotations

import math

import torch

TARGET = dict(q_heads=12, kv_heads=2, head_dim=128, layers=28)
DRAFT = dict(q_heads=14, kv_heads=2, head_dim=64, layers=24)


def gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def randn_bf16(shape, g: torch.Generator, device="cpu") -> torch.Tensor:
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)


def config0(seed: int = 0, device="cpu"):
    """q (1,12,1,128), k/v (1,2,2048,128) BF16 (v before quantization)."""
    g = gen(seed, device)
    q = randn_bf16((1, 12, 1, 128), g, device)
    k = randn_bf16((1, 2, 2048, 128), g, device)
    v = randn_bf16((1, 2, 2048, 128), g, device)
    return q, k, v


def outlier_mask(layers: int, kv_heads: int, head_dim: int, frac: float, g: torch.Generator, device="cpu"):
    """(layers, kv_heads, head_dim) float multiplier: 20 on a seeded `frac` of channels, else 1."""
    n = max(1, round(frac * kv_heads * head_dim))
    m = torch.ones((layers, kv_heads * head_dim), dtype=torch.float32, device=device)
    for layer in range(layers):
        idx = torch.randperm(kv_heads * head_dim, generator=g, device=device)[:n]
        m[layer, idx] = 20.0
    return m.reshape(layers, kv_heads, head_dim)


def config1(seed: int = 1, device="cpu", tokens: int = 2048, layers: int = 28, kv_heads: int = 2,
            head_dim: int = 128):
    """V (layers, tokens, KV, D) BF16 with outlier channels and zero rows; slots (tokens,) int32."""
    g = gen(seed, device)
    v = torch.randn((layers, tokens, kv_heads, head_dim), generator=g, device=device)
    v = v * outlier_mask(layers, kv_heads, head_dim, 0.01, g, device)[:, None]
    n_zero = max(1, round(0.001 * tokens * layers))
    rows = torch.randperm(tokens * layers, generator=g, device=device)[:n_zero]
    v.view(layers * tokens, kv_heads, head_dim)[rows] = 0.0
    v = v.to(torch.bfloat16)
    nblk = -(-tokens // 16)
    perm = torch.randperm(nblk, generator=g, device=device).to(torch.int32)
    pos = torch.arange(tokens, device=device, dtype=torch.int32)
    slots = perm[pos // 16] * 16 + pos % 16
    return v, slots, perm


def ragged_lengths(batch: int, lo: int, hi: int, seed: int):
    g = gen(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (batch,), generator=g)]


def bytes_attn(T: int, S: int, H: int, KV: int, D: int) -> int:
    """Algorithmic HBM bytes of one (sequence, layer) attention call: K, V, scales, Q, O, table."""
    return T * KV * D * 2 + T * KV * D + T * KV * 4 + 2 * S * H * D * 2 + math.ceil(T / 16) * 4


def bytes_quant_append(tokens: int, KV: int, D: int, with_k: bool) -> int:
    """Algorithmic HBM bytes of kernel 1 per call: V in, payload out, scale out, slot (+K in/out)."""
    per = KV * D * 2 + KV * D + KV * 4 + 4
    if with_k:
        per += KV * D * 2 * 2
    return tokens * per


def prefill_chunk(q_heads: int, kv_heads: int, head_dim: int, rows: int, keys: int, seed: int = 901, device="cuda"):
    """One layer's prefill chunk (f3): a paged cache of `keys` tokens (the chunk's `rows` new
    tokens last) and q in the projection layout (1, rows, q_heads, head_dim).  Returns
    (cache, q)."""
    from .engine.paged_cache import PagedKVCache

    g = gen(seed, device)
    cache = PagedKVCache(kv_heads, head_dim, num_blocks=keys // 16 + 8, device=device, seed=seed + 1, growable=False)
    cache.prefill(0, randn_bf16((keys, kv_heads, head_dim), g, device), randn_bf16((keys, kv_heads, head_dim), g, device),
                  [keys])
    return cache, randn_bf16((1, rows, q_heads, head_dim), g, device)


def _main(argv=None) -> None:
    """python -m specdec_amd.workloads prefill [--calls N]: the reference's prefill chunk (2048
    query rows over 8192 keys) for the target (12/2/128) and the draft (14/2/64), N eager calls
    each -- a fixed workload for rocprofv3 counter runs."""
    import argparse

    from .kernels import ops

    ap = argparse.ArgumentParser(prog="python -m specdec_amd.workloads")
    ap.add_argument("workload", choices=("prefill",))
    ap.add_argument("--calls", type=int, default=3)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    for h, kv, d in ((TARGET["q_heads"], TARGET["kv_heads"], TARGET["head_dim"]),
                     (DRAFT["q_heads"], DRAFT["kv_heads"], DRAFT["head_dim"])):
        cache, q = prefill_chunk(h, kv, d, 2048, 8192, device=dev)
        kp, vp, vs = cache.layer(0)
        ws = ops.new_workspace(dev, ops.attention_workspace_bytes(1, 1, h, kv, 2048, d, 8192))
        for _ in range(args.calls):
            ops.paged_attention(q, kp, vp, vs, cache.block_table(), cache.seq_lens_tensor(), 8192,
                                q_token_major=True, workspace_tensor=ws)
        torch.cuda.synchronize()
        print(f"prefill {h}/{kv}/{d} 2048x8192: {args.calls} calls", flush=True)


if __name__ == "__main__":
    _main()
