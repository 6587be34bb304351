"""Kernel 1 (sdv_quant_append) parity: FP8 payload bytes and fp32 scales bit-exact.

Reference: quantize_kv_fp8 (specdec/engine/model_self.py:304-314) on the current V and the
v_fp8 append (model_self.py:795-799); oracle: oracle.quant on the CPU, placed into the
page layout by oracle.paged.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, announce
from helpers import bits16, quantize_rows, to_dev
from oracle import fp8 as ofp8
from oracle import paged as opaged
from specdec_amd.kernels import ops
from specdec_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _pages(dev, layers, nb, kv, d):
    k = torch.zeros((layers, nb, kv, d // 8, 16, 8), dtype=torch.bfloat16, device=dev)
    v = torch.full((layers, nb, kv, d, 16), 0xA5, dtype=torch.uint8, device=dev)  # poison
    s = torch.full((layers, nb, kv, 16), -7.0, dtype=torch.float32, device=dev)
    return k, v, s


@pytest.mark.parametrize("mode", ["div", "rcp"])
def test_config1_bit_exact(cuda_device, mode):
    """2048-token prefill write into 28 layers x 2 KV heads x 128 dims, one launch."""
    announce(f"quant config1 mode={mode}")
    v, slots, perm = wl.config1(seed=1)                  # (28, 2048, 2, 128)
    k = wl.randn_bf16(v.shape, wl.gen(2))
    L, n, kv, d = v.shape
    kp, vp, vs = _pages(cuda_device, L, 128, kv, d)
    ops.quant_append(v.to(cuda_device), slots.to(cuda_device), kp, vp, vs, k.to(cuda_device), scale_mode=mode)
    torch.cuda.synchronize()
    q, s = quantize_rows(v, mode)                        # (28, 2048, 2, 128), (28, 2048, 2)
    kp_h, vp_h, vs_h = kp.cpu(), vp.cpu().numpy(), vs.cpu().numpy()
    kb = bits16(k)
    for layer in range(L):
        ek, ev, es = opaged.alloc(128, kv, d)
        opaged.write(ek, ev, es, kb[layer], q[layer], s[layer], slots.numpy())
        assert np.array_equal(vp_h[layer], ev), f"payload layer {layer}"
        assert np.array_equal(vs_h[layer].view(np.uint32), es.view(np.uint32)), f"scale layer {layer}"
        assert np.array_equal(bits16(kp_h[layer]), ek), f"K layer {layer}"
    zero_rows = (v.float().abs().amax(-1) == 0)
    assert zero_rows.any()


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("mode", ["div", "rcp"])
def test_golden_edge_rows(cuda_device, d, mode):
    announce(f"quant golden edges d={d} mode={mode}")
    z = np.load(GOLDEN / "quant_edge.npz")
    vbits = z[f"d{d}_v"]                                 # (48, 2, d)
    n, kv, _ = vbits.shape
    slots = np.arange(n, dtype=np.int32)[::-1].copy()   # reversed: partial-block byte path
    kp, vp, vs = _pages(cuda_device, 1, 4, kv, d)
    ops.quant_append(to_dev(vbits, cuda_device), to_dev(slots, cuda_device), kp[0], vp[0], vs[0], scale_mode=mode)
    ek, ev, es = opaged.alloc(4, kv, d)
    opaged.write(None, ev, es, None, z[f"d{d}_{mode}_q"], z[f"d{d}_{mode}_s"], slots)
    got_v = vp[0].cpu().numpy()
    got_s = vs[0].cpu().numpy()
    used = np.zeros_like(ev, dtype=bool)
    blk, off = slots // 16, slots % 16
    used[blk, :, :, off] = True
    assert np.array_equal(got_v[used], ev[used])
    assert np.array_equal(got_s[blk, :, off].view(np.uint32), es[blk, :, off].view(np.uint32))
    assert (kp == 0).all()                               # k_new=None leaves K untouched


def test_decode_appends_ragged_and_skips(cuda_device):
    """One token per sequence per step into partially filled blocks, with padding slots."""
    announce("quant ragged decode appends")
    g = wl.gen(31)
    kv, d, nb = 2, 128, 64
    kp, vp, vs = _pages(cuda_device, 1, nb, kv, d)
    alloc = list(torch.randperm(nb, generator=g).numpy())
    rows = [alloc[0:5], alloc[5:9], alloc[9:20]]
    lens = [37, 50, 170]
    ek, ev, es = opaged.alloc(nb, kv, d)
    for step in range(3):
        vv = wl.randn_bf16((len(rows) + 1, kv, d), g)
        kk = wl.randn_bf16((len(rows) + 1, kv, d), g)
        slots = [int(opaged.slots_for(rows[b], lens[b] + step, 1)[0]) for b in range(len(rows))] + [-1]
        slots = np.array(slots, dtype=np.int32)
        ops.quant_append(vv.to(cuda_device), to_dev(slots, cuda_device), kp[0], vp[0], vs[0], kk.to(cuda_device))
        q, s = quantize_rows(vv)
        opaged.write(ek, ev, es, bits16(kk), q, s, slots)
    torch.cuda.synchronize()
    written = np.zeros((nb, kv, 16), dtype=bool)
    for b in range(len(rows)):
        for p in range(lens[b], lens[b] + 3):
            sl = int(opaged.slots_for(rows[b], p, 1)[0])
            written[sl // 16, :, sl % 16] = True
    got_v = vp[0].cpu().numpy().transpose(0, 1, 3, 2)   # (nb, kv, 16, d)
    want_v = ev.transpose(0, 1, 3, 2)
    assert np.array_equal(got_v[written], want_v[written])
    assert (got_v[~written] == 0xA5).all()               # nothing else touched
    got_s = vs[0].cpu().numpy()
    assert np.array_equal(got_s[written].view(np.uint32), es[written].view(np.uint32))
    assert (got_s[~written] == -7.0).all()
    got_k = bits16(kp[0])                                # (nb, kv, d/8, 16, 8)
    blk_i, kv_i, off_i = np.nonzero(written)
    assert np.array_equal(got_k[blk_i, kv_i, :, off_i, :], ek[blk_i, kv_i, :, off_i, :])
    unwritten = np.ones(nb, dtype=bool)
    unwritten[blk_i] = False
    assert (got_k[unwritten] == 0).all()


def test_d64_draft_shape_multi_layer(cuda_device):
    announce("quant d64 24 layers")
    v, slots, _ = wl.config1(seed=4, tokens=512, layers=24, head_dim=64)
    k = wl.randn_bf16(v.shape, wl.gen(5))
    kp, vp, vs = _pages(cuda_device, 24, 32, 2, 64)
    ops.quant_append(v.to(cuda_device), slots.to(cuda_device), kp, vp, vs, k.to(cuda_device))
    q, s = quantize_rows(v)
    kb = bits16(k)
    for layer in (0, 11, 23):
        ek, ev, es = opaged.alloc(32, 2, 64)
        opaged.write(ek, ev, es, kb[layer], q[layer], s[layer], slots.numpy())
        assert np.array_equal(vp[layer].cpu().numpy(), ev)
        assert np.array_equal(vs[layer].cpu().numpy().view(np.uint32), es.view(np.uint32))
        assert np.array_equal(bits16(kp[layer]), ek)


def test_device_encoder_exhaustive(cuda_device):
    """sdv_fp8_encode over every fp32 bit pattern == torch's cast (pinned to the C codec)."""
    announce("fp8 encode exhaustive")
    chunk = 1 << 28
    for lo in range(0, 1 << 32, chunk):
        bits = torch.arange(lo, lo + chunk, dtype=torch.int64, device=cuda_device).to(torch.int32)
        x = bits.view(torch.float32)
        ours = ops.fp8_encode(x)
        th = x.to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(ours, th), hex(lo)
        del bits, x, ours, th
    # and a random sample straight against the C oracle
    g = torch.Generator().manual_seed(5)
    samp = torch.randint(-(1 << 31), (1 << 31) - 1, (1 << 20,), generator=g, dtype=torch.int64).to(torch.int32)
    ours = ops.fp8_encode(samp.view(torch.float32).to(cuda_device)).cpu().numpy()
    assert np.array_equal(ours, ofp8.encode(samp.view(torch.float32).numpy()))


@pytest.mark.parametrize("d", [128, 64])
def test_prefill_mixed_tiles(cuda_device, d):
    """One launch whose 16-token tiles take every path: whole aligned blocks (16-byte
    dimension stores), a contiguous run that starts mid-block, a reversed run, a run with a
    padding slot and an out-of-range slot, and a partial last tile; K written too."""
    announce(f"quant mixed tiles d={d}")
    g = wl.gen(77 + d)
    kv, nb = 2, 16
    slots = list(range(2 * 16, 5 * 16))                 # tiles 0-2: blocks 2, 3, 4 whole
    slots += list(range(6 * 16 + 3, 7 * 16 + 3))        # tile 3: contiguous, not block aligned
    slots += list(range(9 * 16 + 15, 8 * 16 - 1, -1))   # tile 4: block 8 reversed
    t5 = list(range(10 * 16, 11 * 16))
    t5[5], t5[11] = -1, nb * 16 + 40                     # padding and out-of-range slots: skipped
    slots += t5
    slots += list(range(12 * 16, 12 * 16 + 7))          # tile 6: 7 tokens of block 12
    slots = np.array(slots, dtype=np.int32)
    n = len(slots)
    v = wl.randn_bf16((n, kv, d), g)
    k = wl.randn_bf16((n, kv, d), g)
    kp, vp, vs = _pages(cuda_device, 1, nb, kv, d)
    ops.quant_append(v.to(cuda_device), to_dev(slots, cuda_device), kp[0], vp[0], vs[0], k.to(cuda_device))
    torch.cuda.synchronize()
    q, s = quantize_rows(v)
    keep = (slots >= 0) & (slots < nb * 16)
    ek, ev, es = opaged.alloc(nb, kv, d)
    ev[:] = 0xA5
    es[:] = -7.0
    opaged.write(ek, ev, es, bits16(k)[keep], q[keep], s[keep], slots[keep])
    assert np.array_equal(vp[0].cpu().numpy(), ev)
    assert np.array_equal(vs[0].cpu().numpy().view(np.uint32), es.view(np.uint32))
    assert np.array_equal(bits16(kp[0]), ek)


@pytest.mark.parametrize("d", [128, 64])
def test_varlen_prefill_tile_table(cuda_device, d):
    """A packed varlen prefill through sdv_quant_append_tiles: sequences of ragged lengths
    whose first tokens land at various positions of their first page block (a whole prompt,
    or an append to a partly filled block), an empty sequence, fragmented pages.  Bytes and
    scales bit-exact against the oracle, and equal to the launch without a table."""
    announce(f"quant varlen prefill tile table d={d}")
    lengths = [37, 16, 5, 0, 100, 33, 700]
    starts = [0, 0, 3, 0, 15, 16, 9]
    kv, nb = 2, 128
    perm = np.random.default_rng(5).permutation(nb)
    parts, at = [], 0
    for n, p0 in zip(lengths, starts):
        need = (p0 + n + 15) // 16
        blocks = perm[at:at + need]
        at += need
        pos = np.arange(p0, p0 + n)
        parts.append(blocks[pos // 16] * 16 + pos % 16)
    slots = np.concatenate(parts).astype(np.int32)
    n = len(slots)
    g = wl.gen(91 + d)
    v = wl.randn_bf16((n, kv, d), g)
    k = wl.randn_bf16((n, kv, d), g)
    tiles = torch.tensor(ops.varlen_tile_starts(lengths, starts), dtype=torch.int32, device=cuda_device)
    kp, vp, vs = _pages(cuda_device, 1, nb, kv, d)
    ops.quant_append(v.to(cuda_device), to_dev(slots, cuda_device), kp[0], vp[0], vs[0], k.to(cuda_device),
                     tile_starts=tiles)
    kp2, vp2, vs2 = _pages(cuda_device, 1, nb, kv, d)
    ops.quant_append(v.to(cuda_device), to_dev(slots, cuda_device), kp2[0], vp2[0], vs2[0], k.to(cuda_device))
    torch.cuda.synchronize()
    q, s = quantize_rows(v)
    ek, ev, es = opaged.alloc(nb, kv, d)
    ev[:] = 0xA5
    es[:] = -7.0
    opaged.write(ek, ev, es, bits16(k), q, s, slots)
    assert np.array_equal(vp[0].cpu().numpy(), ev)
    assert np.array_equal(vs[0].cpu().numpy().view(np.uint32), es.view(np.uint32))
    assert np.array_equal(bits16(kp[0]), ek)
    assert torch.equal(vp, vp2) and torch.equal(vs.view(torch.int32), vs2.view(torch.int32))
    assert torch.equal(kp.view(torch.int16), kp2.view(torch.int16))
