"""Kernels 2/3 (sdv_paged_attention) parity against the eager BF16 path.

Reference: model_self.py:715-776 (dequantize the FP8 V cache, kv_repeat, BF16 q.k^T,
/sqrt(D), offset-causal mask, fp32 softmax, BF16 probabilities, BF16 p.v).  Oracle:
oracle.attention.eager_attention on the CPU.  Bar (BASELINE): max-abs <= 2e-2 and
rel-L2 <= 1e-3 against the eager output, for every row of every case.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, announce
from helpers import assert_close, bits16, build_pages, eager_ref, to_dev
from oracle import attention as oatt
from specdec_amd import _native, workloads as wl
from specdec_amd.engine.paged_cache import PagedKVCache
from specdec_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _run_case(dev, h, kv, d, lens, s, *, seed, fragmented=True, extra_blocks=7, q_token_major=False, split=False):
    """Random q/k/v per sequence, oracle-built pages, one kernel call (split: the three launches
    called one at a time on one workspace, the profiling split); returns (got, want)."""
    g = wl.gen(seed)
    B = len(lens)
    nbs = [-(-t // 16) for t in lens]
    nb = sum(nbs) + extra_blocks
    order = torch.randperm(nb, generator=g).tolist() if fragmented else list(range(nb))
    rows, at = [], 0
    for n in nbs:
        rows.append(order[at:at + n])
        at += n
    ks = [wl.randn_bf16((kv, t, d), g) for t in lens]
    vs = [wl.randn_bf16((kv, t, d), g) for t in lens]
    qs = [wl.randn_bf16((h, s, d), g) for _ in lens]
    kp, vp, sp = build_pages(ks, vs, nb, rows)
    mb = max(nbs)
    bt = np.full((B, mb), -1, dtype=np.int32)
    for b, r in enumerate(rows):
        bt[b, :len(r)] = r
    q = torch.stack(qs)                                   # (B, H, S, D)
    qd = q.transpose(1, 2).contiguous() if q_token_major else q
    args = (qd.to(dev), to_dev(kp, dev), to_dev(vp, dev), to_dev(sp, dev), to_dev(bt, dev),
            to_dev(np.array(lens, dtype=np.int32), dev), max(lens))
    if split:
        ws = ops.new_workspace(dev, ops.attention_workspace_bytes(1, B, h, kv, s, d, max(lens)))
        out = torch.empty_like(args[0])
        for ph in (_native.PHASE_QK, _native.PHASE_PV, _native.PHASE_REDUCE):
            ops.paged_attention(*args, q_token_major=q_token_major, phases=ph, out=out, workspace_tensor=ws)
    else:
        out = ops.paged_attention(*args, q_token_major=q_token_major)
    torch.cuda.synchronize()
    if q_token_major:
        out = out.transpose(1, 2)
    want = [eager_ref(qs[b][None], ks[b][None], vs[b][None], d)[0] for b in range(B)]
    return out.cpu(), torch.stack(want)


def test_config0_golden(cuda_device):
    """One 1.5B layer, decode, T=2048, V written by kernel 1 (product path end to end)."""
    announce("attn config0 golden")
    q, k, v = wl.config0(seed=0)
    cache = PagedKVCache(2, 128, capacity_tokens=2048, device=cuda_device)
    kt = k[0].transpose(0, 1).unsqueeze(0).contiguous()   # (1, T, KV, D)
    vt = v[0].transpose(0, 1).unsqueeze(0).contiguous()
    cache.append(0, kt.to(cuda_device), vt.to(cuda_device))
    out = cache.attend(0, q.to(cuda_device)).cpu()
    z = np.load(GOLDEN / "attn_eager.npz")
    want = torch.from_numpy(z["cfg0_out"].view(np.int16)).view(torch.bfloat16)
    stats = assert_close(out, want, "cfg0 vs golden")
    print("cfg0", stats)
    assert_close(out, eager_ref(q, k, v, 128), "cfg0 vs oracle on this host")


@pytest.mark.parametrize("t", [2048, 8192])
def test_decode_target_shape(cuda_device, t):
    announce(f"attn decode 12/2/128 T={t}")
    got, want = _run_case(cuda_device, 12, 2, 128, [t], 1, seed=40 + t)
    print("decode", t, assert_close(got, want, f"decode T={t}"))


@pytest.mark.parametrize("t", [2048, 4096, 8192])
def test_verify_five_rows(cuda_device, t):
    announce(f"attn verify S=5 T={t}")
    got, want = _run_case(cuda_device, 12, 2, 128, [t], 5, seed=50 + t)
    for i in range(5):
        assert_close(got[:, :, i], want[:, :, i], f"verify T={t} row {i}")


@pytest.mark.parametrize("t", [2048, 4096, 8192])
def test_draft_shape_d64(cuda_device, t):
    announce(f"attn draft 14/2/64 T={t}")
    got, want = _run_case(cuda_device, 14, 2, 64, [t], 1, seed=60 + t)
    print("draft", t, assert_close(got, want, f"draft T={t}"))


def test_small_and_ragged_edges(cuda_device):
    """T=1, T<16, T not a multiple of 16 or 32, odd block counts, S>T-1 edges."""
    announce("attn ragged small edges")
    lens = [1, 5, 16, 17, 31, 33, 48, 100, 1000]
    got, want = _run_case(cuda_device, 12, 2, 128, lens, 1, seed=70)
    for b, t in enumerate(lens):
        assert_close(got[b], want[b], f"T={t}")
    lens = [5, 6, 21, 64, 129]
    got, want = _run_case(cuda_device, 12, 2, 128, lens, 5, seed=71)
    for b, t in enumerate(lens):
        assert_close(got[b], want[b], f"S=5 T={t}")


@pytest.mark.parametrize("s,lens", [(64, [300, 64, 1000]), (77, [77]), (16, [2048])])
def test_prefill_rows(cuda_device, s, lens):
    """Prefill/chunked-prefill blocks: S query rows per sequence, row i sees keys j <= T-S+i
    (model_self.py:755-764); S=77 over T=77 is a prefill from an empty cache (row 0 sees one key)."""
    announce(f"attn prefill rows S={s} lens={lens}")
    got, want = _run_case(cuda_device, 12, 2, 128, lens, s, seed=90 + s)
    for b, t in enumerate(lens):
        print("prefill", s, t, assert_close(got[b], want[b], f"S={s} T={t}"))


def test_token_major_q_layout(cuda_device):
    announce("attn token-major q")
    got, want = _run_case(cuda_device, 12, 2, 128, [300, 777], 5, seed=72, q_token_major=True)
    assert_close(got, want, "token-major")


@pytest.mark.parametrize("split", [False, True])
def test_config4_batch32_ragged(cuda_device, split):
    """B=32, T_b ~ U{2048..32768}, fragmented pool: every sequence within the bar, through the
    single launch (items sized per sequence) and through the three launches one at a time."""
    announce(f"attn config4 B=32 ragged split={split}")
    lens = wl.ragged_lengths(32, 2048, 32768, seed=4)
    got, want = _run_case(cuda_device, 12, 2, 128, lens, 1, seed=73, split=split)
    worst = 0.0
    for b, t in enumerate(lens):
        worst = max(worst, assert_close(got[b], want[b], f"b={b} T={t}")["rel_l2"])
    print("config4 worst rel_l2", worst)


def test_many_groups_band(cuda_device):
    """More one-tile groups than the single launch holds at once, one layer (160 sequences x 2
    KV heads): the persistent per-group kernel, which took this band over from the three
    launches; every sequence checked."""
    announce("attn per-group kernel, 160 ragged sequences")
    g = np.random.default_rng(77)
    lens = [int(x) for x in g.integers(17, 3000, size=160)]
    assert ops.single_launch_workgroups(1, len(lens), 12, 2, 1, 128, max(lens)) == 0
    got, want = _run_case(cuda_device, 12, 2, 128, lens, 1, seed=78)
    for b, t in enumerate(lens):
        assert_close(got[b], want[b], f"b={b} T={t}")


def test_deterministic_bitwise(cuda_device):
    announce("attn determinism")
    g = wl.gen(80)
    t = 5000
    kp, vp, sp = build_pages([wl.randn_bf16((2, t, 128), g)], [wl.randn_bf16((2, t, 128), g)], 320,
                             [list(range(313))])
    bt = to_dev(np.arange(313, dtype=np.int32)[None], cuda_device)
    args = (to_dev(kp, cuda_device), to_dev(vp, cuda_device), to_dev(sp, cuda_device), bt,
            torch.tensor([t], dtype=torch.int32, device=cuda_device), t)
    q = wl.randn_bf16((1, 12, 5, 128), g).to(cuda_device)
    o1 = ops.paged_attention(q, *args).clone()
    o2 = ops.paged_attention(q, *args)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


def test_invalid_block_ids_are_masked(cuda_device):
    """Block-table entries outside [0, num_blocks) are never read; their tokens drop out."""
    announce("attn invalid block ids")
    g = wl.gen(81)
    t, d = 64, 128
    k = wl.randn_bf16((2, t, d), g)
    v = wl.randn_bf16((2, t, d), g)
    kp, vp, sp = build_pages([k], [v], 4, [[0, 1, 2, 3]])
    q = wl.randn_bf16((1, 12, 1, d), g)
    bt = np.array([[0, 1000, 2, -5]], dtype=np.int32)      # blocks 1 and 3 invalid
    out = ops.paged_attention(q.to(cuda_device), to_dev(kp, cuda_device), to_dev(vp, cuda_device),
                              to_dev(sp, cuda_device), to_dev(bt, cuda_device),
                              torch.tensor([t], dtype=torch.int32, device=cuda_device), t).cpu()
    keep = torch.cat([torch.arange(0, 16), torch.arange(32, 48)])
    want = eager_ref(q, k[None][:, :, keep], v[None][:, :, keep], d)
    assert_close(out, want, "masked blocks")


def test_reference_op_signature(cuda_device):
    """ops.attention(q, k, (payload, scale)) over a contiguous v_fp8 cache (the engine's dicts)."""
    announce("ops.attention contiguous v_fp8")
    g = wl.gen(82)
    q = wl.randn_bf16((1, 12, 5, 128), g)
    k = wl.randn_bf16((1, 2, 333, 128), g)
    v = wl.randn_bf16((1, 2, 333, 128), g)
    from oracle import quant as oq
    pq, ps = oq.quantize_kv_fp8(v, 128)
    out = ops.attention(q.to(cuda_device), k.to(cuda_device), (pq.to(cuda_device), ps.to(cuda_device)),
                        backend="hip").cpu()
    assert_close(out, eager_ref(q, k, v, 128), "ops.attention")
    with pytest.raises(ValueError):
        ops.attention(q.to(cuda_device), k.to(cuda_device), (pq, ps), backend="triton")


def test_multi_layer_launch_matches_per_layer(cuda_device):
    """L layers in one launch agree with L single-layer launches (the split of each layer's
    keys into per-workgroup items depends on how many layers share the launch, so the fp32
    summation order -- not the result beyond rounding -- may differ) and each launch shape is
    bitwise repeatable."""
    announce("attn multi-layer launch")
    L, t = 4, 3000
    cache = PagedKVCache(2, 128, num_layers=L, capacity_tokens=t, device=cuda_device, seed=3)
    g = wl.gen(83)
    for layer in range(L):
        cache.append(layer, wl.randn_bf16((1, t, 2, 128), g).to(cuda_device),
                     wl.randn_bf16((1, t, 2, 128), g).to(cuda_device), starts=[0])
    q = wl.randn_bf16((L, 1, 12, 1, 128), g).to(cuda_device)
    multi = ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                                cache.seq_lens_tensor(), t)
    again = ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                                cache.seq_lens_tensor(), t)
    assert torch.equal(multi.view(torch.int16), again.view(torch.int16))
    for layer in range(L):
        single = cache.attend(layer, q[layer])
        k, v, sc = cache.gather(layer, 0)
        from oracle import quant as oq
        v_hat = oq.dequantize_kv_fp8(v.cpu()[None], sc.cpu()[None], torch.bfloat16)
        want = oatt.eager_attention(q[layer].cpu(), k.cpu()[None], v_hat)
        assert_close(single.cpu(), want, f"layer {layer} single launch")
        assert_close(multi[layer].cpu(), want, f"layer {layer} multi-layer launch")
        d = (single.float() - multi[layer].float()).abs().max().item()
        assert d <= 2.0 ** -8 * multi[layer].float().abs().max().item(), f"layer {layer}: {d}"


def test_single_launch_leaves_sync_area_clean(cuda_device):
    """The single-launch path records no expired waits and leaves its header and statistics
    area zero (the replays of a graph reuse their tag, so nothing tagged may survive a call);
    partial slots are zeroed by each item at the start of a call, so they may hold data."""
    announce("attn single-launch sync area")
    from specdec_amd import _native
    ws = ops.new_workspace(cuda_device, ops.attention_workspace_bytes(1, 3, 12, 2, 5, 128, 700))
    for s in (1, 5):
        got, want = None, None
        g = wl.gen(95 + s)
        lens = [700, 333, 17]
        nbs = [-(-t // 16) for t in lens]
        rows, at = [], 0
        for n_ in nbs:
            rows.append(list(range(at, at + n_)))
            at += n_
        ks = [wl.randn_bf16((2, t, 128), g) for t in lens]
        vs = [wl.randn_bf16((2, t, 128), g) for t in lens]
        q = wl.randn_bf16((3, 12, s, 128), g)
        kp, vp, sp = build_pages(ks, vs, at, rows)
        bt = np.full((3, max(nbs)), -1, dtype=np.int32)
        for b, r in enumerate(rows):
            bt[b, :len(r)] = r
        for _ in range(3):
            out = ops.paged_attention(q.to(cuda_device), to_dev(kp, cuda_device), to_dev(vp, cuda_device),
                                      to_dev(sp, cuda_device), to_dev(bt, cuda_device),
                                      to_dev(np.array(lens, dtype=np.int32), cuda_device), 700,
                                      workspace_tensor=ws)
        torch.cuda.synchronize()
        for b in range(3):
            assert_close(out[b].cpu(), eager_ref(q[b][None], ks[b][None], vs[b][None], 128)[0], f"S={s} b={b}")
    stats_end = 256 + 4096 * 64 * 16   # header + (max, tag), (sum, tag) words of every item row
    sync = ws[:stats_end].view(torch.int32).cpu()
    assert ops.workspace_status(ws) == (0, False), "expired waits"
    assert int(sync.abs().sum()) == 0, "statistics not cleared"


def _check_multi_layer(dev, cache, h, s, layers, seqs, label, seed):
    """One multi-layer launch over every layer of `cache` against the eager oracle on the
    (layer, sequence) pairs named, reading back what the append kernel wrote."""
    from oracle import quant as oq
    g = wl.gen(seed, dev)
    L, B = cache.num_layers, cache.batch
    q = torch.randn((L, B, h, s, cache.head_dim), generator=g, device=dev).to(torch.bfloat16)
    lens = list(cache.lengths)
    ws = ops.new_workspace(dev, ops.attention_workspace_bytes(L, B, h, cache.kv_heads, s, cache.head_dim,
                                                              max(lens)))
    out = ops.paged_attention(q, cache.k_pages, cache.v_pages, cache.v_scales, cache.block_table(),
                              cache.seq_lens_tensor(), max(lens), workspace_tensor=ws)
    torch.cuda.synchronize()
    assert ops.sync_errors(ws) == 0, f"{label}: expired waits"
    for layer in layers:
        for b in seqs:
            k, v, sc = cache.gather(layer, b)
            v_hat = oq.dequantize_kv_fp8(v.cpu()[None], sc.cpu()[None], torch.bfloat16)
            want = oatt.eager_attention(q[layer, b:b + 1].cpu(), k.cpu()[None], v_hat)
            assert_close(out[layer, b:b + 1].cpu(), want, f"{label} layer {layer} seq {b} T={lens[b]}")


def _filled_cache(dev, layers, kv, d, lens, seed, outliers=False):
    g = wl.gen(seed, dev)
    cache = PagedKVCache(kv, d, num_layers=layers, batch=len(lens), num_blocks=sum(-(-t // 16) for t in lens) + 9,
                         device=dev, seed=seed, growable=False)
    mult = wl.outlier_mask(layers, kv, d, 0.01, g, dev) if outliers else None
    slots = None
    for layer in range(layers):
        k = torch.randn((sum(lens), kv, d), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((sum(lens), kv, d), generator=g, device=dev)
        if mult is not None:
            v = v * mult[layer]
        slots = cache.prefill(layer, k, v.to(torch.bfloat16), lens, slots)
    return cache


def test_multi_layer_draft_d64(cuda_device):
    """The 0.5B draft shape (14q/2kv, D=64) over 24 layers at 8K in one launch."""
    announce("attn multi-layer draft 24x14/2/64 T=8192")
    cache = _filled_cache(cuda_device, 24, 2, 64, [8192], seed=501)
    _check_multi_layer(cuda_device, cache, 14, 1, (0, 13, 23), (0,), "draft", seed=502)


def test_multi_layer_decode_28(cuda_device):
    """The headline decode shape (28 layers, 12/2/128, T=8192) in one launch, checked on the
    first, two middle and the last layer."""
    announce("attn multi-layer decode 28x12/2/128 T=8192")
    cache = _filled_cache(cuda_device, 28, 2, 128, [8192], seed=530)
    _check_multi_layer(cuda_device, cache, 12, 1, (0, 13, 14, 27), (0,), "decode 28L", seed=531)


@pytest.mark.parametrize("layers,kv,h,lens", [(37, 1, 6, [7000]), (8, 2, 12, [8192, 3000, 17])])
def test_single_launch_odd_groups_and_ragged(cuda_device, layers, kv, h, lens):
    """The single launch with an odd number of groups (37 layers, one KV head) and with ragged
    sequences in one batch (items past a short sequence's end own nothing)."""
    announce(f"attn single launch L={layers} kv={kv} h={h} lens={lens}")
    assert ops.single_launch_workgroups(layers, len(lens), h, kv, 1, 128, max(lens)) > 0
    cache = _filled_cache(cuda_device, layers, kv, 128, lens, seed=540 + layers)
    seqs = tuple(range(len(lens)))
    _check_multi_layer(cuda_device, cache, h, 1, tuple(sorted({0, layers // 2, layers - 1})), seqs,
                       f"L={layers} lens={lens}", seed=541)


@pytest.mark.parametrize("d,h", [(128, 12), (64, 14)])
def test_single_launch_large_items_batch32(cuda_device, d, h):
    """One layer of a 32-sequence ragged batch of 2K-32K tokens (config 4's per-layer call) in
    one launch: 64 groups cut into items per sequence length, the longest of about 340 page
    blocks (each wavefront sums its p.V units in registers; the LDS is sized for 512).  Checked
    on the longest, the shortest, the first and the last sequence."""
    lens = wl.ragged_lengths(32, 2048, 32768, seed=41)
    announce(f"attn single launch B=32 ragged one layer {h}/2/{d} max T={max(lens)}")
    grid = ops.single_launch_workgroups(1, 32, h, 2, 1, d, max(lens))
    assert grid > 0 and grid % 64 == 0
    assert -(-max(lens) // 16) // min(32, grid // 64) >= 256  # LDS width of the items (blocks)
    cache = _filled_cache(cuda_device, 1, 2, d, lens, seed=575 + d)
    seqs = tuple(sorted({0, 31, int(np.argmax(lens)), int(np.argmin(lens))}))
    _check_multi_layer(cuda_device, cache, h, 1, (0,), seqs, f"B=32 ragged d={d}", seed=576)


@pytest.mark.parametrize("t", [2048, 8192])
def test_multi_layer_verify_s5(cuda_device, t):
    """The k+1=5-row verify over all 28 target layers in one launch."""
    announce(f"attn multi-layer verify 28x12/2/128 S=5 T={t}")
    cache = _filled_cache(cuda_device, 28, 2, 128, [t], seed=510 + t)
    _check_multi_layer(cuda_device, cache, 12, 5, (0, 27), (0,), f"verify T={t}", seed=511)


@pytest.mark.parametrize("layers,h,d,lens", [(1, 12, 128, [32768, 9000]), (1, 12, 64, [32768]), (16, 12, 128, [8192])])
def test_verify_wide_split(cuda_device, layers, h, d, lens):
    """Verify (S=5, two row tiles) on items of 64 blocks or more, where p.V splits wider
    dimension tiles over block parts and the polling wavefronts load V after the group wait:
    a ragged pair (items past the short sequence's end own nothing), D=64, and 16 layers."""
    announce(f"attn verify wide split L={layers} {h}/2/{d} lens={lens}")
    grid = ops.single_launch_workgroups(layers, len(lens), h, 2, 5, d, max(lens))
    groups = layers * len(lens) * 2
    assert grid > 0 and grid % groups == 0
    assert -(-max(lens) // 16) // min(32, grid // groups) >= 64  # blocks per item (at most 32 items a group)
    cache = _filled_cache(cuda_device, layers, 2, d, lens, seed=560 + layers + d)
    _check_multi_layer(cuda_device, cache, h, 5, tuple(sorted({0, layers - 1})), tuple(range(len(lens))),
                       f"wide L={layers} d={d}", seed=561)


def test_multi_layer_batch32_ragged(cuda_device):
    """Config 4: B=32 contexts U{2048..32768}, fragmented pool, 1% outlier V channels x20,
    28 layers in one call, which runs one single launch per layer (the whole call has more
    groups than the device holds at once, one layer does not); the shortest, the longest and
    the first sequence are checked on the first, a middle and the last layer."""
    lens = wl.ragged_lengths(32, 2048, 32768, seed=41)
    announce(f"attn multi-layer B=32 ragged 28x12/2/128 T={min(lens)}..{max(lens)}")
    assert ops.single_launch_workgroups(28, 32, 12, 2, 1, 128, max(lens)) == 0
    assert ops.single_launch_workgroups(1, 32, 12, 2, 1, 128, max(lens)) > 0
    cache = _filled_cache(cuda_device, 28, 2, 128, lens, seed=520, outliers=True)
    seqs = sorted({0, lens.index(min(lens)), lens.index(max(lens))})
    _check_multi_layer(cuda_device, cache, 12, 1, (0, 13, 27), seqs, "B=32 ragged", seed=521)
    fp = cache.footprint()
    assert fp["tokens"] == sum(lens)
    assert abs(fp["saved_frac"] - (1 - 776 / 1024)) < 1e-9


@pytest.mark.parametrize("h,d,s,t,layers", [(12, 128, 8, 3000, 1), (12, 128, 10, 1500, 1), (14, 64, 5, 2048, 1),
                                            (12, 128, 8, 4096, 4), (14, 64, 5, 4096, 6)])
def test_single_launch_three_and_four_row_tiles(cuda_device, h, d, s, t, layers):
    """Query-row groups of 3 and 4 MFMA row tiles (R = G*S = 48, 60, 35 rows) on the single
    launch: probabilities formed once per item in LDS, statistics of several rows per
    wavefront merged in one pass."""
    announce(f"attn single launch {h}/2/{d} S={s} T={t} L={layers}")
    r = (h // 2) * s
    assert r > 32, r  # three or four row tiles
    assert ops.single_launch_workgroups(layers, 1, h, 2, s, d, t) > 0
    cache = _filled_cache(cuda_device, layers, 2, d, [t], seed=600 + s + t)
    _check_multi_layer(cuda_device, cache, h, s, tuple(sorted({0, layers - 1})), (0,), f"{h}/{d} S={s}", seed=601)
