#!/usr/bin/env python3
"""Decode-attention benchmark: HBM GB/s and us/layer at 8K context over a 28-layer FP8-V
paged cache (Qwen2.5-1.5B shape, B=1, S=1, 12q/2kv heads, D=128,
T=8192, block size 16, blocks placed by a seeded permutation).

One step = single-token decode attention over all 28 layers, inputs resident in HBM.
  --mode multi : the 28 layers in one sdv_paged_attention call (one launch of the
                 single-launch kernel at this shape; the three-launch split is timed beside it)
  --mode graph : 28 per-layer calls captured in one HIP graph
The cache is written by the library's own quantize+append kernel from synthetic N(0,1)
K/V.  Several cache replicas (default 4 x 178 MB) are rotated step by step so the 256 MB
Infinity Cache cannot hold the working set.

Prints ONE JSON line.  `value` is whole-step throughput in GB/s of algorithmic bytes
(K + V + scales + Q + O + block table per layer).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "specdec-context-scaling_amd"))

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_decode8k_multi.json"


def library_sha256() -> str:
    """Digest of the native library this run loads (libsdv.so; rebuilding the same sources gives
    the same bytes): a traffic figure measured on another build is not this build's."""
    from specdec_amd import _native

    return hashlib.sha256(_native.LIB_PATH.read_bytes()).hexdigest()


def stamped_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary, and where they came from; the bytes are None when that summary was measured on
    another build of the native library than the one this run loads."""
    if not TRAFFIC_FILE.exists():
        return None, {"file": None, "reason": "no traffic summary committed"}
    rec = json.loads(TRAFFIC_FILE.read_text())
    cur = library_sha256()
    src = {"file": str(TRAFFIC_FILE.relative_to(ROOT)), "summary": rec.get("summary"),
           "measured_library_sha256": rec.get("library_sha256"), "this_library_sha256": cur}
    if rec.get("library_sha256") != cur:
        src["reason"] = "measured on another build of libsdv.so: stale, not reported"
        return None, src
    return rec.get("bytes_per_launch", {}).get(kernel), src


L, B, H, KV, D, T, S = 28, 1, 12, 2, 128, 8192, 1


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=("multi", "graph"), default="multi")
    ap.add_argument("--replicas", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline leg")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph-leg", action="store_true", help="skip the per-layer HIP-graph figure")
    ap.add_argument("--no-suite", action="store_true", help="skip the other BASELINE configurations")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run 3 plain device copies of MIB MiB (calibrates rocprof byte counters)")
    return ap.parse_args()


def phase_bytes():
    """Algorithmic bytes per (sequence, layer) of each launch and of the whole call."""
    from specdec_amd import workloads as wl

    nblk = math.ceil(T / 16)
    return {
        "qk": T * KV * D * 2 + S * H * D * 2 + nblk * 4,
        "pv": T * KV * D + T * KV * 4 + nblk * 4,
        "reduce": S * H * D * 2,
        "all": wl.bytes_attn(T, S, H, KV, D),
    }


def build_replicas(torch, dev, n, scattered=True):
    from specdec_amd.engine.paged_cache import PagedKVCache
    from specdec_amd.kernels import ops

    reps = []
    for r in range(n):
        g = torch.Generator(device=dev)
        g.manual_seed(1000 + r)
        cache = PagedKVCache(KV, D, num_layers=L, batch=B, num_blocks=T // 16 + 64, device=dev,
                             seed=(2000 + r) if scattered else None, growable=False)
        cache.reserve(0, T)
        slots = cache.slot_mapping([0], T)
        k = torch.randn((L, T, KV, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((L, T, KV, D), generator=g, device=dev).to(torch.bfloat16)
        ops.quant_append(v, slots, cache.k_pages, cache.v_pages, cache.v_scales, k)
        cache.lengths[0] = T
        del k, v
        q = torch.randn((L, B, H, S, D), generator=g, device=dev).to(torch.bfloat16)
        reps.append(dict(cache=cache, q=q, bt=cache.block_table(), sl=cache.seq_lens_tensor(),
                         out=torch.empty_like(q)))
    torch.cuda.synchronize()
    return reps


def time_steps(torch, step, steps, warmup, nrep):
    """Average ms per step of step(i) for i = 0..steps-1 (replica i % nrep).

    Exactly `warmup` steps, then exactly `steps` steps, each set captured into one HIP graph
    (cycling through the cache replicas) and replayed once, so the timed region holds only GPU
    work: a Python call costs ~20 us of host time, more than some of the kernels being timed.
    Both graphs are captured first and replayed back to back, so the GPU goes from the warm-up
    steps straight into the timed ones (an idle gap lets its clocks drop: a 20-step timing
    right after one reads 3-6% slower).  HIP events bracket the timed replay on torch's
    current stream, the stream the library launches on.
    """
    def capture(n):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n):
                step(i % nrep)
        return graph

    warm = capture(warmup) if warmup > 0 else None
    timed = capture(steps)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if warm is not None:
        warm.replay()
    e0.record()
    timed.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from specdec_amd import _native
    from specdec_amd.kernels import ops

    _native.load()
    dev = torch.device("cuda:0")
    reps = build_replicas(torch, dev, args.replicas)
    _progress(f"{args.replicas} cache replicas built")
    ws_multi = ops.workspace(dev, ops.attention_workspace_bytes(L, B, H, KV, S, D, T))

    def multi_step(r, phases=_native.PHASE_ALL):
        rep = reps[r]
        c = rep["cache"]
        ops.paged_attention(rep["q"], c.k_pages, c.v_pages, c.v_scales, rep["bt"], rep["sl"], T,
                            out=rep["out"], workspace_tensor=ws_multi, phases=phases)

    def per_layer_calls(r):
        rep = reps[r]
        c = rep["cache"]
        for layer in range(L):
            kp, vp, vs = c.layer(layer)
            ops.paged_attention(rep["q"][layer], kp, vp, vs, rep["bt"], rep["sl"], T, out=rep["out"][layer],
                                workspace_tensor=ws_layer)

    ws_layer = torch.empty(ops.attention_workspace_bytes(1, B, H, KV, S, D, T), dtype=torch.uint8, device=dev)
    graphs = []

    def build_graphs():
        for r in range(args.replicas):
            per_layer_calls(r)  # warm the path outside capture
        torch.cuda.synchronize()
        for r in range(args.replicas):
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                per_layer_calls(r)
            graphs.append(gph)
        torch.cuda.synchronize()

    # the per-layer graphs are recorded after the headline timing unless it uses them, so that
    # their recording (host work, the GPU idle) does not sit between the cache fill and it
    if args.mode == "graph":
        build_graphs()

    def graph_step(r):
        graphs[r].replay()

    def time_graphs(steps, warmup):
        for i in range(warmup):
            graph_step(i % args.replicas)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            graph_step(i % args.replicas)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    pb = phase_bytes()
    bytes_step = L * B * pb["all"]
    if args.mode == "multi":
        ms = time_steps(torch, multi_step, args.steps, args.warmup, args.replicas)
    else:
        ms = time_graphs(args.steps, args.warmup)
    value = bytes_step / (ms * 1e-3) / 1e9

    # The multi-layer call is one launch of the single-launch kernel (fused_kernel) when the
    # grid fits the device, which is the case at this shape; its per-launch time is the step
    # time above (one launch per step, back to back in the graph).  For reference, the same
    # call split into its three launches (q.k^T, p.V, reduce) is timed launch by launch.
    fused_wgs = ops.single_launch_workgroups(L, B, H, KV, S, D, T)
    names = {"qk": _native.PHASE_QK, "pv": _native.PHASE_PV, "reduce": _native.PHASE_REDUCE}
    three = {}
    for name, ph in names.items():
        three[name] = time_steps(torch, lambda r, ph=ph: multi_step(r, ph), args.steps, args.warmup,
                                 args.replicas) * 1e3
    if fused_wgs and args.mode == "multi":
        dom, dom_us, dom_bytes = "fused", ms * 1e3, bytes_step
    else:
        dom = max(("qk", "pv"), key=lambda n: three[n])
        dom_us, dom_bytes = three[dom], L * B * pb[dom]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9

    graph_leg = None
    if args.mode == "multi" and not args.no_graph_leg:
        build_graphs()
    if graphs:
        gms = time_graphs(args.steps, args.warmup)
        graph_leg = {"us_per_step": round(gms * 1e3, 2), "us_per_layer": round(gms * 1e3 / L, 3),
                     "GBps": round(bytes_step / (gms * 1e-3) / 1e9, 1),
                     "frac_of_peak": round(bytes_step / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "launches_per_step": L * (1 if ops.single_launch_workgroups(1, B, H, KV, S, D, T) else 3)}

    traffic, traffic_src = stamped_traffic(dom)

    if args.copy_probe:
        src = torch.empty(args.copy_probe << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    _progress("config 2 timed")
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
    configs = None
    if not args.no_suite:
        configs = suite(torch, dev, reps, time_steps, cpu=not args.no_cpu_baseline)

    line = {
        "metric": "decode-attn HBM GB/s (% of ~8 TB/s peak) + us/layer at 8K ctx, FP8-V cache",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_layer": round(ms * 1e3 / L, 3),
        "frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 K / fp8-e4m3 V, fp32 accumulate",
        "data": "synthetic N(0,1) K/V (quantized by the library's append kernel), seeded",
        "config": {"workload": "config 2: single-token decode attention, 28-layer Qwen2.5-1.5B-shaped "
                               "FP8-V paged cache, T=8192",
                   "batch": B, "q_heads": H, "kv_heads": KV, "head_dim": D, "seq_len": T, "layers": L,
                   "block_size": 16, "launch": args.mode, "cache_replicas_rotated": args.replicas,
                   "bytes_per_step": bytes_step, "parallelism": "none (1 GPU)"},
        "single_launch": {"workgroups": fused_wgs, "launches_per_step": 1 if fused_wgs else 3},
        "three_launch_us": {k: round(v, 3) for k, v in three.items()},
        "roofline": {"bound": "hbm", "kernel": f"{dom}_kernel (multi-layer call)", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": dom_bytes, "us_per_launch": round(dom_us, 3), "traffic": traffic,
                     "traffic_source": traffic_src},
        "per_layer_graph": graph_leg,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


def _progress(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _gbs(nbytes, us):
    return round(nbytes / (us * 1e-6) / 1e9, 1)


def _cpu_time(fn, budget_s):
    """Median seconds of fn() over a bounded sample (warm-up 1, at least 3 runs)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def suite(torch, dev, reps8k, time_steps, cpu=True):
    """The other BASELINE configurations on this GPU (and their CPU rows, briefly timed).

    Decode/verify rows reuse the 8K cache replicas (a shorter context reads the first blocks
    of the same scattered block table); the draft rows build 0.5B-shaped caches (14q/2kv,
    D=64, 24 layers); config 4 builds B=32 ragged sequences in a fragmented pool.  Each
    figure is us per call (GPU, graph replays over rotated inputs) and GB/s of algorithmic
    bytes.  "per_layer" rows are the engine's call pattern (one call per layer, in a graph).
    """
    from specdec_amd import workloads as wl
    from specdec_amd.engine.paged_cache import PagedKVCache
    from specdec_amd.kernels import ops

    out = {"note": "working_set_MB below ~256 MB can stay in the MI355X Infinity Cache, so such rows "
                   "are not HBM-bound"}

    def attn_rows(reps, L, H, KV, D, T, S, label, per_layer=True, steps=64):
        _progress(label)
        B = reps[0]["bt"].shape[0]
        qs = [torch.randn((L, B, H, S, D), device=dev).to(torch.bfloat16) for _ in reps]
        outs = [torch.empty_like(x) for x in qs]
        sls = [torch.full((B,), T, dtype=torch.int32, device=dev) if isinstance(T, int) else r["sl"] for r in reps]
        tmax = T if isinstance(T, int) else max(reps[0]["lens"])
        ws = ops.new_workspace(dev, ops.attention_workspace_bytes(L, B, H, KV, S, D, tmax))
        ws1 = ops.new_workspace(dev, ops.attention_workspace_bytes(1, B, H, KV, S, D, tmax))
        lens = [T] * B if isinstance(T, int) else reps[0]["lens"]
        nbytes = L * sum(wl.bytes_attn(t, S, H, KV, D) for t in lens)

        def multi(r):
            c = reps[r]["cache"]
            ops.paged_attention(qs[r], c.k_pages, c.v_pages, c.v_scales, reps[r]["bt"], sls[r], tmax,
                                out=outs[r], workspace_tensor=ws)

        def layers(r):
            c = reps[r]["cache"]
            for layer in range(L):
                kp, vp, vs = c.layer(layer)
                ops.paged_attention(qs[r][layer], kp, vp, vs, reps[r]["bt"], sls[r], tmax, out=outs[r][layer],
                                    workspace_tensor=ws1)

        us = time_steps(torch, multi, steps, 8, len(reps)) * 1e3
        row = {"layers": L, "batch": B, "q_len": S, "T": T if isinstance(T, int) else "ragged",
               "bytes": nbytes, "working_set_MB": round(len(reps) * nbytes / 1e6, 1),
               "us_per_call": round(us, 2), "us_per_layer": round(us / L, 3),
               "GBps": _gbs(nbytes, us), "single_launch_workgroups":
                   ops.single_launch_workgroups(L, B, H, KV, S, D, tmax)}
        if per_layer:
            usl = time_steps(torch, layers, 16, 4, len(reps)) * 1e3
            row["per_layer_calls_us_per_layer"] = round(usl / L, 3)
            row["per_layer_calls_GBps"] = _gbs(nbytes, usl)
        out[label] = row
        return row

    # config 0: one layer, T=2048, decode
    reps1 = [dict(cache=_LayerView(r["cache"], 0), bt=r["bt"], sl=r["sl"]) for r in reps8k]
    attn_rows(reps1, 1, H, KV, D, 2048, 1, "cfg0_one_layer_T2048", per_layer=False, steps=128)
    # config 3, target verify (S=5) at 2K/4K/8K over the 28-layer cache
    for t in (2048, 4096, 8192):
        attn_rows(reps8k, L, H, KV, D, t, 5, f"cfg3_verify_S5_T{t}")
    # config 3, draft chain: 5 sequential single-token decodes, 0.5B shape (14q/2kv, D=64, 24 layers)
    dH, dKV, dD, dL = wl.DRAFT["q_heads"], wl.DRAFT["kv_heads"], wl.DRAFT["head_dim"], wl.DRAFT["layers"]
    dreps = _build(torch, dev, dL, dKV, dD, [8192], 6, seed0=3000)
    for t in (2048, 4096, 8192):
        row = attn_rows(dreps, dL, dH, dKV, dD, t, 1, f"cfg3_draft_decode_T{t}")
        row["five_decodes_us"] = round(5 * row["per_layer_calls_us_per_layer"] * dL, 1)
    _progress("cfg3 chains")
    out["cfg3_draft_chain_5x24_T8192"] = chain_row(torch, dev, dreps, dL, dH, dKV, dD, 8192, 1, 5)
    out["cfg3_draft_chain_5x24_T8192_fused"] = chain_row(torch, dev, dreps, dL, dH, dKV, dD, 8192, 1, 5,
                                                         fused=True)
    del dreps
    out["cfg3_target_verify_step_28_T8192"] = chain_row(torch, dev, reps8k, L, H, KV, D, 8192, 5, 1)
    out["cfg3_target_verify_step_28_T8192_fused"] = chain_row(torch, dev, reps8k, L, H, KV, D, 8192, 5, 1,
                                                              fused=True)
    # config 4: B=32 ragged contexts U{2048..32768}, fragmented pool, 1% outlier channels x20
    lens = wl.ragged_lengths(32, 2048, 32768, seed=41)
    creps = _build(torch, dev, L, KV, D, lens, 1, seed0=4000, outliers=True)
    row = attn_rows(creps, L, H, KV, D, None, 1, "cfg4_batch32_ragged", steps=8)
    fp = creps[0]["cache"].footprint()
    row["mean_T"] = round(sum(lens) / len(lens))
    row["footprint"] = {"fp8v_bytes": fp["fp8v_bytes"], "bf16_bytes": fp["bf16_bytes"],
                        "saved_frac": round(fp["saved_frac"], 4), "scale_frac_of_fp8v": round(fp["scale_frac_of_fp8v"], 4)}
    del creps
    torch.cuda.empty_cache()

    # row f2: the engine's draft chain and verify block through the pack, eager and from a graph
    out["f2_engine_graph"] = engine_rows(torch, dev)

    # row f3: the reference's prefill chunk (2048 query rows over 8192 keys), target and draft
    out["f3_prefill_chunk_target_2048x8192"] = prefill_row(torch, dev, 12, 2, 128, 2048, 8192,
                                                           ref={"cudnn_sdpa_ms": 4.56, "cudnn_sdpa_transient_MiB": 74.1,
                                                                "eager_ms": 34.01, "eager_transient_MiB": 1998.1})
    out["f3_prefill_chunk_draft_2048x8192"] = prefill_row(torch, dev, 14, 2, 64, 2048, 8192,
                                                          ref={"cudnn_sdpa_ms": 4.12, "cudnn_sdpa_transient_MiB": 59.4,
                                                               "eager_ms": 38.54, "eager_transient_MiB": 2288.4})

    # config 1: fused quantize + append of a 2048-token chunk into 28 layers (V only, and with K)
    v1s, slots1, k1s, pages1 = [], None, [], []
    for r in range(4):
        v1, slots1, _ = wl.config1(seed=10 + r, device=dev)
        v1s.append(v1)
        k1s.append(torch.randn_like(v1, dtype=torch.float32).to(torch.bfloat16))
        pc = PagedKVCache(KV, D, num_layers=L, num_blocks=2048 // 16, device=dev, growable=False)
        pages1.append(pc)

    def qa(r, with_k):
        pc = pages1[r]
        ops.quant_append(v1s[r], slots1, pc.k_pages, pc.v_pages, pc.v_scales, k1s[r] if with_k else None)

    for with_k in (False, True):
        _progress(f"cfg1 quant_append with_k={with_k}")
        us = time_steps(torch, lambda r, w=with_k: qa(r, w), 64, 8, 4) * 1e3
        nb = L * wl.bytes_quant_append(2048, KV, D, with_k)
        out["cfg1_quant_append_2048x28" + ("_with_k" if with_k else "")] = {
            "bytes": nb, "us_per_call": round(us, 2), "GBps": _gbs(nb, us)}

    if cpu:
        _progress("cpu rows")
        out["cpu"] = cpu_rows(budget_s=2.0)
    return out


def prefill_row(torch, dev, h, kv, d, s, t, ref, nrep=2):
    """One layer's prefill-chunk attention: s query rows (the chunk's new tokens, already in the
    pages) over t keys with the offset-causal mask, q in the projection layout (B, S, H, D) as
    the engine pack passes it.  Reports time, MFMA rate and the call's transient device memory
    (workspace + output) beside the reference's measurement on its RTX 4060 Laptop
    (docs/data_ledger.md:1145-1152)."""
    from specdec_amd.engine.paged_cache import PagedKVCache
    from specdec_amd.kernels import ops

    _progress(f"prefill {h}/{kv}/{d} {s}x{t}")
    g = torch.Generator(device=dev)
    g.manual_seed(901)
    reps = []
    for r in range(nrep):
        c = PagedKVCache(kv, d, num_blocks=t // 16 + 8, device=dev, seed=902 + r, growable=False)
        c.prefill(0, torch.randn((t, kv, d), generator=g, device=dev).to(torch.bfloat16),
                  torch.randn((t, kv, d), generator=g, device=dev).to(torch.bfloat16), [t])
        q = torch.randn((1, s, h, d), generator=g, device=dev).to(torch.bfloat16)
        reps.append((c, q, torch.empty_like(q), c.block_table(), c.seq_lens_tensor()))
    nbytes = ops.attention_workspace_bytes(1, 1, h, kv, s, d, t)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    ws = ops.new_workspace(dev, nbytes)
    c0, q0, _, bt0, sl0 = reps[0]
    kp, vp, vs = c0.layer(0)
    o = ops.paged_attention(q0, kp, vp, vs, bt0, sl0, t, q_token_major=True, workspace_tensor=ws)
    torch.cuda.synchronize()
    transient = torch.cuda.max_memory_allocated(dev) - base
    del o

    def call(r):
        c, q, out, bt, sl = reps[r]
        kp, vp, vs = c.layer(0)
        ops.paged_attention(q, kp, vp, vs, bt, sl, t, q_token_major=True, out=out, workspace_tensor=ws)

    # 200 warm-up calls (about 50 ms): the GPU's clocks take tens of milliseconds of load to
    # ramp after the idle host work that builds the row's caches (with 4 warm-up calls the
    # timed calls read about 10% slower, with 64 about 4%)
    us = time_steps(torch, call, 64, 200, nrep) * 1e3
    keys = s * (t - s) + s * (s + 1) // 2          # visible (row token, key) pairs per head
    flops = 4 * h * keys * d                         # q.k^T and p.V, as the eager path computes them
    executed = 6 * h * keys * d                      # pass 1 recomputes q.k^T
    return {"q_heads": h, "kv_heads": kv, "head_dim": d, "q_rows": s, "keys": t, "us_per_call": round(us, 1),
            "launches": 2, "workspace_MiB": round(nbytes / 2 ** 20, 2),
            "transient_MiB_workspace_plus_output": round(transient / 2 ** 20, 2),
            "TFLOPs_algorithmic": round(flops / (us * 1e-6) / 1e12, 1),
            "TFLOPs_executed": round(executed / (us * 1e-6) / 1e12, 1),
            "reference_rtx4060": ref}


# ---------------------------------------------------------------------------- engine host for the pack
# The pack (specdec_amd.kernels.patch) replaces SelfAttention.forward of an engine module, as the
# reference's kernels/patch.py does for specdec.engine.model_self.  The rows below need a
# full-size host to record the engine's own steps: a Qwen2-shaped decoder (RMSNorm, rotate-half
# RoPE, biased q/k/v projections, SiLU-gated MLP, tied LM head) with random weights, built here;
# every attention call goes through the pack.
def _qwen_module(torch):
    import types

    nn = torch.nn
    F = torch.nn.functional
    mod = types.ModuleType("bench_qwen")

    class RMSNorm(nn.Module):
        def __init__(self, n):
            super().__init__()
            self.weight = nn.Parameter(torch.ones(n))

        def forward(self, x):
            xf = x.float()
            return self.weight * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype)

    def rope(head_dim, n, start, device, dtype):
        inv = 1.0 / (1e6 ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
        ang = torch.outer(torch.arange(start, start + n, device=device, dtype=torch.float32), inv)
        return torch.cat([ang.cos()] * 2, -1)[None, None].to(dtype), torch.cat([ang.sin()] * 2, -1)[None, None].to(dtype)

    def apply_rope(x, cos, sin):
        h = x.shape[-1] // 2
        return x * cos + torch.cat([-x[..., h:], x[..., :h]], -1) * sin

    class SelfAttention(nn.Module):
        def __init__(self, hidden, heads, kv, hd):
            super().__init__()
            self.q_proj = nn.Linear(hidden, heads * hd)
            self.k_proj = nn.Linear(hidden, kv * hd)
            self.v_proj = nn.Linear(hidden, kv * hd)
            self.o_proj = nn.Linear(heads * hd, hidden, bias=False)
            self.heads, self.kv_heads, self.head_dim, self.kv_format = heads, kv, hd, "v_fp8"

        def forward(self, x, cos, sin, cache=None):
            raise RuntimeError("install the fp8v pack")

    class Layer(nn.Module):
        def __init__(self, hidden, heads, kv, hd, inter):
            super().__init__()
            self.self_attn = SelfAttention(hidden, heads, kv, hd)
            self.input_layernorm, self.post_attention_layernorm = RMSNorm(hidden), RMSNorm(hidden)
            self.gate_proj = nn.Linear(hidden, inter, bias=False)
            self.up_proj = nn.Linear(hidden, inter, bias=False)
            self.down_proj = nn.Linear(inter, hidden, bias=False)

        def forward(self, x, cos, sin, cache):
            a, c = self.self_attn(self.input_layernorm(x), cos, sin, cache)
            x = x + a
            y = self.post_attention_layernorm(x)
            return x + self.down_proj(F.silu(self.gate_proj(y)) * self.up_proj(y)), c

    class Model(nn.Module):
        def __init__(self, vocab, hidden, heads, kv, hd, inter, layers):
            super().__init__()
            self.embed = nn.Embedding(vocab, hidden)
            self.layers = nn.ModuleList(Layer(hidden, heads, kv, hd, inter) for _ in range(layers))
            self.norm = RMSNorm(hidden)
            self.head_dim = hd

        def run(self, ids, cache):
            """Logits of ids (1, s) given the per-layer cache list (None: prefill)."""
            x = self.embed(ids)
            start = 0 if cache is None else cache[0]["k"].shape[2]
            cos, sin = rope(self.head_dim, ids.shape[1], start, x.device, x.dtype)
            new = []
            for i, layer in enumerate(self.layers):
                x, c = layer(x, cos, sin, None if cache is None else cache[i])
                new.append(c)
            return self.norm(x) @ self.embed.weight.T, new

    mod.SelfAttention, mod.apply_rope, mod.Model = SelfAttention, apply_rope, Model
    return mod


def engine_rows(torch, dev):
    """The engine's own speculative steps through the pack, eager and replayed from a HIP graph, at
    8K context: the draft chain (5 proposal steps of the 0.5B shape: hidden 896, 14/2/64, 24
    layers, vocab 151936) and the target verify block (5 rows of the 1.5B shape: hidden 1536,
    12/2/128, 28 layers), beside the reference's graph experiments (README.md:113-115:
    draft-chain speed-up 3.7-6.0x and verify 1.4-2.6x on its RTX 4060 Laptop, graph pools 2.0 /
    0.89 GiB).  Weights are random (no checkpoints offline); the contexts are prefilled through
    the pack in 2048-token chunks (the prefill kernels), then recorded at that fixed length."""
    from specdec_amd.kernels import patch

    mod = _qwen_module(torch)
    out = {}
    shapes = {"draft_chain_0p5B_5x24_T8192": (896, 14, 2, 64, 4864, 24, "propose"),
              "target_verify_1p5B_5rows_28L_T8192": (1536, 12, 2, 128, 8960, 28, "verify")}
    g = torch.Generator(device=dev)
    g.manual_seed(951)
    patch.install("fp8v", mod, scale_mode="rcp", capacity_tokens=8192 + 64, seed=17)
    try:
        for name, (hidden, heads, kv, hd, inter, layers, phase) in shapes.items():
            _progress(f"engine {name}")
            with torch.device(dev):
                model = mod.Model(151936, hidden, heads, kv, hd, inter, layers).to(torch.bfloat16).eval()
            with torch.no_grad():
                for prm in model.parameters():
                    if prm.dim() == 2:
                        prm.normal_(0.0, 1.0 / prm.shape[1] ** 0.5, generator=g)
                model.embed.weight.mul_(0.05)
            ids = torch.randint(0, 151936, (1, 8192), generator=g, device=dev)
            toks = torch.randint(0, 151936, (1, 5), generator=g, device=dev)
            with torch.no_grad():
                cache = None
                for c0 in range(0, 8192, 2048):
                    _, cache = model.run(ids[:, c0:c0 + 2048], cache)
                patch.reserve(cache, 8192 + 5)

            def step():
                view = [dict(layer) for layer in cache]
                with torch.no_grad():
                    if phase == "verify":
                        return model.run(toks, view)[0]
                    lg = None
                    for i in range(5):
                        lg, view = model.run(toks[:, i:i + 1], view)
                    return lg

            for _ in range(3):
                step()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            e0.record()
            for _ in range(reps):
                step()
            e1.record()
            torch.cuda.synchronize()
            eager_us = e0.elapsed_time(e1) * 1e3 / reps
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                step()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            # the graph's memory: the peak of what the recorded step allocated (activations and
            # logits; the cache is written in place, so nothing of it lands in the graph's pool).
            # Recording on the warmed-up side stream keeps the BLAS library's per-stream
            # workspace, made on that stream's first GEMM, out of the figure.
            alloc0 = torch.cuda.memory_allocated(dev)
            torch.cuda.reset_peak_memory_stats(dev)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                logits = step()
            torch.cuda.synchronize()
            pool_peak = torch.cuda.max_memory_allocated(dev) - alloc0
            pool_kept = torch.cuda.memory_allocated(dev) - alloc0
            graph.replay()
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            graph_us = e0.elapsed_time(e1) * 1e3 / reps
            out[name] = {"eager_us": round(eager_us, 1), "graph_us": round(graph_us, 1),
                         "speedup": round(eager_us / graph_us, 2),
                         "graph_pool_peak_MiB": round(pool_peak / 2 ** 20, 1),
                         "graph_outputs_MiB": round(pool_kept / 2 ** 20, 1),
                         "logits_shape": list(logits.shape),
                         "attention_calls": layers * (5 if phase == "propose" else 1),
                         "reference_rtx4060": {"graph_pool_GiB": 2.0 if phase == "propose" else 0.89,
                                               "speedup": "3.7-6.0x" if phase == "propose" else "1.4-2.6x"}}
            del graph, model, cache, logits
            torch.cuda.empty_cache()
    finally:
        patch.restore()
    return out


def chain_row(torch, dev, reps, layers, h, kv, d, T, s, steps, fused=False):
    """The engine's per-layer call pattern for `steps` speculative steps, in one HIP graph: per
    step and layer, kernel 1 appends the step's s new tokens (BF16 K copy and FP8 V) at the end
    of the context, then the layer's attention runs over it (T tokens after the last step).
    Draft chain: s=1, 5 steps; target verify: s=5, 1 step.  fused: both in one
    sdv_paged_attention_append call per layer (the single launch writes the new tokens)."""
    from specdec_amd import workloads as wl
    from specdec_amd.kernels import ops

    ws = ops.new_workspace(dev, ops.attention_workspace_bytes(1, 1, h, kv, s, d, T))
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    per = []
    for r in reps:
        c = r["cache"]
        k_new = torch.randn((steps, layers, s, kv, d), generator=g, device=dev).to(torch.bfloat16)
        v_new = torch.randn((steps, layers, s, kv, d), generator=g, device=dev).to(torch.bfloat16)
        q = torch.randn((steps, layers, 1, h, s, d), generator=g, device=dev).to(torch.bfloat16)
        out = torch.empty_like(q[0, 0])
        starts = [T - s * (steps - j) for j in range(steps)]
        slots = [c.slot_mapping([p0], s) for p0 in starts]
        lens = [torch.full((1,), p0 + s, dtype=torch.int32, device=dev) for p0 in starts]
        per.append((c, k_new, v_new, q, out, slots, lens, r["bt"]))

    def chain(ri):
        c, k_new, v_new, q, out, slots, lens, bt = per[ri]
        for j in range(steps):
            for layer in range(layers):
                kp, vp, vs = c.layer(layer)
                if fused:
                    ops.paged_attention(q[j, layer], kp, vp, vs, bt, lens[j], T, out=out, workspace_tensor=ws,
                                        append=(k_new[j, layer], v_new[j, layer], slots[j]))
                    continue
                ops.quant_append(v_new[j, layer], slots[j], kp, vp, vs, k_new[j, layer])
                ops.paged_attention(q[j, layer], kp, vp, vs, bt, lens[j], T, out=out, workspace_tensor=ws)

    # the graph-capture helper replays several chains per graph; keep the graph small
    us = _time_chain(torch, chain, len(reps))
    nbytes = steps * layers * (wl.bytes_attn(T, s, h, kv, d) + wl.bytes_quant_append(s, kv, d, True))
    return {"layers": layers, "steps": steps, "q_len": s, "T": T, "launches": (1 if fused else 2) * steps * layers,
            "us_per_chain": round(us, 1), "us_per_layer_step": round(us / (steps * layers), 3),
            "GBps": _gbs(nbytes, us)}


def _time_chain(torch, chain, nrep, replays=6):
    """Average us of chain(r): one HIP graph holding one chain per replica, replayed."""
    graph = torch.cuda.CUDAGraph()
    for r in range(nrep):
        chain(r)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for r in range(nrep):
            chain(r)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (replays * nrep)


class _LayerView:
    """One layer of a multi-layer cache, shaped as a 1-layer cache (views, no copy)."""

    def __init__(self, cache, layer):
        self.k_pages = cache.k_pages[layer:layer + 1]
        self.v_pages = cache.v_pages[layer:layer + 1]
        self.v_scales = cache.v_scales[layer:layer + 1]

    def layer(self, i):
        return self.k_pages[i], self.v_pages[i], self.v_scales[i]


def _build(torch, dev, layers, kv, d, lens, nrep, seed0, outliers=False):
    """Scattered paged caches for sequences of the given lengths (N(0,1) K/V, V quantized by the
    library's append kernel), one layer at a time to bound memory."""
    from specdec_amd import workloads as wl
    from specdec_amd.engine.paged_cache import PagedKVCache

    reps = []
    B = len(lens)
    nblocks = sum(-(-t // 16) for t in lens) + 64
    total = sum(lens)
    for r in range(nrep):
        g = torch.Generator(device=dev)
        g.manual_seed(seed0 + r)
        cache = PagedKVCache(kv, d, num_layers=layers, batch=B, num_blocks=nblocks, device=dev,
                             seed=seed0 + 100 + r, growable=False)
        mult = wl.outlier_mask(layers, kv, d, 0.01, g, dev) if outliers else None
        slots = None
        for layer in range(layers):
            k = torch.randn((total, kv, d), generator=g, device=dev).to(torch.bfloat16)
            v = torch.randn((total, kv, d), generator=g, device=dev)
            if mult is not None:
                v = v * mult[layer]
            slots = cache.prefill(layer, k, v.to(torch.bfloat16), lens, slots)
        reps.append(dict(cache=cache, bt=cache.block_table(), sl=cache.seq_lens_tensor(), lens=list(lens)))
    torch.cuda.synchronize()
    return reps


def cpu_rows(budget_s: float):
    """The reference path restated in torch-CPU (oracle) for configs 0, 1 and 3 (one layer each)."""
    import torch

    sys.path.insert(0, str(ROOT))
    from oracle import attention as oatt
    from oracle import quant as oq
    from specdec_amd import workloads as wl

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    rows = {"cores": n, "kind": "port", "budget_s_per_row": budget_s}
    g = wl.gen(11)
    for label, t, s in (("cfg0_one_layer_T2048", 2048, 1), ("cfg3_verify_S5_T8192_per_layer", 8192, 5)):
        k = wl.randn_bf16((1, KV, t - s, D), g)
        v = wl.randn_bf16((1, KV, t - s, D), g)
        _, cache = oatt.vfp8_decode_step(None, wl.randn_bf16((1, H, 1, D), g), k, v)
        q = wl.randn_bf16((1, H, s, D), g)
        kn = wl.randn_bf16((1, KV, s, D), g)
        vn = wl.randn_bf16((1, KV, s, D), g)
        med, nrun = _cpu_time(lambda: oatt.vfp8_decode_step(cache, q, kn, vn), budget_s)
        nbytes = wl.bytes_attn(t, s, H, KV, D)
        rows[label] = {"us": round(med * 1e6, 1), "GBps": round(nbytes / med / 1e9, 3), "runs": nrun}
    v1, _, _ = wl.config1(seed=10)
    med, nrun = _cpu_time(lambda: [oq.quantize_kv_fp8(v1[layer], D) for layer in range(L)], budget_s)
    nb = L * wl.bytes_quant_append(2048, KV, D, False)
    rows["cfg1_quant_2048x28"] = {"us": round(med * 1e6, 1), "GBps": round(nb / med / 1e9, 3), "runs": nrun}
    return rows


def cpu_baseline(budget_s: float):
    """The reference path restated in torch-CPU (oracle), one 8K layer per sample, timed here."""
    import torch

    sys.path.insert(0, str(ROOT))
    from oracle import attention as oatt
    from specdec_amd import workloads as wl

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    g = wl.gen(7)
    k = wl.randn_bf16((1, KV, T - 1, D), g)
    v = wl.randn_bf16((1, KV, T - 1, D), g)
    _, cache = oatt.vfp8_decode_step(None, wl.randn_bf16((1, H, 1, D), g), k, v)  # cache of T-1 tokens
    q = wl.randn_bf16((1, H, 1, D), g)
    kn = wl.randn_bf16((1, KV, 1, D), g)
    vn = wl.randn_bf16((1, KV, 1, D), g)
    oatt.vfp8_decode_step(cache, q, kn, vn)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        oatt.vfp8_decode_step(cache, q, kn, vn)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    per_layer_bytes = wl.bytes_attn(T, S, H, KV, D)
    cpu_name = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(per_layer_bytes / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "us_per_layer": round(med * 1e6, 1),
            "sample": f"{len(times)} single-layer 8K v_fp8 decode steps (quantize current V, cat K, dequantize + "
                      f"cat V, kv_repeat, BF16 eager attention, append) in torch-CPU, median; a 28-layer step "
                      f"is 28x this", "cpu": cpu_name, "torch": torch.__version__}


if __name__ == "__main__":
    main()
