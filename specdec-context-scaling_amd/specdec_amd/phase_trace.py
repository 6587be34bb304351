"""Per-phase timeline of the single-launch decode/verify attention, workgroup by workgroup.

The single launch (csrc/sdv_attn.hip, fused_kernel) runs q.k^T, a statistics exchange, p.V, a
partial exchange and the output sum in one kernel; its time per call splits into those phases.
A trace build of the same sources (``python -m specdec_amd.build --trace`` ->
specdec_amd/libsdv_trace.so, compiled with SDV_PHASE_TRACE) has thread 0 of every workgroup
stamp the GPU's 100 MHz wall clock at ten phase boundaries.  This module installs that build as
the process's library, records each workload's call (four cache replicas in turn, so the pages
are not still in the last-level cache from the previous call) into a HIP graph, replays it and
reads the stamps of the last call, and prints, per phase boundary, the minimum, median and
maximum over workgroups of the time since the first workgroup started (the median over
replays, in microseconds).

    python -m specdec_amd.phase_trace [--replays 8] [--workloads one_layer_decode,...]

Workloads (the Qwen2.5-1.5B attention shape, 12 query / 2 KV heads of 128, T = 8192):
one_layer_decode (an engine decode call), one_layer_verify (S=5), multi_layer_decode (all 28
layers in one call, the headline), multi_layer_verify (S=5); and the 0.5B draft's shape (14 / 2
heads of 64): draft_one_layer_decode, draft_multi_layer_decode (24 layers).
"""
from __future__ import annotations

import argparse
import ctypes

import numpy as np
import torch

from . import _native, build
from .engine.paged_cache import PagedKVCache
from .kernels import ops

PHASES = ("start", "block table + append done", "q.k^T done", "statistics published",
          "group statistics read", "p.V done", "partial published", "owner polls + output sums done",
          "output written", "end")
SLOTS = 16          # stamp words per workgroup (kPhaseSlots)
MAX_GROUPS = 4096   # workgroups traced (kPhaseTraceGroups)
TICK_US = 0.01      # wall clock at 100 MHz

WORKLOADS = {
    # name: (layers in the call, q_heads, kv_heads, head_dim, q_len, T)
    "one_layer_decode": (1, 12, 2, 128, 1, 8192),
    "one_layer_verify": (1, 12, 2, 128, 5, 8192),
    "multi_layer_decode": (28, 12, 2, 128, 1, 8192),
    "multi_layer_verify": (28, 12, 2, 128, 5, 8192),
    "draft_one_layer_decode": (1, 14, 2, 64, 1, 8192),
    "draft_multi_layer_decode": (24, 14, 2, 64, 1, 8192),
}


def _install_trace_library() -> ctypes.CDLL:
    lib = _native.load(build.TRACE_LIB_PATH, make_default=True)
    lib.sdv_phase_trace_read.restype = ctypes.c_int
    lib.sdv_phase_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    return lib


def _replica(dev, layers, kv, d, t, h, s, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    cache = PagedKVCache(kv, d, num_layers=layers, num_blocks=t // 16 + 64, device=dev, seed=seed,
                         growable=False)
    cache.reserve(0, t)
    slots = cache.slot_mapping([0], t)
    k = torch.randn((layers, t, kv, d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((layers, t, kv, d), generator=g, device=dev).to(torch.bfloat16)
    ops.quant_append(v, slots, cache.k_pages, cache.v_pages, cache.v_scales, k)
    cache.lengths[0] = t
    q = torch.randn((layers, 1, h, s, d), generator=g, device=dev).to(torch.bfloat16)
    return dict(cache=cache, q=q if layers > 1 else q[0], bt=cache.block_table(), sl=cache.seq_lens_tensor(),
                out=torch.empty_like(q if layers > 1 else q[0]))


def trace(lib, dev, name, replays=8, n_rep=4):
    """Median-over-replays stamps (groups, 10) in microseconds for one workload."""
    layers, h, kv, d, s, t = WORKLOADS[name]
    grid = ops.single_launch_workgroups(layers, 1, h, kv, s, d, t)
    if grid == 0 or grid > MAX_GROUPS:
        raise _native.SdvError(f"{name}: not a single-launch shape ({grid} workgroups)")
    reps = [_replica(dev, layers, kv, d, t, h, s, 4100 + r) for r in range(n_rep)]
    ws = ops.new_workspace(dev, ops.attention_workspace_bytes(layers, 1, h, kv, s, d, t))

    def call(r):
        rep = reps[r]
        c = rep["cache"]
        if layers > 1:
            kp, vp, vs = c.k_pages, c.v_pages, c.v_scales
        else:
            kp, vp, vs = c.layer(0)
        ops.paged_attention(rep["q"], kp, vp, vs, rep["bt"], rep["sl"], t, out=rep["out"], workspace_tensor=ws)

    call(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for r in range(n_rep):
            call(r)
    buf = np.zeros(grid * SLOTS, dtype=np.uint64)
    samples = []
    for _ in range(replays):
        graph.replay()
        torch.cuda.synchronize()
        _native.check(lib.sdv_phase_trace_read(buf.ctypes.data, buf.size), "sdv_phase_trace_read")
        st = buf.reshape(grid, SLOTS)[:, :len(PHASES)].astype(np.float64)
        samples.append((st - st[:, 0].min()) * TICK_US)
    ops.check_workspace(ws)
    del graph, reps
    torch.cuda.empty_cache()
    return grid, np.median(np.stack(samples), axis=0)


def table(name, grid, med) -> str:
    layers, h, kv, d, s, t = WORKLOADS[name]
    lines = [f"### {name}: {layers} layer(s), {h}/{kv} heads of {d}, S={s}, T={t}; {grid} workgroups",
             "", "| phase boundary | min µs | median µs | max µs |", "|---|---|---|---|"]
    for k, nm in enumerate(PHASES):
        col = med[:, k]
        lines.append(f"| {nm} | {col.min():.2f} | {np.median(col):.2f} | {col.max():.2f} |")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--replays", type=int, default=8)
    ap.add_argument("--workloads", default=",".join(WORKLOADS))
    args = ap.parse_args(argv)
    lib = _install_trace_library()
    dev = torch.device("cuda:0")
    for name in args.workloads.split(","):
        print(f"[phase_trace] {name}", flush=True)
        grid, med = trace(lib, dev, name, args.replays)
        print(table(name, grid, med), "\n", flush=True)


if __name__ == "__main__":
    main()
