"""Torch-facing operators of the FP8-V path (mirror of specdec/kernels/ops.py).

torch is plumbing here: tensors provide device memory and the current HIP stream; every
computation runs in libsdv's gfx950 kernels through the C ABI (include/sdv.h).  Argument
problems raise ``RuntimeError`` (:class:`specdec_amd.SdvError`), the way the reference
op's TORCH_CHECKs do (specdec/kernels/cuda/attention.cu:245-262); an unknown backend raises
``ValueError`` as in specdec/kernels/ops.py:76.

Operators
---------
``quant_append``      kernel 1: V -> FP8 (per token and KV head max-abs/448 scale) plus the
                      BF16 K copy, written into page slots.
``paged_attention``   kernels 2/3: GQA decode / k+1-row verify over BF16 K + FP8 V pages.
``attention``         the reference op's signature ``attention(q, k, v, backend)``
                      (ops.py:67-76) over a contiguous v_fp8 cache: k BF16 (B,KV,T,D) and
                      v given as the (payload, scale) pair the engine stores.
``fp8_encode``        elementwise fp32 -> E4M3FN on the device.
"""
from __future__ import annotations

import ctypes
import functools
import os
import weakref

import torch

from .. import _native
from .._native import SdvError

BLOCK = _native.BLOCK_SIZE
_SCALE_MODES = {"div": _native.SCALE_DIV, "rcp": _native.SCALE_RCP}
_BACKENDS = ("hip", "cuda")  # "cuda" is what reference call sites pass (patch.py:107)

_WORKSPACES: dict = {}
# Cached workspaces replaced by larger ones that a call recorded into a HIP graph used (the
# graph still points at them).  A replacement is at least twice the size of the buffer it
# replaces, so these hold at most as many bytes as the current workspace of their stream.
_RETIRED: list = []
_RECORDED = weakref.WeakSet()  # cached workspaces handed to a call while its stream was recording
_READY: dict = {}  # id(tensor) -> weakref of workspaces whose sync prefix is known to be zero
# SDV_CHECK_SYNC=1: every paged_attention call reads its workspace's failure count afterwards
# and raises SdvError when a single-launch wait expired (synchronises; a debugging aid)
_CHECK_SYNC = os.environ.get("SDV_CHECK_SYNC", "0") not in ("", "0")


def _fail(msg: str):
    raise SdvError(msg, _native.SDV_ERR_SHAPE)


# The eager engine calls these operators once per layer and step, so their host cost is part of
# every decoded token: pointers go to ctypes as plain ints (the argtypes are c_void_p), the
# current stream comes from torch's raw query when it has one, and workspace sizes are cached.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


def _p(t):
    return t.data_ptr() if t is not None else None


def _need(t, name, dtypes, dev=None, ndim=None):
    if not isinstance(t, torch.Tensor):
        _fail(f"{name} must be a tensor")
    if not t.is_cuda:
        _fail(f"{name} must be on a HIP device (got {t.device})")
    if dev is not None and t.device != dev:
        _fail(f"{name} is on {t.device}, expected {dev}")
    if t.dtype not in dtypes:
        _fail(f"{name} must have dtype in {dtypes} (got {t.dtype})")
    if not t.is_contiguous():
        _fail(f"{name} must be contiguous")
    if ndim is not None and t.dim() not in ndim:
        _fail(f"{name} must have {ndim} dims (got {tuple(t.shape)})")


def _pages_dims(k_pages, v_pages, v_scales, layered: bool):
    lead = 1 if layered else 0
    if k_pages.dim() != 5 + lead or v_pages.dim() != 4 + lead or v_scales.dim() != 3 + lead:
        _fail(f"page tensors must be (..., num_blocks, KV, D/8, 16, 8) / (..., num_blocks, KV, D, 16) / "
              f"(..., num_blocks, KV, 16); got {tuple(k_pages.shape)}, {tuple(v_pages.shape)}, "
              f"{tuple(v_scales.shape)}")
    nb, kv, dc, blk, eight = k_pages.shape[lead:]
    d = dc * 8
    if blk != BLOCK or eight != 8 or tuple(v_pages.shape[lead:]) != (nb, kv, d, BLOCK) or \
            tuple(v_scales.shape[lead:]) != (nb, kv, BLOCK):
        _fail(f"page shapes disagree: k {tuple(k_pages.shape)}, v {tuple(v_pages.shape)}, s {tuple(v_scales.shape)}")
    if layered and not (k_pages.shape[0] == v_pages.shape[0] == v_scales.shape[0]):
        _fail("page tensors disagree on the layer count")
    return nb, kv, d


def new_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A fresh uint8 workspace of at least nbytes whose synchronisation prefix is zeroed
    (sdv_attention_workspace_init on the current stream)."""
    dev = torch.device(device)
    ws = torch.empty(max(int(nbytes), _native.SYNC_BYTES), dtype=torch.uint8, device=dev)
    _init_workspace(ws)
    return ws


def _init_workspace(ws: torch.Tensor) -> None:
    _native.check(_native.load().sdv_attention_workspace_init(_p(ws), ws.numel(), _stream(ws.device)),
                  "sdv_attention_workspace_init")
    key = id(ws)
    _READY[key] = weakref.ref(ws, lambda _r, key=key: _READY.pop(key, None))


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A cached uint8 workspace of at least nbytes on (device, current stream).

    A cached buffer that is too small is replaced by one at least twice its size.  The old
    buffer is freed, unless a call recorded into a HIP graph used it: the graph still points
    at it, so it is kept alive (at most the current buffer's size in all, by the doubling).
    Callers that record graphs should rather pass their own buffer (``workspace_tensor``)
    and keep it for the graph's lifetime.
    """
    dev = torch.device(device)
    key = (dev, _stream(dev))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        grow = 0
        if ws is not None:
            grow = 2 * ws.numel()
            if ws in _RECORDED:
                _RETIRED.append(ws)
        ws = new_workspace(dev, max(nbytes, grow, 1 << 20))
        _WORKSPACES[key] = ws
    if torch.cuda.is_current_stream_capturing():
        _RECORDED.add(ws)
    return ws


def single_launch_workgroups(num_layers: int, batch: int, q_heads: int, kv_heads: int, q_len: int, head_dim: int,
                             max_seq_len: int) -> int:
    """Workgroups of the single-launch kernel for these sizes on the current device, or 0
    when paged_attention takes the three-launch path."""
    return int(_native.load().sdv_attention_single_launch(num_layers, batch, q_heads, kv_heads, q_len, head_dim,
                                                           max_seq_len))


def _ws_args(ws: torch.Tensor | None):
    """(pointer, bytes, stream) of a workspace; None: the current device's no-allocation scratch
    (the workspace of sdv_paged_attention_noalloc), which the library names by a NULL pointer."""
    if ws is None:
        return None, 0, _stream(torch.device("cuda", torch.cuda.current_device()))
    return _p(ws), ws.numel(), _stream(ws.device)


def workspace_status(ws: torch.Tensor | None = None) -> tuple[int, bool]:
    """(failures, poisoned) of a workspace (sdv_attention_workspace_status; synchronises the
    current stream): failures = expired waits and refused calls of the single-launch path
    since the workspace was initialised; poisoned = graph-recorded calls are being refused
    until reset_workspace().  ws None: the no-allocation entry point's scratch on the current
    device."""
    fail, poison = ctypes.c_uint32(0), ctypes.c_uint32(0)
    ptr, n, st = _ws_args(ws)
    _native.check(_native.load().sdv_attention_workspace_status(ptr, n, ctypes.byref(fail), ctypes.byref(poison), st),
                  "sdv_attention_workspace_status")
    return int(fail.value), bool(poison.value)


def sync_errors(ws: torch.Tensor | None = None) -> int:
    """Expired waits and refused calls of the single-launch path recorded in a workspace
    (synchronises)."""
    return workspace_status(ws)[0]


def check_workspace(ws: torch.Tensor | None = None) -> None:
    """Raise SdvError when a single-launch call on this workspace could not complete (its
    outputs hold NaN where it failed); the reference raises every error (model_self.py:331-332).
    ws None: the no-allocation entry point's scratch on the current device."""
    fail, poison = workspace_status(ws)
    if fail or poison:
        raise SdvError(f"single-launch attention: {fail} wait(s) expired or call(s) refused on this workspace"
                       f"{' (graph-recorded calls poisoned)' if poison else ''}; outputs of the failed calls are NaN. "
                       f"Call ops.reset_workspace() before recording new graphs on it", _native.SDV_ERR_HIP)


def reset_workspace(ws: torch.Tensor | None = None) -> None:
    """Zero a workspace's synchronisation area (clears the failure count and the graph poison).
    ws None: the no-allocation entry point's scratch on the current device."""
    if ws is not None:
        _init_workspace(ws)
        return
    ptr, n, st = _ws_args(None)
    _native.check(_native.load().sdv_attention_workspace_init(ptr, n, st), "sdv_attention_workspace_init")


def set_wait_limit(polls: int) -> None:
    """Bound of the single launch's cross-workgroup waits for later calls (0: the default);
    tests use a tiny bound to drive the failure path."""
    _native.check(_native.load().sdv_attention_set_wait_limit(int(polls)), "sdv_attention_set_wait_limit")


@functools.lru_cache(maxsize=256)
def attention_workspace_bytes(num_layers: int, batch: int, q_heads: int, kv_heads: int, q_len: int,
                              head_dim: int, max_seq_len: int) -> int:
    n = _native.load().sdv_attention_workspace_size(num_layers, batch, q_heads, kv_heads, q_len,
                                                    head_dim, max_seq_len)
    if n == 0:
        _fail(f"unsupported attention sizes L={num_layers} B={batch} H={q_heads} KV={kv_heads} "
              f"S={q_len} D={head_dim} T={max_seq_len}")
    return int(n)


def quant_append(v_new: torch.Tensor, slot_mapping: torch.Tensor, k_pages: torch.Tensor,
                 v_pages: torch.Tensor, v_scales: torch.Tensor, k_new: torch.Tensor | None = None,
                 *, scale_mode: str = "div", tile_starts: torch.Tensor | None = None) -> None:
    """Quantize V to FP8 and write V (and BF16 K when given) into page slots, in place.

    v_new/k_new: BF16 (n_tokens, KV, D), or (L, n_tokens, KV, D) with layered pages.
    slot_mapping: int32 (n_tokens,), slot = block * 16 + offset, negative = skip.
    Pages: k (…, num_blocks, KV, D/8, 16, 8) BF16; v (…, num_blocks, KV, D, 16) uint8 or
    float8_e4m3fn; scales (…, num_blocks, KV, 16) fp32.
    tile_starts: optional int32 (n_tiles + 1,) on the device: tile i is rows
    [tile_starts[i], min(tile_starts[i] + 16, tile_starts[i+1])) (see varlen_tile_starts).
    """
    lib = _native.load()
    _need(v_new, "v_new", (torch.bfloat16,), ndim=(3, 4))
    dev = v_new.device
    layered = v_new.dim() == 4
    _need(k_pages, "k_pages", (torch.bfloat16,), dev)
    _need(v_pages, "v_pages", (torch.uint8, torch.float8_e4m3fn), dev)
    _need(v_scales, "v_scales", (torch.float32,), dev)
    _need(slot_mapping, "slot_mapping", (torch.int32,), dev, ndim=(1,))
    nb, kv, d = _pages_dims(k_pages, v_pages, v_scales, layered)
    L = v_new.shape[0] if layered else 1
    n_tokens = v_new.shape[-3]
    if tuple(v_new.shape[-2:]) != (kv, d) or slot_mapping.shape[0] != n_tokens:
        _fail(f"v_new {tuple(v_new.shape)} / slot_mapping {tuple(slot_mapping.shape)} do not match "
              f"pages (KV={kv}, D={d})")
    if layered and k_pages.shape[0] != L:
        _fail(f"v_new has {L} layers, pages have {k_pages.shape[0]}")
    if k_new is not None:
        _need(k_new, "k_new", (torch.bfloat16,), dev)
        if k_new.shape != v_new.shape:
            _fail(f"k_new {tuple(k_new.shape)} != v_new {tuple(v_new.shape)}")
    if scale_mode not in _SCALE_MODES:
        raise ValueError(f"scale_mode must be one of {sorted(_SCALE_MODES)}")
    # the kernel moves 16-byte pieces of each row; a view starting mid-row is copied first
    if v_new.data_ptr() % 16:
        v_new = v_new.clone()
    if k_new is not None and k_new.data_ptr() % 16:
        k_new = k_new.clone()
    per = lambda t: t[0].numel() if layered else 0  # noqa: E731  (elements per layer)
    if tile_starts is None:
        st = lib.sdv_quant_append(_p(v_new), _p(k_new), _p(slot_mapping), n_tokens, kv, d, d, L,
                                  per(v_new), _p(k_pages), _p(v_pages), _p(v_scales), nb,
                                  per(k_pages), per(v_pages), per(v_scales), _SCALE_MODES[scale_mode],
                                  _stream(dev))
        _native.check(st, "sdv_quant_append")
        return
    _need(tile_starts, "tile_starts", (torch.int32,), dev, ndim=(1,))
    if tile_starts.shape[0] < 1:
        _fail("tile_starts needs n_tiles + 1 entries")
    st = lib.sdv_quant_append_tiles(_p(v_new), _p(k_new), _p(slot_mapping), n_tokens, kv, d, d, L,
                                    per(v_new), _p(k_pages), _p(v_pages), _p(v_scales), nb,
                                    per(k_pages), per(v_pages), per(v_scales), _SCALE_MODES[scale_mode],
                                    _p(tile_starts), tile_starts.shape[0] - 1, _stream(dev))
    _native.check(st, "sdv_quant_append_tiles")


def varlen_tile_starts(lengths: list[int], starts: list[int] | None = None) -> list[int]:
    """Tile table for a packed varlen input of sequences with `lengths` tokens whose first token
    lands at position `starts[b]` of its sequence (0: a whole prompt): tiles break where a page
    block begins, so every whole block is one tile.  n_tiles + 1 entries; the last is the
    total row count."""
    starts = starts or [0] * len(lengths)
    out, row = [], 0
    for n, p0 in zip(lengths, starts):
        if n < 0 or p0 < 0:
            raise ValueError("negative length or start position")
        i = 0
        while i < n:
            step = min(n - i, 16 - (p0 + i) % 16)
            out.append(row + i)
            i += step
        row += n
    out.append(row)
    return out


def paged_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, v_scales: torch.Tensor,
                    block_table: torch.Tensor, seq_lens: torch.Tensor, max_seq_len: int, *,
                    q_token_major: bool = False, out: torch.Tensor | None = None,
                    workspace_tensor: torch.Tensor | None = None,
                    phases: int = _native.PHASE_ALL,
                    append: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
                    scale_mode: str = "div") -> torch.Tensor:
    """GQA attention of q over paged BF16 K / FP8 V.

    q: BF16 (B, H, S, D) (or (B, S, H, D) with q_token_major=True); a leading layer dimension
    (L, ...) processes L layers in one launch with layered pages (L, num_blocks, ...).
    block_table int32 (B, max_blocks); seq_lens int32 (B,) = context length including the S
    new tokens, each <= max_seq_len, or None: every sequence has max_seq_len tokens (nothing
    to copy to the device, so the call can be recorded into a HIP graph).  Returns out shaped
    like q (BF16).
    ``phases`` (profiling) runs a subset of the three launches; see sdv_paged_attention_phases.
    ``append`` = (k_new, v_new, slot_mapping): first write the S new tokens of every sequence
    into the pages (as quant_append with ``scale_mode`` would; k_new/v_new BF16 (B*S, KV, D),
    or (L, B*S, KV, D) with layers, token b*S + i at position seq_lens[b] - S + i), in the same
    call (sdv_paged_attention_append); slot_mapping None takes each token's slot from the block
    table on the device.
    """
    lib = _native.load()
    _need(q, "q", (torch.bfloat16,), ndim=(4, 5))
    dev = q.device
    layered = q.dim() == 5
    _need(k_pages, "k_pages", (torch.bfloat16,), dev)
    _need(v_pages, "v_pages", (torch.uint8, torch.float8_e4m3fn), dev)
    _need(v_scales, "v_scales", (torch.float32,), dev)
    _need(block_table, "block_table", (torch.int32,), dev, ndim=(2,))
    if seq_lens is not None:
        _need(seq_lens, "seq_lens", (torch.int32,), dev, ndim=(1,))
    nb, kv, d = _pages_dims(k_pages, v_pages, v_scales, layered)
    L = q.shape[0] if layered else 1
    if layered and k_pages.shape[0] != L:
        _fail(f"q has {L} layers, pages have {k_pages.shape[0]}")
    if q_token_major:
        B, S, H, Dq = q.shape[-4:]
    else:
        B, H, S, Dq = q.shape[-4:]
    if Dq != d or H % kv:
        _fail(f"q {tuple(q.shape)} does not match pages (KV={kv}, D={d})")
    if block_table.shape[0] != B or (seq_lens is not None and seq_lens.shape[0] != B):
        _fail(f"block_table {tuple(block_table.shape)} / seq_lens "
              f"{None if seq_lens is None else tuple(seq_lens.shape)} need batch {B}")
    max_seq_len = int(max_seq_len)
    if max_seq_len <= 0 or block_table.shape[1] * BLOCK < max_seq_len:
        _fail(f"max_seq_len {max_seq_len} must be in [1, 16 * max_blocks = {block_table.shape[1] * BLOCK}]")
    if out is None:
        out = torch.empty_like(q)
    else:
        _need(out, "out", (torch.bfloat16,), dev)
        if out.shape != q.shape:
            _fail(f"out {tuple(out.shape)} != q {tuple(q.shape)}")
    nbytes = attention_workspace_bytes(L, B, H, kv, S, d, max_seq_len)
    if workspace_tensor is None:
        workspace_tensor = workspace(dev, nbytes)
    else:
        _need(workspace_tensor, "workspace_tensor", (torch.uint8,), dev)
        if workspace_tensor.numel() < nbytes:
            _fail(f"workspace_tensor holds {workspace_tensor.numel()} bytes, {nbytes} needed")
        ref = _READY.get(id(workspace_tensor))
        if ref is None or ref() is not workspace_tensor:  # a caller's own buffer: zero its sync prefix once
            _init_workspace(workspace_tensor)
    per = lambda t: t[0].numel() if layered else 0  # noqa: E731
    args = (_p(q), _p(k_pages), _p(v_pages), _p(v_scales), nb, per(k_pages), per(v_pages), per(v_scales),
            _p(block_table), block_table.shape[1], _p(seq_lens), L, B, H, kv, S, d, max_seq_len,
            int(bool(q_token_major)), _p(workspace_tensor), workspace_tensor.numel(), _p(out), _stream(dev))
    if append is not None:
        if phases != _native.PHASE_ALL:
            raise ValueError("append runs with the whole call (phases=PHASE_ALL)")
        if scale_mode not in _SCALE_MODES:
            raise ValueError(f"scale_mode must be one of {sorted(_SCALE_MODES)}")
        k_new, v_new, slots = append
        want = ((L,) if layered else ()) + (B * S, kv, d)
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            _need(t, name, (torch.bfloat16,), dev)
            if tuple(t.shape) != want:
                _fail(f"{name} {tuple(t.shape)} != {want}")
        if slots is not None:
            _need(slots, "slot_mapping", (torch.int32,), dev, ndim=(1,))
            if slots.shape[0] != B * S:
                _fail(f"slot_mapping {tuple(slots.shape)} needs {B * S} entries")
        if k_new.data_ptr() % 16:
            k_new = k_new.clone()
        if v_new.data_ptr() % 16:
            v_new = v_new.clone()
        st = lib.sdv_paged_attention_append(*args[:-1], _p(k_new), _p(v_new), _p(slots), per(v_new),
                                            _SCALE_MODES[scale_mode], args[-1])
        _native.check(st, "sdv_paged_attention_append")
        if _CHECK_SYNC:
            check_workspace(workspace_tensor)
        return out
    if phases == _native.PHASE_ALL:
        st = lib.sdv_paged_attention(*args)
    else:
        st = lib.sdv_paged_attention_phases(*args, int(phases))
    _native.check(st, "sdv_paged_attention")
    if _CHECK_SYNC:
        check_workspace(workspace_tensor)
    return out


def pack_contiguous(k: torch.Tensor, v_payload: torch.Tensor, v_scale: torch.Tensor):
    """Copy a contiguous v_fp8 cache (B,KV,T,D) into pages (one copy; block b*nbps + j is
    tokens 16j.. of sequence b).  Returns (k_pages, v_pages, v_scales, block_table, seq_lens)."""
    B, KV, T, D = k.shape
    nbps = -(-T // BLOCK)
    Tp = nbps * BLOCK
    pad = Tp - T
    kk = torch.nn.functional.pad(k, (0, 0, 0, pad)) if pad else k
    vv = v_payload.view(torch.uint8)
    vv = torch.nn.functional.pad(vv, (0, 0, 0, pad)) if pad else vv
    ss = v_scale.reshape(B, KV, T)
    ss = torch.nn.functional.pad(ss, (0, pad), value=1.0) if pad else ss
    k_pages = (kk.reshape(B, KV, nbps, BLOCK, D // 8, 8).permute(0, 2, 1, 4, 3, 5)
               .reshape(B * nbps, KV, D // 8, BLOCK, 8).contiguous())
    v_pages = vv.reshape(B, KV, nbps, BLOCK, D).permute(0, 2, 1, 4, 3).reshape(B * nbps, KV, D, BLOCK).contiguous()
    v_scales = ss.reshape(B, KV, nbps, BLOCK).permute(0, 2, 1, 3).reshape(B * nbps, KV, BLOCK).contiguous()
    block_table = torch.arange(B * nbps, dtype=torch.int32, device=k.device).reshape(B, nbps)
    seq_lens = torch.full((B,), T, dtype=torch.int32, device=k.device)
    return k_pages, v_pages, v_scales, block_table, seq_lens


def attention(q: torch.Tensor, k: torch.Tensor, v, backend: str = "hip") -> torch.Tensor:
    """Reference op signature (specdec/kernels/ops.py:67-76) for the v_fp8 cache format.

    q (B,H,S,D) BF16; k (B,KV,T,D) BF16; v = (payload float8_e4m3fn (B,KV,T,D),
    scale fp32 (B,KV,T,1)) exactly as the reference cache stores it.  The FP8 payload is
    dequantized inside the kernel; row i of the S-row block sees keys j <= T - S + i.
    """
    if backend not in _BACKENDS:
        raise ValueError(backend)
    if isinstance(v, torch.Tensor):
        raise SdvError("the FP8-V backend needs v as (payload float8_e4m3fn, scale fp32); "
                       "BF16 V is the reference's 'fp16' cache format, which this library does not serve",
                       _native.SDV_ERR_UNSUPPORTED)
    payload, scale = v
    _need(q, "q", (torch.bfloat16,), ndim=(4,))
    _need(k, "k", (torch.bfloat16,), q.device, ndim=(4,))
    if payload.shape != k.shape or tuple(scale.shape) != tuple(k.shape[:3]) + (1,):
        _fail(f"v payload {tuple(payload.shape)} / scale {tuple(scale.shape)} do not match k {tuple(k.shape)}")
    kp, vp, vs, bt, sl = pack_contiguous(k.contiguous(), payload.contiguous(), scale.contiguous())
    return torch.ops.sdv.paged_attention(q.contiguous(), kp, vp, vs, bt, sl, k.shape[2])


def fp8_encode(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> uint8 E4M3FN codes (RNE; NaN beyond 464), computed on the device."""
    _need(x, "x", (torch.float32,))
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _native.check(_native.load().sdv_fp8_encode(_p(x), _p(out), x.numel(), _stream(x.device)), "sdv_fp8_encode")
    return out


# ---------------------------------------------------------------------------- torch.library
# The ops as torch custom operators (namespace "sdv"), so torch.compile and fake-tensor tracing
# see them: the real implementations are the functions above (the C ABI through ctypes); the
# fake implementations only produce outputs of the right shape and dtype.  The page tensors of
# the appending ops are declared mutated.
@torch.library.custom_op("sdv::paged_attention", mutates_args=())
def _lib_paged_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, v_scales: torch.Tensor,
                         block_table: torch.Tensor, seq_lens: torch.Tensor | None, max_seq_len: int,
                         q_token_major: bool = False) -> torch.Tensor:
    return paged_attention(q, k_pages, v_pages, v_scales, block_table, seq_lens, max_seq_len,
                           q_token_major=q_token_major)


@_lib_paged_attention.register_fake
def _(q, k_pages, v_pages, v_scales, block_table, seq_lens, max_seq_len, q_token_major=False):
    return torch.empty_like(q)


@torch.library.custom_op("sdv::paged_attention_append", mutates_args=("k_pages", "v_pages", "v_scales"))
def _lib_paged_attention_append(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                                v_scales: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor | None,
                                max_seq_len: int, k_new: torch.Tensor, v_new: torch.Tensor,
                                slot_mapping: torch.Tensor | None, scale_mode: str = "div",
                                q_token_major: bool = False) -> torch.Tensor:
    return paged_attention(q, k_pages, v_pages, v_scales, block_table, seq_lens, max_seq_len,
                           q_token_major=q_token_major, append=(k_new, v_new, slot_mapping), scale_mode=scale_mode)


@_lib_paged_attention_append.register_fake
def _(q, k_pages, v_pages, v_scales, block_table, seq_lens, max_seq_len, k_new, v_new, slot_mapping,
      scale_mode="div", q_token_major=False):
    return torch.empty_like(q)


@torch.library.custom_op("sdv::quant_append", mutates_args=("k_pages", "v_pages", "v_scales"))
def _lib_quant_append(v_new: torch.Tensor, slot_mapping: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                      v_scales: torch.Tensor, k_new: torch.Tensor | None = None, scale_mode: str = "div") -> None:
    quant_append(v_new, slot_mapping, k_pages, v_pages, v_scales, k_new, scale_mode=scale_mode)


@_lib_quant_append.register_fake
def _(v_new, slot_mapping, k_pages, v_pages, v_scales, k_new=None, scale_mode="div"):
    return None
