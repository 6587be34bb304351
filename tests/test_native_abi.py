"""libsdv.so loads on a machine without a GPU, exports every symbol include/sdv.h declares,
and rejects bad arguments on the host before any HIP call (no compute calls here)."""
from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT
from specdec_amd import _native, build


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        build.build()
    return _native.load()


def _declared():
    text = (ROOT / "include" / "sdv.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|size_t|const char\*)\s+(sdv_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert names == sorted(_native.SIGNATURES), names
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version_and_status_strings(lib):
    assert lib.sdv_abi_version() == _native.ABI_VERSION
    for st in range(0, -7, -1):
        assert _native.status_string(st) not in ("", "unknown status"), st
    assert _native.status_string(-99) == "unknown status"


P = ctypes.c_void_p(0x1000)   # fake, 256-aligned non-null device pointers: never dereferenced
N = None


def _attn(lib, **kw):
    a = dict(q=P, k=P, v=P, s=P, nb=8, kls=0, vls=0, sls=0, bt=P, mb=4, sl=P, L=1, B=1, H=12, KV=2, S=1,
             D=128, T=64, tm=0, ws=P, wsb=1 << 30, out=P, st=N)
    a.update(kw)
    return lib.sdv_paged_attention(a["q"], a["k"], a["v"], a["s"], a["nb"], a["kls"], a["vls"], a["sls"],
                                   a["bt"], a["mb"], a["sl"], a["L"], a["B"], a["H"], a["KV"], a["S"], a["D"],
                                   a["T"], a["tm"], a["ws"], a["wsb"], a["out"], a["st"])


def test_attention_host_validation(lib):
    assert _attn(lib, q=N) == _native.SDV_ERR_NULL
    assert _attn(lib, D=96) == _native.SDV_ERR_UNSUPPORTED
    assert _attn(lib, H=13) == _native.SDV_ERR_SHAPE            # H % KV != 0
    assert _attn(lib, T=0) == _native.SDV_ERR_SHAPE
    assert _attn(lib, mb=3) == _native.SDV_ERR_SHAPE            # 3 blocks < 64 tokens
    assert _attn(lib, tm=2) == _native.SDV_ERR_SHAPE
    assert _attn(lib, L=2, kls=10) == _native.SDV_ERR_SHAPE     # layer stride smaller than a layer
    assert _attn(lib, ws=N) == _native.SDV_ERR_WORKSPACE
    assert _attn(lib, wsb=16) == _native.SDV_ERR_WORKSPACE
    assert _attn(lib, ws=ctypes.c_void_p(0x1010)) == _native.SDV_ERR_WORKSPACE   # not 256-aligned
    assert _attn(lib, q=ctypes.c_void_p(0x1002)) == _native.SDV_ERR_ALIGN


def _quant(lib, **kw):
    a = dict(v=P, k=N, sl=P, n=16, KV=2, D=128, gs=128, L=1, ils=0, kp=P, vp=P, vs=P, nb=8, kls=0, vls=0,
             sls=0, mode=0, st=N)
    a.update(kw)
    return lib.sdv_quant_append(a["v"], a["k"], a["sl"], a["n"], a["KV"], a["D"], a["gs"], a["L"], a["ils"],
                                a["kp"], a["vp"], a["vs"], a["nb"], a["kls"], a["vls"], a["sls"], a["mode"],
                                a["st"])


def test_quant_host_validation(lib):
    assert _quant(lib, v=N) == _native.SDV_ERR_NULL
    assert _quant(lib, k=P, kp=N) == _native.SDV_ERR_NULL
    assert _quant(lib, gs=32) == _native.SDV_ERR_UNSUPPORTED    # GROUP_SIZE ablation is not v_fp8
    assert _quant(lib, D=256, gs=256) == _native.SDV_ERR_UNSUPPORTED
    assert _quant(lib, mode=7) == _native.SDV_ERR_UNSUPPORTED
    assert _quant(lib, n=-1) == _native.SDV_ERR_SHAPE
    assert _quant(lib, L=2, ils=5) == _native.SDV_ERR_SHAPE
    assert _quant(lib, vp=ctypes.c_void_p(0x1004)) == _native.SDV_ERR_ALIGN
    assert _quant(lib, v=ctypes.c_void_p(0x1008)) == _native.SDV_ERR_ALIGN    # rows move as 16-byte pieces
    assert _quant(lib, k=ctypes.c_void_p(0x1008)) == _native.SDV_ERR_ALIGN
    assert _quant(lib, kp=ctypes.c_void_p(0x1008), k=P) == _native.SDV_ERR_ALIGN
    assert _quant(lib, L=2, ils=16 * 2 * 128 + 4, vls=1 << 20, sls=1 << 20) == _native.SDV_ERR_ALIGN
    assert _quant(lib, n=0) == _native.SDV_OK                  # nothing to do, no launch


def test_append_attention_host_validation(lib):
    def f(**kw):
        a = dict(q=P, k=P, v=P, s=P, nb=8, kls=0, vls=0, sls=0, bt=P, mb=4, sl=P, L=1, B=1, H=12, KV=2, S=1,
                 D=128, T=64, tm=0, ws=P, wsb=1 << 30, out=P, kn=P, vn=P, slots=P, nls=0, mode=0, st=N)
        a.update(kw)
        return lib.sdv_paged_attention_append(a["q"], a["k"], a["v"], a["s"], a["nb"], a["kls"], a["vls"], a["sls"],
                                              a["bt"], a["mb"], a["sl"], a["L"], a["B"], a["H"], a["KV"], a["S"],
                                              a["D"], a["T"], a["tm"], a["ws"], a["wsb"], a["out"], a["kn"], a["vn"],
                                              a["slots"], a["nls"], a["mode"], a["st"])
    assert f(kn=N) == _native.SDV_ERR_NULL
    assert f(slots=N, D=96) == _native.SDV_ERR_UNSUPPORTED         # NULL slots (from the block table) are valid
    assert f(sl=N, D=96) == _native.SDV_ERR_UNSUPPORTED            # NULL lengths (all max_seq_len) are valid
    assert f(q=N) == _native.SDV_ERR_NULL                         # the attention checks apply
    assert f(mode=5) == _native.SDV_ERR_UNSUPPORTED
    assert f(vn=ctypes.c_void_p(0x1008)) == _native.SDV_ERR_ALIGN
    assert f(L=2, nls=8) == _native.SDV_ERR_SHAPE                   # layer stride below one layer
    assert f(D=96) == _native.SDV_ERR_UNSUPPORTED


def test_quant_tiles_host_validation(lib):
    def q(**kw):
        a = dict(v=P, k=N, sl=P, n=16, KV=2, D=128, gs=128, L=1, ils=0, kp=P, vp=P, vs=P, nb=8, kls=0, vls=0,
                 sls=0, mode=0, t=P, nt=1, st=N)
        a.update(kw)
        return lib.sdv_quant_append_tiles(a["v"], a["k"], a["sl"], a["n"], a["KV"], a["D"], a["gs"], a["L"],
                                          a["ils"], a["kp"], a["vp"], a["vs"], a["nb"], a["kls"], a["vls"],
                                          a["sls"], a["mode"], a["t"], a["nt"], a["st"])
    assert q(t=N) == _native.SDV_ERR_NULL
    assert q(nt=-1) == _native.SDV_ERR_SHAPE
    assert q(t=ctypes.c_void_p(0x1002)) == _native.SDV_ERR_ALIGN
    assert q(v=N) == _native.SDV_ERR_NULL                       # the checks of sdv_quant_append apply
    assert q(gs=32) == _native.SDV_ERR_UNSUPPORTED
    assert q(nt=0) == _native.SDV_OK                            # no tiles: nothing to do, no launch
    assert q(n=0) == _native.SDV_OK


def test_workspace_size_is_pure_host(lib):
    a = lib.sdv_attention_workspace_size(1, 1, 12, 2, 1, 128, 8192)
    b = lib.sdv_attention_workspace_size(28, 1, 12, 2, 1, 128, 8192)
    c = lib.sdv_attention_workspace_size(1, 1, 12, 2, 5, 128, 8192)
    assert 0 < a < b and a < c
    assert a % 256 == 0
    assert lib.sdv_attention_workspace_size(1, 1, 12, 2, 1, 96, 8192) == 0
    assert lib.sdv_attention_workspace_size(1, 1, 12, 5, 1, 128, 8192) == 0


def test_workspace_init_validation(lib):
    # NULL names the current device's no-allocation scratch: with no device there is none
    assert lib.sdv_attention_workspace_init(N, 1 << 21, N) in (_native.SDV_ERR_HIP, _native.SDV_OK)
    f, p = ctypes.c_uint32(0), ctypes.c_uint32(0)
    assert lib.sdv_attention_workspace_status(N, 0, None, ctypes.byref(p), N) == _native.SDV_ERR_NULL
    assert lib.sdv_attention_workspace_status(N, 0, ctypes.byref(f), ctypes.byref(p), N) in (_native.SDV_ERR_HIP,
                                                                                          _native.SDV_OK)
    assert lib.sdv_attention_workspace_init(P, _native.SYNC_BYTES - 4, N) == _native.SDV_ERR_WORKSPACE
    assert lib.sdv_attention_workspace_init(ctypes.c_void_p(0x1010), 1 << 21, N) == _native.SDV_ERR_WORKSPACE
    # every attention workspace holds the synchronisation prefix
    assert lib.sdv_attention_workspace_size(1, 1, 12, 2, 1, 128, 16) >= _native.SYNC_BYTES
    header = (ROOT / "include" / "sdv.h").read_text()
    assert f"#define SDV_SYNC_BYTES {_native.SYNC_BYTES}" in header


def test_encode_validation(lib):
    assert lib.sdv_fp8_encode(N, P, 4, N) == _native.SDV_ERR_NULL
    assert lib.sdv_fp8_encode(P, P, -1, N) == _native.SDV_ERR_SHAPE
    assert lib.sdv_fp8_encode(P, P, 0, N) == _native.SDV_OK


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_native.SdvError, match="not built"):
        _native.load(tmp_path / "libsdv.so")


def test_phase_trace_stays_out_of_the_product_library(lib):
    """The phase stamps (SDV_PHASE_TRACE) exist only in libsdv_trace.so, which exports the same
    C-ABI plus its reader; the product library compiles them away."""
    assert not hasattr(lib, "sdv_phase_trace_read")
    if not build.TRACE_LIB_PATH.exists():
        pytest.skip("libsdv_trace.so not built")
    tlib = ctypes.CDLL(str(build.TRACE_LIB_PATH))
    for n in _declared():
        assert hasattr(tlib, n), n
    tlib.sdv_phase_trace_read.restype = ctypes.c_int
    tlib.sdv_phase_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    assert tlib.sdv_phase_trace_read(None, 1) == _native.SDV_ERR_NULL
    buf = (ctypes.c_uint64 * 1)()
    assert tlib.sdv_phase_trace_read(buf, 1 << 40) == _native.SDV_ERR_SHAPE


def test_group_shapes_workspace_and_no_split(lib):
    """A batch of 256 or more one-tile groups (one per workgroup of the per-group kernel) that
    no single launch serves runs in one launch of the per-group kernel: its workspace is the
    synchronisation prefix plus 256 score rows per query row of the longest sequence, and the
    profiling split refuses it (before any launch)."""
    L, B, H, KV, D, T = 28, 32, 12, 2, 128, 32768          # 1792 groups of 6 rows
    need = lib.sdv_attention_workspace_size(L, B, H, KV, 1, D, T)
    assert need == _native.SYNC_BYTES + 256 * (H // KV) * T * 2
    # 448 groups, at least one per workgroup: the per-group kernel
    assert lib.sdv_attention_workspace_size(L, 8, H, KV, 1, D, T) == need
    # 112 groups, fewer than one per workgroup: the three launches' layout (scores of every
    # group: 112 x 6 x 32768 x 2 bytes and more), not the per-group kernel's
    three = lib.sdv_attention_workspace_size(L, 2, H, KV, 1, D, T)
    assert three != need and three > _native.SYNC_BYTES + 112 * (H // KV) * T * 2

    def phases(mask):
        return lib.sdv_paged_attention_phases(P, P, P, P, 8, 1 << 30, 1 << 30, 1 << 30, P, T // 16, P, L, B, H,
                                              KV, 1, D, T, 0, P, 1 << 40, P, N, mask)
    for mask in (_native.PHASE_QK, _native.PHASE_PV, 4):
        assert phases(mask) == _native.SDV_ERR_UNSUPPORTED


def _round256(x):
    return (x + 255) // 256 * 256


def test_prefill_workspace_follows_the_part_plan(lib):
    """The prefill workspace is the synchronisation prefix, pass 1's (max, sum) per row and key
    part, pass 2's fp32 part slots (128 rows per row group, as many slots as its most-split row
    group) and V dequantized once (one 1 KiB tile per 16 dimensions and two blocks).  2048 x 8192
    (12/2/128): pass 1 in 8 parts (1,536 workgroups of 128 rows), pass 2 by key count, at most 3
    parts (the last 10 of each head's 16 row groups); with S not a multiple of 128 (S = T =
    1000) pass 1 takes 7 parts (no fewer than 8 blocks each) and pass 2 splits every row group
    alike, in 5."""
    H, KV, D, S, T = 12, 2, 128, 2048, 8192
    R, groups = H // KV * S, KV
    want = (_native.SYNC_BYTES + _round256(groups * R * 8 * 8) + _round256(groups * (R // 128) * 3 * 128 * D * 4)
            + groups * (T // 32) * (D // 16) * 1024)
    assert lib.sdv_attention_workspace_size(1, 1, H, KV, S, D, T) == want
    S = T = 1000
    R = H // KV * S
    nrg1, nrg2 = -(-R // 128), -(-R // 128)
    split1 = min(64, (T // 16) // 8, 1536 // (groups * nrg1))
    parts2 = min(8, (T // 16) // 8, 512 // (groups * nrg2))
    want = (_native.SYNC_BYTES + _round256(groups * R * 8 * split1) + _round256(groups * nrg2 * parts2 * 128 * D * 4)
            + groups * (-(-(-(-T // 16)) // 2)) * (D // 16) * 1024)
    assert lib.sdv_attention_workspace_size(1, 1, H, KV, S, D, T) == want
