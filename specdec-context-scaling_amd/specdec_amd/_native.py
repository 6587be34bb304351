"""ctypes binding of libsdv.so (the C ABI declared in include/sdv.h).

The library is built in-tree by ``specdec_amd.build.build()`` (hipcc, gfx950) and loaded
from this package directory.  There is no fallback: if the library is missing, every
native call raises :class:`SdvError` that says how to build it.

Error behaviour mirrors the reference op (specdec/kernels/cuda/attention.cu:244-288, whose
TORCH_CHECK failures surface as ``RuntimeError``): a non-zero status from the library
raises :class:`SdvError`, a ``RuntimeError`` subclass carrying ``.status``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_NAME = "libsdv.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

SDV_OK = 0
SDV_ERR_NULL = -1
SDV_ERR_SHAPE = -2
SDV_ERR_UNSUPPORTED = -3
SDV_ERR_WORKSPACE = -4
SDV_ERR_ALIGN = -5
SDV_ERR_HIP = -6

SCALE_DIV = 0
SCALE_RCP = 1

PHASE_QK = 1
PHASE_PV = 2
PHASE_REDUCE = 4
PHASE_ALL = 7

BLOCK_SIZE = 16
SYNC_BYTES = 12583168       # SDV_SYNC_BYTES: workspace prefix the single-launch path synchronises through
NOALLOC_MAX_WORKSPACE = 33554432  # SDV_NOALLOC_MAX_WORKSPACE: the no-allocation entry point's scratch per GPU
ABI_VERSION = 1

# Every symbol include/sdv.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
SIGNATURES = {
    "sdv_quant_append": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I64,
                                        _P, _P, _P, _I32, _I64, _I64, _I64, _I32, _P]),
    "sdv_quant_append_tiles": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I64,
                                              _P, _P, _P, _I32, _I64, _I64, _I64, _I32, _P, _I32, _P]),
    "sdv_attention_workspace_size": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "sdv_attention_workspace_init": (ctypes.c_int, [_P, _SZ, _P]),
    "sdv_attention_workspace_status": (ctypes.c_int, [_P, _SZ, ctypes.POINTER(ctypes.c_uint32),
                                                      ctypes.POINTER(ctypes.c_uint32), _P]),
    "sdv_attention_set_wait_limit": (ctypes.c_int, [ctypes.c_uint32]),
    "sdv_attention_single_launch": (ctypes.c_int32, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "sdv_paged_attention": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I64, _I64, _I64, _P, _I32, _P,
                                           _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                           _P, _SZ, _P, _P]),
    "sdv_paged_attention_phases": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I64, _I64, _I64, _P, _I32, _P,
                                                  _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                                  _P, _SZ, _P, _P, _I32]),
    "sdv_paged_attention_append": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I64, _I64, _I64, _P, _I32, _P,
                                                  _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                                  _P, _SZ, _P, _P, _P, _P, _I64, _I32, _P]),
    "sdv_paged_attention_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I64, _I64, _I64, _P, _I32, _P,
                                                   _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P]),
    "sdv_fp8_encode": (ctypes.c_int, [_P, _P, _I64, _P]),
    "sdv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "sdv_abi_version": (ctypes.c_int, []),
}


class SdvError(RuntimeError):
    """A libsdv entry point returned a non-zero status (or the library is unavailable)."""

    def __init__(self, msg: str, status: int | None = None):
        super().__init__(msg)
        self.status = status


_LIB = None


def load(path: os.PathLike | str | None = None, make_default: bool = False) -> ctypes.CDLL:
    """Load libsdv.so once and attach the C signatures.  Raises SdvError when it is absent.

    path: another build of the same sources (the phase-trace variant); make_default=True makes
    it the library every op of this process calls from then on."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise SdvError(f"{p} is not built; run `python -m specdec_amd.build` (or "
                       f"__graft_entry__.build()) on a machine with hipcc")
    lib = ctypes.CDLL(os.fspath(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.sdv_abi_version() != ABI_VERSION:
        raise SdvError(f"{p} has ABI {lib.sdv_abi_version()}, expected {ABI_VERSION}; rebuild it")
    if path is None or make_default:
        _LIB = lib
    return lib


def status_string(status: int) -> str:
    return load().sdv_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    if status != SDV_OK:
        raise SdvError(f"{what}: {status_string(status)} (status {status})", status)
