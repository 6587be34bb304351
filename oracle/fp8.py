"""From-spec OCP E4M3FN codec (TEST INFRASTRUCTURE ONLY).

Thin ctypes front-end for ``oracle/fp8_e4m3.c``.  The C file is compiled on first use
(``make -C oracle``) into ``oracle/_build/liboracle_fp8.so``.

Pinned by: the exhaustive comparison with torch's CPU ``float8_e4m3fn`` cast over every
fp32 bit pattern (tests/test_oracle_fp8.py), plus the spec's fixed points (0x7E = 448,
0x01 = 2^-9, 0x08 = 2^-6, ties-to-even at 464 and at subnormal half-steps).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle_fp8.so"
_LIB = None


def build() -> Path:
    """Compile the codec (gcc) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        src = _HERE / "fp8_e4m3.c"
        if not _LIB_PATH.exists() or _LIB_PATH.stat().st_mtime < src.stat().st_mtime:
            build()
        lib = ctypes.CDLL(os.fspath(_LIB_PATH))
        lib.oracle_e4m3fn_encode_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        lib.oracle_e4m3fn_encode_range.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t]
        lib.oracle_e4m3fn_decode_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        _LIB = lib
    return _LIB


def encode(x: np.ndarray) -> np.ndarray:
    """fp32 array -> uint8 E4M3FN codes (round to nearest even, NaN on overflow)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint8)
    _lib().oracle_e4m3fn_encode_n(a.ctypes.data, out.ctypes.data, a.size)
    return out


def encode_range(lo: int, n: int) -> np.ndarray:
    """Encode the n fp32 values whose bit patterns are lo, lo+1, ..., lo+n-1."""
    out = np.empty(n, dtype=np.uint8)
    _lib().oracle_e4m3fn_encode_range(lo, out.ctypes.data, n)
    return out


def decode(b: np.ndarray) -> np.ndarray:
    """uint8 E4M3FN codes -> fp32 values (exact)."""
    a = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(a.shape, dtype=np.float32)
    _lib().oracle_e4m3fn_decode_n(a.ctypes.data, out.ctypes.data, a.size)
    return out
