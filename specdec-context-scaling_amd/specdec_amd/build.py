"""Build and load the native library (mirror of specdec/kernels/build.py:17-52).

The reference JIT-compiles its CUDA extension with ``torch.utils.cpp_extension.load``.
Here the native code is a plain C-ABI shared library compiled ahead of time, in-tree, by
``hipcc --offload-arch=gfx950`` (it cross-compiles without a GPU), and loaded with ctypes;
``load()`` keeps the reference's name and its "build once, cache the module" behaviour.

    python -m specdec_amd.build          # compile specdec_amd/libsdv.so
    python -m specdec_amd.build --trace  # compile specdec_amd/libsdv_trace.so (phase stamps)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

from . import _native

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops stay off on this hardware pool (the host pass warns that it does
    # not know the feature; that is expected).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs rather than accumulation registers: no copy out of the
    # AGPRs per result, and one register budget (the prefill passes: 2048 x 8192, 12/2/128
    # 350 -> 332 us; the decode kernels measured unchanged)
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise _native.SdvError("hipcc not found (ROCm is required to build libsdv.so)")


TRACE_LIB_PATH = PKG_DIR / "libsdv_trace.so"


def build(verbose: bool = False, trace: bool = False) -> Path:
    """Compile every HIP source into specdec_amd/libsdv.so (always recompiles).

    trace=True builds the phase-trace variant, specdec_amd/libsdv_trace.so: the same kernels
    with wall-clock stamps at the single launch's phase boundaries (SDV_PHASE_TRACE), read by
    specdec_amd.phase_trace.  The product path never loads it."""
    out = TRACE_LIB_PATH if trace else _native.LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    defs = ["-DSDV_PHASE_TRACE"] if trace else []
    cmd = [_hipcc(), *HIPCC_FLAGS, *defs, f"-I{INCLUDE}", f"-I{CSRC}", "-o", str(tmp), *map(str, sources())]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise _native.SdvError(f"hipcc failed ({res.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, file=sys.stderr)
    os.replace(tmp, out)
    return out


def load():
    """The loaded native library (ctypes.CDLL); raises SdvError if it has not been built."""
    return _native.load()


if __name__ == "__main__":
    print(build(verbose=True, trace="--trace" in sys.argv))
