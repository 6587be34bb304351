"""specdec_amd -- MI355X-native FP8-V paged decode hot path of SpecDec-Context-Scaling.

Layout:
  specdec_amd._native        ctypes binding of libsdv.so (C ABI: include/sdv.h)
  specdec_amd.build          in-tree hipcc build of libsdv.so (gfx950)
  specdec_amd.kernels.ops    torch-facing operators (quant_append, paged_attention, attention)
  specdec_amd.kernels.patch  engine pack install/restore (mirror of specdec/kernels/patch.py)
  specdec_amd.engine         paged cache, cache API (spec_cache), attention accounting
"""
from ._native import SdvError  # noqa: F401

__all__ = ["SdvError"]
