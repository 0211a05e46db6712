"""crb_amd: MI355X-native (gfx950) CRB layer-wise binarization quantizer.

Drop-in replacements for the reference's per-layer quantizer API:
``BRAGPTQ`` (bigptq.py:18-298) and ``Binarization`` (binary.py:2850-2890),
backed by hand-written HIP kernels in ``libcrbq.so`` (C ABI in
include/crbq.h).  There is no CPU fallback.
"""
from .bigptq import BRAGPTQ  # noqa: F401
from .binary import Binarization  # noqa: F401

__all__ = ["BRAGPTQ", "Binarization"]
