"""coachwhip_amd: the quantized mixture-of-experts expert path on AMD MI355X (gfx950).

HIP kernels behind a C ABI (include/cwmoe.h, built as libcwmoe.so) with a thin Python mirror of
the reference engine's QMatMul / MoE-layer interfaces (``coachwhip_amd.ops``, which needs torch)
and the host bank bookkeeping (``coachwhip_amd.slots``).
"""
from . import formats
from ._lib import CW_MOE_STATE_BYTES, CW_MOE_STATUS_OFFSET, NO_SLOT, CwError, CwNotSupported, lib
from .slots import Plan, Slots

__all__ = ["formats", "lib", "CwError", "CwNotSupported", "NO_SLOT", "CW_MOE_STATE_BYTES", "CW_MOE_STATUS_OFFSET", "Slots", "Plan"]
