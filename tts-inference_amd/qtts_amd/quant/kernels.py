"""Availability of the fused dequantize-in-registers GEMM.

Mirrors qtts/quant/kernels.py:83-84 (``kernel_available``), backed by the hand-written
gfx950 kernels in libqtts_amd.so instead of a Triton kernel.  The reference's wrapper
(``w8_gemm``, kernels.py:138-178) is ``ops.w8a16_gemm`` / ``ops.w8a16_gemm_strips``.
"""

from __future__ import annotations

import torch

from .. import _lib, ops


def kernel_available() -> tuple[bool, str]:
    """(True, "") when libqtts_amd.so loads and the current device is a gfx950."""
    try:
        _lib.load()
    except Exception as exc:
        return False, f"libqtts_amd unavailable: {exc}"
    if not torch.cuda.is_available():
        return False, "no GPU visible"
    if not ops.device_supported():
        name = torch.cuda.get_device_name()
        return False, f"device {name!r} is not a gfx950 (MI355X-class) GPU"
    return True, ""
