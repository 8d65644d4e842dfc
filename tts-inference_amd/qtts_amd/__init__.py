"""qtts_amd: the quantized-linear hot path of qtts, native to MI355X (gfx950).

The GPU work runs in libqtts_amd.so (hand-written HIP, C ABI in
include/qtts_amd.h); this package is the host side that mirrors the reference's
``qtts.layers.linear`` / ``qtts.quant`` interfaces on top of it.
"""

from . import ops, torch_ops  # torch_ops registers torch.ops.qtts.*
from .config import QuantConfig
from .layers.linear import LinearBase, MergedLinear, iter_linears
from .quant import apply_quantization, build_method, fp8_supported, quantize_module

__all__ = ["ops", "torch_ops", "QuantConfig", "LinearBase", "MergedLinear", "iter_linears", "apply_quantization",
           "build_method", "fp8_supported", "quantize_module"]
