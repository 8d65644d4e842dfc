"""fp8 (OCP e4m3) quantization methods (qtts/quant/fp8.py).

``Fp8Method`` is W8A8: per-output-channel e4m3 weights, per-token e4m3
activations quantized at run time, and a gfx950 fp8 MFMA GEMM with the rowwise x
columnwise scale epilogue in place of torch._scaled_mm.  It is applied
uniformly, as in the reference (qtts/quant/fp8.py:52-89).

``Fp8WeightOnlyMethod`` raises NotImplementedError, as the reference does
(qtts/quant/fp8.py:92-123).
"""

from __future__ import annotations

import torch

from .. import _lib, ops
from .base import QuantMethodBase

_FP8_MAX = 448.0


def quantize_weight_fp8(weight: torch.Tensor, div_mode: int = _lib.DIV_DEVICE):
    """Symmetric per-output-channel e4m3 on the GPU: ``(q [N,K] float8_e4m3fn, scale [N] fp32)``."""
    return ops.pack_fp8(weight, div_mode)


class Fp8Method(QuantMethodBase):
    """W8A8 e4m3 on CDNA4 fp8 MFMA."""

    name = "fp8"

    def __init__(self, div_mode: int = _lib.DIV_DEVICE) -> None:
        self.div_mode = div_mode

    def process_weights(self, layer) -> None:
        weight = layer.weight
        q, scale = quantize_weight_fp8(weight, self.div_mode)
        # The reference keeps the [K, N] column-major view of the packed bytes for
        # _scaled_mm; this backend keeps the MFMA-native strip layout of the same
        # bytes instead (fp8_weight_rowmajor recovers them).  The scale is [1, N]
        # fp32 as in the reference.
        if layer.in_features % 32 == 0:
            layer.register_buffer("fp8_weight", ops.to_strips(q, _lib.STRIP_FP8), persistent=False)
            layer.fp8_layout = "strips"
        else:  # the strip kernels need K % 32 == 0; keep the reference's [K, N] view
            layer.register_buffer("fp8_weight", q.t(), persistent=False)
            layer.fp8_layout = "rowmajor"
        layer.register_buffer("fp8_scale", scale.reshape(1, -1), persistent=False)
        ops.reserve_workspace(weight.device, max(
            ops.workspace_bytes(_lib.OP_W8A8_FP8, m, layer.out_features, layer.in_features) for m in (16, 64, 256)))
        layer.weight = torch.nn.Parameter(torch.empty(0, dtype=weight.dtype, device=weight.device),
                                          requires_grad=False)

    def applies_to(self, layer) -> bool:
        return getattr(layer, "fp8_weight", None) is not None

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        if layer.fp8_layout == "strips":
            return ops.fp8_linear_strips(x, layer.fp8_weight, layer.out_features, layer.fp8_scale.reshape(-1), bias,
                                         self.div_mode)
        return ops.fp8_linear(x, layer.fp8_weight.t(), layer.fp8_scale.reshape(-1), bias, self.div_mode)


def fp8_weight_rowmajor(layer) -> torch.Tensor:
    """The packer's row-major ``[N, K]`` e4m3 bytes of a converted layer."""
    if getattr(layer, "fp8_layout", "rowmajor") == "strips":
        return ops.from_strips(layer.fp8_weight, layer.out_features, layer.in_features, _lib.STRIP_FP8)
    return layer.fp8_weight.t()


class Fp8WeightOnlyMethod(QuantMethodBase):
    """fp8 weights with model-dtype activations: not implemented, as in the reference."""

    name = "fp8_weight_only"

    def __init__(self) -> None:
        raise NotImplementedError(
            "fp8 weight-only is not implemented: use --quant-method int8_weight_only for the same "
            "footprint, or --quant-method fp8 for the W8A8 hardware path.")
