"""The quant methods and the call that attaches them to a model's linears once its weights are
loaded (the package interface of qtts/quant/__init__.py)."""

from .base import apply_quantization, build_method, fp8_supported, quantize_module

__all__ = ["apply_quantization", "build_method", "fp8_supported", "quantize_module"]
