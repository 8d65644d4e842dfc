"""Quantization dispatch: build a method, attach it to the chosen linears, report.

Same contract as qtts/quant/base.py:41-183.  A method is an object assigned to
``layer.quant_method`` after the checkpoint has loaded; ``process_weights``
replaces the weight with quantized buffers or declines the layer, and the
report counts converted / excluded-by-name / declined layers and the bytes
before and after.
"""

from __future__ import annotations

import logging

import torch
from torch import nn

from ..config import QuantConfig
from ..layers.linear import iter_linears

logger = logging.getLogger("qtts_amd.quant")

#: The MI355X Infinity Cache.  A submodel whose quantized weights exceed it cannot keep them
#: cached from one decode step to the next, so each step streams every weight byte from HBM
#: once; its layers then load weights non-temporally (the weight policy, ALGO_STREAM), which
#: keeps that stream from evicting what is reused: the activations, and the weights of a
#: smaller submodel (the code predictor's, read 15 times a frame).
CACHE_RESIDENT_BYTES = 256 << 20


def weight_flags(layer) -> int:
    """The algo flags of ``layer``'s weight policy: ``ALGO_STREAM`` for a streamed submodel."""
    from .. import _lib

    return _lib.ALGO_STREAM if getattr(layer, "quant_stream", False) else 0


class QuantMethodBase:
    """Base of the assign-after-load quant methods (qtts/quant/base.py:41-63)."""

    name = "base"
    #: The weight policy of the submodel being converted (set by quantize_module before its
    #: layers are processed; process_weights records it on each layer as ``quant_stream``).
    stream_weights = False

    def process_weights(self, layer) -> None:
        raise NotImplementedError

    def applies_to(self, layer) -> bool:
        """Whether ``process_weights`` converted this layer (a method may decline one)."""
        return True

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        raise NotImplementedError


def _param_bytes(module: nn.Module) -> int:
    return sum(p.numel() * p.element_size() for p in module.parameters(recurse=True))


def _buffer_bytes(module: nn.Module) -> int:
    return sum(b.numel() * b.element_size() for b in module.buffers(recurse=True))


def _human(n: int) -> str:
    for unit in ("B", "KiB", "MiB", "GiB"):
        if abs(n) < 1024 or unit == "GiB":
            return f"{n:.1f} {unit}" if unit != "B" else f"{n} B"
        n /= 1024  # type: ignore[assignment]
    return str(n)


def streams_weights(module: nn.Module, config: QuantConfig) -> bool:
    """Whether the eligible linears' codes (one byte per weight) exceed ``CACHE_RESIDENT_BYTES``."""
    codes = sum(layer.weight.numel() for name, layer in iter_linears(module)
                if not config.excludes(name) and getattr(layer, "weight", None) is not None)
    return codes > CACHE_RESIDENT_BYTES


def quantize_module(module: nn.Module, method: QuantMethodBase, config: QuantConfig, label: str) -> dict[str, int]:
    """Attach ``method`` to every eligible linear under ``module`` (qtts/quant/base.py:74-113)."""
    before = _param_bytes(module) + _buffer_bytes(module)
    converted = excluded = declined = kept_weight = 0
    stream = streams_weights(module, config)
    method.stream_weights = stream
    for name, layer in iter_linears(module):
        if config.excludes(name):
            excluded += 1
            continue
        method.process_weights(layer)
        if not method.applies_to(layer):
            declined += 1
            continue
        layer.quant_method = method
        layer.quant_stream = stream
        converted += 1
        # a converted layer whose calibration routed some row bucket to F.linear keeps its weight
        weight = getattr(layer, "weight", None)
        kept_weight += int(weight is not None and weight.numel() > 0)
    after = _param_bytes(module) + _buffer_bytes(module)
    logger.info("%s: %s converted %d linears (%d keeping their weight for F.linear at some row bucket), "
                "skipped %d by exclusion, kept %d on F.linear; weights %s -> %s, %s",
                label, method.name, converted, kept_weight, excluded, declined, _human(before), _human(after),
                "streamed past the caches" if stream else "cache-resident")
    return {"converted": converted, "excluded": excluded, "declined": declined, "bytes_before": before,
            "bytes_after": after, "kept_weight": kept_weight, "stream_weights": int(stream)}


def fp8_supported() -> tuple[bool, str]:
    """Whether the fp8 W8A8 path can run here, and why not (qtts/quant/base.py:133-152)."""
    if not torch.cuda.is_available():
        return False, "no GPU device"
    if not hasattr(torch, "float8_e4m3fn"):
        return False, f"torch {torch.__version__} has no float8_e4m3fn dtype"
    from .kernels import kernel_available

    ok, reason = kernel_available()
    if not ok:
        return False, reason
    return True, ""


def build_method(config: QuantConfig, calibration_batch: int = 16) -> QuantMethodBase:
    """Method object for ``config.method`` (qtts/quant/base.py:116-130)."""
    from .fp8 import Fp8Method, Fp8WeightOnlyMethod
    from .int8 import Int8Method, Int8WeightOnlyMethod

    method = config.method
    if method in ("fp8", "fp8_weight_only"):
        supported, reason = fp8_supported()
        if not supported:
            raise RuntimeError(f"the fp8 method cannot run here: {reason}")
        if method == "fp8_weight_only":
            return Fp8WeightOnlyMethod(calibrate=config.calibrate, calibration_batch=calibration_batch)
        return Fp8Method()
    if method == "int8_weight_only":
        return Int8WeightOnlyMethod(calibrate=config.calibrate, calibration_batch=calibration_batch)
    if method == "int8":
        return Int8Method()
    raise ValueError(f"no quantization method named {method!r}")


def apply_quantization(config: QuantConfig, *, talker: nn.Module | None = None,
                       code_predictor: nn.Module | None = None, code2wav: nn.Module | None = None,
                       calibration_batch: int = 16) -> dict[str, dict[str, int]]:
    """Quantize the submodels named in ``config.targets`` (qtts/quant/base.py:155-183)."""
    if not config.enabled:
        return {}
    unknown = set(config.targets) - {"talker", "code_predictor", "code2wav"}
    if unknown:
        raise ValueError(f"quant targets {sorted(unknown)} name no submodel (talker, code_predictor, code2wav)")
    method = build_method(config, calibration_batch=calibration_batch)
    report: dict[str, dict[str, int]] = {}
    if config.targets_submodel("talker"):
        if talker is not None:
            report["talker"] = quantize_module(talker, method, config, "talker")
        if code_predictor is not None:
            report["code_predictor"] = quantize_module(code_predictor, method, config, "code_predictor")
    if config.targets_submodel("code2wav") and code2wav is not None:
        report["code2wav"] = quantize_module(code2wav, method, config, "code2wav")
    return report
