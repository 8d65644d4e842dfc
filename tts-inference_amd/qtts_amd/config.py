"""Quantization flags (qtts/config.py:50-98), same fields and semantics."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

METHODS = ("none", "fp8", "fp8_weight_only", "int8", "int8_weight_only")


@dataclass
class QuantConfig:
    method: Literal["none", "fp8", "fp8_weight_only", "int8", "int8_weight_only"] = "none"
    #: Submodels to quantize; the code predictor follows "talker" (qtts/quant/base.py:176-180).
    targets: tuple[str, ...] = ("talker",)
    #: Layers whose name contains any of these keep full precision (qtts/config.py:71-76).
    exclude_substrings: tuple[str, ...] = ("lm_head", "codec_head", "text_projection", "small_to_mtp_projection")
    #: Time each distinct linear shape at load and keep the fastest kernel (qtts/config.py:85).
    calibrate: bool = True

    @property
    def enabled(self) -> bool:
        return self.method != "none"

    @property
    def weight_only(self) -> bool:
        return self.method.endswith("_weight_only")

    def targets_submodel(self, name: str) -> bool:
        return self.enabled and name in self.targets

    def excludes(self, layer_name: str) -> bool:
        return any(s in layer_name for s in self.exclude_substrings)
