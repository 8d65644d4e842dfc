"""The linear layer with one quantization hook.

Same duck-typed contract as the reference's qtts/layers/linear.py:25-104: a model
builds ``LinearBase`` / ``MergedLinear`` modules, loads real weights into
``weight``, and a quant method assigned to ``quant_method`` afterwards takes over
``forward`` (linear.py:57-60).  Models written against the reference's layer run
unchanged on this one, and the reference's own layers work with this package's
quant methods, because only attribute names are relied on.
"""

from __future__ import annotations

from typing import Protocol

import torch
import torch.nn.functional as F
from torch import nn


class QuantMethod(Protocol):
    """qtts/layers/linear.py:25-30 (plus ``applies_to``, qtts/quant/base.py:49-58)."""

    name: str

    def process_weights(self, layer: "LinearBase") -> None: ...

    def applies_to(self, layer: "LinearBase") -> bool: ...

    def apply(self, layer: "LinearBase", x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor: ...


class LinearBase(nn.Module):
    """``y = x W^T + b`` whose GEMM a quant method can replace (qtts/layers/linear.py:33-64)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=dtype, device=device),
                                   requires_grad=False)
        if bias:
            self.bias: nn.Parameter | None = nn.Parameter(torch.empty(out_features, dtype=dtype, device=device),
                                                          requires_grad=False)
        else:
            self.register_parameter("bias", None)
        self.quant_method: QuantMethod | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        method = self.quant_method
        if method is not None:
            return method.apply(self, x, self.bias)
        return F.linear(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        q = self.quant_method.name if self.quant_method is not None else "none"
        return f"{self.in_features} -> {self.out_features}, bias={self.bias is not None}, quant_method={q}"


class MergedLinear(LinearBase):
    """Output partitions fused into one weight along dim 0 (qtts/layers/linear.py:67-100).

    The fused qkv and gate_up projections quantize as one ``[sum(N_i), K]`` matrix
    with per-row scales; ``split`` cuts the output afterwards.
    """

    def __init__(self, in_features: int, partitions: list[int], bias: bool = False,
                 dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> None:
        super().__init__(in_features, sum(partitions), bias=bias, dtype=dtype, device=device)
        self.partitions = list(partitions)
        self.offsets = [0]
        for size in self.partitions:
            self.offsets.append(self.offsets[-1] + size)

    def load_partition(self, index: int, tensor: torch.Tensor) -> None:
        lo, hi = self.offsets[index], self.offsets[index + 1]
        if tuple(tensor.shape) != (hi - lo, self.in_features):
            raise ValueError(f"weight slice {index} must be {(hi - lo, self.in_features)}, not {tuple(tensor.shape)}")
        self.weight.data[lo:hi].copy_(tensor)

    def load_bias_partition(self, index: int, tensor: torch.Tensor) -> None:
        if self.bias is None:
            raise ValueError("this linear was built without a bias")
        lo, hi = self.offsets[index], self.offsets[index + 1]
        self.bias.data[lo:hi].copy_(tensor)

    def split(self, out: torch.Tensor) -> tuple[torch.Tensor, ...]:
        return tuple(out.split(self.partitions, dim=-1))


def iter_linears(module: nn.Module) -> list[tuple[str, nn.Module]]:
    """Every hooked linear under ``module`` in ``named_modules`` order (qtts/layers/linear.py:103-104).

    A module counts when it has the hook's attributes (``quant_method``,
    ``weight``, ``in_features``, ``out_features``), so the reference's own
    ``LinearBase`` modules are found as well as this package's.
    """
    found = []
    for name, m in module.named_modules():
        if isinstance(m, LinearBase) or (
            hasattr(m, "quant_method") and hasattr(m, "weight") and hasattr(m, "in_features")
            and hasattr(m, "out_features")
        ):
            found.append((name, m))
    return found
