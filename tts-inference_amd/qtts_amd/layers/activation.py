"""GatedMLP whose activation runs inside its GEMMs (qtts/layers/activation.py:121-147).

Same constructor and forward contract as the reference's ``GatedMLP``: ``gate_up_proj``
(a ``MergedLinear`` of [intermediate, intermediate], gate first) or ``gate_proj`` /
``up_proj``, then ``down_proj(F.silu(gate) * up)``.  When ``gate_up_proj``'s quant method
has ``apply_gate_up_silu`` (the int8 weight-only method), it returns ``silu(gate) * up``
itself: decode rows get it from the gate_up GEMM's epilogue, which never stores the
gate_up output.  Otherwise, when ``down_proj``'s quant method has ``apply_silu_mul``, the
fused gate_up output goes to it whole (a single decode row has the activation computed
inside the down GEMM).  Torch's rounding either way.  Any other MLP gets
``F.silu(gate) * up`` first, exactly as the reference computes it.

``fuse_gated_mlps(model)`` gives the reference's own ``GatedMLP`` instances (anything
with ``gate_up_proj``, ``down_proj`` and ``fuse``) this forward, so a model built from
the reference's layers switches over after ``apply_quantization`` with no code change.
"""

from __future__ import annotations

import types

import torch
import torch.nn.functional as F
from torch import nn

from .linear import LinearBase, MergedLinear


def gated_mlp_forward(mlp: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """The forward of GatedMLP (activation.py:142-147): the activation computed by gate_up_proj's
    quant method when it can (from the GEMM's epilogue), else handed to the down projection's."""
    if mlp.fuse:
        up_method = getattr(mlp.gate_up_proj, "quant_method", None)
        pair = getattr(up_method, "apply_gate_up_silu", None)
        if pair is not None:
            act = pair(mlp.gate_up_proj, x, mlp.gate_up_proj.bias)
            if act is not None:
                return mlp.down_proj(act)
        gate_up = mlp.gate_up_proj(x)
        method = getattr(mlp.down_proj, "quant_method", None)
        fused = getattr(method, "apply_silu_mul", None)
        if fused is not None:
            return fused(mlp.down_proj, gate_up, mlp.down_proj.bias)
        gate, up = mlp.gate_up_proj.split(gate_up)
    else:
        gate, up = mlp.gate_proj(x), mlp.up_proj(x)
    return mlp.down_proj(F.silu(gate) * up)


class GatedMLP(nn.Module):
    """SwiGLU feed-forward; ``fuse`` merges gate and up into one GEMM (activation.py:121-147)."""

    def __init__(self, hidden_size: int, intermediate_size: int, fuse: bool = True,
                 dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> None:
        super().__init__()
        self.fuse = fuse
        if fuse:
            self.gate_up_proj = MergedLinear(hidden_size, [intermediate_size, intermediate_size], bias=False,
                                             dtype=dtype, device=device)
        else:
            self.gate_proj = LinearBase(hidden_size, intermediate_size, bias=False, dtype=dtype, device=device)
            self.up_proj = LinearBase(hidden_size, intermediate_size, bias=False, dtype=dtype, device=device)
        self.down_proj = LinearBase(intermediate_size, hidden_size, bias=False, dtype=dtype, device=device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return gated_mlp_forward(self, x)


def fuse_gated_mlps(model: nn.Module) -> int:
    """Bind :func:`gated_mlp_forward` to every GatedMLP-shaped submodule of ``model``; returns how many."""
    count = 0
    for module in model.modules():
        if isinstance(module, GatedMLP):
            count += 1
        elif all(hasattr(module, a) for a in ("gate_up_proj", "down_proj", "fuse")):
            module.forward = types.MethodType(gated_mlp_forward, module)
            count += 1
    return count
