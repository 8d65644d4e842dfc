"""The talker decoder layer's linears with their neighbours fused (qtts/models/talker.py:246-271).

The reference's decode loop runs, per layer::

    q, k, v = attn.project(layer.input_layernorm(hidden))         # norm, qkv_proj
    ...attention...
    hidden = residual + attn.o_proj(out)                           # o_proj, add
    hidden = hidden + layer.mlp(layer.post_attention_layernorm(hidden))   # norm, MLP, add

Each helper here computes one of those lines from the reference's own modules (anything
with the same attributes): ``norm_linear`` is ``linear(norm(x))``, ``linear_residual`` is
``residual + linear(x)`` and ``norm_mlp_residual`` is ``hidden + mlp(norm(hidden))``.  When
the linears carry the int8 weight-only method on strip weights, the norm runs inside the
GEMM that follows it, the residual add in the GEMM's epilogue and GatedMLP's activation in
the gate_up GEMM's epilogue, so a layer is four launches.  Anything else computes the
reference's composition unchanged, so a caller can switch its loop over unconditionally.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import ops, torch_ops  # noqa: F401  (torch_ops registers torch.ops.qtts)
from ..quant.base import weight_flags


def _int8_strips(linear: nn.Module, x: torch.Tensor) -> bool:
    """Whether ``linear`` runs x through the int8 weight-only strip kernels: its method, layout and
    x's dtype allow it, and its calibration routed x's row bucket to a kernel (not to F.linear on
    the kept weight, nor to the prefill route)."""
    method = getattr(linear, "quant_method", None)
    if not (getattr(method, "name", None) == "int8_weight_only" and getattr(linear, "int8_weight", None) is not None
            and getattr(linear, "int8_layout", None) == "strips" and x.is_cuda
            and x.dtype in (torch.bfloat16, torch.float16) and linear.in_features % 64 == 0):
        return False
    routed = getattr(method, "routes_to_kernel", None)
    return routed is None or routed(linear, x)


def _norm_eps(norm: nn.Module) -> float:
    for attr in ("eps", "variance_epsilon"):
        if hasattr(norm, attr):
            return float(getattr(norm, attr))
    raise AttributeError(f"{type(norm).__name__} has no eps")


def norm_linear(norm: nn.Module, linear: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """``linear(norm(x))``: input_layernorm + qkv_proj (talker.py:249), with the RMSNorm computed
    inside the int8 weight-only GEMM's prologue."""
    if _int8_strips(linear, x):
        return torch.ops.qtts.w8a16_fused_gemm_strips(x, linear.int8_weight, linear.out_features, linear.int8_scale,
                                                      linear.bias, ops.PRO_RMS_NORM, norm.weight, _norm_eps(norm),
                                                      None, ops.ALGO_AUTO | weight_flags(linear))
    return linear(norm(x))


def linear_residual(linear: nn.Module, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """``residual + linear(x)``: o_proj and the residual add (talker.py:270), the add in the GEMM's
    epilogue (the linear's output rounded to the activation dtype first, as torch adds two tensors)."""
    if _int8_strips(linear, x) and residual.shape[:-1] == x.shape[:-1] and residual.dtype == x.dtype:
        return torch.ops.qtts.w8a16_fused_gemm_strips(x, linear.int8_weight, linear.out_features, linear.int8_scale,
                                                      linear.bias, ops.PRO_NONE, None, 1e-6, residual,
                                                      ops.ALGO_AUTO | weight_flags(linear))
    return residual + linear(x)


def norm_mlp_residual(norm: nn.Module, mlp: nn.Module, hidden: torch.Tensor) -> torch.Tensor:
    """``hidden + mlp(norm(hidden))`` for a GatedMLP (talker.py:271; activation.py:142-147): the norm
    in the gate_up GEMM's prologue, ``silu(gate) * up`` in its epilogue, the residual add in the
    down GEMM's epilogue: two launches."""
    fused = getattr(mlp, "fuse", False)
    if fused and _int8_strips(mlp.gate_up_proj, hidden) and mlp.gate_up_proj.out_features % 2 == 0:
        up = mlp.gate_up_proj
        act = torch.ops.qtts.w8a16_gate_up_silu_strips(hidden, up.int8_weight, up.out_features, up.int8_scale,
                                                       up.bias, ops.PRO_RMS_NORM, norm.weight, _norm_eps(norm),
                                                       ops.ALGO_AUTO | weight_flags(up))
        return linear_residual(mlp.down_proj, act, hidden)
    if fused:
        gate, up = mlp.gate_up_proj.split(mlp.gate_up_proj(norm(hidden)))
    else:
        h = norm(hidden)
        gate, up = mlp.gate_proj(h), mlp.up_proj(h)
    return hidden + mlp.down_proj(F.silu(gate) * up)
