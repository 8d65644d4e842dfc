"""The quantized-linear entry points as torch custom ops (``torch.ops.qtts.*``).

The quant methods' ``apply`` and the decoder-layer helpers call these, so graph capture,
``torch.compile`` and ``torch._dynamo`` see each quantized linear as one opaque op with a
known output shape instead of a ctypes call they cannot trace (the reference compiles the
code predictor's prefix forward with ``torch.compile(dynamic=True)``,
qtts/models/code_predictor.py:186-192).  Each op's real implementation is the ``ops``
wrapper of the same name (one C-ABI call on torch's current stream); its fake
implementation only computes the output's shape and dtype, so tracing never touches a
device.  The ops are functional: every output is a fresh tensor.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import ops

_LIB = "qtts"


def _rows_shape(x: torch.Tensor, n) -> tuple:
    return (*x.shape[:-1], n)


# ---- int8 weight-only (W8A16), qtts/quant/kernels.py:138-178 -------------------------------

@torch.library.custom_op(f"{_LIB}::w8a16_gemm", mutates_args=())
def w8a16_gemm(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor, bias: Optional[torch.Tensor],
               algo: int) -> torch.Tensor:
    return ops.w8a16_gemm(x, q, scale, bias, algo)


@w8a16_gemm.register_fake
def _(x, q, scale, bias, algo):
    return x.new_empty(_rows_shape(x, q.shape[0]))


@torch.library.custom_op(f"{_LIB}::w8a16_gemm_strips", mutates_args=())
def w8a16_gemm_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor, bias: Optional[torch.Tensor],
                      algo: int) -> torch.Tensor:
    return ops.w8a16_gemm_strips(x, qs, n, scale, bias, algo)


@w8a16_gemm_strips.register_fake
def _(x, qs, n, scale, bias, algo):
    return x.new_empty(_rows_shape(x, n))


# ---- fp8 W8A8 (Fp8Method.apply, qtts/quant/fp8.py:72-89) ------------------------------------

@torch.library.custom_op(f"{_LIB}::fp8_linear", mutates_args=())
def fp8_linear(x: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor, bias: Optional[torch.Tensor], div_mode: int,
               algo: int) -> torch.Tensor:
    return ops.fp8_linear(x, qw, sw, bias, div_mode, algo)


@fp8_linear.register_fake
def _(x, qw, sw, bias, div_mode, algo):
    return x.new_empty(_rows_shape(x, qw.shape[0]))


@torch.library.custom_op(f"{_LIB}::fp8_linear_strips", mutates_args=())
def fp8_linear_strips(x: torch.Tensor, qws: torch.Tensor, n: int, sw: torch.Tensor, bias: Optional[torch.Tensor],
                      div_mode: int, algo: int) -> torch.Tensor:
    return ops.fp8_linear_strips(x, qws, n, sw, bias, div_mode, algo)


@fp8_linear_strips.register_fake
def _(x, qws, n, sw, bias, div_mode, algo):
    return x.new_empty(_rows_shape(x, n))


# ---- int8 W8A8 (Int8Method.apply, qtts/quant/int8.py:145-160) -------------------------------

@torch.library.custom_op(f"{_LIB}::int8_linear", mutates_args=())
def int8_linear(x: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor, bias: Optional[torch.Tensor], div_mode: int,
                algo: int) -> torch.Tensor:
    return ops.int8_linear(x, qw, sw, bias, div_mode, algo)


@int8_linear.register_fake
def _(x, qw, sw, bias, div_mode, algo):
    return x.new_empty(_rows_shape(x, qw.shape[0]))


@torch.library.custom_op(f"{_LIB}::int8_linear_strips", mutates_args=())
def int8_linear_strips(x: torch.Tensor, qws: torch.Tensor, n: int, sw: torch.Tensor, bias: Optional[torch.Tensor],
                       div_mode: int, algo: int) -> torch.Tensor:
    return ops.int8_linear_strips(x, qws, n, sw, bias, div_mode, algo)


@int8_linear_strips.register_fake
def _(x, qws, n, sw, bias, div_mode, algo):
    return x.new_empty(_rows_shape(x, n))


# ---- fp8 weight-only (Fp8WeightOnlyMethod, qtts/quant/fp8.py:92-123) ------------------------

@torch.library.custom_op(f"{_LIB}::fp8w_gemm_strips", mutates_args=())
def fp8w_gemm_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor, bias: Optional[torch.Tensor],
                     algo: int) -> torch.Tensor:
    return ops.fp8w_gemm_strips(x, qs, n, scale, bias, algo)


@fp8w_gemm_strips.register_fake
def _(x, qs, n, scale, bias, algo):
    return x.new_empty(_rows_shape(x, n))


# ---- the weight-only methods' prefill route (quant/prefill.py) ------------------------------

@torch.library.custom_op(f"{_LIB}::dequant_linear", mutates_args=())
def dequant_linear(x: torch.Tensor, qs: torch.Tensor, codes: int, n: int, k: int, scale: torch.Tensor,
                   bias: Optional[torch.Tensor]) -> torch.Tensor:
    """``F.linear(x, dtype(codes * scale[:, None]), bias)``: the codes dequantized into the device's
    scratch buffer, then the library GEMM."""
    w = ops.dequant_scratch(x.device, n, k, x.dtype)
    ops.dequant_strips(qs, n, k, scale, x.dtype, codes, out=w)
    return F.linear(x, w, bias)


@dequant_linear.register_fake
def _(x, qs, codes, n, k, scale, bias):
    return x.new_empty(_rows_shape(x, n))


# ---- decoder-layer neighbours (qtts/layers/norm.py, activation.py; talker.py:246-271) -------

@torch.library.custom_op(f"{_LIB}::rms_norm", mutates_args=())
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return ops.rms_norm(x, weight, eps)


@rms_norm.register_fake
def _(x, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_LIB}::silu_mul", mutates_args=())
def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    return ops.silu_mul(gate_up)


@silu_mul.register_fake
def _(gate_up):
    return gate_up.new_empty(_rows_shape(gate_up, gate_up.shape[-1] // 2))


@torch.library.custom_op(f"{_LIB}::w8a16_silu_mul_gemm_strips", mutates_args=())
def w8a16_silu_mul_gemm_strips(gate_up: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                               bias: Optional[torch.Tensor], algo: int) -> torch.Tensor:
    return ops.w8a16_silu_mul_gemm_strips(gate_up, qs, n, scale, bias, algo)


@w8a16_silu_mul_gemm_strips.register_fake
def _(gate_up, qs, n, scale, bias, algo):
    return gate_up.new_empty(_rows_shape(gate_up, n))


@torch.library.custom_op(f"{_LIB}::w8a16_fused_gemm_strips", mutates_args=())
def w8a16_fused_gemm_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                            bias: Optional[torch.Tensor], prologue: int, norm_weight: Optional[torch.Tensor],
                            eps: float, residual: Optional[torch.Tensor], algo: int) -> torch.Tensor:
    return ops.w8a16_fused_gemm_strips(x, qs, n, scale, bias, prologue=prologue, norm_weight=norm_weight, eps=eps,
                                       residual=residual, algo=algo)


@w8a16_fused_gemm_strips.register_fake
def _(x, qs, n, scale, bias, prologue, norm_weight, eps, residual, algo):
    return x.new_empty(_rows_shape(x, n))


@torch.library.custom_op(f"{_LIB}::w8a16_gate_up_silu_strips", mutates_args=())
def w8a16_gate_up_silu_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                              bias: Optional[torch.Tensor], prologue: int, norm_weight: Optional[torch.Tensor],
                              eps: float, algo: int) -> torch.Tensor:
    return ops.w8a16_gate_up_silu_strips(x, qs, n, scale, bias, prologue=prologue, norm_weight=norm_weight, eps=eps,
                                         algo=algo)


@w8a16_gate_up_silu_strips.register_fake
def _(x, qs, n, scale, bias, prologue, norm_weight, eps, algo):
    return x.new_empty(_rows_shape(x, n // 2))


#: Every op this module registers, by name (``torch.ops.qtts.<name>``).
OPS = ("w8a16_gemm", "w8a16_gemm_strips", "fp8_linear", "fp8_linear_strips", "int8_linear", "int8_linear_strips",
       "fp8w_gemm_strips", "dequant_linear", "rms_norm", "silu_mul", "w8a16_silu_mul_gemm_strips",
       "w8a16_fused_gemm_strips", "w8a16_gate_up_silu_strips")
