"""The reference's CPU path for the quantized linear, restated with torch on the CPU.

TEST INFRASTRUCTURE ONLY: used by bench.py's cpu_baseline leg and by tests, never
by the product package.

* ``naive_dequant_linear`` is the eager weight-only formula the reference uses as
  its baseline and as ``configs[0]``'s CPU path:
  ``F.linear(x, q.to(dtype) * scale[:, None])`` (examples/kernels/tune_w8_gemm.py:73-79,
  qtts/quant/kernels.py:6-15).  The dequantized weight is rounded to the
  activation dtype before the GEMM, exactly as that expression does.
* ``fp8_dequant_linear`` is the CPU form of the fp8 W8A8 path,
  ``(qx * sx) @ (qw * sw)^T`` in fp32, cast to the output dtype, bias added in the
  output dtype afterwards (qtts/quant/fp8.py:79-89).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def naive_dequant_linear(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor,
                         bias: torch.Tensor | None = None) -> torch.Tensor:
    return F.linear(x, q.to(x.dtype) * scale[:, None].to(x.dtype), bias)


def fp8_dequant_linear(qx: torch.Tensor, sx: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor,
                       out_dtype: torch.dtype = torch.bfloat16,
                       bias: torch.Tensor | None = None) -> torch.Tensor:
    a = qx.view(torch.float8_e4m3fn).float() * sx.reshape(-1, 1).float()
    b = qw.view(torch.float8_e4m3fn).float() * sw.reshape(-1, 1).float()
    out = (a @ b.t()).to(out_dtype)
    if bias is not None:
        out = out + bias.to(out_dtype)
    return out
