"""Prefill route of the weight-only methods: dequantize the stored codes, then a library GEMM.

At prefill row counts a GEMM is compute-bound and the weight bytes no longer set its
time, so the bf16 baseline the calibration times against (F.linear, hipBLASLt on ROCm)
can beat the fused dequantize-in-registers tile kernel.  A quantized layer no longer
holds its bf16 weight, so the route rebuilds it: ``qtts_dequant_strips`` writes
``dtype(code * scale[n])`` -- the reference's dequantize-then-matmul form,
``q.to(dtype) * scale[:, None]`` (qtts/quant/kernels.py:144-148) -- into a per-device
scratch buffer, and F.linear multiplies by it.  The calibration times both per prefill
bucket (qtts/quant/calibrate.py:77-114 answers the same question at the calibration
batch) and records the route where it wins; every other call keeps the HIP kernels.
"""

from __future__ import annotations

from typing import Callable

import torch
import torch.nn.functional as F

from .. import ops
from .calibrate import pick_fastest

#: Algo value (Python side only) that sends a bucket's calls through dequantize + F.linear.
ALGO_DEQUANT_GEMM = -1

#: Row buckets whose route the calibration decides (the M_BUCKETS entries past 128 rows;
#: the last one also serves every larger call).
PREFILL_BUCKETS = (256, 1024, 2048)


def reserve(device: torch.device, n: int, k: int, dtype: torch.dtype) -> None:
    """Room for one ``[N, K]`` weight of ``dtype`` in the device's dequantization scratch."""
    ops.reserve_dequant_scratch(device, n * k * torch.empty((), dtype=dtype).element_size())


def dequant_linear(qs: torch.Tensor, codes: int, n: int, k: int, scale: torch.Tensor, x: torch.Tensor,
                   bias: torch.Tensor | None) -> torch.Tensor:
    """``F.linear(x, dtype(codes * scale[:, None]), bias)`` through the device's scratch buffer."""
    w = ops.dequant_scratch(x.device, n, k, x.dtype)
    ops.dequant_strips(qs, n, k, scale, x.dtype, codes, out=w)
    return F.linear(x, w, bias)


def calibrate(table: dict, key: str, qs: torch.Tensor, codes: int, n: int, k: int, scale: torch.Tensor,
              dtype: torch.dtype, device: torch.device,
              kernel_call: Callable[[torch.Tensor], object]) -> dict[int, bool]:
    """For each prefill bucket, time ``kernel_call(x)`` (the HIP kernel) against
    :func:`dequant_linear` on random rows; where the latter is faster by 3%, record
    ``table[(n, k, bucket)] = ALGO_DEQUANT_GEMM``.  Returns the verdict per bucket."""
    reserve(device, n, k, dtype)
    verdicts = {}
    for rows in PREFILL_BUCKETS:
        gen = torch.Generator(device=device).manual_seed(rows)
        x = torch.randn(rows, k, device=device, dtype=dtype, generator=gen)
        best = pick_fastest({"dequant": lambda x=x: dequant_linear(qs, codes, n, k, scale, x, None)},
                            lambda x=x: kernel_call(x), key=(key, n, k, rows, str(dtype)), margin=1.03)
        verdicts[rows] = best is not None
        if best is not None:
            table.setdefault((n, k, rows), ALGO_DEQUANT_GEMM)
    return verdicts
