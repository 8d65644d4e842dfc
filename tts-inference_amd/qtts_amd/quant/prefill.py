"""Prefill route of the weight-only methods: dequantize the stored codes, then a library GEMM.

At prefill row counts a GEMM is compute-bound and the weight bytes no longer set its
time, so the bf16 baseline the calibration times against (F.linear, hipBLASLt on ROCm)
can beat the fused dequantize-in-registers tile kernel.  A quantized layer no longer
holds its bf16 weight, so the route rebuilds it: ``qtts_dequant_strips`` writes
``dtype(code * scale[n])`` -- the reference's dequantize-then-matmul form,
``q.to(dtype) * scale[:, None]`` (qtts/quant/kernels.py:144-148) -- into a per-device
scratch buffer, and F.linear multiplies by it.  The calibration (calibrate.calibrate_buckets)
times it as one more candidate at each prefill bucket and records the route where it is
the fastest; every other call keeps the HIP kernels.
"""

from __future__ import annotations

import torch

from .. import ops, torch_ops  # noqa: F401  (torch_ops registers torch.ops.qtts)

#: Algo value (Python side only) that sends a bucket's calls through dequantize + F.linear.
ALGO_DEQUANT_GEMM = -1

#: Row buckets where the calibration times this route (the M_BUCKETS entries past 128 rows;
#: the last one also serves every larger call).
PREFILL_BUCKETS = (256, 1024, 2048)


def reserve(device: torch.device, n: int, k: int, dtype: torch.dtype) -> None:
    """Room for one ``[N, K]`` weight of ``dtype`` in the device's dequantization scratch."""
    ops.reserve_dequant_scratch(device, n * k * torch.empty((), dtype=dtype).element_size())


def dequant_linear(qs: torch.Tensor, codes: int, n: int, k: int, scale: torch.Tensor, x: torch.Tensor,
                   bias: torch.Tensor | None) -> torch.Tensor:
    """``F.linear(x, dtype(codes * scale[:, None]), bias)`` through the device's scratch buffer
    (``torch.ops.qtts.dequant_linear``)."""
    return torch.ops.qtts.dequant_linear(x, qs, codes, n, k, scale, bias)
