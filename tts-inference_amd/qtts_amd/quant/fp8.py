"""fp8 (OCP e4m3) quantization methods (qtts/quant/fp8.py).

``Fp8Method`` is W8A8: per-output-channel e4m3 weights, per-token e4m3
activations quantized at run time, and a gfx950 fp8 MFMA GEMM with the rowwise x
columnwise scale epilogue in place of torch._scaled_mm.  It is applied
uniformly, as in the reference (qtts/quant/fp8.py:52-89).

``Fp8WeightOnlyMethod`` (fp8 weights, bf16 / fp16 activations) is the fused kernel
the reference's stub names as the right home for fp8 weights (qtts/quant/fp8.py:92-123,
where it raises NotImplementedError because Triton could not load e4m3): the W8A16
kernels with the e4m3 codes converted in registers.  Calibrated per layer shape
like the int8 weight-only method, with the same per-layer bucket table and the same
F.linear route for buckets no quantized route wins.
"""

from __future__ import annotations

import torch

import torch.nn.functional as F

from .. import _lib, ops
from . import prefill
from .base import QuantMethodBase, weight_flags
from .calibrate import ALGO_REFERENCE_GEMM, calibrate_buckets, rotating, rotation
from .int8 import layer_algo, tile8_candidates
from .kernels import kernel_available

_FP8_MAX = 448.0


def quantize_weight_fp8(weight: torch.Tensor, div_mode: int = _lib.DIV_DEVICE):
    """Symmetric per-output-channel e4m3 on the GPU: ``(q [N,K] float8_e4m3fn, scale [N] fp32)``."""
    return ops.pack_fp8(weight, div_mode)


class Fp8Method(QuantMethodBase):
    """W8A8 e4m3 on CDNA4 fp8 MFMA."""

    name = "fp8"

    def __init__(self, div_mode: int = _lib.DIV_DEVICE) -> None:
        self.div_mode = div_mode

    def process_weights(self, layer) -> None:
        weight = layer.weight
        q, scale = quantize_weight_fp8(weight, self.div_mode)
        # The reference keeps the [K, N] column-major view of the packed bytes for
        # _scaled_mm; this backend keeps the MFMA-native strip layout of the same
        # bytes instead (fp8_weight_rowmajor recovers them).  The scale is [1, N]
        # fp32 as in the reference.
        if layer.in_features % 32 == 0:
            layer.register_buffer("fp8_weight", ops.to_strips(q, _lib.STRIP_FP8), persistent=False)
            layer.fp8_layout = "strips"
        else:  # the strip kernels need K % 32 == 0; keep the reference's [K, N] view
            layer.register_buffer("fp8_weight", q.t(), persistent=False)
            layer.fp8_layout = "rowmajor"
        layer.register_buffer("fp8_scale", scale.reshape(1, -1), persistent=False)
        # apply never allocates up to ops.WORKSPACE_ROWS rows (and under capture never does)
        for op in (_lib.OP_FP8_LINEAR, _lib.OP_W8A8_FP8):
            ops.reserve_for_rows(weight.device, op, layer.out_features, layer.in_features)
        layer.weight = torch.nn.Parameter(torch.empty(0, dtype=weight.dtype, device=weight.device),
                                          requires_grad=False)

    def applies_to(self, layer) -> bool:
        return getattr(layer, "fp8_weight", None) is not None

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        algo = _lib.ALGO_AUTO | weight_flags(layer)
        if layer.fp8_layout == "strips":
            return torch.ops.qtts.fp8_linear_strips(x, layer.fp8_weight, layer.out_features,
                                                    layer.fp8_scale.reshape(-1), bias, self.div_mode, algo)
        return torch.ops.qtts.fp8_linear(x, layer.fp8_weight.t(), layer.fp8_scale.reshape(-1), bias, self.div_mode,
                                         algo)


def fp8_weight_rowmajor(layer) -> torch.Tensor:
    """The packer's row-major ``[N, K]`` e4m3 bytes of a converted layer."""
    if getattr(layer, "fp8_layout", "rowmajor") == "strips":
        return ops.from_strips(layer.fp8_weight, layer.out_features, layer.in_features, _lib.STRIP_FP8)
    return layer.fp8_weight.t()


def _fp8w_candidates(rows: int) -> dict[str, int]:
    """Kernel configurations worth timing at ``rows`` (the algo bits of include/qtts_amd.h)."""
    # the automatic choice (row-split strips where whole strips leave compute units idle), kept
    # unless a pin beats it clearly (calibrate.AUTO_MARGIN)
    c: dict[str, int] = {"auto": _lib.ALGO_AUTO}
    if rows <= 16:
        c["skinny"] = _lib.algo_code(_lib.ALGO_SKINNY)
        for s in (1, 2, 4):
            for w in (4, 8, 16):
                c[f"skinny_s{s}_w{w}"] = _lib.algo_code(_lib.ALGO_SKINNY, splits=s, waves=w)
    else:
        c["tile"] = _lib.algo_code(_lib.ALGO_TILE)
        for s in (1, 2, 4):
            c[f"tile_s{s}"] = _lib.algo_code(_lib.ALGO_TILE, splits=s)
        for bm in (32, 64, 128):
            for bn in (64, 128):
                c[f"tile_bm{bm}_bn{bn}"] = _lib.algo_code(_lib.ALGO_TILE, 0, 0, _lib.tile_shape(bm, bn))
        c.update(tile8_candidates())
    return c


def fp8w_weight_rowmajor(layer) -> torch.Tensor:
    """The packer's row-major ``[N, K]`` e4m3 codes of an fp8 weight-only layer."""
    q = ops.from_strips(layer.fp8w_weight, layer.out_features, layer.in_features, _lib.STRIP_INT8)
    return q.view(torch.float8_e4m3fn)


class Fp8WeightOnlyMethod(QuantMethodBase):
    """fp8 (e4m3) weights, bf16 / fp16 activations, converted inside the GEMM.

    The weight is packed as quantize_weight_fp8 packs it (qtts/quant/fp8.py:45-49: per
    channel fp32 scale, e4m3 codes) and stored in the 64-column strip layout
    (``fp8w_weight``, ``fp8w_scale``).  Layers the kernels cannot take (K % 64 != 0 or
    a non-16-bit weight dtype) and, with ``calibrate``, layers where no kernel
    configuration beats F.linear by 5% keep their weight and F.linear.
    """

    name = "fp8_weight_only"

    def __init__(self, calibrate: bool = True, calibration_batch: int = 16, div_mode: int = _lib.DIV_DEVICE,
                 calibration_rows: tuple[int, ...] | None = None, timer=None, keep_reference_routes: bool = True,
                 rotate_weights: bool = True) -> None:
        from .int8 import M_BUCKETS
        available, reason = kernel_available()
        if not available:
            raise RuntimeError(f"fp8 weight-only needs the gfx950 fused kernel: {reason}")
        self.calibrate = calibrate
        self.calibration_batch = calibration_batch
        self.calibration_rows = tuple(sorted(set(calibration_rows or M_BUCKETS)))
        self.timer = timer
        self.keep_reference_routes = keep_reference_routes
        self.rotate_weights = rotate_weights
        self.calibration_report: dict[tuple[int, int], dict] = {}
        self.div_mode = div_mode
        self.quantized = 0
        self.declined = 0
        self.kept_reference = 0

    def _profitable(self, layer, qs: torch.Tensor, scale: torch.Tensor) -> tuple[bool, dict[int, int]]:
        """Per-bucket calibration, as Int8WeightOnlyMethod._profitable (calibrate.calibrate_buckets)."""
        if not self.calibrate:
            return True, {}
        weight = layer.weight
        n, k = layer.out_features, layer.in_features
        ops.reserve_workspace(weight.device, max(ops.workspace_bytes(_lib.OP_FP8W, r, n, k, a)
                                                 for r in self.calibration_rows for a in _fp8w_candidates(r).values()))
        copies = rotation(n * k) if self.rotate_weights else 1
        qss = [qs] + [qs.clone() for _ in range(copies - 1)]
        ws = [weight] + [weight.detach().clone() for _ in range(copies - 1)]
        routes = {}
        if any(r in prefill.PREFILL_BUCKETS for r in self.calibration_rows):
            prefill.reserve(weight.device, n, k, weight.dtype)
            route = (prefill.ALGO_DEQUANT_GEMM,
                     rotating([lambda x, q=q_: prefill.dequant_linear(q, _lib.CODE_E4M3, n, k, scale, x, None)
                               for q_ in qss]))
            routes = {r: {"dequant": route} for r in self.calibration_rows if r in prefill.PREFILL_BUCKETS}
        f = _lib.ALGO_STREAM if self.stream_weights else 0  # timed under the layer's weight policy
        accept, table, report = calibrate_buckets(  # the policy is part of the cache key
            "fp8_wo_stream" if self.stream_weights else "fp8_wo", n, k, weight.dtype, weight.device,
            self.calibration_rows, max(1, self.calibration_batch),
            _fp8w_candidates,
            rotating([lambda x, a, q=q_: ops.fp8w_gemm_strips(x, q, n, scale, None, a | f) for q_ in qss]),
            rotating([lambda x, w=w_: F.linear(x, w, None) for w_ in ws]), routes, timer=self.timer,
            keep_reference=self.keep_reference_routes, inner=copies)
        del qss, ws
        self.calibration_report[(n, k)] = report
        return accept, table

    def _decline(self, layer) -> None:
        self.declined += 1
        layer.register_buffer("fp8w_weight", None, persistent=False)

    def process_weights(self, layer) -> None:
        weight = layer.weight
        if layer.in_features % 64 or weight.dtype not in (torch.bfloat16, torch.float16):
            self._decline(layer)
            return
        q, scale = quantize_weight_fp8(weight, self.div_mode)
        qs = ops.fp8w_strips(q)
        accept, table = self._profitable(layer, qs, scale)
        if not accept:
            self._decline(layer)
            return
        ops.reserve_for_rows(weight.device, _lib.OP_FP8W, layer.out_features, layer.in_features)
        layer.register_buffer("fp8w_weight", qs, persistent=False)
        layer.register_buffer("fp8w_scale", scale, persistent=False)
        layer.quant_algos = dict(table)
        self.quantized += 1
        if ALGO_REFERENCE_GEMM in table.values():
            self.kept_reference += 1  # F.linear serves some bucket: the weight stays
            return
        layer.weight = torch.nn.Parameter(torch.empty(0, dtype=weight.dtype, device=weight.device),
                                          requires_grad=False)

    def applies_to(self, layer) -> bool:
        return getattr(layer, "fp8w_weight", None) is not None

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"fp8 weight-only layers take bf16 or fp16 activations, got {x.dtype}")
        n, k = layer.out_features, layer.in_features
        rows = x.numel() // k if k else 0
        algo = layer_algo(layer, rows)
        if algo == ALGO_REFERENCE_GEMM and layer.weight.numel() > 0 and x.dtype == layer.weight.dtype:
            return F.linear(x, layer.weight, bias)
        if algo == prefill.ALGO_DEQUANT_GEMM:  # x is bf16 / fp16 here, as the scratch was sized for
            return prefill.dequant_linear(layer.fp8w_weight, _lib.CODE_E4M3, n, k, layer.fp8w_scale, x, bias)
        return torch.ops.qtts.fp8w_gemm_strips(x, layer.fp8w_weight, n, layer.fp8w_scale, bias,
                                               max(algo, 0) | weight_flags(layer))
