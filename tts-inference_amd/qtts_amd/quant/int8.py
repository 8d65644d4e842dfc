"""int8 quantization methods (qtts/quant/int8.py).

``Int8WeightOnlyMethod`` (W8A16) stores the weight as int8 with one scale per
output channel, keeps activations in the model dtype, and runs the gfx950 fused
dequantize-in-registers GEMM.  With ``calibrate`` it times, per layer shape, the
HIP kernel candidates against the unquantized F.linear (hipBLASLt on ROCm) inside
a HIP graph and keeps the fastest; a layer where no candidate wins by 5% keeps
its original weight and GEMM (qtts/quant/int8.py:79-111).  The timing runs at every
row bucket the callers produce (decode rows 1..16, code-predictor rows up to 128,
prefill buckets), the verdict comes from the decode buckets, and each bucket keeps
its fastest route: a skinny or tile kernel configuration, or at the prefill buckets
dequantizing the codes into a scratch buffer and calling F.linear (quant/prefill.py).
A converted layer that still loses to F.linear at some bucket keeps its weight too and
sends that bucket's calls to F.linear (``keep_reference_routes``), so no bucket runs
slower than the unquantized layer.  The per-bucket choices live on the layer
(``layer.quant_algos``), so layers of one shape but another dtype or device never share them.

``Int8Method`` (W8A8) quantizes activations per token at run time and multiplies
int8 codes on the int8 matrix cores (v_mfma_i32_16x16x64_i8) with exact int32
accumulation and the reference's fp32 epilogue, so its output is bit-identical to
the reference's torch._int_mm path for the same weights (qtts/quant/int8.py:129-160).
"""

from __future__ import annotations

import logging

import torch
import torch.nn.functional as F

from .. import _lib, ops
from . import prefill
from .base import QuantMethodBase, weight_flags
from .calibrate import ALGO_REFERENCE_GEMM, calibrate_buckets, rotating, rotation
from .kernels import kernel_available

logger = logging.getLogger("qtts_amd.quant.int8")

_INT8_MAX = 127.0

#: Row counts the kernel choice is tuned for: each call uses the entry of the
#: smallest bucket that holds its row count (decode rows 1..16 go to the skinny
#: kernel, prefill rows to the tile kernel).
M_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256, 1024, 2048)


def bucket_of(rows: int) -> int:
    for b in M_BUCKETS:
        if rows <= b:
            return b
    return M_BUCKETS[-1]


def quantize_weight_per_channel(weight: torch.Tensor, div_mode: int = _lib.DIV_DEVICE):
    """Symmetric per-output-channel int8 on the GPU: ``(q [N,K] int8, scale [N] fp32)``.

    Bit-exact with qtts/quant/int8.py:53-55 evaluated by torch on the GPU
    (``div_mode=DIV_DEVICE``) or on the CPU (``DIV_IEEE``).
    """
    return ops.pack_int8(weight, torch.float32, div_mode)


def layer_algo(layer, rows: int) -> int:
    """The calibrated route of ``layer`` for a call of ``rows`` rows (``ALGO_AUTO`` if none)."""
    return getattr(layer, "quant_algos", {}).get(bucket_of(rows), _lib.ALGO_AUTO)


def _candidates(rows: int, k: int | None = None) -> dict[str, int]:
    """Kernel configurations worth timing at ``rows`` for a weight of ``k`` input features (the
    algo bits of include/qtts_amd.h)."""
    # the automatic choice (row-split strips where whole strips leave compute units idle; the
    # skinny kernel, its m-blocks or the tile kernel by rows), kept unless a pin beats it clearly
    # (calibrate.AUTO_MARGIN)
    c: dict[str, int] = {"auto": _lib.ALGO_AUTO}
    if rows <= 64 and k is not None and k % 128 == 0:  # half strips (past 8 rows: in row parts of 8)
        c["skinny_half"] = _lib.algo_code(_lib.ALGO_SKINNY_HALF)
    if rows <= 64:  # skinny: up to 16 rows, or 64 on strip weights
        c["skinny"] = _lib.algo_code(_lib.ALGO_SKINNY)
        for s in (1, 2, 4):
            for w in (4, 8, 16):
                c[f"skinny_s{s}_w{w}"] = _lib.algo_code(_lib.ALGO_SKINNY, splits=s, waves=w)
    if rows > 16:  # tile: split counts, stages and tile shapes (4 waves: BM 32/64/128 x BN 64/128)
        c["tile"] = _lib.algo_code(_lib.ALGO_TILE)
        for s in (1, 2, 4):
            c[f"tile_s{s}"] = _lib.algo_code(_lib.ALGO_TILE, splits=s)
        for bm in (32, 64, 128):
            for bn in (64, 128):
                shape = _lib.tile_shape(bm, bn)
                for p in (3, 4):
                    c[f"tile_bm{bm}_bn{bn}_p{p}"] = _lib.algo_code(_lib.ALGO_TILE, 0, p, shape)
                c[f"tile_bm{bm}_bn{bn}_p4ra"] = _lib.algo_code(_lib.ALGO_TILE, 0, 4 | _lib.TILE_READ_AHEAD, shape)
        if k is not None and k % 128 == 0:  # two chunks a stage (an odd chunk count a split drops the candidate)
            for s in (1, 2):
                c[f"tile_bm32_bn64_c2_s{s}"] = _lib.algo_code(
                    _lib.ALGO_TILE, s, 4 | _lib.TILE_READ_AHEAD | _lib.TILE_TWO_CHUNKS, _lib.tile_shape(32, 64))
        c.update(tile8_candidates())
    return c


def tile8_candidates() -> dict[str, int]:
    """The 8-wave tiles (4 stages read ahead) in one and two splits."""
    c: dict[str, int] = {}
    for bm, bn, grid2 in ((64, 128, False), (64, 256, False), (128, 256, False), (128, 128, True)):
        for s in (1, 2):
            c[f"tile8_bm{bm}_bn{bn}{'_g2' if grid2 else ''}_s{s}"] = _lib.algo_code(
                _lib.ALGO_TILE, s, 4 | _lib.TILE_READ_AHEAD, _lib.tile_shape(bm, bn, 8, grid2))
    return c


def int8_weight_rowmajor(layer) -> torch.Tensor:
    """The packer's row-major ``[N, K]`` int8 bytes of a converted layer."""
    if getattr(layer, "int8_layout", "rowmajor") == "strips":
        return ops.from_strips(layer.int8_weight, layer.out_features, layer.in_features, _lib.STRIP_INT8)
    return layer.int8_weight


def _strips_ok(layer) -> bool:
    """The strip kernels take 16-bit activations and K % 16 == 0; other layers stay row-major."""
    return layer.in_features % 16 == 0 and layer.weight.dtype in (torch.bfloat16, torch.float16)


class Int8WeightOnlyMethod(QuantMethodBase):
    """int8 weights, model-dtype activations, dequantized inside the GEMM."""

    name = "int8_weight_only"

    def __init__(self, calibrate: bool = True, calibration_batch: int = 16, div_mode: int = _lib.DIV_DEVICE,
                 calibration_rows: tuple[int, ...] = M_BUCKETS, timer=None, keep_reference_routes: bool = True,
                 rotate_weights: bool = True) -> None:
        available, reason = kernel_available()
        if not available:
            raise RuntimeError(f"int8 weight-only needs the gfx950 fused kernel: {reason}")
        self.calibrate = calibrate
        self.calibration_batch = calibration_batch
        self.calibration_rows = tuple(sorted(set(calibration_rows)))
        self.timer = timer
        #: Keep a converted layer's weight for the buckets where F.linear on it beat every
        #: quantized route (else those buckets run the fastest quantized route anyway).
        self.keep_reference_routes = keep_reference_routes
        #: Time each shape over copies of its weight that together exceed the L2s (calibrate.rotation),
        #: as the weights stream in a decode step, rather than one weight's repeated calls.
        self.rotate_weights = rotate_weights
        #: (N, K) -> per-bucket timings of the last calibration (calibrate_buckets' report)
        self.calibration_report: dict[tuple[int, int], dict] = {}
        self.div_mode = div_mode
        self.quantized = 0
        self.declined = 0
        #: converted layers that kept their weight for F.linear at some bucket
        self.kept_reference = 0

    def _profitable(self, layer, q: torch.Tensor, scale: torch.Tensor, layout: str) -> tuple[bool, dict[int, int]]:
        """Per-bucket calibration (calibrate.calibrate_buckets): every HIP candidate, and the
        prefill route at the prefill buckets, against F.linear at each row bucket in
        ``calibration_rows``; the layer converts when it wins over the decode buckets (rows up
        to ``calibration_batch``) and each bucket then runs its fastest route, F.linear on the
        kept weight where that was faster than every quantized one.  Returns the verdict and
        the per-bucket table."""
        if not self.calibrate:
            return True, {}
        weight = layer.weight
        if not torch.cuda.is_available() or weight.device.type != "cuda":
            return False, {}
        n, k = layer.out_features, layer.in_features
        strips = layout == "strips"
        kk = k if strips else None  # row-split strips exist on strip weights only
        ops.reserve_workspace(weight.device, max(ops.workspace_bytes(_lib.OP_W8A16, r, n, k, a)
                                                 for r in self.calibration_rows
                                                 for a in _candidates(r, kk).values()))
        copies = rotation(n * k) if self.rotate_weights else 1
        qs = [q] + [q.clone() for _ in range(copies - 1)]
        ws = [weight] + [weight.detach().clone() for _ in range(copies - 1)]
        f = _lib.ALGO_STREAM if self.stream_weights else 0  # timed under the layer's weight policy
        if strips:
            kernel = rotating([lambda x, a, q=q_: ops.w8a16_gemm_strips(x, q, n, scale, None, a | f) for q_ in qs])
        else:
            kernel = rotating([lambda x, a, q=q_: ops.w8a16_gemm(x, q, scale, None, a | f) for q_ in qs])
        routes = {}
        if strips and any(r in prefill.PREFILL_BUCKETS for r in self.calibration_rows):
            prefill.reserve(weight.device, n, k, weight.dtype)
            route = (prefill.ALGO_DEQUANT_GEMM,
                     rotating([lambda x, q=q_: prefill.dequant_linear(q, _lib.CODE_INT8, n, k, scale, x, None)
                               for q_ in qs]))
            routes = {r: {"dequant": route} for r in self.calibration_rows if r in prefill.PREFILL_BUCKETS}
        accept, table, report = calibrate_buckets(  # the policy is part of the cache key
            "int8_wo_stream" if self.stream_weights else "int8_wo", n, k, weight.dtype, weight.device,
            self.calibration_rows, max(1, self.calibration_batch),
            lambda rows: _candidates(rows, kk), kernel, rotating([lambda x, w=w_: F.linear(x, w, None) for w_ in ws]),
            routes, timer=self.timer, keep_reference=self.keep_reference_routes, inner=copies)
        del qs, ws
        self.calibration_report[(n, k)] = report
        return accept, table

    def process_weights(self, layer) -> None:
        weight = layer.weight
        q, scale = ops.pack_int8(weight, weight.dtype, self.div_mode)
        # Keep the MFMA-native strip layout only: a permutation of the packed bytes
        # (int8_weight_rowmajor recovers them), read by 1 KiB-contiguous wave loads.
        layout = "strips" if _strips_ok(layer) else "rowmajor"
        if layout == "strips":
            q = ops.to_strips(q, _lib.STRIP_INT8)
        accept, table = self._profitable(layer, q, scale, layout)
        if not accept:
            self.declined += 1
            # Leaving quant_method unset keeps the layer on F.linear.
            layer.register_buffer("int8_weight", None, persistent=False)
            return
        # apply (and the decoder helpers' fused forms) never allocate up to ops.WORKSPACE_ROWS rows
        for op in (_lib.OP_W8A16, _lib.OP_W8A16_SILU, _lib.OP_W8A16_FUSED):
            ops.reserve_for_rows(weight.device, op, layer.out_features, layer.in_features)
        layer.register_buffer("int8_weight", q, persistent=False)
        layer.register_buffer("int8_scale", scale, persistent=False)
        layer.int8_layout = layout
        layer.quant_algos = dict(table)
        self.quantized += 1
        if ALGO_REFERENCE_GEMM in table.values():
            # F.linear serves some bucket: the weight stays (and counts in the memory report).
            self.kept_reference += 1
            return
        # Drop the full-precision weight, or the memory report would claim a saving it did not make.
        layer.weight = torch.nn.Parameter(torch.empty(0, dtype=weight.dtype, device=weight.device),
                                          requires_grad=False)

    def applies_to(self, layer) -> bool:
        return getattr(layer, "int8_weight", None) is not None

    @staticmethod
    def _reference_route(layer, x: torch.Tensor, algo: int) -> bool:
        """Whether this call goes to F.linear on the layer's kept weight."""
        return algo == ALGO_REFERENCE_GEMM and layer.weight.numel() > 0 and x.dtype == layer.weight.dtype

    def routes_to_kernel(self, layer, x: torch.Tensor) -> bool:
        """Whether a call of ``x`` on this layer runs a HIP kernel (not F.linear or the prefill route)."""
        k = layer.in_features
        algo = layer_algo(layer, x.numel() // k if k else 0)
        return algo not in (ALGO_REFERENCE_GEMM, prefill.ALGO_DEQUANT_GEMM)

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        n, k = layer.out_features, layer.in_features
        rows = x.numel() // k if k else 0
        algo = layer_algo(layer, rows)
        if self._reference_route(layer, x, algo):
            return F.linear(x, layer.weight, bias)
        if algo == prefill.ALGO_DEQUANT_GEMM and layer.int8_layout == "strips" and x.dtype in (torch.bfloat16,
                                                                                             torch.float16):
            return prefill.dequant_linear(layer.int8_weight, _lib.CODE_INT8, n, k, layer.int8_scale, x, bias)
        if algo < 0:  # a route's marker never reaches a kernel
            algo = _lib.ALGO_AUTO
        f = weight_flags(layer)
        if layer.int8_layout == "strips":
            if x.dtype in (torch.bfloat16, torch.float16):
                return torch.ops.qtts.w8a16_gemm_strips(x, layer.int8_weight, n, layer.int8_scale, bias, algo | f)
            # e.g. fp32 activations into a bf16-calibrated layer: correct, not fast
            return torch.ops.qtts.w8a16_gemm(x, int8_weight_rowmajor(layer), layer.int8_scale, bias, _lib.ALGO_AUTO)
        return torch.ops.qtts.w8a16_gemm(x, layer.int8_weight, layer.int8_scale, bias, algo | f)

    def apply_gate_up_silu(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor | None:
        """``F.silu(gate) * up`` of this fused gate_up layer's output (qtts/layers/activation.py:142-147)
        in one call; on strip weights with 16-bit activations, decode rows get the activation from
        the GEMM's epilogue.  None when this layer cannot (the caller then runs the plain path)."""
        if layer.int8_layout != "strips" or x.dtype not in (torch.bfloat16, torch.float16):
            return None
        n, k = layer.out_features, layer.in_features
        if n % 2:
            return None
        rows = x.numel() // k if k else 0
        algo = layer_algo(layer, rows)
        if algo < 0:  # F.linear or the prefill route serves this bucket: the plain path
            return None
        if (algo & 0xFF) in (_lib.ALGO_SKINNY_HALF, _lib.ALGO_SKINNY_QUARTER):
            algo = _lib.ALGO_AUTO  # the pair kernel runs whole strips (two per workgroup)
        return torch.ops.qtts.w8a16_gate_up_silu_strips(x, layer.int8_weight, n, layer.int8_scale, bias,
                                                       ops.PRO_NONE, None, 1e-6, algo | weight_flags(layer))

    def apply_silu_mul(self, layer, gate_up: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        """``layer(F.silu(gate) * up)`` from GatedMLP's fused gate_up output (qtts/layers/activation.py:
        142-147): on strip weights one call, with the activation inside the GEMM for a single row."""
        n, k = layer.out_features, layer.in_features
        if gate_up.shape[-1] != 2 * k:
            raise ValueError(f"gate_up has {gate_up.shape[-1]} columns for a down projection with K={k}")
        if layer.int8_layout == "strips" and gate_up.dtype in (torch.bfloat16, torch.float16):
            rows = gate_up.numel() // (2 * k) if k else 0
            algo = layer_algo(layer, rows)
            if algo >= 0:
                return torch.ops.qtts.w8a16_silu_mul_gemm_strips(gate_up, layer.int8_weight, n, layer.int8_scale,
                                                                 bias, algo | weight_flags(layer))
        return self.apply(layer, torch.ops.qtts.silu_mul(gate_up), bias)


class Int8Method(QuantMethodBase):
    """W8A8: per-token activation scales, per-channel weight scales, int8 GEMM (qtts/quant/int8.py:129-160).

    ``process_weights`` packs the weight exactly as quantize_weight_per_channel does
    and keeps the unrounded fp32 scale (int8.py:136-140); the codes go into the strip
    layout when K % 16 == 0 (row-major otherwise) instead of the reference's [K, N]
    transpose for torch._int_mm.  ``apply`` is one C call: per-token quantization in
    the activation dtype, the int8 GEMM, and ``(f32(acc) * sx) * sw + bias`` rounded
    once to the activation dtype.  No row padding (int8.py:150-155) is needed.
    """

    name = "int8"

    def __init__(self, div_mode: int = _lib.DIV_DEVICE) -> None:
        self.div_mode = div_mode

    def process_weights(self, layer) -> None:
        weight = layer.weight
        q, scale = quantize_weight_per_channel(weight, self.div_mode)
        n, k = layer.out_features, layer.in_features
        if k % 16 == 0:
            layer.register_buffer("int8_weight", ops.to_strips(q, _lib.STRIP_INT8), persistent=False)
            layer.int8_layout = "strips"
        else:
            layer.register_buffer("int8_weight", q, persistent=False)
            layer.int8_layout = "rowmajor"
        layer.register_buffer("int8_scale", scale, persistent=False)
        ops.reserve_for_rows(weight.device, _lib.OP_INT8_LINEAR, n, k)
        layer.weight = torch.nn.Parameter(torch.empty(0, dtype=weight.dtype, device=weight.device),
                                          requires_grad=False)

    def applies_to(self, layer) -> bool:
        return getattr(layer, "int8_weight", None) is not None

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        algo = _lib.ALGO_AUTO | weight_flags(layer)
        if layer.int8_layout == "strips":
            return torch.ops.qtts.int8_linear_strips(x, layer.int8_weight, layer.out_features, layer.int8_scale, bias,
                                                     self.div_mode, algo)
        return torch.ops.qtts.int8_linear(x, layer.int8_weight, layer.int8_scale, bias, self.div_mode, algo)
