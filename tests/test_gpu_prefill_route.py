"""GPU parity of the weight-only methods' prefill route: dequantize the stored codes
(``qtts_dequant_strips``), then F.linear (quant/prefill.py).

* ``dequant_strips`` against torch evaluating the reference's dequantized weight,
  ``q.to(dtype) * scale[:, None]`` (qtts/quant/kernels.py:144-148), bit for bit: int8
  and e4m3 codes, bf16 / fp16 / fp32 scales, ragged N and K, a strided destination;
* a layer whose prefill bucket is routed there returns F.linear of that weight, bit for
  bit, and stays within the W8A16 bound of the fp64 oracle; smaller row counts keep the
  HIP kernels; the GatedMLP forward and graph replays take the route too;
* the calibration records a verdict for every prefill bucket and the layer's output
  is within the bound whichever route it chose.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from test_gpu_gemm import half_ulp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _bound(ref, dtype):
    rms = float(np.sqrt(np.mean(ref * ref)))
    return 1e-2 * rms + half_ulp(ref, dtype)


@pytest.mark.parametrize("n,k", [(12288, 2048), (2048, 6144), (100, 80), (33, 1000), (16, 16)])
def test_dequant_strips_matches_torch(ops, n, k):
    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = torch.randn(n, k, device="cuda", generator=g) * 0.02
    for wdt in (torch.bfloat16, torch.float16, torch.float32):
        for sdt in ({torch.float32, wdt} if wdt != torch.float32 else {torch.float32, torch.bfloat16}):
            q, s = ops.pack_int8(w.to(wdt if wdt != torch.float32 else torch.bfloat16), sdt)
            qs = ops.to_strips(q)
            want = q.to(wdt) * s.to(wdt)[:, None] if sdt == wdt else (q.float() * s.float()[:, None]).to(wdt)
            got = ops.dequant_strips(qs, n, k, s, wdt)
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), (wdt, sdt, int((got != want).sum()))
    # e4m3 codes (the fp8 weight-only layout: 64-column strips of e4m3 bytes), fp32 scale
    if k % 64 == 0:
        q8, s8 = ops.pack_fp8(w)
        qs8 = ops.fp8w_strips(q8)
        prod = q8.view(torch.float8_e4m3fn).float() * s8.reshape(-1, 1)  # exact codes times the scale, fp32
        # Bits, not values (torch.equal takes -0 for +0): products that tie at 16-bit precision
        # and -0 codes are where one rounding of the exact product (a fused multiply-convert)
        # differs from fp32 then 16-bit; numpy's IEEE conversion of the same fp32 products
        # agrees with torch's.
        for wdt, npdt in ((torch.bfloat16, None), (torch.float16, np.float16)):
            got = ops.dequant_strips(qs8, n, k, s8.reshape(-1), wdt, ops.CODE_E4M3)
            want = prod.to(wdt)
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
                (wdt, int((got.view(torch.int16) != want.view(torch.int16)).sum()))
            if npdt is not None:
                ieee = prod.cpu().numpy().astype(npdt).view(np.uint16)
                np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), ieee)
    # a strided destination leaves the columns past k alone
    q, s = ops.pack_int8(w.to(torch.bfloat16), torch.bfloat16)
    wide = torch.full((n, k + 24), 7.0, device="cuda", dtype=torch.bfloat16)
    ops.dequant_strips(ops.to_strips(q), n, k, s, torch.bfloat16, out=wide[:, :k])
    assert torch.equal(wide[:, :k], q.to(torch.bfloat16) * s[:, None])
    assert bool((wide[:, k:] == 7.0).all())


def _layer(n, k, seed, bias=True):
    from qtts_amd.layers import LinearBase
    torch.manual_seed(seed)
    lin = LinearBase(k, n, bias=bias, dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        for p in lin.parameters():
            p.normal_(0.0, 0.02)
    return lin


def test_int8_route_bits_and_bound(ops, monkeypatch):
    from qtts_amd.quant import int8 as I, prefill
    n, k = 4096, 2048
    lin = _layer(n, k, seed=1)
    w_bf16 = lin.weight.detach().clone()
    method = I.Int8WeightOnlyMethod(calibrate=False)
    method.process_weights(lin)
    lin.quant_method = method
    prefill.reserve(torch.device("cuda"), n, k, torch.bfloat16)
    lin.quant_algos = {1024: prefill.ALGO_DEQUANT_GEMM, 2048: prefill.ALGO_DEQUANT_GEMM}
    wq = ops.dequant_strips(lin.int8_weight, n, k, lin.int8_scale, torch.bfloat16)
    q = I.int8_weight_rowmajor(lin)
    assert torch.equal(wq, q.to(torch.bfloat16) * lin.int8_scale[:, None])
    for rows in (300, 1024, 1500):
        x = torch.randn(rows, k, device="cuda").to(torch.bfloat16)
        y = lin(x)
        assert torch.equal(y, F.linear(x, wq, lin.bias)), rows  # the route: exactly F.linear of that weight
        ref = O.w8a16_ref(x.float().cpu().numpy(), q.cpu().numpy(), lin.int8_scale.float().cpu().numpy(),
                          lin.bias.float().cpu().numpy())
        err = np.abs(y.double().cpu().numpy() - ref)
        assert (err <= _bound(ref, torch.bfloat16)).all(), (rows, float(err.max()))
    # rows outside the routed bucket keep the HIP kernels, and so do fp32 activations inside it
    x = torch.randn(64, k, device="cuda").to(torch.bfloat16)
    assert torch.equal(lin(x), ops.w8a16_gemm_strips(x, lin.int8_weight, n, lin.int8_scale, lin.bias))
    x32 = torch.randn(300, k, device="cuda")
    assert torch.equal(lin(x32), ops.w8a16_gemm(x32, q, lin.int8_scale, lin.bias))
    del w_bf16


def test_route_graph_replays_and_gated_mlp(ops, monkeypatch):
    from qtts_amd.layers import GatedMLP
    from qtts_amd.quant import int8 as I, prefill
    torch.manual_seed(2)
    mlp = GatedMLP(2048, 6144, dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        for p in mlp.parameters():
            p.normal_(0.0, 0.02)
    method = I.Int8WeightOnlyMethod(calibrate=False)
    for lin in (mlp.gate_up_proj, mlp.down_proj):
        method.process_weights(lin)
        lin.quant_method = method
        prefill.reserve(torch.device("cuda"), lin.out_features, lin.in_features, torch.bfloat16)
    x = torch.randn(512, 2048, device="cuda").to(torch.bfloat16)
    kernels = mlp(x)  # the HIP tile kernels
    mlp.gate_up_proj.quant_algos = {1024: prefill.ALGO_DEQUANT_GEMM}
    mlp.down_proj.quant_algos = {1024: prefill.ALGO_DEQUANT_GEMM}
    routed = mlp(x)
    assert torch.equal(routed, mlp.down_proj(ops.silu_mul(mlp.gate_up_proj(x))))  # both GEMMs on the route
    # against the HIP tile kernels: two GEMMs, each within the bar, and the rounded activation between
    ref = kernels.double().cpu().numpy()
    err = np.abs(routed.double().cpu().numpy() - ref)
    assert (err <= 3 * _bound(ref, torch.bfloat16)).all(), float(err.max())
    # graph capture: replays with fresh inputs match eager
    static_x = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        mlp(static_x)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = mlp(static_x)
    for i in range(3):
        static_x.copy_(torch.randn(512, 2048, device="cuda").to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, mlp(static_x)), f"replay {i}"


def test_calibration_records_prefill_verdicts(ops):
    """Both weight-only methods with calibration: every bucket decided; F.linear on the kept weight
    exactly where it beat every quantized route, else the prefill route exactly where it was the
    fastest candidate; the layer's output at the prefill row counts is F.linear of the original
    weight bit for bit on the F.linear route, and otherwise within the W8A16 bound of the HIP kernel
    on the same codes."""
    from qtts_amd.quant import fp8 as P, int8 as I, prefill
    from qtts_amd.quant.calibrate import ALGO_REFERENCE_GEMM, clear_cache
    clear_cache()
    n, k = 12288, 2048
    for method, kernel in (
            (I.Int8WeightOnlyMethod(calibrate=True),
             lambda lin, x: ops.w8a16_gemm_strips(x, lin.int8_weight, n, lin.int8_scale)),
            (P.Fp8WeightOnlyMethod(calibrate=True),
             lambda lin, x: ops.fp8w_gemm_strips(x, lin.fp8w_weight, n, lin.fp8w_scale))):
        lin = _layer(n, k, seed=3, bias=False)
        w_bf16 = lin.weight.detach().clone()
        method.process_weights(lin)
        report = method.calibration_report[(n, k)]
        assert sorted(report) == list(method.calibration_rows)
        if not method.applies_to(lin):
            continue  # declined over the decode buckets: stays on F.linear
        lin.quant_method = method
        table = lin.quant_algos
        assert sorted(table) == list(method.calibration_rows), "every bucket decided"
        loses = {rows for rows in method.calibration_rows
                 if report[rows]["timings"][report[rows]["best"]] > report[rows]["reference"]}
        assert {r for r, a in table.items() if a == ALGO_REFERENCE_GEMM} == loses, method.name
        assert (lin.weight.numel() > 0) == bool(loses), "the weight stays exactly when F.linear serves a bucket"
        for rows in prefill.PREFILL_BUCKETS:
            x = torch.randn(rows, k, device="cuda").to(torch.bfloat16)
            y = lin(x)
            if rows in loses:
                assert torch.equal(y, F.linear(x, w_bf16)), (method.name, rows)
                continue
            routed = table[rows] == prefill.ALGO_DEQUANT_GEMM
            assert routed == (report[rows]["best"] == "dequant"), (method.name, rows)
            ref = kernel(lin, x).double().cpu().numpy()
            err = np.abs(y.double().cpu().numpy() - ref)
            assert (err <= 2 * _bound(ref, torch.bfloat16)).all(), (method.name, rows, routed, float(err.max()))


def test_reference_route_keeps_weight_and_calls_f_linear(ops, monkeypatch):
    """Calibration where F.linear wins the 256-row bucket (timings forced on the host): the layer
    converts on its decode buckets, keeps its weight, reports it, and its 256-row calls are
    F.linear of that weight bit for bit while decode calls stay on the HIP kernel."""
    from qtts_amd import QuantConfig, quantize_module
    from qtts_amd.quant import calibrate as cal, int8 as I

    def fake_times(candidates, reference_call, *, key, use_graph=True, timer=None):
        rows = key[3]
        return 1.0, {name: (2.0 if rows == 256 else 0.5) for name in candidates}

    monkeypatch.setattr(cal, "time_candidates", fake_times)
    n, k = 2048, 2048
    lin = _layer(n, k, seed=4, bias=True)
    w_bf16 = lin.weight.detach().clone()
    model = torch.nn.Module()
    model.o_proj = lin
    method = I.Int8WeightOnlyMethod(calibrate=True, calibration_rows=(1, 8, 256))
    report = quantize_module(model, method, QuantConfig(method="int8_weight_only"), "talker")
    assert report["converted"] == 1 and report["kept_weight"] == 1 and method.kept_reference == 1
    assert lin.quant_algos[256] == cal.ALGO_REFERENCE_GEMM and lin.quant_algos[1] >= 0
    assert torch.equal(lin.weight, w_bf16)
    x = torch.randn(256, k, device="cuda").to(torch.bfloat16)
    assert torch.equal(lin(x), F.linear(x, w_bf16, lin.bias))
    x1 = torch.randn(1, k, device="cuda").to(torch.bfloat16)
    assert torch.equal(lin(x1), ops.w8a16_gemm_strips(x1, lin.int8_weight, n, lin.int8_scale, lin.bias,
                                                      lin.quant_algos[1]))
    # without keep_reference_routes the bucket keeps its fastest quantized route and the weight goes
    lin2 = _layer(n, k, seed=4, bias=True)
    method2 = I.Int8WeightOnlyMethod(calibrate=True, calibration_rows=(1, 8, 256), keep_reference_routes=False)
    method2.process_weights(lin2)
    assert lin2.quant_algos[256] >= 0 and lin2.weight.numel() == 0


def test_calibrated_half_strips_reach_the_kernel(ops, monkeypatch):
    """A talker down_proj whose calibration finds half strips fastest at the decode buckets (timings
    forced on the host): its table holds the half-strip code there, and its calls run that kernel --
    bit for bit the explicit half-strip call, and within the bar of the oracle -- with graph replays
    equal to eager."""
    from qtts_amd import _lib
    from qtts_amd.quant import calibrate as cal, int8 as I

    def fake_times(candidates, reference_call, *, key, use_graph=True, timer=None):
        return 1.0, {name: (0.1 if name == "skinny_half" else 0.5) for name in candidates}

    monkeypatch.setattr(cal, "time_candidates", fake_times)
    n, k = 2048, 6144
    lin = _layer(n, k, seed=6, bias=False)
    method = I.Int8WeightOnlyMethod(calibrate=True, calibration_rows=(1, 2, 4, 8, 16))
    method.process_weights(lin)
    lin.quant_method = method
    half = _lib.algo_code(_lib.ALGO_SKINNY_HALF)
    assert all(lin.quant_algos[r] == half for r in (1, 2, 4, 8, 16))
    q = I.int8_weight_rowmajor(lin)
    for m in (1, 3, 8, 12):  # 12: two row parts of 8 on half strips
        x = torch.randn(m, k, device="cuda").to(torch.bfloat16)
        y = lin(x)
        assert torch.equal(y, ops.w8a16_gemm_strips(x, lin.int8_weight, n, lin.int8_scale, None, half)), m
        ref = O.w8a16_ref(x.float().cpu().numpy(), q.cpu().numpy(), lin.int8_scale.float().cpu().numpy())
        err = np.abs(y.double().cpu().numpy() - ref)
        assert (err <= _bound(ref, torch.bfloat16)).all(), (m, float(err.max()))
    static_x = torch.randn(4, k, device="cuda").to(torch.bfloat16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lin(static_x)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = lin(static_x)
    for i in range(3):
        static_x.copy_(torch.randn(4, k, device="cuda").to(torch.bfloat16))
        lin(static_x * 0.5)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, lin(static_x)), f"replay {i}"
