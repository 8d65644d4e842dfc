"""The weight policy flag (``QTTS_ALGO_STREAM``) on the GPU: the same bits with and without it.

The flag only changes how the decode kernels load the weight (non-temporal loads for a
submodel whose weights are streamed from HBM each step, include/qtts_amd.h), so every entry
point that can run a decode kernel must return identical outputs with it, at every row count
and forced configuration, and the tile kernels (more rows) must ignore it.  The method path
sets it per layer from ``quantize_module``'s decision (``layer.quant_stream``).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(2048, 2048), (2048, 6144), (12288, 2048), (1024, 3072), (96, 512)]
ROWS = (1, 2, 3, 4, 5, 8, 12, 16, 40)


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _weights(ops, n, k, seed, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype)
    return w, b


def _x(m, k, seed, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(m, k, device="cuda", generator=g) * 2).to(dtype)


def _same(fn, what):
    """fn(flags) with and without the weight policy flag: equal bits."""
    from qtts_amd import _lib
    a = fn(0)
    b = fn(_lib.ALGO_STREAM)
    torch.cuda.synchronize()
    assert torch.equal(a, b), (what, int((a != b).sum()))


@pytest.mark.parametrize("n,k", SHAPES)
def test_w8a16_stream_flag_same_bits(ops, n, k):
    for dtype in (torch.bfloat16, torch.float16):
        w, b = _weights(ops, n, k, seed=n + k, dtype=dtype)
        q, s = ops.pack_int8(w, dtype)
        qs = ops.to_strips(q)
        for m in ROWS:
            x = _x(m, k, seed=m * 7 + k, dtype=dtype)
            what = f"{dtype} n={n} k={k} m={m}"
            print(what, flush=True)
            algos = [ops.ALGO_AUTO]
            if m <= 16:
                algos.append(ops.algo_code(1, 2))  # two K splits: the split-K meeting
            if m <= 8 and k % 128 == 0:
                algos.append(ops.algo_code(ops.ALGO_SKINNY_HALF))
            for algo in algos:
                _same(lambda f: ops.w8a16_gemm_strips(x, qs, n, s, b, algo | f), f"{what} strips algo={algo:#x}")
            _same(lambda f: ops.w8a16_gemm(x, q, s, b, ops.ALGO_AUTO | f), f"{what} row-major")


@pytest.mark.parametrize("n,k", [(4096, 2048), (12288, 2048), (2048, 6144), (96, 512)])
def test_fused_forms_stream_flag_same_bits(ops, n, k):
    for m in (1, 2, 4, 8, 12):
        w, b = _weights(ops, n, k, seed=3 * n + k)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        g = torch.Generator(device="cuda").manual_seed(m + n)
        nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
        res = _x(m, n, seed=m + 5)
        x = _x(m, k, seed=m + 11)
        what = f"n={n} k={k} m={m}"
        print(what, flush=True)
        _same(lambda f: ops.w8a16_fused_gemm_strips(x, qs, n, s, b, prologue=ops.PRO_RMS_NORM, norm_weight=nw,
                                                    algo=f), f"{what} rmsnorm")
        _same(lambda f: ops.w8a16_fused_gemm_strips(x, qs, n, s, b, residual=res, algo=f), f"{what} residual")
        if n % 2 == 0:
            _same(lambda f: ops.w8a16_gate_up_silu_strips(x, qs, n, s, b, prologue=ops.PRO_RMS_NORM,
                                                          norm_weight=nw, algo=f), f"{what} gate_up+silu")
        gu = _x(m, 2 * k, seed=m + 17)
        _same(lambda f: ops.w8a16_silu_mul_gemm_strips(gu, qs, n, s, b, f), f"{what} silu_mul")


@pytest.mark.parametrize("n,k", [(2048, 2048), (2048, 6144), (1024, 3072)])
def test_fp8_and_int8_stream_flag_same_bits(ops, n, k):
    w, b = _weights(ops, n, k, seed=7 * n + k)
    qf, sf = ops.pack_fp8(w)
    qfs = ops.to_strips(qf)
    qfw = ops.fp8w_strips(qf)
    qi, si = ops.pack_int8(w, torch.float32)
    qis = ops.to_strips(qi)
    for m in ROWS + (64,):
        x = _x(m, k, seed=m * 3 + n)
        what = f"n={n} k={k} m={m}"
        print(what, flush=True)
        _same(lambda f: ops.fp8w_gemm_strips(x, qfw, n, sf, b, ops.ALGO_AUTO | f), f"{what} fp8 weight-only")
        _same(lambda f: ops.fp8_linear_strips(x, qfs, n, sf, b, ops.DIV_DEVICE, ops.ALGO_AUTO | f), f"{what} fp8")
        _same(lambda f: ops.int8_linear_strips(x, qis, n, si, b, ops.DIV_DEVICE, ops.ALGO_AUTO | f), f"{what} int8")
        if m <= 8:  # the two-kernel forms' skinny GEMMs on their own
            qx, sx = ops.quant_act_fp8(x)
            _same(lambda f: ops.w8a8_fp8_gemm_strips(qx, sx, qfs, n, sf, b, torch.bfloat16, ops.algo_code(1, 1) | f),
                  f"{what} fp8 skinny")


def test_method_layers_carry_the_policy(ops):
    """A converted layer with ``quant_stream`` set gives the bits it gives without it."""
    from qtts_amd.layers.linear import LinearBase
    from qtts_amd.quant.int8 import Int8WeightOnlyMethod
    torch.manual_seed(0)
    lin = LinearBase(2048, 2048, bias=True).cuda().to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
        lin.bias.normal_(0, 0.1)
    method = Int8WeightOnlyMethod(calibrate=False)
    method.process_weights(lin)
    lin.quant_method = method
    for m in (1, 4, 8, 16):
        x = _x(m, 2048, seed=m)
        lin.quant_stream = False
        a = lin(x)
        lin.quant_stream = True
        b = lin(x)
        assert torch.equal(a, b), m
