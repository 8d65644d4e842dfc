"""GPU parity of the fp8 weight-only GEMM (Fp8WeightOnlyMethod, qtts/quant/fp8.py:92-123), through the C ABI.

Reference: the oracle's fp64 dequantize-then-matmul of the same e4m3 codes and fp32
scales (oracle/qtts_oracle.c), with the W8A16 tolerance of tests/test_gpu_gemm.py
(|y - ref| <= 1e-2 RMS + half an ulp of the output dtype).  The conversion of every
finite e4m3 code, at every byte position of a weight fragment, is checked exactly
through one-hot activation rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from test_gpu_gemm import PREDICTOR, TALKER, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _make(ops, m, n, k, dtype=torch.bfloat16, bias=False, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    x = torch.randn(m, k, device="cuda", generator=g).to(dtype)
    b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if bias else None
    q, s = ops.pack_fp8(w)
    return x, q, s, b


def _oracle(x, q, s, b):
    return O.fp8w_ref(x.float().cpu().numpy(), q.view(torch.uint8).cpu().numpy(), s.cpu().numpy(),
                      None if b is None else b.float().cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8w_every_code_every_position(ops, dtype):
    """One-hot activation rows read single codes: y = e4m3(q) exactly (unit scales), for all
    254 finite codes at all 64 columns of a chunk, through the staged skinny (M = 8), the
    direct skinny (M = 16) and the tile kernel (M = 64)."""
    n, k = 256, 64
    lut = O.e4m3_decode_table()
    codes = (np.arange(n)[:, None] + 37 * np.arange(k)[None, :]) % 256
    codes[(codes == 0x7F) | (codes == 0xFF)] = 0
    q = torch.from_numpy(codes.astype(np.uint8)).cuda()
    qs = ops.fp8w_strips(q)
    ones = torch.ones(n, device="cuda")  # bf16 and fp16 hold every e4m3 value exactly
    for rows in (range(0, 8), range(8, 24), range(0, 64)):
        cols = list(rows)
        x = torch.zeros(len(cols), k, device="cuda", dtype=dtype)
        x[torch.arange(len(cols)), torch.tensor(cols)] = 1.0
        y = ops.fp8w_gemm_strips(x, qs, n, ones)
        want = lut[codes[:, cols]].T
        np.testing.assert_array_equal(y.float().cpu().numpy(), want, err_msg=f"{dtype} rows {cols[0]}..{cols[-1]}")


@pytest.mark.parametrize("n,k", TALKER + PREDICTOR)
def test_fp8w_decode_shapes(ops, n, k):
    for m in (1, 2, 3, 4, 8, 12, 16):
        x, q, s, b = _make(ops, m, n, k, bias=(m % 2 == 0), seed=n + 3 * k + m)
        qs = ops.fp8w_strips(q)
        ref = _oracle(x, q, s, b)
        assert_close(ops.fp8w_gemm_strips(x, qs, n, s, b), ref, f"auto m={m} n={n} k={k}")
        for splits, waves, cpw in ((1, 4, 8), (2, 8, 8), (1, 16, 6), (3, 2, 8)):
            y = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(1, splits, waves, cpw))
            assert_close(y, ref, f"m={m} n={n} k={k} S={splits} W={waves} C={cpw}")
            # staged rows (9-16: in row parts of 8 on at most 128 strips with one split) and direct loads
            direct = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(1, splits, waves, cpw | 0x40))
            assert torch.equal(y, direct), f"staged != direct m={m} n={n} k={k} S={splits} W={waves}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8w_prefill_and_ragged(ops, dtype):
    for m, n, k in ((17, 4096, 2048), (64, 2048, 6144), (256, 12288, 2048), (130, 1030, 1024), (5, 100, 128),
                    (33, 48, 64), (24, 1024, 3072), (40, 2048, 2048), (64, 1000, 2048)):  # the last three: half
        # strips in row parts of 8 by the automatic choice
        x, q, s, b = _make(ops, m, n, k, dtype=dtype, bias=True, seed=m + n + k)
        qs = ops.fp8w_strips(q)
        ref = _oracle(x, q, s, b)
        assert_close(ops.fp8w_gemm_strips(x, qs, n, s, b), ref, f"auto m={m} n={n} k={k} {dtype}")
        if m > 16:
            eight = (ops.tile_shape(64, 128, 8), ops.tile_shape(64, 256, 8), ops.tile_shape(128, 256, 8),
                     ops.tile_shape(128, 128, 8, grid2=True), ops.tile_shape(128, 384, 8))
            for splits, shape in ((1, 0), (2, 0), (0, 0x21), (0, 0x12), (0, 0x23)) + tuple((0, e) for e in eight):
                y = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, 0, shape))
                assert_close(y, ref, f"tile m={m} n={n} k={k} S={splits} shape={shape:#x} {dtype}")
                if shape and shape != ops.tile_shape(128, 384, 8):  # 4 stages with and without read-ahead: the same bits
                    y4 = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, 4, shape))
                    y4ra = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, 4 | ops.TILE_READ_AHEAD, shape))
                    assert torch.equal(y4, y4ra), f"read-ahead m={m} n={n} k={k} shape={shape:#x} {dtype}"
            if (k // 64) % 2 == 0:  # two chunks a stage on the 4-wave 32 x 64 tile: the same bits as one
                t3264, ra = ops.tile_shape(32, 64), ops.TILE_READ_AHEAD
                for splits in (1, 2):
                    y1 = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, 4 | ra, t3264))
                    y2 = ops.fp8w_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, 4 | ra | ops.TILE_TWO_CHUNKS, t3264))
                    assert torch.equal(y1, y2), f"two chunks m={m} n={n} k={k} S={splits} {dtype}"


def test_fp8w_graph_replays(ops):
    x, q, s, b = _make(ops, 4, 2048, 6144, bias=True, seed=9)
    qs = ops.fp8w_strips(q)
    algo = ops.algo_code(1, 4, 8)
    eager = ops.fp8w_gemm_strips(x, qs, 2048, s, b, algo)
    static_x = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.fp8w_gemm_strips(static_x, qs, 2048, s, b, algo)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.fp8w_gemm_strips(static_x, qs, 2048, s, b, algo)
    for i in range(4):
        junk = ops.fp8w_gemm_strips(x * (i + 2), qs, 2048, s, b, ops.algo_code(1, 2, 16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"
        assert_close(junk, _oracle(x * (i + 2), q, s, b), f"junk {i}")


def test_fp8w_errors(ops):
    x, q, s, _ = _make(ops, 2, 64, 128)
    qs = ops.fp8w_strips(q)
    with pytest.raises(ValueError):
        ops.fp8w_gemm_strips(x[:, :64], qs, 64, s)  # the buffer holds K = 128
    with pytest.raises(ValueError, match="M <= 16"):
        ops.fp8w_gemm_strips(torch.randn(17, 128, device="cuda", dtype=torch.bfloat16), qs, 64, s, None,
                             ops.algo_code(1))
    x2, q2, s2, _ = _make(ops, 2, 64, 96)
    with pytest.raises(ValueError, match="64"):
        ops.fp8w_gemm_strips(x2, ops.fp8w_strips(q2), 64, s2)


def test_fp8w_method_hook(ops):
    """--quant-method fp8_weight_only: converted layers match the oracle on their stored codes;
    a layer with K % 64 != 0 is declined and keeps F.linear."""
    from qtts_amd import QuantConfig, apply_quantization
    from qtts_amd.layers.linear import LinearBase
    from qtts_amd.quant.fp8 import fp8w_weight_rowmajor
    torch.manual_seed(0)
    mod = torch.nn.Module()
    mod.o_proj = LinearBase(2048, 2048, dtype=torch.bfloat16, device="cuda")
    mod.text_proj_fc1 = LinearBase(2048, 1024, bias=True, dtype=torch.bfloat16, device="cuda")
    mod.odd = LinearBase(96, 64, dtype=torch.bfloat16, device="cuda")
    for p in mod.parameters():
        p.data.normal_(0, 0.02)
    w_ref = {name: getattr(mod, name).weight.detach().clone() for name in ("o_proj", "text_proj_fc1")}
    report = apply_quantization(QuantConfig(method="fp8_weight_only", calibrate=False), talker=mod)
    assert report["talker"]["converted"] == 2 and report["talker"]["declined"] == 1
    assert mod.odd.quant_method is None and mod.odd.weight.numel() == 96 * 64
    for name in ("o_proj", "text_proj_fc1"):
        lin = getattr(mod, name)
        q, s = ops.pack_fp8(w_ref[name])
        assert torch.equal(fp8w_weight_rowmajor(lin).view(torch.uint8), q.view(torch.uint8))
        assert torch.equal(lin.fp8w_scale, s)
        for m in (1, 8, 40):
            x = torch.randn(m, lin.in_features, device="cuda").to(torch.bfloat16)
            assert_close(lin(x), _oracle(x, q, s, lin.bias), f"{name} m={m}")
