"""GPU parity of the decoder layer around the W8A16 GEMM (qtts/models/talker.py:246-271), through the C ABI.

* ``qtts_rms_norm`` against the fp64 oracle (qtts/layers/norm.py:50-76): every element
  within one unit in the last place, at most one in a hundred not the oracle's value
  rounded; and against torch-CPU's eager RMSNorm fixtures within one unit (the bound
  the reference's own tests/test_norm.py:56-72 sets between its fused and eager paths).
* ``qtts_w8a16_fused_gemm_strips`` with the RMSNorm prologue against the oracle's GEMM of
  the oracle's normalized rows (W8A16 tolerance: |y - ref| <= 1e-2 RMS + half an ulp),
  and, where the norm runs as its own pass, bit for bit against qtts_rms_norm followed
  by qtts_w8a16_gemm_strips.
* The residual epilogue against torch's ``residual + linear(x)`` on this library's own
  GEMM output, bit for bit, fused (up to 8 rows) or not, in place or not; with the
  SiLU prologue as well (the down projection).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O
from test_gpu_gemm import PREDICTOR, TALKER, assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NORMED = [TALKER[0], TALKER[2], PREDICTOR[0], PREDICTOR[2], (100, 512)]  # qkv and gate_up
RESIDUAL = [TALKER[1], TALKER[3], PREDICTOR[1], PREDICTOR[3], (48, 512)]  # o_proj and down
_TD = {torch.bfloat16: O.DT_BF16, torch.float16: O.DT_F16, torch.float32: O.DT_F32}


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def _ulp(v: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[dtype]
    lo = {torch.bfloat16: -126, torch.float16: -14, torch.float32: -126}[dtype]
    e = np.maximum(np.floor(np.log2(np.maximum(np.abs(v), 1e-38))), lo)
    return 2.0 ** (e - mant)


def _round(v: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(v, np.float64)).to(dtype)


def _weights(ops, n, k, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    q, s = ops.pack_int8(w, dtype)
    return q, s, ops.to_strips(q)


def _oracle_gemm(h: torch.Tensor, q, s, b):
    return O.w8a16_ref(h.float().cpu().numpy(), q.cpu().numpy(), s.float().cpu().numpy(),
                       None if b is None else b.float().cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rms_norm_vs_oracle(ops, dtype):
    for m, k in ((1, 2048), (5, 1024), (3, 512), (4, 100), (2, 6144), (9, 8)):
        g = torch.Generator(device="cuda").manual_seed(m * 31 + k)
        x = (torch.randn(m, k, device="cuda", generator=g) * 2).to(dtype)
        x[0, : k // 4] *= 30.0
        w = (1 + 0.2 * torch.randn(k, device="cuda", generator=g)).to(dtype)
        y = ops.rms_norm(x, w, 1e-6)
        ref = O.rms_norm(_bits(x), _bits(w), 1e-6, _TD[dtype])
        got = y.double().cpu().numpy()
        units = 4 if dtype == torch.float32 else 1  # fp32: the roundings of inv and two products
        assert np.all(np.abs(got - ref) <= units * _ulp(ref, dtype)), f"{dtype} m={m} k={k}"
        if dtype != torch.float32:
            off = int((y.cpu() != _round(ref, dtype)).sum())
            assert off <= max(1, y.numel() // 100), f"{dtype} m={m} k={k}: {off} elements not rounded"


def test_rms_norm_golden(ops):
    z = np.load(os.path.join(GOLDEN, "rms_norm.npz"))
    eps = float(z["eps"])
    for dt, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        for width in (2048, 1024, 512):
            x = torch.from_numpy(z[f"{dt}.{width}.x"].view(np.int16)).view(tdt).cuda()
            w = torch.from_numpy(z[f"{dt}.{width}.w"].view(np.int16)).view(tdt).cuda()
            want = torch.from_numpy(z[f"{dt}.{width}.y"].view(np.int16)).view(tdt)
            y = ops.rms_norm(x, w, eps).cpu()
            diff = (y.double() - want.double()).abs().numpy()
            assert np.all(diff <= _ulp(want.double().numpy(), tdt)), f"{dt} width={width}"


@pytest.mark.parametrize("n,k", NORMED)
def test_norm_prologue(ops, n, k):
    from qtts_amd.ops import PRO_RMS_NORM
    for dtype in (torch.bfloat16, torch.float16):
        q, s, qs = _weights(ops, n, k, dtype, seed=n + k)
        for m in (1, 2, 3, 5, 8, 9, 12, 16):  # 9-16: fused in two row parts of 8
            g = torch.Generator(device="cuda").manual_seed(m + 5 * k)
            x = (torch.randn(m, k, device="cuda", generator=g) * 3).to(dtype)
            nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(dtype)
            b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if m != 2 else None
            h_ref = _round(O.rms_norm(_bits(x), _bits(nw), 1e-6, _TD[dtype]), dtype)
            ref = _oracle_gemm(h_ref, q, s, b)
            h = ops.rms_norm(x, nw, 1e-6)
            for algo in (0, ops.algo_code(1, 0, 4, 8), ops.algo_code(1, 0, 2, 8), ops.algo_code(1, 2, 8, 8),
                         ops.algo_code(1, 0, 16, 6)):
                what = f"{dtype} n={n} k={k} m={m} algo={algo:#x}"
                y = ops.w8a16_fused_gemm_strips(x, qs, n, s, b, prologue=PRO_RMS_NORM, norm_weight=nw, algo=algo)
                assert_close(y, ref, what)
                plain = ops.w8a16_gemm_strips(h, qs, n, s, b, algo)
                if ((algo >> 8) & 0xFF) > 1:  # split K: the norm runs as its own pass
                    assert torch.equal(y, plain), what
                else:  # up to 16 rows: fused, its sums in another order
                    assert_close(y, _oracle_gemm(h, q, s, b), what + " vs separate norm")


@pytest.mark.parametrize("n,k", RESIDUAL)
def test_residual_epilogue(ops, n, k):
    for dtype in (torch.bfloat16, torch.float16):
        q, s, qs = _weights(ops, n, k, dtype, seed=3 * n + k)
        for m in (1, 2, 3, 5, 8, 12, 16, 24, 40):  # past 16: half strips in row parts, else the separate add
            g = torch.Generator(device="cuda").manual_seed(m + n)
            x = torch.randn(m, k, device="cuda", generator=g).to(dtype)
            r = (torch.randn(m, n, device="cuda", generator=g) * 4).to(dtype)
            b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if m % 2 else None
            half = ops.algo_code(ops.ALGO_SKINNY_HALF)
            for algo in (0, ops.algo_code(1, 0, 4, 8), ops.algo_code(1, 3, 2, 8), ops.algo_code(1, 0, 8, 12), half):
                if m > 16 and algo not in (0, half):
                    continue  # past 16 rows: the automatic choice and half strips in row parts
                if algo == ops.algo_code(1, 0, 8, 12) and m > 8 and n > 2048:
                    continue  # 8 waves of 12 chunks: staged rows only (9-16 rows: on at most 128 strips)
                what = f"{dtype} n={n} k={k} m={m} algo={algo:#x}"
                lin = ops.w8a16_gemm_strips(x, qs, n, s, b, algo)
                want = r + lin
                y = ops.w8a16_fused_gemm_strips(x, qs, n, s, b, residual=r, algo=algo)
                assert torch.equal(y, want), what
                hidden = r.clone()
                out = ops.w8a16_fused_gemm_strips(x, qs, n, s, b, residual=hidden, out=hidden, algo=algo)
                assert out is hidden and torch.equal(hidden, want), what + " in place"
            assert_close(lin, _oracle_gemm(x, q, s, b), f"{dtype} n={n} k={k} m={m} vs oracle")


@pytest.mark.parametrize("n,k", [TALKER[3], PREDICTOR[3], (48, 512)])
def test_silu_and_residual(ops, n, k):
    from qtts_amd.ops import PRO_SILU_MUL
    for dtype in (torch.bfloat16, torch.float16):
        _, s, qs = _weights(ops, n, k, dtype, seed=n * k)
        f32 = s.float()
        for m in (1, 2, 3):
            g = torch.Generator(device="cuda").manual_seed(11 * m + k)
            gu = (torch.randn(m, 2 * k, device="cuda", generator=g) * 3).to(dtype)
            r = torch.randn(m, n, device="cuda", generator=g).to(dtype)
            for scale in (s, f32):
                for algo in (0, ops.algo_code(1, 0, 16, 6), ops.algo_code(1, 2, 4, 8),
                             ops.algo_code(ops.ALGO_SKINNY_HALF)):
                    what = f"{dtype} n={n} k={k} m={m} algo={algo:#x} scale {scale.dtype}"
                    want = r + ops.w8a16_silu_mul_gemm_strips(gu, qs, n, scale, None, algo)
                    y = ops.w8a16_fused_gemm_strips(gu, qs, n, scale, prologue=PRO_SILU_MUL, residual=r, algo=algo)
                    assert torch.equal(y, want), what


def test_fused_graph_replays(ops):
    """The norm prologue (a workgroup barrier over per-wave sums) and the residual epilogue
    under graph capture: every replay equals the eager result, with other calls between."""
    from qtts_amd.ops import PRO_RMS_NORM
    n, k = 12288, 2048
    _, s, qs = _weights(ops, n, k, torch.bfloat16, seed=1)
    x = torch.randn(1, k, device="cuda").to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, device="cuda")).to(torch.bfloat16)
    r = torch.randn(1, n, device="cuda").to(torch.bfloat16)

    def call(xx):
        return ops.w8a16_fused_gemm_strips(xx, qs, n, s, prologue=PRO_RMS_NORM, norm_weight=nw, residual=None), \
            ops.w8a16_fused_gemm_strips(xx, qs, n, s, residual=r[:, :n])

    eager = call(x)
    static = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        call(static)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call(static)
    for i in range(4):
        other = call(torch.randn(1, k, device="cuda").to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], eager[0]) and torch.equal(out[1], eager[1]), f"replay {i}"
        assert other[0].shape == (1, n)


def test_fused_errors(ops):
    from qtts_amd import _lib
    n, k = 64, 128
    _, s, qs = _weights(ops, n, k, torch.bfloat16, seed=2)
    x = torch.randn(2, k, device="cuda").to(torch.bfloat16)
    with pytest.raises(ValueError, match="norm weight"):
        ops.w8a16_fused_gemm_strips(x, qs, n, s, prologue=ops.PRO_RMS_NORM)
    with pytest.raises(ValueError, match="residual"):
        ops.w8a16_fused_gemm_strips(x, qs, n, s, residual=torch.zeros(2, n + 1, device="cuda", dtype=torch.bfloat16))
    buf = torch.zeros(2 * n + 8, device="cuda", dtype=torch.bfloat16)
    st = _lib.load().qtts_w8a16_fused_gemm_strips(
        x.data_ptr(), _lib.BF16, 2, k, k, 0, None, 0.0, qs.data_ptr(), n, s.data_ptr(), _lib.BF16, None,
        buf[8:].data_ptr(), n, buf.data_ptr(), n, 0, None, 0, None)
    assert st != 0 and "overlaps" in _lib.last_error()
    st = _lib.load().qtts_w8a16_fused_gemm_strips(
        x.data_ptr(), _lib.BF16, 2, k, k, 7, None, 0.0, qs.data_ptr(), n, s.data_ptr(), _lib.BF16, None,
        None, 0, buf.data_ptr(), n, 0, None, 0, None)
    assert st != 0 and "prologue" in _lib.last_error()
