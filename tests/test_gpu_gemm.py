"""GPU parity of the W8A16 and fp8 W8A8 GEMMs, through the C ABI.

Reference: the fp64 dequantize-then-matmul of the oracle (oracle/qtts_oracle.c)
on the same packed bytes and stored scales, at sizes it finishes in seconds;
a torch fp32 GEMM on the GPU at the large prefill shapes.

Tolerance (north star: max |err| <= 1e-2 x output RMS, bf16 outputs): every
element must satisfy |y - ref| <= 1e-2 * RMS(ref) + ulp_bf16(ref) / 2.  The
half-ulp term is what rounding even the exact result to bf16 costs: at a 4-sigma
output (|y| in [4, 8), RMS ~0.9) it is 0.0156, already above 1e-2 * RMS, so no
bf16-output kernel could meet the bar without it.  Errors of a real defect (a
dropped K chunk, a wrong scale row, a missing bias) are O(RMS) and still fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

TALKER = [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144)]
PREDICTOR = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def half_ulp(ref: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    mant = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}[dtype]
    a = np.abs(ref).astype(np.float64)
    e = np.floor(np.log2(np.maximum(a, 1e-30)))
    if dtype == torch.float16:
        e = np.maximum(e, -14)
    return np.ldexp(1.0, (e - (mant - 1)).astype(np.int64)) / 2


def assert_close(y: torch.Tensor, ref: np.ndarray, what: str = "", inter: np.ndarray | None = None) -> float:
    """``inter``: an intermediate the reference formula itself rounds to y's dtype (the fp8 path
    rounds the scaled product before adding the bias, qtts/quant/fp8.py:79-89); its half-ulp is
    part of the reference's own rounding budget and is added to the bound."""
    yv = y.float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, np.float64)
    assert yv.shape == ref.shape, (yv.shape, ref.shape)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    err = np.abs(yv - ref)
    bound = 1e-2 * rms + half_ulp(ref, y.dtype)
    if inter is not None:
        bound = bound + half_ulp(np.asarray(inter, np.float64), y.dtype)
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements out of tolerance; max err {err.max():.4g}, "
                           f"rms {rms:.4g}, worst at {np.unravel_index(np.argmax(err - bound), err.shape)}")
    return float(err.max() / rms) if rms else 0.0


def _make(m, n, k, dtype=torch.bfloat16, bias=False, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    x = torch.randn(m, k, device="cuda", generator=g).to(dtype)
    b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if bias else None
    return x, w, b


def _oracle_w8a16(x, q, scale, b):
    return O.w8a16_ref(x.float().cpu().numpy(), q.cpu().numpy(), scale.float().cpu().numpy(),
                       None if b is None else b.float().cpu().numpy())


def _sample_rows(m: int) -> torch.Tensor:
    """Rows of a large-M output checked against the fp64 oracle: the first and last, both sides of
    every 64- and 128-row tile edge up to 256, and about 20 more spread over M."""
    rows = {0, m - 1} | {r for e in (32, 64, 128, 256) for r in (e - 1, e) if r < m}
    rows |= set(range(1, m, max(1, m // 20)))
    return torch.tensor(sorted(rows), device="cuda")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_w8a16_brute_force_small(ops, dtype):
    """Tails in M, N and K, bias on and off, every dtype; includes the generic path (K % 16 != 0)."""
    for m in (1, 2, 3):
        for n in (1, 7, 16, 17, 33):
            for k in (16, 64, 130, 257):
                for has_bias in (False, True):
                    x, w, b = _make(m, n, k, dtype, has_bias, seed=m * 1000 + n * 10 + k)
                    q, s = ops.pack_int8(w, dtype)
                    y = ops.w8a16_gemm(x, q, s, b)
                    assert y.dtype == dtype and y.shape == (m, n)
                    assert_close(y, _oracle_w8a16(x, q, s, b), f"m={m} n={n} k={k} bias={has_bias}")


@pytest.mark.parametrize("n,k", TALKER + PREDICTOR)
def test_w8a16_skinny_decode_shapes(ops, n, k):
    for m in (1, 2, 4, 8, 16):
        print(f"skinny n={n} k={k} m={m}", flush=True)
        x, w, b = _make(m, n, k, seed=n + k + m)
        q, s = ops.pack_int8(w, torch.bfloat16)
        y = ops.w8a16_gemm(x, q, s, None, ops.algo_code(1))
        assert_close(y, _oracle_w8a16(x, q, s, None), f"skinny m={m} n={n} k={k}")


def test_w8a16_skinny_configs_agree(ops):
    """Every split / wave count gives an in-tolerance, run-to-run deterministic answer."""
    m, n, k = 5, 2048, 6144
    x, w, b = _make(m, n, k, bias=True, seed=9)
    q, s = ops.pack_int8(w, torch.bfloat16)
    ref = _oracle_w8a16(x, q, s, b)
    for splits in (1, 2, 3, 4, 8, 16):
        for waves in (1, 2, 4, 8, 16):
            algo = ops.algo_code(1, splits, waves)
            y1 = ops.w8a16_gemm(x, q, s, b, algo)
            y2 = ops.w8a16_gemm(x, q, s, b, algo)
            assert torch.equal(y1, y2), f"non-deterministic at splits={splits} waves={waves}"
            assert_close(y1, ref, f"splits={splits} waves={waves}")


@pytest.mark.parametrize("m", [17, 32, 33, 64, 100, 128, 256])
def test_w8a16_tile_vs_oracle(ops, m):
    for n, k in ((2048, 2048), (1024, 3072), (130 * 16, 1024)):
        x, w, b = _make(m, n, k, bias=(m % 2 == 1), seed=m + n)
        q, s = ops.pack_int8(w, torch.bfloat16)
        ref = _oracle_w8a16(x, q, s, b)
        y = ops.w8a16_gemm(x, q, s, b, ops.algo_code(2))
        assert_close(y, ref, f"tile m={m} n={n} k={k}")
        for splits in (1, 2, 4):
            y2 = ops.w8a16_gemm(x, q, s, b, ops.algo_code(2, splits))
            assert_close(y2, ref, f"tile m={m} n={n} k={k} splits={splits}")


@pytest.mark.parametrize("n,k", TALKER)
def test_w8a16_prefill_full_shapes_vs_fp32(ops, n, k):
    """configs[3] shapes at M in {64, 256, 1024} against a torch fp32 GEMM of the dequantized weight."""
    for m in (64, 256, 1024):
        x, w, _ = _make(m, n, k, seed=n * 3 + m)
        q, s = ops.pack_int8(w, torch.bfloat16)
        y = ops.w8a16_gemm(x, q, s)
        ref = (x.float() @ (q.float() * s.float()[:, None]).t()).double().cpu().numpy()
        assert_close(y, ref, f"prefill m={m} n={n} k={k}")


def test_w8a16_hip_graph_replays(ops):
    """Capture split-K GEMMs into a graph; every replay, between eager work, matches eager."""
    x, w, b = _make(4, 2048, 2048, bias=True, seed=5)
    q, s = ops.pack_int8(w, torch.bfloat16)
    algo = ops.algo_code(1, 4)
    eager = ops.w8a16_gemm(x, q, s, b, algo)
    static_x = x.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        ops.w8a16_gemm(static_x, q, s, b, algo)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.w8a16_gemm(static_x, q, s, b, algo)
    for i in range(5):
        junk = ops.w8a16_gemm(x * (i + 2), q, s, b, algo)  # eager work sharing the workspace
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"
        assert_close(junk, _oracle_w8a16(x * (i + 2), q, s, b))


def test_w8a16_errors(ops):
    x, w, _ = _make(2, 32, 64)
    q, s = ops.pack_int8(w, torch.bfloat16)
    with pytest.raises(ValueError, match="K=48"):
        ops.w8a16_gemm(x[:, :48], q, s)
    with pytest.raises(ValueError):
        ops.w8a16_gemm(torch.randn(17, 64, device="cuda", dtype=torch.bfloat16), q, s, None, ops.algo_code(1))
    # an explicit split count with no room for it in the workspace is an error, not a silent downgrade
    from qtts_amd import _lib
    x2, w2, _ = _make(2, 64, 1024)
    q2, s2 = ops.pack_int8(w2, torch.bfloat16)
    y2 = torch.empty(2, 64, dtype=torch.bfloat16, device="cuda")
    st = _lib.load().qtts_w8a16_gemm(x2.data_ptr(), 1, 2, 1024, 1024, q2.data_ptr(), 64, 1024, s2.data_ptr(), 1,
                                     None, y2.data_ptr(), 64, ops.algo_code(1, 2), None, 0,
                                     torch.cuda.current_stream().cuda_stream)
    assert st == _lib.ERR_WORKSPACE


def test_w8a16_empty(ops):
    q = torch.zeros(8, 64, dtype=torch.int8, device="cuda")
    s = torch.ones(8, dtype=torch.bfloat16, device="cuda")
    y = ops.w8a16_gemm(torch.zeros(0, 64, dtype=torch.bfloat16, device="cuda"), q, s)
    assert y.shape == (0, 8)
    # K = 0: the sum is empty, the output is the bias (0 without one), as in the reference kernel
    q0 = torch.zeros(8, 0, dtype=torch.int8, device="cuda")
    b = torch.arange(8, dtype=torch.bfloat16, device="cuda")
    y0 = ops.w8a16_gemm(torch.zeros(3, 0, dtype=torch.bfloat16, device="cuda"), q0, s, b)
    assert torch.equal(y0, b.expand(3, 8))


# ---- fp8 W8A8 -----------------------------------------------------------------------------

def _oracle_w8a8(qx, sx, qw, sw, bias):
    """(exact fp64 result, the scaled product the reference rounds before its bias add)."""
    y = O.w8a8_ref(qx.view(torch.uint8).cpu().numpy(), sx.cpu().numpy(), qw.view(torch.uint8).cpu().numpy(),
                   sw.cpu().numpy())
    if bias is None:
        return y, None
    return y + bias.double().cpu().numpy(), y


def _fp8_inputs(m, n, k, seed, outliers=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g)
    if outliers:
        mask = torch.rand(m, k, device="cuda", generator=g) < 0.01
        x = torch.where(mask, torch.sign(x) * 20.0, x)
    w = torch.randn(n, k, device="cuda", generator=g) * 0.02
    return x.to(torch.bfloat16), w.to(torch.bfloat16)


@pytest.mark.parametrize("n,k", TALKER)
def test_fp8_gemm_vs_oracle(ops, n, k):
    for m in (1, 8, 16, 17, 64):
        x, w = _fp8_inputs(m, n, k, seed=n + m)
        qw, sw = ops.pack_fp8(w)
        qx, sx = ops.quant_act_fp8(x)
        y = ops.w8a8_fp8_gemm(qx, sx, qw, sw, None, torch.bfloat16)
        ref, _ = _oracle_w8a8(qx, sx, qw, sw, None)
        assert_close(y, ref, f"fp8 m={m} n={n} k={k}")


def test_fp8_gemm_m256_vs_fp32(ops):
    for n, k in TALKER:
        x, w = _fp8_inputs(256, n, k, seed=n)
        qw, sw = ops.pack_fp8(w)
        qx, sx = ops.quant_act_fp8(x)
        y = ops.w8a8_fp8_gemm(qx, sx, qw, sw, None, torch.bfloat16)
        a = qx.float() * sx[:, None]
        bm = qw.float() * sw[:, None]
        ref = (a @ bm.t()).double().cpu().numpy()
        assert_close(y, ref, f"fp8 m=256 n={n} k={k}")


def test_fp8_small_and_odd(ops):
    for m, n, k in ((1, 1, 32), (3, 17, 64), (2, 33, 130), (5, 16, 96), (20, 40, 256)):
        x, w = _fp8_inputs(m, n, k, seed=m * n + k, outliers=False)
        b = torch.randn(n, device="cuda").to(torch.bfloat16)
        qw, sw = ops.pack_fp8(w)
        y = ops.fp8_linear(x, qw, sw, b)
        qx, sx = ops.quant_act_fp8(x)
        ref, inter = _oracle_w8a8(qx, sx, qw, sw, b)
        assert_close(y, ref, f"fp8 m={m} n={n} k={k}", inter)


# ---- strip layout ---------------------------------------------------------------------------

def _strips_numpy(q: np.ndarray, ch: int) -> np.ndarray:
    """The strip layout written straight from its definition (include/qtts_amd.h)."""
    n, k = q.shape
    strips, nch = -(-n // 16), -(-k // ch)
    pad = np.zeros((strips * 16, nch * ch), q.dtype)
    pad[:n, :k] = q
    out = np.zeros(strips * nch * 16 * ch, q.dtype)
    for s in range(strips):
        for c in range(nch):
            base = (s * nch + c) * 16 * ch
            for h in range(ch // 64):
                for lane in range(64):
                    row = 16 * s + lane % 16
                    col = c * ch + (lane // 16) * (ch // 4) + 16 * h
                    off = base + h * 1024 + lane * 16
                    out[off:off + 16] = pad[row, col:col + 16]
    return out


@pytest.mark.parametrize("kind,ch", [(0, 64), (1, 128)])
def test_strip_layout_definition_and_roundtrip(ops, kind, ch):
    rng = np.random.default_rng(kind)
    for n, k in ((1, 16), (16, 64), (17, 100), (33, 130), (40, 256), (5, 2048)):
        q = rng.integers(-127, 128, (n, k)).astype(np.int8)
        qt = torch.from_numpy(q).cuda()
        if kind == 1:
            qt = qt.view(torch.float8_e4m3fn)
        qs = ops.to_strips(qt, kind)
        assert qs.numel() == ops.strip_bytes(n, k, kind)
        got = qs.reshape(-1).view(torch.int8).cpu().numpy()
        np.testing.assert_array_equal(got, _strips_numpy(q, ch), err_msg=f"n={n} k={k}")
        back = ops.from_strips(qs, n, k, kind)
        assert torch.equal(back.view(torch.int8), torch.from_numpy(q).cuda())


@pytest.mark.parametrize("n,k", TALKER + PREDICTOR)
def test_w8a16_strips_decode_shapes(ops, n, k):
    for m in (1, 2, 4, 8, 16):
        print(f"strips n={n} k={k} m={m}", flush=True)
        x, w, b = _make(m, n, k, bias=(m == 4), seed=n + 3 * k + m)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        ref = _oracle_w8a16(x, q, s, b)
        y = ops.w8a16_gemm_strips(x, qs, n, s, b)
        assert_close(y, ref, f"strips auto m={m} n={n} k={k}")
        for splits, waves, cpw in ((1, 4, 4), (2, 8, 8), (4, 16, 6), (3, 2, 8), (1, 16, 4), (1, 1, 4)):
            y2 = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(1, splits, waves, cpw))
            assert_close(y2, ref, f"strips m={m} n={n} k={k} S={splits} W={waves} C={cpw}")


@pytest.mark.parametrize("xdt,sdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                      (torch.bfloat16, torch.float32)])
def test_w8a16_strips_staged_rows_match_direct(ops, xdt, sdt):
    """Decode rows (M <= 8, and 9-16 in two row parts of 8 without a split) stage their
    activation rows through LDS; algo bit 30 loads them straight from global memory instead.  Same
    operands in the same order: equal bits, for every (waves, chunks) pair built with staging,
    ragged N and a bias, and the oracle bound."""
    for (n, k) in ((2048, 2048), (2048, 6144), (1000, 1024), (1030, 3072), (48, 512)):
        for m in (1, 2, 3, 4, 5, 8, 9, 12, 16):
            x, w, b = _make(m, n, k, dtype=xdt, bias=(m % 2 == 1), seed=n + k + m)
            q, s = ops.pack_int8(w, sdt)
            qs = ops.to_strips(q)
            ref = _oracle_w8a16(x, q, s, b)
            # the automatic choice (its waves may differ from the direct kernel's: oracle only)
            assert_close(ops.w8a16_gemm_strips(x, qs, n, s, b), ref, f"auto m={m} n={n} k={k} {xdt} {sdt}")
            for splits, waves, cpw in ((1, 1, 8), (1, 2, 8), (1, 4, 8), (2, 8, 8), (1, 16, 6)):
                staged = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(1, splits, waves, cpw))
                direct = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(1, splits, waves, cpw | 0x40))
                what = f"m={m} n={n} k={k} S={splits} W={waves} C={cpw} {xdt} {sdt}"
                assert torch.equal(staged, direct), what
                assert_close(staged, ref, what)
            # 8 waves of 12 chunks: staged only (the automatic choice for K = 6144 from 2 rows)
            y = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(1, 0, 8, 12))
            assert_close(y, ref, f"m={m} n={n} k={k} W=8 C=12 {xdt} {sdt}")


def test_w8a16_strips_ragged_and_tile(ops):
    for m, n, k in ((3, 17, 16), (5, 100, 80), (1, 33, 2064), (16, 1000, 1008), (17, 100, 80), (64, 2040, 2048),
                    (130, 1030, 1040), (256, 2048, 2048)):
        x, w, b = _make(m, n, k, bias=True, seed=m * 7 + n + k)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        y = ops.w8a16_gemm_strips(x, qs, n, s, b)
        assert_close(y, _oracle_w8a16(x, q, s, b), f"strips m={m} n={n} k={k}")
        if m > 16:
            for splits in (1, 2, 4):
                y2 = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits))
                assert_close(y2, _oracle_w8a16(x, q, s, b), f"strips tile m={m} n={n} k={k} S={splits}")


def test_w8a16_strips_graph_replays_split(ops):
    x, w, b = _make(8, 2048, 6144, bias=True, seed=77)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    algo = ops.algo_code(1, 4, 8)
    eager = ops.w8a16_gemm_strips(x, qs, 2048, s, b, algo)
    assert torch.equal(eager, ops.w8a16_gemm_strips(x, qs, 2048, s, b, algo)), "split-K result is not deterministic"
    static_x = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.w8a16_gemm_strips(static_x, qs, 2048, s, b, algo)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.w8a16_gemm_strips(static_x, qs, 2048, s, b, algo)
    for i in range(4):
        ops.w8a16_gemm_strips(x * 3, qs, 2048, s, b, ops.algo_code(1, 2, 16))  # another split count in between
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


@pytest.mark.parametrize("n,k", TALKER)
def test_fp8_strips_vs_oracle(ops, n, k):
    for m in (1, 8, 16, 17, 256):
        x, w = _fp8_inputs(m, n, k, seed=n + m + 1)
        qw, sw = ops.pack_fp8(w)
        qws = ops.to_strips(qw)
        qx, sx = ops.quant_act_fp8(x)
        ref, _ = _oracle_w8a8(qx, sx, qw, sw, None) if m <= 64 else (None, None)
        if ref is None:
            ref = ((qx.float() * sx[:, None]) @ (qw.float() * sw[:, None]).t()).double().cpu().numpy()
        y = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, None, torch.bfloat16)
        assert_close(y, ref, f"fp8 strips m={m} n={n} k={k}")
        if m > 64:  # and the fp64 oracle itself on a sample of the rows
            idx = _sample_rows(m)
            assert_close(y[idx], _oracle_w8a8(qx[idx].contiguous(), sx[idx].contiguous(), qw, sw, None)[0],
                         f"fp8 strips m={m} n={n} k={k} oracle")
        if m <= 16:
            for splits, waves in ((1, 4), (2, 8), (4, 16)):
                y2 = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, None, torch.bfloat16, ops.algo_code(1, splits, waves))
                assert_close(y2, ref, f"fp8 strips m={m} n={n} k={k} S={splits} W={waves}")
        y3 = ops.fp8_linear_strips(x, qws, n, sw)
        assert_close(y3, ref, f"fp8 linear strips m={m} n={n} k={k}")


def test_fp8_strips_half_strips(ops):
    """Decode rows on layers with few strips (at most 64, or 128 with K >= 4096) take half strips in
    the fp8 GEMM: two workgroups of 8 weight rows per strip, two 128-column chunks per MFMA on its
    diagonal blocks.  Every M in 1..8, ragged N, bias on and off, and every output dtype, against
    the oracle and the whole-strip kernel (forced), which sums the chunks in another order."""
    for n, k in ((2048, 6144), (1000, 512), (40, 256), (72, 768)):
        print(f"fp8 half strips n={n} k={k}", flush=True)
        x8, w = _fp8_inputs(8, n, k, seed=n + k + 5)
        qw, sw = ops.pack_fp8(w)
        qws = ops.to_strips(qw)
        for m in range(1, 9):
            qx, sx = ops.quant_act_fp8(x8[:m].contiguous())
            odt = (torch.bfloat16, torch.float16, torch.float32)[m % 3]
            b = (torch.randn(n, device="cuda") * 0.1).to(odt) if m % 2 else None
            ref, inter = _oracle_w8a8(qx, sx, qw, sw, b)
            y = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt)
            assert_close(y, ref, f"fp8 half strips m={m} n={n} k={k} {odt}", inter)
            whole = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt, ops.algo_code(1))
            assert_close(whole, ref, f"fp8 whole strips m={m} n={n} k={k} {odt}", inter)


def test_kernel_timer_times_eager_launches_only(ops):
    """The bench's kernel timer: one event pair per eager launch, none for captured launches,
    and the timed launches still compute the same result."""
    x, w, b = _make(4, 2048, 2048, bias=True, seed=91)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    ref = ops.w8a16_gemm_strips(x, qs, 2048, s, b)
    with ops.KernelTimer(max_launches=8) as t:
        outs = [ops.w8a16_gemm_strips(x, qs, 2048, s, b) for _ in range(5)]
    assert t.launches == 5 and t.untimed == 0
    assert 0.0 < t.mean_ms < 10.0, t.mean_ms
    for o in outs:
        assert torch.equal(o, ref)
    with ops.KernelTimer(max_launches=2) as t:
        for _ in range(3):
            ops.w8a16_gemm_strips(x, qs, 2048, s, b)
    assert t.launches == 2 and t.untimed == 1
    static_x = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.w8a16_gemm_strips(static_x, qs, 2048, s, b)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with ops.KernelTimer(max_launches=4) as t:
        with torch.cuda.graph(graph):
            out = ops.w8a16_gemm_strips(static_x, qs, 2048, s, b)
    assert t.launches == 0 and t.untimed == 0
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("m", [17, 33, 64, 65, 128, 129, 256])
def test_w8a16_strips_tile_vs_oracle(ops, m):
    """The pipelined strip-layout tile kernel (M > 16, K % 64 == 0): ragged M and N, every scale dtype,
    fp16 activations, forced split counts."""
    for n, k, sdt, xdt in ((2048, 2048, torch.bfloat16, torch.bfloat16), (1000, 1024, torch.float32, torch.bfloat16),
                           (2080, 3072, torch.float16, torch.float16), (24, 64, torch.bfloat16, torch.bfloat16)):
        print(f"strips tile m={m} n={n} k={k} scale={sdt} x={xdt}", flush=True)
        x, w, b = _make(m, n, k, dtype=xdt, bias=(m % 2 == 1), seed=m * 5 + n + k)
        q, s = ops.pack_int8(w, sdt)
        qs = ops.to_strips(q)
        ref = _oracle_w8a16(x, q, s, b)
        y = ops.w8a16_gemm_strips(x, qs, n, s, b)
        assert_close(y, ref, f"strips tile auto m={m} n={n} k={k}")
        for splits in (1, 2, 3, 4):
            y2 = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits))
            assert_close(y2, ref, f"strips tile m={m} n={n} k={k} S={splits}")
            if splits > 1:
                assert torch.equal(y2, ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits))), \
                    f"split-K not deterministic m={m} n={n} k={k} S={splits}"


@pytest.mark.parametrize("n,k", TALKER + PREDICTOR)
def test_w8a16_strips_prefill_vs_fp32(ops, n, k):
    """configs[3] rows (and the batch-8 code-predictor rows) on the strip layout against a torch fp32
    GEMM of the dequantized weight."""
    for m in (48, 120, 256, 1024):
        print(f"strips prefill m={m} n={n} k={k}", flush=True)
        x, w, b = _make(m, n, k, bias=(m == 120), seed=n * 7 + m)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        y = ops.w8a16_gemm_strips(x, qs, n, s, b)
        ref = x.float() @ (q.float() * s.float()[:, None]).t()
        if b is not None:
            ref = ref + b.float()
        assert_close(y, ref.double().cpu().numpy(), f"strips prefill m={m} n={n} k={k}")
        # and the fp64 oracle itself on a sample of the rows (every tile edge up to 256 among them)
        idx = _sample_rows(m)
        assert_close(y[idx], _oracle_w8a16(x[idx].contiguous(), q, s, b), f"strips prefill m={m} n={n} k={k} oracle")


def test_w8a16_strips_tile_graph_replays_split(ops):
    x, w, b = _make(40, 1024, 3072, bias=True, seed=78)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    algo = ops.algo_code(2, 4)
    eager = ops.w8a16_gemm_strips(x, qs, 1024, s, b, algo)
    static_x = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.w8a16_gemm_strips(static_x, qs, 1024, s, b, algo)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.w8a16_gemm_strips(static_x, qs, 1024, s, b, algo)
    for i in range(4):
        ops.w8a16_gemm_strips(x * 2, qs, 1024, s, b, ops.algo_code(2, 3))  # another split count in between
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


@pytest.mark.parametrize("m", [17, 40, 128, 200])
def test_fp8_strips_tile_vs_oracle(ops, m):
    """The pipelined fp8 tile kernel (M > 16, K % 128 == 0): ragged M and N, bias, every output dtype,
    forced tile shapes and split counts, with and without read-ahead."""
    for n, k, odt in ((2048, 2048, torch.bfloat16), (1000, 1024, torch.float16), (24, 256, torch.float32),
                      (2080, 3072, torch.bfloat16)):
        print(f"fp8 strips tile m={m} n={n} k={k} out={odt}", flush=True)
        x, w = _fp8_inputs(m, n, k, seed=m * 3 + n + k)
        b = (torch.randn(n, device="cuda") * 0.1).to(odt)
        qw, sw = ops.pack_fp8(w)
        qws = ops.to_strips(qw)
        qx, sx = ops.quant_act_fp8(x)
        ref, inter = _oracle_w8a8(qx, sx, qw, sw, b)
        y = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt)
        assert_close(y, ref, f"fp8 strips tile auto m={m} n={n} k={k}", inter)
        for splits, stages, shape in ((1, 2, 0x11), (2, 3, 0x22), (3, 4, 0x21), (4, 3, 0x12),
                                      (1, 4, 0x2A), (2, 3, 0x3A), (1, 4, 0x2B), (3, 3, 0x3B)):  # 8 waves: 0x_A, 0x_B
            algo = ops.algo_code(2, splits, stages, shape)
            y2 = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt, algo)
            assert_close(y2, ref, f"fp8 strips tile m={m} n={n} k={k} S={splits} P={stages} shape={shape:#x}", inter)
            if splits > 1:
                assert torch.equal(y2, ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt, algo)), \
                    f"fp8 split-K not deterministic m={m} n={n} k={k} S={splits}"
            if stages >= 3:  # read-ahead: the same MFMAs in the same order, so the same bits
                ra = ops.algo_code(2, splits, stages | ops.TILE_READ_AHEAD, shape)
                assert torch.equal(y2, ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt, ra)), \
                    f"fp8 read-ahead m={m} n={n} k={k} S={splits} P={stages} shape={shape:#x}"
            if shape & 8:  # 8 waves: the same sums as 4 waves over the same split
                four = ops.algo_code(2, splits, 3, 0x11)
                assert torch.equal(y2, ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, odt, four)), \
                    f"fp8 8 waves m={m} n={n} k={k} S={splits} P={stages} shape={shape:#x}"


def test_w8a16_strips_tile_forced_shapes(ops):
    """Every tile shape, wave grid and stage count the tile kernel is built for, against the oracle,
    and each with read-ahead (bit-identical to it); K ranges longer than the stage ring, as long,
    and shorter (one, two and three 64-column stages)."""
    for m, n, k, splits in ((70, 520, 1024, 2), (40, 200, 128, 1), (40, 200, 128, 2), (33, 72, 256, 1),
                            (48, 96, 192, 1)):
        x, w, b = _make(m, n, k, bias=True, seed=4242 + k)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        ref = _oracle_w8a16(x, q, s, b)
        for bmc in (1, 2, 3):
            for bnc in (1, 2, 3):
                for grid in (0, 4):  # 1 x 4 or 2 x 2 waves over the tile
                    for stages in (2, 3, 4, 6, 8):
                        algo = ops.algo_code(2, splits, stages, bmc | grid | (bnc << 4))
                        what = f"tile m={m} n={n} k={k} S={splits} BM={16 << bmc} BN={32 << bnc} grid={grid} P={stages}"
                        try:
                            y = ops.w8a16_gemm_strips(x, qs, n, s, b, algo)
                        except ValueError as e:
                            assert "stages are not built" in str(e), (what, e)
                            continue
                        assert_close(y, ref, what)
                        # read-ahead: the same MFMAs in the same order, so the same bits
                        ra = ops.algo_code(2, splits, stages | ops.TILE_READ_AHEAD, bmc | grid | (bnc << 4))
                        if stages < 3:
                            with pytest.raises(ValueError, match="read-ahead needs 3 stages"):
                                ops.w8a16_gemm_strips(x, qs, n, s, b, ra)
                            continue
                        y_ra = ops.w8a16_gemm_strips(x, qs, n, s, b, ra)
                        assert torch.equal(y_ra, y), what + " read-ahead"


def test_w8a16_strips_tile_two_chunks_a_stage(ops):
    """Two 64-column chunks a stage (stage bit 23) on the 4-wave 32 x 64 tile with read-ahead: against the
    oracle and bit for bit the one-chunk kernel with the same split (the same MFMAs in the same order),
    over one to eight stages a split; the automatic choice, which takes it on at most 256 such tiles,
    gives the same bits; an odd chunk count a split, another tile or no read-ahead is rejected."""
    two = ops.TILE_TWO_CHUNKS | ops.TILE_READ_AHEAD
    t3264 = ops.tile_shape(32, 64)
    for m, n, k, splits in ((70, 520, 1024, 2), (40, 200, 128, 1), (33, 72, 256, 1), (48, 96, 384, 3),
                            (130, 272, 2048, 4), (64, 4096, 1024, 0), (17, 1040, 3072, 0)):
        x, w, b = _make(m, n, k, bias=True, seed=6161 + k + m)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        ref = _oracle_w8a16(x, q, s, b)
        for p in (3, 4):
            what = f"two chunks m={m} n={n} k={k} S={splits} P={p}"
            print(what, flush=True)
            y1 = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, p | ops.TILE_READ_AHEAD, t3264))
            y2 = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, p | two, t3264))
            assert_close(y2, ref, what)
            assert torch.equal(y1, y2), what
        if (m, n, k) == (64, 4096, 1024):  # 128 tiles, 16 chunks, one split: the automatic choice takes two a stage
            assert torch.equal(ops.w8a16_gemm_strips(x, qs, n, s, b), y1), "auto"
    x, w, b = _make(48, 200, 640, bias=True, seed=17)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    with pytest.raises(ValueError, match="even chunk count"):  # 10 chunks in two splits of 5
        ops.w8a16_gemm_strips(x, qs, 200, s, b, ops.algo_code(2, 2, 4 | two, t3264))
    with pytest.raises(ValueError, match="even chunk count"):  # 3 chunks
        ops.w8a16_gemm_strips(x[:, :192].contiguous(), ops.to_strips(q[:, :192].contiguous()), 200, s, b,
                              ops.algo_code(2, 1, 4 | two, t3264))
    with pytest.raises(ValueError, match="two chunks a stage are built"):
        ops.w8a16_gemm_strips(x, qs, 200, s, b, ops.algo_code(2, 1, 4 | two, ops.tile_shape(64, 128)))
    with pytest.raises(ValueError, match="two chunks a stage are built"):
        ops.w8a16_gemm_strips(x, qs, 200, s, b, ops.algo_code(2, 1, 4 | ops.TILE_TWO_CHUNKS, t3264))


def test_w8a16_strips_tile_eight_waves(ops):
    """Every 8-wave tile the kernel is built for (two waves a SIMD), 3 and 4 stages, with and without
    read-ahead: against the oracle, and bit for bit equal to the 4-wave 32 x 64 tile with the same
    split (same K ranges, same MFMAs in the same order); ragged M and N, short and long K."""
    built = ((32, 64, True), (64, 128, False), (64, 128, True), (64, 256, False), (128, 128, True),
             (256, 128, True), (128, 256, False), (128, 256, True), (128, 384, False))
    for m, n, k, splits in ((70, 520, 1024, 2), (40, 200, 128, 1), (300, 1040, 2048, 1), (130, 272, 192, 3)):
        x, w, b = _make(m, n, k, bias=True, seed=5151 + k + m)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        ref = _oracle_w8a16(x, q, s, b)
        y4 = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, 3, ops.tile_shape(32, 64)))
        assert_close(y4, ref, f"tile m={m} n={n} k={k} S={splits} 4 waves")
        for bm, bn, grid2 in built:
            shape = ops.tile_shape(bm, bn, 8, grid2)
            for stages in (3, 4):
                for ra in (0, ops.TILE_READ_AHEAD):
                    what = f"tile m={m} n={n} k={k} S={splits} {bm}x{bn} 8 waves grid2={grid2} P={stages} ra={ra}"
                    print(what, flush=True)
                    try:
                        y = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(2, splits, stages | ra, shape))
                    except ValueError as e:
                        if bn == 384:  # 3 stages without read-ahead only
                            assert (stages, ra) != (3, 0) and "128x384 tiles are built" in str(e), (what, e)
                        else:
                            assert stages == 4 and bm == 256 and "stages are not built" in str(e), (what, e)
                        continue
                    assert torch.equal(y, y4), what


def _fused_waves(n: int, k: int) -> int:
    """The fused fp8 linear's wave count (fp8_fused.hip: fused_cfg)."""
    nch = k // 128
    c = 2 if nch <= 32 else 3
    w = 1
    while w * c < nch:
        w *= 2
    while w < 16 and -(-n // 16) * w < 2048:
        w *= 2
    return w


@pytest.mark.parametrize("n,k", TALKER + PREDICTOR + [(40, 256), (1000, 128)])
def test_fp8_linear_fused_matches_two_kernel_path(ops, n, k):
    """Decode rows (M <= 8) can take the fused kernel (quantization inside the GEMM).  Forced to a
    wave count (the one the automatic rule picks, which does not depend on M, and twice it), it must
    equal the two-kernel path (stand-alone quantization, bit-exact with the reference, then the GEMM
    with the same wave split, so the same accumulation order) bit for bit: any difference in the
    fused per-token scale or e4m3 codes shows.  The automatic choice at every M is within tolerance
    of the oracle, with bias."""
    waves = _fused_waves(n, k)
    for m in (1, 2, 3, 4, 5, 8, 16):
        x, w = _fp8_inputs(m, n, k, seed=n + 5 * m + k)
        b = (torch.randn(n, device="cuda") * 0.1).to(torch.bfloat16)
        qw, sw = ops.pack_fp8(w)
        qws = ops.to_strips(qw)
        qx, sx = ops.quant_act_fp8(x)
        if m <= 8:
            for wf in sorted({waves, min(16, 2 * waves)}):
                print(f"fp8 fused n={n} k={k} m={m} W={wf}", flush=True)
                y = ops.fp8_linear_strips(x, qws, n, sw, b, ops.DIV_DEVICE, ops.algo_code(1, 0, wf))
                two = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, b, torch.bfloat16, ops.algo_code(1, 1, wf))
                assert torch.equal(y, two), f"fused differs from the two-kernel path: n={n} k={k} m={m} W={wf}"
        y = ops.fp8_linear_strips(x, qws, n, sw, b)
        ref, inter = _oracle_w8a8(qx, sx, qw, sw, b)
        assert_close(y, ref, f"fp8 linear n={n} k={k} m={m}", inter)
    # fp16 activations and the CPU division mode take the same kernel
    x, w = _fp8_inputs(4, n, k, seed=n + k)
    x = x.to(torch.float16)
    qw, sw = ops.pack_fp8(w)
    qws = ops.to_strips(qw)
    qx, sx = ops.quant_act_fp8(x, ops.DIV_IEEE)
    for wf in sorted({waves, min(16, 2 * waves)}):  # the automatic wave count, and twice it
        y = ops.fp8_linear_strips(x, qws, n, sw, None, ops.DIV_IEEE, ops.algo_code(1, 0, wf))
        two = ops.w8a8_fp8_gemm_strips(qx, sx, qws, n, sw, None, torch.float16, ops.algo_code(1, 1, wf))
        assert torch.equal(y, two), f"fused fp16 / IEEE differs: n={n} k={k} W={wf}"


@pytest.mark.parametrize("n,k", TALKER + PREDICTOR)
def test_w8a16_strips_skinny_blocks(ops, n, k):
    """The skinny kernel with 2 and 4 m-blocks (17 <= M <= 64 on strip weights): the automatic choice and
    every built (waves, chunks) pair, forced splits, bias, against the oracle."""
    for m in (17, 24, 32, 33, 48, 64):
        print(f"skinny blocks n={n} k={k} m={m}", flush=True)
        x, w, b = _make(m, n, k, bias=(m % 2 == 0), seed=n + 11 * m + k)
        q, s = ops.pack_int8(w, torch.bfloat16)
        qs = ops.to_strips(q)
        ref = _oracle_w8a16(x, q, s, b)
        assert_close(ops.w8a16_gemm_strips(x, qs, n, s, b), ref, f"auto m={m} n={n} k={k}")
        combos = ((1, 4, 8), (1, 8, 8), (1, 16, 4), (2, 8, 4), (3, 4, 8)) if m <= 32 else ((1, 8, 4), (2, 4, 4), (3, 8, 4))
        for splits, waves, cpw in combos:
            y = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(1, splits, waves, cpw))
            assert_close(y, ref, f"skinny m={m} n={n} k={k} S={splits} W={waves} C={cpw}")


def test_w8a16_strips_skinny_blocks_dtypes(ops):
    for sdt, xdt in ((torch.float32, torch.bfloat16), (torch.float16, torch.float16)):
        for m in (20, 40):
            x, w, b = _make(m, 1000, 1024, dtype=xdt, bias=True, seed=m + 7)
            q, s = ops.pack_int8(w, sdt)
            qs = ops.to_strips(q)
            assert_close(ops.w8a16_gemm_strips(x, qs, 1000, s, b), _oracle_w8a16(x, q, s, b),
                         f"skinny blocks m={m} scale={sdt} x={xdt}")
    x, w, _ = _make(65, 64, 128)
    q, s = ops.pack_int8(w, torch.bfloat16)
    with pytest.raises(ValueError, match="M <= 64"):
        ops.w8a16_gemm_strips(x, ops.to_strips(q), 64, s, None, ops.algo_code(1))


# (SUB, waves, units per wave) pairs built for row-split strips (w8a16_xrows_sub.hip)
SUB_PAIRS = {2: ((1, 8), (2, 8), (4, 4), (4, 8), (8, 6), (16, 3)),
             4: ((1, 8), (2, 6), (4, 6))}


@pytest.mark.parametrize("xdt,sdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
                                     (torch.float16, torch.float16)])
def test_w8a16_strips_row_split(ops, xdt, sdt):
    """Row-split strips (2 or 4 workgroups per 16-row strip, SUB chunks per MFMA) against the oracle:
    every built (waves, units) pair that covers K in one group, ragged N, a bias on odd M, every M
    the split allows (half strips: up to 64 rows in row parts of 8); the automatic choice too, and
    the same bits on a second call."""
    for (n, k) in ((2048, 2048), (2048, 6144), (1024, 3072), (1000, 1024), (40, 512), (24, 256)):
        nch = k // 64
        q = s = qs = None
        for m in list(range(1, 17)) + [23, 40, 64]:
            x, w, b = _make(m, n, k, dtype=xdt, bias=(m % 2 == 1), seed=3 * n + k + m)
            if q is None:
                q, s = ops.pack_int8(w, sdt)
                qs = ops.to_strips(q)
            ref = _oracle_w8a16(x, q, s, b)
            y = ops.w8a16_gemm_strips(x, qs, n, s, b)
            assert_close(y, ref, f"auto m={m} n={n} k={k} {xdt} {sdt}")
            assert torch.equal(y, ops.w8a16_gemm_strips(x, qs, n, s, b)), f"auto not deterministic m={m} n={n}"
            for sub, family in ((2, ops.ALGO_SKINNY_HALF), (4, ops.ALGO_SKINNY_QUARTER)):
                if m > (64 if sub == 2 else 16 // sub) or nch % sub:
                    with pytest.raises(ValueError, match="row-split"):
                        ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(family))
                    continue
                units = nch // sub
                for waves, cpw in SUB_PAIRS[sub]:
                    if waves * cpw < units or cpw > 2 * units:
                        continue
                    what = f"sub={sub} W={waves} C={cpw} m={m} n={n} k={k} {xdt} {sdt}"
                    print(what, flush=True)
                    y = ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(family, 0, waves, cpw))
                    assert_close(y, ref, what)
                # the default waves for this split
                assert_close(ops.w8a16_gemm_strips(x, qs, n, s, b, ops.algo_code(family)), ref,
                             f"sub={sub} default m={m} n={n} k={k}")


def test_w8a16_strips_row_split_rejects(ops):
    x, w, b = _make(65, 256, 512, seed=5)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    with pytest.raises(ValueError, match="row-split"):  # 65 rows: more than eight row parts of 8
        ops.w8a16_gemm_strips(x, qs, 256, s, b, ops.algo_code(ops.ALGO_SKINNY_HALF))
    with pytest.raises(ValueError, match="row-split"):  # 5 rows: more than the 4 a quarter strip takes
        ops.w8a16_gemm_strips(x[:5], qs, 256, s, b, ops.algo_code(ops.ALGO_SKINNY_QUARTER))
    with pytest.raises(ValueError, match="row-split"):  # an explicit split count
        ops.w8a16_gemm_strips(x[:2], qs, 256, s, b, ops.algo_code(ops.ALGO_SKINNY_HALF, 2))
    with pytest.raises(ValueError, match="cover less"):  # 1 wave of 3 units for 4 units of K
        ops.w8a16_gemm_strips(x[:2], qs, 256, s, b, ops.algo_code(ops.ALGO_SKINNY_HALF, 0, 1, 3))
    with pytest.raises(ValueError, match="not built"):
        ops.w8a16_gemm_strips(x[:2], qs, 256, s, b, ops.algo_code(ops.ALGO_SKINNY_HALF, 0, 1, 5))
    xr, wr, _ = _make(2, 64, 640, seed=6)  # K = 10 chunks: not a multiple of 4
    qr, sr = ops.pack_int8(wr, torch.bfloat16)
    with pytest.raises(ValueError, match="row-split"):
        ops.w8a16_gemm_strips(xr, ops.to_strips(qr), 64, sr, None, ops.algo_code(ops.ALGO_SKINNY_QUARTER))
