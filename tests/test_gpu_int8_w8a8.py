"""GPU parity of the int8 W8A8 path (Int8Method.apply, qtts/quant/int8.py:145-160), through the C ABI.

The int32 accumulation is exact and the epilogue is three fp32 roundings and one
rounding to the activation dtype, so the bar here is bit-exact, everywhere:

* the activation codes and scales against the oracle (oracle/qtts_oracle.c) and
  against torch on the GPU evaluating the reference's own expressions;
* the GEMM against the oracle at small sizes and, at the full talker / code
  predictor shapes, against torch on the GPU (an fp64 matmul of the codes, which is
  exact, followed by the reference's fp32 epilogue expression);
* whole linears against the golden fixtures written by torch._int_mm on the CPU;
* the fused decode kernel (quantization inside the GEMM) against the two-kernel path.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TALKER = [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144)]
PREDICTOR = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]
ODT = {torch.bfloat16: O.DT_BF16, torch.float16: O.DT_F16, torch.float32: O.DT_F32}


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _np_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 / fp16 as uint16 bit patterns, fp32 as values (the oracle's encoding)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def _from_bits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.float32:
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).view(dtype).cuda()


def _assert_bits(y: torch.Tensor, want: np.ndarray, what: str) -> None:
    got = _np_bits(y)
    if got.dtype == np.float32:
        got, want = got.view(np.uint32), np.ascontiguousarray(want, np.float32).view(np.uint32)
    bad = got != want
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outputs differ, first at " \
                          f"{np.unravel_index(np.argmax(bad), bad.shape)}"


def _acts(m, k, dtype, seed):
    """N(0,1) rows with 20-sigma outliers; from 4 rows on a zero row, a row below the
    1e-6 clamp and a row of rounding ties."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g)
    out = torch.rand(m, k, device="cuda", generator=g) < 0.01
    x[out] = 20.0
    if m >= 4:
        x[1] = 0.0
        x[2] *= 1e-7
        x[3] = (torch.arange(k, device="cuda") % 16).float() - 7.5
        x[3, 0] = 127.0
    return x.to(dtype)


def _torch_act_int8(x: torch.Tensor):
    """qtts/quant/int8.py:146-149 evaluated by torch on the GPU, as the reference runs it."""
    flat = x.reshape(-1, x.shape[-1])
    scale_x = flat.abs().amax(dim=1, keepdim=True).clamp_min(1e-6) / 127.0
    q = (flat / scale_x).round().clamp_(-127.0, 127.0).to(torch.int8)
    return q, scale_x.reshape(-1)


def _torch_int8_out(qx, sx, qw, sw, bias, dtype):
    """torch._int_mm and the epilogue of qtts/quant/int8.py:151-160 on the GPU; the integer
    product as an fp64 matmul of the codes (exact: |sum| < 2^53)."""
    acc = (qx.double() @ qw.double().t()).to(torch.int32)
    out = acc.float() * sx.float().reshape(-1, 1) * sw.reshape(1, -1)
    if bias is not None:
        out += bias.float()
    return out.to(dtype)


# ---- activations ---------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_act_int8_vs_oracle(ops, dtype):
    """Vector kernel (16-bit, k % 8 == 0, k <= 8192) and scalar kernel (fp32, odd k, long rows)."""
    for (m, k) in ((1, 2048), (8, 2048), (5, 130), (16, 1024), (3, 6144), (2, 16384), (4, 8)):
        x = _acts(m, k, dtype, seed=m * 31 + k)
        for mode in (O.DIV_DEVICE, O.DIV_IEEE):
            qx, sx = ops.quant_act_int8(x, mode)
            q_ref, s_ref = O.quant_act_int8(_np_bits(x), ODT[dtype], mode)
            what = f"{dtype} m={m} k={k} mode={mode}"
            np.testing.assert_array_equal(qx.cpu().numpy(), q_ref, err_msg=what)
            np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), s_ref.view(np.uint32), err_msg=what)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_act_int8_vs_torch_gpu_expression(ops, dtype):
    """DIV_DEVICE is what torch's GPU kernels compute for the reference's expression."""
    for (m, k) in ((1, 2048), (8, 2048), (5, 130), (16, 6144)):
        x = _acts(m, k, dtype, seed=k + m)
        qx, sx = ops.quant_act_int8(x, O.DIV_DEVICE)
        q_t, s_t = _torch_act_int8(x)
        assert torch.equal(qx, q_t), f"{dtype} m={m} k={k}: codes differ"
        assert torch.equal(sx, s_t.float()), f"{dtype} m={m} k={k}: scales differ"


def test_act_int8_golden(ops):
    z = np.load(os.path.join(GOLDEN, "int8_w8a8.npz"))
    cases = sorted({k.rsplit(".", 1)[0] for k in z.files if k.startswith("act.") and k.endswith(".x")})
    dts = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    for case in cases:
        dtype = dts[case.rsplit(".", 1)[1]]
        x = _from_bits(z[f"{case}.x"], dtype)
        for mode, code in (("ieee", O.DIV_IEEE), ("device", O.DIV_DEVICE)):
            qx, sx = ops.quant_act_int8(x, code)
            np.testing.assert_array_equal(qx.cpu().numpy(), z[f"{case}.{mode}.q"], err_msg=case)
            np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32),
                                          err_msg=case)


# ---- GEMM ------------------------------------------------------------------------------

def _codes(m, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    qx = torch.randint(-127, 128, (m, k), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    qw = torch.randint(-127, 128, (n, k), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
    sx = torch.rand(m, device="cuda", generator=g) * 0.05 + 1e-3
    sw = torch.rand(n, device="cuda", generator=g) * 0.01 + 1e-4
    return qx, sx, qw, sw


def _oracle_gemm(qx, sx, qw, sw, bias, dtype):
    y = O.int8_linear_out(qx.cpu().numpy(), sx.cpu().numpy(), qw.cpu().numpy(), sw.cpu().numpy(),
                          None if bias is None else _np_bits(bias), ODT[dtype])
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_int8_gemm_small_vs_oracle(ops, dtype):
    """Tails in M, N and K, bias on and off; skinny, tile and generic kernels; both layouts."""
    g = torch.Generator(device="cuda").manual_seed(1)
    for (m, n, k) in ((1, 33, 256), (3, 16, 64), (5, 40, 384), (16, 72, 128), (17, 48, 256), (40, 130, 512),
                      (70, 64, 1024), (9, 20, 80), (2, 24, 130)):
        qx, sx, qw, sw = _codes(m, n, k, seed=m * 1000 + n + k)
        for with_bias in (False, True):
            bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if with_bias else None
            want = _oracle_gemm(qx, sx, qw, sw, bias, dtype)
            for fam in (0, 1, 2):
                algo = ops.algo_code(fam)
                what = f"{dtype} m={m} n={n} k={k} bias={with_bias} family={fam}"
                _assert_bits(ops.w8a8_int8_gemm(qx, sx, qw, sw, bias, dtype, algo), want, what + " rowmajor")
                if k % 16 == 0:
                    qs = ops.to_strips(qw)
                    _assert_bits(ops.w8a8_int8_gemm_strips(qx, sx, qs, n, sw, bias, dtype, algo), want,
                                 what + " strips")


def test_int8_gemm_generic_path(ops):
    """Unaligned rows (odd leading dimensions) take the generic kernel; still exact."""
    m, n, k = 6, 37, 200
    qx, sx, qw, sw = _codes(m, n, k + 3, seed=9)
    qx, qw = qx[:, 1:k + 1], qw[:, 2:k + 2]  # row strides k + 3, misaligned starts
    bias = torch.randn(n, device="cuda").to(torch.bfloat16)
    want = _oracle_gemm(qx.contiguous(), sx, qw.contiguous(), sw, bias, torch.bfloat16)
    _assert_bits(ops.w8a8_int8_gemm(qx, sx, qw, sw, bias, torch.bfloat16), want, "generic")


def test_int8_gemm_every_config_identical(ops):
    """Exact integer sums: every split count, wave count, tile shape and stage depth gives the
    same bits (the split-K meeting adds int32 partials)."""
    m, n, k = 24, 512, 2048
    qx, sx, qw, sw = _codes(m, n, k, seed=3)
    qs = ops.to_strips(qw)
    bias = torch.randn(n, device="cuda").to(torch.bfloat16)
    want = _oracle_gemm(qx, sx, qw, sw, bias, torch.bfloat16)
    algos = [ops.algo_code(1, s, w) for s in (0, 1, 2, 4, 8) for w in (0, 1, 4, 16)]
    def fits(p, shape):  # the stage ring must fit the 160 KiB of LDS; 8 waves build 3 and 4 stages
        bm, bn = (32, 64) if shape == 0 else (16 << (shape & 7), 32 << (shape >> 4))
        return (p & 0x3f) * (bm // 8 + bn // 8) * 1024 + 64 <= 160 * 1024 and not (shape & 8 and p & 0x3f == 2)
    ra = ops.TILE_READ_AHEAD  # operands read one stage ahead
    eight = (0x2A, 0x3A, 0x2B, 0x3B)  # 8 waves: 64 x 128, 64 x 256, 128 x 128, 128 x 256
    algos += [ops.algo_code(2, s, p, shape) for s in (0, 1, 2, 4) for p in (2, 3, 4, 3 | ra, 4 | ra)
              for shape in (0, 0x11, 0x21, 0x12, 0x22, 0x32, 0x13, 0x23) + eight if fits(p, shape)]
    with pytest.raises(ValueError, match="read-ahead needs 3 stages"):
        ops.w8a8_int8_gemm_strips(qx, sx, qs, n, sw, bias, torch.bfloat16, ops.algo_code(2, 0, 2 | ra, 0x11))
    for algo in algos:
        _assert_bits(ops.w8a8_int8_gemm_strips(qx, sx, qs, n, sw, bias, torch.bfloat16, algo), want,
                     f"strips algo={algo:#x}")
    for algo in algos[::3]:
        _assert_bits(ops.w8a8_int8_gemm(qx, sx, qw, sw, bias, torch.bfloat16, algo), want, f"rowmajor algo={algo:#x}")


def test_int8_gemm_half_strips(ops):
    """Decode rows on layers with few strips take half strips (two workgroups of 8 weight rows per
    strip, two chunks per MFMA): exactly the oracle, and exactly the whole-strip kernel, for every
    M in 1..8, ragged N, bias on and off."""
    for (n, k) in ((40, 256), (1000, 512), (72, 384), (2048, 6144)):
        qx8, sx8, qw, sw = _codes(8, n, k, seed=n + k)
        qs = ops.to_strips(qw)
        for m in range(1, 9):
            qx, sx = qx8[:m].contiguous(), sx8[:m].contiguous()
            bias = (torch.randn(n, device="cuda") * 0.1).to(torch.bfloat16) if m % 2 else None
            want = _oracle_gemm(qx, sx, qw, sw, bias, torch.bfloat16)
            what = f"n={n} k={k} m={m}"
            print(what, flush=True)
            half = ops.w8a8_int8_gemm_strips(qx, sx, qs, n, sw, bias, torch.bfloat16)
            _assert_bits(half, want, what + " automatic (half strips)")
            whole = ops.w8a8_int8_gemm_strips(qx, sx, qs, n, sw, bias, torch.bfloat16, ops.algo_code(1, 0, 16))
            assert torch.equal(half, whole), what + ": half strips differ from whole strips"


@pytest.mark.parametrize("shape", TALKER + PREDICTOR)
def test_int8_linear_full_shapes(ops, shape):
    """Whole Int8Method.apply at the talker / code predictor shapes, decode and prefill rows,
    against torch on the GPU evaluating the reference's expressions.  From 17 to 128 rows the
    automatic choice on strips is the skinny kernel where ceil(M / 16) * N * K <= 24 MiB and the
    tile kernel elsewhere; both are checked against the other family too."""
    n, k = shape
    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    qw, sw = ops.pack_int8(w, torch.float32)
    qs = ops.to_strips(qw)
    bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    for m in (1, 4, 8, 16, 17, 64, 128, 256):
        x = _acts(m, k, torch.bfloat16, seed=m)
        q_t, s_t = _torch_act_int8(x)
        b = bias if m % 2 else None
        want = _np_bits(_torch_int8_out(q_t, s_t, qw, sw, b, torch.bfloat16))
        _assert_bits(ops.int8_linear_strips(x, qs, n, sw, b), want, f"strips n={n} k={k} m={m}")
        if 17 <= m <= 128:
            for fam in (1, 2):
                _assert_bits(ops.int8_linear_strips(x, qs, n, sw, b, O.DIV_DEVICE, ops.algo_code(fam)), want,
                             f"strips n={n} k={k} m={m} family={fam}")
        if m in (1, 64):
            _assert_bits(ops.int8_linear(x, qw, sw, b), want, f"rowmajor n={n} k={k} m={m}")


def test_int8_linear_golden(ops):
    """Whole linears against torch._int_mm on the CPU (tests/golden/make_golden.py)."""
    z = np.load(os.path.join(GOLDEN, "int8_w8a8.npz"))
    cases = sorted({k.rsplit(".", 1)[0] for k in z.files if k.startswith("lin.") and k.endswith(".x")})
    dts = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    for case in cases:
        dtype = dts[case.rsplit(".", 1)[1]]
        x = _from_bits(z[f"{case}.x"], dtype)
        qw = torch.from_numpy(z[f"{case}.qw"]).cuda()
        sw = torch.from_numpy(z[f"{case}.sw"]).cuda()
        bias = _from_bits(z[f"{case}.bias"], dtype) if f"{case}.bias" in z.files else None
        n, k = qw.shape
        for mode, code in (("ieee", O.DIV_IEEE), ("device", O.DIV_DEVICE)):
            want = z[f"{case}.{mode}.y"]
            _assert_bits(ops.int8_linear(x, qw, sw, bias, code), want, f"{case} {mode} rowmajor")
            if k % 16 == 0:
                _assert_bits(ops.int8_linear_strips(x, ops.to_strips(qw), n, sw, bias, code), want,
                             f"{case} {mode} strips")


def test_int8_linear_graph_replays(ops):
    """Capture a split-K int8 linear; every replay, between eager calls sharing the
    workspace, matches eager."""
    n, k = 2048, 6144
    g = torch.Generator(device="cuda").manual_seed(4)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    qw, sw = ops.pack_int8(w, torch.float32)
    qs = ops.to_strips(qw)
    x = _acts(8, k, torch.bfloat16, seed=5)
    algo = ops.algo_code(1, 4, 8)
    eager = ops.int8_linear_strips(x, qs, n, sw, None, O.DIV_DEVICE, algo)
    static_x = x.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.int8_linear_strips(static_x, qs, n, sw, None, O.DIV_DEVICE, algo)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.int8_linear_strips(static_x, qs, n, sw, None, O.DIV_DEVICE, algo)
    for i in range(4):
        junk = ops.int8_linear_strips(x * (i + 2), qs, n, sw, None, O.DIV_DEVICE, ops.algo_code(1, 2, 16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"
        q_t, s_t = _torch_act_int8(x * (i + 2))
        assert torch.equal(junk, _torch_int8_out(q_t, s_t, qw, sw, None, torch.bfloat16))


def _two_kernel(ops, x, qs, n, sw, bias, mode):
    """The unfused path: quant_act_int8_vec_kernel, then the skinny int8 GEMM."""
    qx, sx = ops.quant_act_int8(x, mode)
    return ops.w8a8_int8_gemm_strips(qx, sx, qs, n, sw, bias, x.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_int8_linear_fused_decode(ops, dtype):
    """Decode rows (M <= 8, K % 64 == 0) run quantization, GEMM and epilogue in one kernel
    (int8_linear_fused_kernel), forced here through an explicit wave count (the fewest the
    shape allows, and 16: runs of 8, 6, 4 and 2 chunks) besides the automatic choice.  Its
    output is the two-kernel path's, bit for bit, at every M in 1..8, for ragged K (runs
    shorter than a wave's, waves with no chunk) and N, strided rows, both division modes,
    with a zero row, a row under the 1e-6 clamp (an fp16 scale of zero: codes +-127 and 0)
    and a row of rounding ties; and the oracle's on small cases."""
    for (n, k) in ((100, 64), (48, 320), (2048, 2048), (12288, 2048), (2048, 6144), (1024, 3072), (64, 8192),
                   (40, 1984)):
        g = torch.Generator(device="cuda").manual_seed(n * 7 + k)
        w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
        qw, sw = ops.pack_int8(w, torch.float32)
        qs = ops.to_strips(qw)
        bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype)
        for m in range(1, 9):
            base = _acts(max(m, 4), k + 64, dtype, seed=m * 17 + k)[-m:]  # the special rows from m = 4 on
            x = base[:, 32:32 + k] if m % 3 == 0 else base[:, :k].contiguous()  # strided rows, 16-byte aligned
            b = bias if m % 2 else None
            wmin = 1
            while wmin * 8 < k // 64:
                wmin *= 2
            for mode in (O.DIV_DEVICE, O.DIV_IEEE):
                want = _two_kernel(ops, x, qs, n, sw, b, mode)
                for algo in (ops.algo_code(0), ops.algo_code(1, 0, wmin), ops.algo_code(1, 0, 16)):
                    what = f"{dtype} n={n} k={k} m={m} mode={mode} bias={b is not None} ldx={x.stride(0)} algo={algo:#x}"
                    got = ops.int8_linear_strips(x, qs, n, sw, b, mode, algo)
                    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
                        (what, int((got.view(torch.int16) != want.view(torch.int16)).sum()))
                if n * k <= 200_000:
                    q_ref, s_ref = O.quant_act_int8(_np_bits(x), ODT[dtype], mode)
                    y_ref = O.int8_linear_out(q_ref, s_ref, qw.cpu().numpy(), sw.cpu().numpy(),
                                              None if b is None else _np_bits(b), ODT[dtype])
                    _assert_bits(got, y_ref, what + " vs oracle")


def test_int8_linear_fused_graph_replays(ops):
    """The fused decode kernel captured in a graph: every replay matches eager."""
    n, k = 4096, 2048
    g = torch.Generator(device="cuda").manual_seed(6)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    qw, sw = ops.pack_int8(w, torch.float32)
    qs = ops.to_strips(qw)
    static_x = _acts(4, k, torch.bfloat16, seed=8)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.int8_linear_strips(static_x, qs, n, sw)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.int8_linear_strips(static_x, qs, n, sw)
    for i in range(3):
        static_x.copy_(_acts(4, k, torch.bfloat16, seed=20 + i))
        graph.replay()
        torch.cuda.synchronize()
        want = _two_kernel(ops, static_x, qs, n, sw, None, O.DIV_DEVICE)
        assert torch.equal(out, want), f"replay {i}"


def test_int8_errors(ops):
    qx, sx, qw, sw = _codes(4, 32, 64, seed=1)
    with pytest.raises(ValueError, match="K=48"):
        ops.w8a8_int8_gemm(qx[:, :48], sx, qw, sw)
    with pytest.raises(ValueError, match="strip-layout"):
        ops.w8a8_int8_gemm_strips(qx, sx, qw, 48, sw)  # 2048 bytes cannot be a [48, 64] strip buffer
    x = torch.randn(4, 64, device="cuda").to(torch.bfloat16)
    with pytest.raises(ValueError):
        ops.int8_linear(x, qw, sw[:8])
    # an explicit split count with no room for it in the workspace is an error
    from qtts_amd import _lib
    qx2, sx2, qw2, sw2 = _codes(2, 64, 4096, seed=2)
    y = torch.empty(2, 64, dtype=torch.bfloat16, device="cuda")
    st = _lib.load().qtts_w8a8_int8_gemm(qx2.data_ptr(), sx2.data_ptr(), 2, 4096, 4096, qw2.data_ptr(), 64, 4096,
                                         sw2.data_ptr(), None, y.data_ptr(), _lib.BF16, 64, ops.algo_code(1, 4),
                                         None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == _lib.ERR_WORKSPACE


def test_int8_method_hook(ops):
    """--quant-method int8 on a talker-like module: every converted linear is bit-exact with
    the reference's Int8Method.apply on the same weights."""
    from qtts_amd import QuantConfig, apply_quantization
    from qtts_amd.layers.linear import LinearBase
    from qtts_amd.quant.int8 import int8_weight_rowmajor
    torch.manual_seed(0)
    lin = LinearBase(2048, 2048, bias=True, dtype=torch.bfloat16, device="cuda")
    lin.weight.data.normal_(0, 0.02)
    lin.bias.data.normal_(0, 0.1)
    mod = torch.nn.Module()
    mod.text_proj_fc1 = lin
    qw_ref, sw_ref = ops.pack_int8(lin.weight.data, torch.float32)
    report = apply_quantization(QuantConfig(method="int8"), talker=mod)
    assert report["talker"]["converted"] == 1
    assert lin.weight.numel() == 0 and lin.int8_layout == "strips"
    assert torch.equal(int8_weight_rowmajor(lin), qw_ref) and torch.equal(lin.int8_scale, sw_ref)
    for m in (1, 8, 100):
        x = _acts(m, 2048, torch.bfloat16, seed=m + 7)
        q_t, s_t = _torch_act_int8(x)
        assert torch.equal(lin(x), _torch_int8_out(q_t, s_t, qw_ref, sw_ref, lin.bias, torch.bfloat16)), f"m={m}"
