"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so that a plausible mistake in the oracle fails it:
golden fixtures from torch evaluating the reference's expressions
(tests/golden/make_golden.py), closed-form rows, an exhaustive e4m3 sweep
against torch's float8_e4m3fn cast, and invariants of the fp64 GEMM.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O
from oracle import cpu_path

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def _cases(z):
    return sorted({k.rsplit(".", 1)[0] for k in z.files if k.endswith(".src")})


MODES = {"ieee": O.DIV_IEEE, "device": O.DIV_DEVICE}


@pytest.mark.parametrize("mode", list(MODES))
def test_int8_pack_matches_golden(mode):
    z = _load("int8_pack")
    for case in _cases(z):
        src = z[f"{case}.src"]
        dt = O.DT_F32 if case.endswith(".f32") else O.DT_BF16
        q, s32, sb = O.pack_int8(src, dt, O.DT_BF16, MODES[mode])
        np.testing.assert_array_equal(q, z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(s32.view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32), err_msg=case)
        np.testing.assert_array_equal(sb, z[f"{case}.{mode}.scale_bf16"], err_msg=case)


@pytest.mark.parametrize("mode", list(MODES))
def test_fp8_pack_matches_golden(mode):
    z = _load("fp8_pack")
    for case in _cases(z):
        src = z[f"{case}.src"]
        dt = O.DT_F32 if case.endswith(".f32") else O.DT_BF16
        q, s = O.pack_fp8(src, dt, MODES[mode])
        np.testing.assert_array_equal(q, z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(s.view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32), err_msg=case)


@pytest.mark.parametrize("mode", list(MODES))
def test_act_fp8_matches_golden(mode):
    z = _load("act_fp8")
    for case in sorted({k.split(".")[0] for k in z.files}):
        qx, sx = O.quant_act_fp8(z[f"{case}.x"], O.DT_BF16, MODES[mode])
        np.testing.assert_array_equal(qx, z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(sx.view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32), err_msg=case)


def test_int8_closed_forms():
    k = 64
    w = np.zeros((5, k), np.float32)
    w[1, :9] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    w[2, 3] = -2.0
    w[3, :] = 0.25
    w[4, 0], w[4, 1] = 1.0, -1.0
    q, s, sb = O.pack_int8(w, O.DT_F32, O.DT_F32, O.DIV_IEEE)
    # all-zero row: amax clamps to 1e-12, q = 0
    assert s[0] == np.float32(np.float32(1e-12) / np.float32(127.0))
    assert not q[0].any()
    # amax 127 -> scale exactly 1 -> round half to even
    assert s[1] == 1.0
    assert list(q[1, :9]) == [127, 0, 2, 2, 0, -2, -2, 126, -126]
    # the absmax element always maps to +/-127, never -128
    assert q[2, 3] == -127 and (q[3] == 127).all()
    assert q[4, 0] == 127 and q[4, 1] == -127
    assert q.min() >= -127


def test_device_scale_is_reciprocal_multiply():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (4096, 32)).astype(np.float32)
    _, s_dev, _ = O.pack_int8(w, O.DT_F32, O.DT_F32, O.DIV_DEVICE)
    _, s_ieee, _ = O.pack_int8(w, O.DT_F32, O.DT_F32, O.DIV_IEEE)
    amax = np.abs(w).max(axis=1)
    np.testing.assert_array_equal(s_ieee, amax / np.float32(127.0))
    np.testing.assert_array_equal(s_dev, amax * (np.float32(1.0) / np.float32(127.0)))
    # The two semantics genuinely differ on some rows (else one mode is untested).
    assert (s_dev != s_ieee).any()


def _all_bf16_values() -> np.ndarray:
    return O.bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))


def test_e4m3_encode_exhaustive_bf16_vs_torch():
    v = _all_bf16_values()
    ours = O.e4m3_encode(v)
    theirs = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_e4m3_encode_fp32_samples_vs_torch():
    rng = np.random.default_rng(11)
    v = np.concatenate([
        rng.normal(0, 100, 20000), rng.normal(0, 1e-2, 20000),
        rng.uniform(-470, 470, 20000), rng.normal(0, 1e-3, 5000),
    ]).astype(np.float32)
    # exact ties between neighbouring e4m3 values (normal and subnormal)
    tab = O.e4m3_decode_table()
    fin = np.sort(tab[np.isfinite(tab)])
    mids = ((fin[1:].astype(np.float64) + fin[:-1]) / 2).astype(np.float32)
    v = np.concatenate([v, mids, -mids, np.float32([464.0, 463.99997, 480.0, -464.0, np.inf, -np.inf, np.nan])])
    ours = O.e4m3_encode(v)
    theirs = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_e4m3_decode_table():
    tab = O.e4m3_decode_table()
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(tab), np.isnan(codes))
    fin = ~np.isnan(tab)
    np.testing.assert_array_equal(tab[fin], codes[fin])
    # OCP E4M3 landmarks
    assert tab[0x7E] == 448.0 and tab[0x01] == 2.0 ** -9 and tab[0x08] == 2.0 ** -6
    assert tab[0x38] == 1.0 and tab[0xB8] == -1.0
    assert np.isnan(tab[0x7F]) and np.isnan(tab[0xFF]) and np.isnan(tab).sum() == 2


def test_gemm_oracle_matches_fp64_golden():
    z = _load("gemm_small")
    for case in sorted({k.split(".")[0] for k in z.files}):
        x = O.bf16_bits_to_f32(z[f"{case}.x"])
        s = O.bf16_bits_to_f32(z[f"{case}.scale_bf16"])
        b = O.bf16_bits_to_f32(z[f"{case}.bias"]) if f"{case}.bias" in z.files else None
        y = O.w8a16_ref(x, z[f"{case}.q"], s, b)
        np.testing.assert_allclose(y, z[f"{case}.y_f64"], rtol=1e-12, atol=1e-12, err_msg=case)


def test_gemm_oracle_invariants():
    rng = np.random.default_rng(5)
    m, n, k = 3, 7, 50
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.01, n).astype(np.float32)
    b = rng.normal(0, 1, n).astype(np.float32)
    y = O.w8a16_ref(x, q, s, b)
    np.testing.assert_allclose(y, x.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T + b,
                               rtol=1e-12, atol=1e-12)
    # linearity in x, and one-hot x selects a scaled weight column (catches a transposed operand)
    x2 = rng.normal(0, 1, (m, k)).astype(np.float32)
    np.testing.assert_allclose(O.w8a16_ref(x + x2, q, s), O.w8a16_ref(x, q, s) + O.w8a16_ref(x2, q, s), rtol=1e-5, atol=1e-5)
    e = np.zeros((1, k), np.float32); e[0, 9] = 1.0
    np.testing.assert_allclose(O.w8a16_ref(e, q, s)[0], q[:, 9] * s.astype(np.float64))


def test_w8a8_oracle_invariants():
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (4, 96)).astype(np.float32)
    w = rng.normal(0, 0.02, (9, 96)).astype(np.float32)
    qx, sx = O.quant_act_fp8(O.f32_to_bf16_bits(x), O.DT_BF16)
    qw, sw = O.pack_fp8(w)
    y = O.w8a8_ref(qx, sx, qw, sw)
    tab = O.e4m3_decode_table().astype(np.float64)
    ref = (tab[qx] * sx[:, None]) @ (tab[qw] * sw[:, None]).T
    np.testing.assert_allclose(y, ref, rtol=1e-12)
    # quantization error of W8A8 against the unquantized product stays within a few %
    exact = O.bf16_bits_to_f32(O.f32_to_bf16_bits(x)).astype(np.float64) @ w.T.astype(np.float64)
    assert O.rel_err(y, exact) < 0.15


def test_naive_cpu_path_matches_golden():
    z = _load("gemm_small")
    for case in sorted({k.split(".")[0] for k in z.files}):
        x = torch.from_numpy(z[f"{case}.x"].view(np.int16)).view(torch.bfloat16)
        s = torch.from_numpy(z[f"{case}.scale_bf16"].view(np.int16)).view(torch.bfloat16)
        b = (torch.from_numpy(z[f"{case}.bias"].view(np.int16)).view(torch.bfloat16)
             if f"{case}.bias" in z.files else None)
        y = cpu_path.naive_dequant_linear(x, torch.from_numpy(z[f"{case}.q"]), s, b).float().numpy()
        exp = O.bf16_bits_to_f32(z[f"{case}.y_naive_bf16"])
        # bf16 GEMM accumulation order is library-dependent: allow one bf16 step.
        np.testing.assert_allclose(y, exp, rtol=2 ** -7, atol=1e-6, err_msg=case)
        # The reference's formula rounds the dequantized weight and the output to
        # bf16, so it sits near (and on a 3-sigma output, just past) the 1e-2 bar.
        assert O.rel_err(y, z[f"{case}.y_f64"]) < 2e-2


def test_bf16_rounding_helpers():
    v = np.float32([1.0, 1.00390625, 1.005859375, -3.0e-39, 65504.0, np.inf])
    ours = O.f32_to_bf16_bits(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


# ---- int8 W8A8 (Int8Method.apply, qtts/quant/int8.py:146-160) ---------------------------

_I8_DT = {"bf16": O.DT_BF16, "f16": O.DT_F16, "f32": O.DT_F32}


@pytest.mark.parametrize("mode", list(MODES))
def test_act_int8_matches_golden(mode):
    z = _load("int8_w8a8")
    cases = sorted({k.rsplit(".", 1)[0] for k in z.files if k.startswith("act.") and k.endswith(".x")})
    assert len(cases) == 12
    for case in cases:
        dt = _I8_DT[case.rsplit(".", 1)[1]]
        q, s = O.quant_act_int8(z[f"{case}.x"], dt, MODES[mode])
        np.testing.assert_array_equal(q, z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(s.view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32), err_msg=case)


@pytest.mark.parametrize("mode", list(MODES))
def test_int8_linear_matches_golden(mode):
    z = _load("int8_w8a8")
    cases = sorted({k.rsplit(".", 1)[0] for k in z.files if k.startswith("lin.") and k.endswith(".x")})
    assert len(cases) == 5
    for case in cases:
        dt = _I8_DT[case.rsplit(".", 1)[1]]
        qx, sx = O.quant_act_int8(z[f"{case}.x"], dt, MODES[mode])
        bias = z[f"{case}.bias"] if f"{case}.bias" in z.files else None
        y = O.int8_linear_out(qx, sx, z[f"{case}.qw"], z[f"{case}.sw"], bias, dt)
        want = z[f"{case}.{mode}.y"]
        np.testing.assert_array_equal(y.view(np.uint32) if dt == O.DT_F32 else y,
                                      want.view(np.uint32) if dt == O.DT_F32 else want, err_msg=case)


def test_act_int8_closed_forms():
    """Rows whose codes follow from the definition alone."""
    k = 16
    # amax 127 in fp32: scale = 127 * fl(1/127) (device) or exactly 1 (ieee); ties go to even
    x = np.zeros((1, k), np.float32)
    x[0, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]
    q, s = O.quant_act_int8(x, O.DT_F32, O.DIV_IEEE)
    assert s[0] == np.float32(1.0)
    np.testing.assert_array_equal(q[0, :8], [127, 0, 2, 2, 0, -2, -2, 126])
    # an all-zero row: scale = dtype(1e-6) / 127, every code 0
    for dt, floor in ((O.DT_F32, np.float32(1e-6)), (O.DT_BF16, O.bf16_bits_to_f32(O.f32_to_bf16_bits(
            np.float32([1e-6])))[0])):
        z0 = np.zeros((1, k), np.float32 if dt == O.DT_F32 else np.uint16)
        q, s = O.quant_act_int8(z0, dt, O.DIV_IEEE)
        assert not q.any()
        want = np.float32(floor) / np.float32(127.0)
        if dt == O.DT_BF16:
            want = O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.float32([want])))[0]
        assert s[0] == want
    # bf16 double rounding: amax 384 gives the bf16 scale 384/127 -> 3.03125; then
    # 204 / 3.03125 = 67.299 rounds to bf16 67.5 and half-to-even gives 68, and
    # 202 / 3.03125 = 66.639 rounds to 66.5 and then 66 (rounding the fp32 quotients
    # directly would give 67 and 67); the absmax itself, 384 / 3.03125 = 126.68, rounds
    # to bf16 126.5 and then to 126, not 127
    xb = O.f32_to_bf16_bits(np.array([[384.0, 204.0, 202.0] + [0.0] * 13], np.float32))
    q, s = O.quant_act_int8(xb, O.DT_BF16, O.DIV_IEEE)
    assert s[0] == np.float32(3.03125)
    np.testing.assert_array_equal(q[0, :3], [126, 68, 66])
    # fp16 scale underflow: amax 2e-6 gives scale 0; nonzero codes saturate, 0/0 gives 0
    xh = np.zeros((1, k), np.float16)
    xh[0, 0], xh[0, 1] = 2e-6, -1e-6
    q, s = O.quant_act_int8(xh.view(np.uint16), O.DT_F16, O.DIV_DEVICE)
    assert s[0] == 0.0
    np.testing.assert_array_equal(q[0, :3], [127, -127, 0])


def test_int8_linear_oracle_invariants():
    """The integer product against numpy's int64 matmul (a transposed operand or a dropped
    term fails it), and the epilogue order: (acc * sx) * sw, then + bias, rounded once."""
    rng = np.random.default_rng(5)
    m, n, k = 3, 7, 96
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ones_m, ones_n = np.ones(m, np.float32), np.ones(n, np.float32)
    y = O.int8_linear_out(qx, ones_m, qw, ones_n, None, O.DT_F32)
    acc = qx.astype(np.int64) @ qw.astype(np.int64).T
    np.testing.assert_array_equal(y, acc.astype(np.float32))
    sx = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, n).astype(np.float32)
    bias = rng.normal(0, 1, n).astype(np.float32)
    y = O.int8_linear_out(qx, sx, qw, sw, bias, O.DT_F32)
    want = (acc.astype(np.float32) * sx[:, None]).astype(np.float32) * sw[None, :] + bias[None, :]
    np.testing.assert_array_equal(y, want.astype(np.float32))
    yb = O.int8_linear_out(qx, sx, qw, sw, O.f32_to_bf16_bits(bias), O.DT_BF16)
    bb = O.bf16_bits_to_f32(O.f32_to_bf16_bits(bias))
    np.testing.assert_array_equal(
        yb, O.f32_to_bf16_bits((acc.astype(np.float32) * sx[:, None]) * sw[None, :] + bb[None, :]))


def test_fp8w_oracle_matches_numpy_and_one_hot():
    """The fp8 weight-only oracle against numpy's matmul of the decoded codes (the decode
    table is pinned above against the OCP spec), and one-hot rows that read single codes."""
    rng = np.random.default_rng(11)
    m, n, k = 3, 9, 70
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    q = rng.choice(finite, (n, k)).astype(np.uint8)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    s = rng.uniform(0.001, 0.01, n).astype(np.float32)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    lut = O.e4m3_decode_table().astype(np.float64)
    want = x.astype(np.float64) @ (lut[q] * s.astype(np.float64)[:, None]).T + b
    np.testing.assert_allclose(O.fp8w_ref(x, q, s, b), want, rtol=1e-12, atol=1e-12)
    eye = np.eye(k, dtype=np.float32)[:5]
    y = O.fp8w_ref(eye, q, np.ones(n, np.float32))
    np.testing.assert_array_equal(y, lut[q[:, :5]].T)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_silu_mul_oracle_matches_golden(dt):
    """GatedMLP's activation against torch-CPU's F.silu(gate) * up.  The exp of the two
    libraries may differ in the last bit of an fp32 result, which the rounding to a
    16-bit dtype nearly always absorbs: every element within one ulp of the output dtype,
    and at most one in a thousand not exact."""
    z = _load("silu_mul")
    code = {"bf16": O.DT_BF16, "f16": O.DT_F16, "f32": O.DT_F32}[dt]
    h = O.silu_mul(z[f"{dt}.gate_up"], code)
    want = z[f"{dt}.h"]
    if dt == "f32":
        got, ref = h.astype(np.float64), want.astype(np.float64)
        assert np.all(np.abs(got - ref) <= 2.0 ** -22 * np.maximum(np.abs(ref), 1e-30))
        return
    diff = np.abs(h.astype(np.int32) - want.astype(np.int32))
    same_sign = (h >> 15) == (want >> 15)
    assert np.all((diff <= 1) & same_sign | (diff == 0)), dt
    assert np.count_nonzero(diff) <= h.size // 1000, (dt, np.count_nonzero(diff))


def test_silu_mul_oracle_closed_forms():
    """silu(0) = 0; silu(g) -> g for large g and -> -0 for very negative g; up = 1 gives silu itself;
    up = 0 gives zeros of the right sign."""
    k = 8
    gu = np.zeros((1, 2 * k), np.float32)
    gu[0, :k] = [0.0, 100.0, -100.0, 1.0, -1.0, 2.0, 30.0, -30.0]
    gu[0, k:] = 1.0
    h = O.silu_mul(gu, O.DT_F32)[0]
    g = gu[0, :k].astype(np.float64)
    finite = np.arange(k) != 2  # exp(100) overflows fp32: -100 / inf is -0 there, as in torch
    np.testing.assert_allclose(h[finite], (g / (1.0 + np.exp(-g)))[finite], rtol=3e-7)
    assert h[0] == 0.0 and h[1] == 100.0 and h[2] == 0.0 and np.signbit(h[2])


# ---- RMSNorm (qtts/layers/norm.py:50-76) ----------------------------------------------

def _ulp16(v: np.ndarray, dt: str) -> np.ndarray:
    """One unit in the last place of bf16 / fp16 at |v| (normal range)."""
    a = np.maximum(np.abs(v), 1e-30)
    if dt == "bf16":
        return 2.0 ** (np.floor(np.log2(a)) - 7)
    return 2.0 ** (np.maximum(np.floor(np.log2(a)), -14) - 10)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_rms_norm_oracle_matches_golden(dt):
    """The fp64 oracle against torch-CPU's eager RMSNorm (the reference's eager path, the one
    its parity suite runs): every torch output within one unit in the last place of the
    oracle's value, and at most one in a hundred not the oracle's value rounded."""
    z = _load("rms_norm")
    code = {"bf16": O.DT_BF16, "f16": O.DT_F16, "f32": O.DT_F32}[dt]
    eps = float(z["eps"])
    for width in (2048, 1024, 512):
        x, w, want = z[f"{dt}.{width}.x"], z[f"{dt}.{width}.w"], z[f"{dt}.{width}.y"]
        ref = O.rms_norm(x, w, eps, code)
        if dt == "f32":
            np.testing.assert_allclose(want, ref, rtol=1e-6, atol=1e-30)
            continue
        got = (O.bf16_bits_to_f32(want) if dt == "bf16" else want.view(np.float16).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(got - ref) <= _ulp16(ref, dt)), (dt, width)
        rounded = O.f32_to_bf16_bits(ref.astype(np.float32)) if dt == "bf16" else ref.astype(np.float16).view(np.uint16)
        assert np.count_nonzero(rounded != want) <= want.size // 100, (dt, width, np.count_nonzero(rounded != want))


def test_rms_norm_oracle_closed_forms():
    """A constant row c gives c w / sqrt(c^2 + eps); a one-hot row a e_j gives
    a w_j / sqrt(a^2 / k + eps) at j and zeros elsewhere; with eps = 0 the result does not
    change when the row is scaled by a power of two; strides and the weight index follow
    the textbook formula on a random matrix."""
    k = 64
    w = np.linspace(0.5, 1.5, k, dtype=np.float32)
    w64 = w.astype(np.float64)
    x = np.zeros((3, k), np.float32)
    x[0, :] = 0.75
    x[1, 9] = -3.0
    x[2, :] = np.sin(np.arange(k)).astype(np.float32)
    eps = 1e-6
    y = O.rms_norm(x, w, eps, O.DT_F32)
    np.testing.assert_allclose(y[0], 0.75 * w64 / np.sqrt(0.5625 + eps), rtol=1e-14)
    want1 = np.zeros(k)
    want1[9] = -3.0 * w64[9] / np.sqrt(9.0 / k + eps)
    np.testing.assert_allclose(y[1], want1, rtol=1e-14, atol=0)
    y0 = O.rms_norm(x, w, 0.0, O.DT_F32)
    y8 = O.rms_norm(x * 8.0, w, 0.0, O.DT_F32)
    np.testing.assert_allclose(y8, y0, rtol=1e-14)
    rng = np.random.default_rng(3)
    xr = rng.normal(0, 2, (5, 96)).astype(np.float32)
    wr = rng.normal(1, 0.3, 96).astype(np.float32)
    x64 = xr.astype(np.float64)
    textbook = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-5) * wr.astype(np.float64)
    np.testing.assert_allclose(O.rms_norm(xr, wr, 1e-5, O.DT_F32), textbook, rtol=1e-13)
