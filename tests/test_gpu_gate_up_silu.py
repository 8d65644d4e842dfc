"""GPU parity of GatedMLP's gate_up_proj with its activation (``qtts_w8a16_gate_up_silu_strips``).

``act = silu(gate) * up`` of ``gate_up_proj(prologue(x))`` (qtts/layers/activation.py:142-147;
the prologue is post_attention_layernorm, qtts/models/talker.py:271), through the C ABI:

* against this library's separate calls (``w8a16_fused_gemm_strips`` with the same prologue,
  then ``silu_mul``) bit for bit at the separate GEMM's own wave configuration: up to 8 rows
  run one launch whose waves split K as the separate GEMM's do and sum gate and up in the
  same order, and the activation rounds as torch does;
* against the fp64 oracle: the W8A16 bar on gate and up (|err| <= 1e-2 RMS + ulp/2)
  carried through silu(g) * u to first order, plus the activation's two roundings;
* graph replays, the GatedMLP forward, and the separate fallback (more than 8 rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from test_gpu_gemm import half_ulp

pytestmark = pytest.mark.gpu

EPS = 1e-6
GATE_UP = [(12288, 2048), (6144, 1024), (96, 512), (64, 1024)]  # talker, predictor, ragged pairs
_TD = {torch.bfloat16: O.DT_BF16, torch.float16: O.DT_F16}


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _bound(ref, dtype):
    rms = float(np.sqrt(np.mean(ref * ref)))
    return 1e-2 * rms + half_ulp(ref, dtype)


def _act_ref_and_bound(gu: np.ndarray, dtype):
    half = gu.shape[1] // 2
    g, u = gu[:, :half], gu[:, half:]
    sig = 1.0 / (1.0 + np.exp(-g))
    sg = g * sig
    dsg = sig * (1.0 + g * (1.0 - sig))
    act = sg * u
    bound = (1.25 * (np.abs(dsg * u) * _bound(g, dtype) + np.abs(sg) * _bound(u, dtype))
             + 2 * half_ulp(act, dtype) + np.abs(u) * half_ulp(sg, dtype))
    return act, bound


def _case(ops, n, k, dtype, sdtype, seed, bias):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    q, s = ops.pack_int8(w, sdtype)
    b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if bias else None
    nw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(dtype)
    return q, s, ops.to_strips(q), b, nw


@pytest.mark.parametrize("n,k", GATE_UP)
def test_gate_up_silu_matches_separate_and_oracle(ops, n, k):
    from qtts_amd.ops import PRO_NONE, PRO_RMS_NORM
    for dtype, sdtype in ((torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)):
        q, s, qs, b, nw = _case(ops, n, k, dtype, sdtype, seed=n + 7 * k, bias=True)
        for m in (1, 2, 3, 4, 5, 8, 11, 16):
            g = torch.Generator(device="cuda").manual_seed(m * 13 + k)
            x = (torch.randn(m, k, device="cuda", generator=g) * 2).to(dtype)
            for pro in (PRO_NONE, PRO_RMS_NORM):
                bias = b if m % 2 else None
                what = f"{dtype} n={n} k={k} m={m} pro={pro} bias={bias is not None}"
                # bit for bit at the plain GEMM's own configuration (same waves, same chunks)
                cfg = ops.algo_code(1, 0, max(1, (k // 64) // 8), 8)
                act8 = ops.w8a16_gate_up_silu_strips(x, qs, n, s, bias, prologue=pro, norm_weight=nw, eps=EPS,
                                                     algo=cfg)
                gu = ops.w8a16_fused_gemm_strips(x, qs, n, s, bias, prologue=pro, norm_weight=nw, eps=EPS, algo=cfg)
                sep = ops.silu_mul(gu)
                assert torch.equal(act8, sep), (what, int((act8 != sep).sum()))
                if m <= 16:
                    # half strips (8 gate rows and their 8 up rows a workgroup, the plain GEMM's grid; 9-16
                    # rows in two row parts of 8): bit for bit the separate calls at the same configuration too
                    half = ops.algo_code(3, 0, max(1, (k // 64) // 8), 8)
                    act_h = ops.w8a16_gate_up_silu_strips(x, qs, n, s, bias, prologue=pro, norm_weight=nw, eps=EPS,
                                                          algo=half)
                    assert torch.equal(act_h, sep), (what, "half strips", int((act_h != sep).sum()))
                # the automatic configuration (half strips up to 8 rows) within tolerance below
                act = ops.w8a16_gate_up_silu_strips(x, qs, n, s, bias, prologue=pro, norm_weight=nw, eps=EPS)
                # the oracle on the same GEMM input (normalized rows as the kernel stages them)
                if pro == PRO_RMS_NORM:
                    h = torch.from_numpy(O.rms_norm(_bits(x), _bits(nw), EPS, _TD[dtype])).to(dtype)
                else:
                    h = x.cpu()
                ref_gu = O.w8a16_ref(h.float().numpy(), q.cpu().numpy(), s.float().cpu().numpy(),
                                     None if bias is None else bias.float().cpu().numpy())
                ref, bound = _act_ref_and_bound(ref_gu, dtype)
                err = np.abs(act.double().cpu().numpy() - ref)
                bad = err > bound
                assert not bad.any(), (what, int(bad.sum()), float(err.max()))


def test_gate_up_silu_graph_replays(ops):
    from qtts_amd.ops import PRO_RMS_NORM
    n, k = 12288, 2048
    q, s, qs, b, nw = _case(ops, n, k, torch.bfloat16, torch.bfloat16, seed=3, bias=False)
    x = torch.randn(4, k, device="cuda").to(torch.bfloat16)
    run = lambda: ops.w8a16_gate_up_silu_strips(x, qs, n, s, prologue=PRO_RMS_NORM, norm_weight=nw)  # noqa: E731
    out = run()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        run()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for rep in range(3):
        x.copy_(torch.randn(4, k, device="cuda").to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = run()
        assert torch.equal(out, want), f"replay {rep}"


def test_gated_mlp_takes_the_pair_path(ops, monkeypatch):
    """GatedMLP.forward with an int8 weight-only gate_up returns down(silu(gate) * up) with the
    activation from gate_up's epilogue, within the W8A16 bound of the reference's composition on
    the same layers (the fused launch splits K across twice the waves)."""
    from qtts_amd.layers import GatedMLP
    from qtts_amd.quant.int8 import Int8WeightOnlyMethod
    calls = []
    real = ops.w8a16_gate_up_silu_strips
    monkeypatch.setattr(ops, "w8a16_gate_up_silu_strips", lambda *a, **k: calls.append(1) or real(*a, **k))
    torch.manual_seed(0)
    mlp = GatedMLP(2048, 6144, dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        for p in mlp.parameters():
            p.normal_(0.0, 0.02)
    method = Int8WeightOnlyMethod(calibrate=False)
    for lin in (mlp.gate_up_proj, mlp.down_proj):
        method.process_weights(lin)
        lin.quant_method = method
    for m in (1, 3, 8):
        x = torch.randn(m, 1, 2048, device="cuda").to(torch.bfloat16)
        y = mlp(x)
        gu = mlp.gate_up_proj(x)
        gate, up = mlp.gate_up_proj.split(gu)
        want = mlp.down_proj(F.silu(gate) * up)
        assert y.shape == want.shape
        ref = want.double().cpu().numpy()
        err = np.abs(y.double().cpu().numpy() - ref)
        assert (err <= _bound(ref, torch.bfloat16)).all(), f"m={m}: max err {err.max():.3g}"
    assert len(calls) == 3


def test_gate_up_silu_errors(ops):
    n, k = 96, 512
    q, s, qs, b, nw = _case(ops, n, k, torch.bfloat16, torch.bfloat16, seed=4, bias=False)
    x = torch.randn(2, k, device="cuda").to(torch.bfloat16)
    with pytest.raises(ValueError):
        ops.w8a16_gate_up_silu_strips(x, qs, 95, s)
    with pytest.raises(ValueError):
        ops.w8a16_gate_up_silu_strips(x[:, :500], qs, n, s)
    with pytest.raises(ValueError):
        ops.w8a16_gate_up_silu_strips(x, qs, n, s, prologue=ops.PRO_RMS_NORM)  # no norm weight
    empty = ops.w8a16_gate_up_silu_strips(x[:0], qs, n, s)
    assert empty.shape == (0, n // 2)


def test_decoder_helpers_fuse_int8_layers(ops, monkeypatch):
    """qtts_amd.layers.decoder on int8 weight-only layers: norm + qkv, o + residual, and norm + MLP +
    residual each run as fused launches (two for the MLP) and agree with the reference's composition
    within the W8A16 bound, stage by stage."""
    from torch import nn

    from qtts_amd.layers import GatedMLP, LinearBase
    from qtts_amd.layers.decoder import linear_residual, norm_linear, norm_mlp_residual
    from qtts_amd.quant.int8 import Int8WeightOnlyMethod

    class Norm(nn.Module):
        def __init__(self, n):
            super().__init__()
            self.weight = nn.Parameter((1 + 0.1 * torch.randn(n, device="cuda")).to(torch.bfloat16),
                                       requires_grad=False)
            self.eps = 1e-6

        def forward(self, x):
            return ops.rms_norm(x, self.weight, self.eps)

    calls = {"fused": 0, "pair": 0}
    real_fused, real_pair = ops.w8a16_fused_gemm_strips, ops.w8a16_gate_up_silu_strips
    monkeypatch.setattr(ops, "w8a16_fused_gemm_strips",
                        lambda *a, **k: calls.__setitem__("fused", calls["fused"] + 1) or real_fused(*a, **k))
    monkeypatch.setattr(ops, "w8a16_gate_up_silu_strips",
                        lambda *a, **k: calls.__setitem__("pair", calls["pair"] + 1) or real_pair(*a, **k))
    torch.manual_seed(1)
    method = Int8WeightOnlyMethod(calibrate=False)
    qkv = LinearBase(2048, 4096, dtype=torch.bfloat16, device="cuda")
    o = LinearBase(2048, 2048, dtype=torch.bfloat16, device="cuda")
    mlp = GatedMLP(2048, 6144, dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        for mod in (qkv, o, mlp):
            for p in mod.parameters():
                p.normal_(0.0, 0.02)
    for lin in (qkv, o, mlp.gate_up_proj, mlp.down_proj):
        method.process_weights(lin)
        lin.quant_method = method
    n_in, n_post = Norm(2048), Norm(2048)

    def check(got, want, what):
        ref = want.double().cpu().numpy()
        err = np.abs(got.double().cpu().numpy() - ref)
        assert (err <= 2 * _bound(ref, torch.bfloat16)).all(), f"{what}: max err {err.max():.3g}"

    for m in (1, 4, 8):
        h = (torch.randn(m, 1, 2048, device="cuda") * 2).to(torch.bfloat16)
        attn = torch.randn(m, 1, 2048, device="cuda").to(torch.bfloat16)
        check(norm_linear(n_in, qkv, h), qkv(n_in(h)), f"m={m} norm+qkv")
        h1 = linear_residual(o, attn, h)
        check(h1, h + o(attn), f"m={m} o+residual")
        gate, up = mlp.gate_up_proj.split(mlp.gate_up_proj(n_post(h1)))
        check(norm_mlp_residual(n_post, mlp, h1), h1 + mlp.down_proj(F.silu(gate) * up), f"m={m} mlp")
    assert calls == {"fused": 9, "pair": 3}, calls
