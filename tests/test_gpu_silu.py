"""GPU parity of GatedMLP's activation and the fused down projection (qtts/layers/activation.py:142-147).

* ``qtts_silu_mul`` against torch on the GPU evaluating ``F.silu(gate) * up`` (the
  reference's own expression), bit for bit, and against the golden fixtures;
* ``qtts_w8a16_silu_mul_gemm_strips`` against ``qtts_w8a16_gemm_strips`` of torch's
  activation with the same kernel configuration, bit for bit (the fused decode path
  computes the activation inside the GEMM), and against the oracle within the W8A16
  tolerance;
* the GatedMLP forward with an int8 weight-only down projection against the
  reference's composition.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from test_gpu_gemm import assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DOWN = [(2048, 6144), (1024, 3072), (2048, 2048), (48, 512)]


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _gate_up(m, k, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(m, 2 * k, device="cuda", generator=g) * 3).to(dtype)


def _torch_act(gu):
    k = gu.shape[-1] // 2
    gate, up = gu.split([k, k], dim=-1)
    return F.silu(gate) * up


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_silu_mul_vs_torch_gpu(ops, dtype):
    for m, k in ((1, 6144), (3, 3072), (8, 1024), (5, 100), (2, 8)):
        gu = _gate_up(m, k, dtype, seed=m + k)
        h = ops.silu_mul(gu)
        ref = _torch_act(gu)
        if dtype == torch.float32:
            torch.testing.assert_close(h, ref, rtol=3e-7, atol=0)
        else:
            assert torch.equal(h, ref), f"{dtype} m={m} k={k}: {int((h != ref).sum())} elements differ"


def test_silu_mul_golden(ops):
    z = np.load(os.path.join(GOLDEN, "silu_mul.npz"))
    for dt, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        gu = torch.from_numpy(z[f"{dt}.gate_up"].view(np.int16)).view(tdt).cuda()
        h = ops.silu_mul(gu).view(torch.int16).cpu().numpy().view(np.uint16)
        want = z[f"{dt}.h"]
        diff = np.abs(h.astype(np.int32) - want.astype(np.int32))
        assert diff.max() <= 1 and np.count_nonzero(diff) <= h.size // 1000, dt


@pytest.mark.parametrize("n,k", DOWN)
def test_silu_down_matches_composition(ops, n, k):
    """Fused (M = 1) and two-pass (M > 1) paths equal the W8A16 GEMM of torch's activation
    under the same configuration, and meet the oracle's tolerance."""
    for dtype in (torch.bfloat16, torch.float16):
        g = torch.Generator(device="cuda").manual_seed(n + k)
        w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
        q, s = ops.pack_int8(w, dtype)
        qs = ops.to_strips(q)
        for m in (1, 2, 3, 8, 17):
            gu = _gate_up(m, k, dtype, seed=7 * m + k)
            b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(dtype) if m % 2 else None
            h = _torch_act(gu)
            for algo in (0, ops.algo_code(1, 0, 4, 8), ops.algo_code(1, 2, 8, 8), ops.algo_code(1, 0, 16, 6)):
                if m > 16 and algo:
                    continue
                y = ops.w8a16_silu_mul_gemm_strips(gu, qs, n, s, b, algo)
                if algo or m > 1:  # the automatic fused choice may pick other waves than the plain GEMM
                    assert torch.equal(y, ops.w8a16_gemm_strips(h, qs, n, s, b, algo)), \
                        f"{dtype} n={n} k={k} m={m} algo={algo:#x}"
                ref = O.w8a16_ref(h.float().cpu().numpy(), q.cpu().numpy(), s.float().cpu().numpy(),
                                  None if b is None else b.float().cpu().numpy())
                assert_close(y, ref, f"{dtype} n={n} k={k} m={m} algo={algo:#x}")


def test_silu_down_graph_replays(ops):
    n, k = 2048, 6144
    w = (torch.randn(n, k, device="cuda") * 0.02).to(torch.bfloat16)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    gu = _gate_up(1, k, torch.bfloat16, seed=3)
    eager = ops.w8a16_silu_mul_gemm_strips(gu, qs, n, s)
    static = gu.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.w8a16_silu_mul_gemm_strips(static, qs, n, s)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.w8a16_silu_mul_gemm_strips(static, qs, n, s)
    for i in range(3):
        other = ops.w8a16_silu_mul_gemm_strips(_gate_up(4, k, torch.bfloat16, seed=i), qs, n, s)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        assert other.shape == (4, n)


def test_gated_mlp_fused_forward(ops):
    """GatedMLP with int8 weight-only projections against the reference's composition
    down_proj(F.silu(gate) * up) on the same quantized layers: within the W8A16 bound at decode
    rows (gate_up's fused launch splits K over other waves than the plain GEMM), bit for bit at
    prefill rows (the activation then runs as its own kernel)."""
    from qtts_amd import QuantConfig, apply_quantization
    from qtts_amd.layers import GatedMLP, gated_mlp_forward
    torch.manual_seed(0)
    mlp = GatedMLP(2048, 6144, dtype=torch.bfloat16, device="cuda")
    for p in mlp.parameters():
        p.data.normal_(0, 0.02)
    holder = torch.nn.Module()
    holder.mlp = mlp
    report = apply_quantization(QuantConfig(method="int8_weight_only", calibrate=False), talker=holder)
    assert report["talker"]["converted"] == 2
    for m in (1, 2, 5, 40):
        x = torch.randn(m, 2048, device="cuda").to(torch.bfloat16)
        fused = mlp(x)
        gate, up = mlp.gate_up_proj.split(mlp.gate_up_proj(x))
        assert torch.equal(fused, gated_mlp_forward(mlp, x))
        composed = mlp.down_proj(F.silu(gate) * up)
        if m > 8:
            assert torch.equal(fused, composed), f"m={m}"
        else:
            assert_close(fused, composed.double().cpu().numpy(), f"m={m}")
