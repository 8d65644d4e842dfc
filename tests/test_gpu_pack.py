"""GPU parity of the packers and the fp8 activation quantizer (bit-exact).

Checked three ways: against the committed golden fixtures, against the C oracle
on seeded full-size rows, and against torch on the GPU evaluating the reference's
literal expressions (which pins the device division semantics).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODES = {"ieee": 1, "device": 0}


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    return _ops


def _cases(z):
    return sorted({k.rsplit(".", 1)[0] for k in z.files if k.endswith(".src")})


def _to_dev(src: np.ndarray, is_f32: bool) -> torch.Tensor:
    if is_f32:
        return torch.from_numpy(src).cuda()
    return torch.from_numpy(src.view(np.int16)).view(torch.bfloat16).cuda()


@pytest.mark.parametrize("mode", list(MODES))
def test_pack_int8_golden(ops, mode):
    z = np.load(os.path.join(GOLDEN, "int8_pack.npz"))
    for case in _cases(z):
        print("case", case, mode, flush=True)
        w = _to_dev(z[f"{case}.src"], case.endswith(".f32"))
        q, sb, s32 = ops.pack_int8(w, torch.bfloat16, MODES[mode], want_f32_scale=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(s32.cpu().numpy().view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32))
        np.testing.assert_array_equal(sb.cpu().view(torch.int16).numpy().view(np.uint16),
                                      z[f"{case}.{mode}.scale_bf16"], err_msg=case)


@pytest.mark.parametrize("mode", list(MODES))
def test_pack_fp8_golden(ops, mode):
    z = np.load(os.path.join(GOLDEN, "fp8_pack.npz"))
    for case in _cases(z):
        w = _to_dev(z[f"{case}.src"], case.endswith(".f32"))
        q, s = ops.pack_fp8(w, MODES[mode])
        np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32))


@pytest.mark.parametrize("mode", list(MODES))
def test_quant_act_fp8_golden(ops, mode):
    z = np.load(os.path.join(GOLDEN, "act_fp8.npz"))
    for case in sorted({k.split(".")[0] for k in z.files}):
        x = torch.from_numpy(z[f"{case}.x"].view(np.int16)).view(torch.bfloat16).cuda()
        qx, sx = ops.quant_act_fp8(x, MODES[mode])
        np.testing.assert_array_equal(qx.view(torch.uint8).cpu().numpy(), z[f"{case}.{mode}.q"], err_msg=case)
        np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), z[f"{case}.{mode}.scale"].view(np.uint32))


@pytest.mark.parametrize("n,k", [(4096, 2048), (2048, 6144), (1024, 3072)])
def test_pack_int8_matches_oracle_full_rows(ops, n, k):
    rng = np.random.default_rng(n + k)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    wb = O.f32_to_bf16_bits(w)
    for src, dt in ((w, O.DT_F32), (wb, O.DT_BF16)):
        qo, so, sbo = O.pack_int8(src, dt, O.DT_BF16, O.DIV_DEVICE)
        q, sb, s32 = ops.pack_int8(_to_dev(src, dt == O.DT_F32), torch.bfloat16, 0, want_f32_scale=True)
        assert torch.equal(q.cpu(), torch.from_numpy(qo))
        np.testing.assert_array_equal(s32.cpu().numpy().view(np.uint32), so.view(np.uint32))
        np.testing.assert_array_equal(sb.cpu().view(torch.int16).numpy().view(np.uint16), sbo)


def test_pack_int8_matches_torch_gpu_literal(ops):
    """The reference's expressions executed by torch on this GPU (qtts/quant/int8.py:53-55, :105)."""
    g = torch.Generator(device="cuda").manual_seed(1)
    for dtype in (torch.float32, torch.bfloat16):
        weight = (torch.randn(2048, 2048, device="cuda", generator=g) * 0.02).to(dtype)
        w = weight.detach().float()
        scale = w.abs().amax(dim=1).clamp_min(1e-12) / 127.0
        q_ref = (w / scale[:, None]).round().clamp_(-127.0, 127.0).to(torch.int8)
        q, sb, s32 = ops.pack_int8(weight, dtype, 0, want_f32_scale=True)
        assert torch.equal(s32, scale), "device division semantics differ from torch on this GPU"
        assert torch.equal(q, q_ref)
        assert torch.equal(sb, scale.to(dtype))


def test_pack_fp8_matches_torch_gpu_literal(ops):
    """qtts/quant/fp8.py:47-49 executed by torch on this GPU."""
    g = torch.Generator(device="cuda").manual_seed(2)
    weight = (torch.randn(1024, 3072, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    w = weight.detach().float()
    scale = w.abs().amax(dim=1).clamp_min(1e-12) / 448.0
    q_ref = (w / scale[:, None]).to(torch.float8_e4m3fn)
    q, s = ops.pack_fp8(weight, 0)
    assert torch.equal(s, scale)
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))


def test_quant_act_fp8_matches_torch_gpu_literal(ops):
    """qtts/quant/fp8.py:76-78 executed by torch on this GPU, with 1% outliers at 20 sigma."""
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(16, 6144, device="cuda", generator=g)
    mask = torch.rand(16, 6144, device="cuda", generator=g) < 0.01
    x = torch.where(mask, torch.sign(x) * 20.0, x).to(torch.bfloat16)
    x[3] = 0
    flat = x.reshape(-1, x.shape[-1]).contiguous()
    scale_x = flat.abs().amax(dim=1, keepdim=True).clamp_min(1e-6).float() / 448.0
    q_ref = (flat.float() / scale_x).to(torch.float8_e4m3fn)
    qx, sx = ops.quant_act_fp8(x, 0)
    assert torch.equal(sx, scale_x.reshape(-1))
    assert torch.equal(qx.view(torch.uint8), q_ref.view(torch.uint8))


def test_pack_edge_shapes(ops):
    """Empty, single-row, single-column and ragged inputs, strided source rows."""
    for n, k in ((0, 16), (1, 1), (3, 1), (5, 257), (17, 33)):
        w = torch.randn(n, k + 3, device="cuda")[:, :k]  # row stride k+3
        q, s, s32 = ops.pack_int8(w, torch.float32, 1, want_f32_scale=True)
        qo, so, _ = O.pack_int8(np.ascontiguousarray(w.cpu().numpy()), O.DT_F32, O.DT_F32, O.DIV_IEEE)
        assert q.shape == (n, k)
        np.testing.assert_array_equal(q.cpu().numpy(), qo)
        np.testing.assert_array_equal(s32.cpu().numpy(), so)
