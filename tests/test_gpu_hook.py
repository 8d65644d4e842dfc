"""The drop-in boundary end to end on the GPU: LinearBase modules quantized by
apply_quantization, run eagerly and from a captured HIP graph, checked against
the oracle's dequantize-then-matmul (qtts/layers/linear.py:57-60 ->
qtts/quant/int8.py:116-117 / qtts/quant/fp8.py:72-89)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from test_gpu_gemm import assert_close

pytestmark = pytest.mark.gpu


class TalkerLayer(nn.Module):
    """The four talker linears plus an excluded head and a biased text projection."""

    def __init__(self, hidden=2048, inter=6144, dtype=torch.bfloat16):
        super().__init__()
        from qtts_amd.layers.linear import LinearBase, MergedLinear
        self.qkv_proj = MergedLinear(hidden, [hidden, hidden // 2, hidden // 2], dtype=dtype, device="cuda")
        self.o_proj = LinearBase(hidden, hidden, dtype=dtype, device="cuda")
        self.gate_up_proj = MergedLinear(hidden, [inter, inter], dtype=dtype, device="cuda")
        self.down_proj = LinearBase(inter, hidden, dtype=dtype, device="cuda")
        self.text_proj_fc1 = LinearBase(hidden, hidden, bias=True, dtype=dtype, device="cuda")
        self.codec_head = LinearBase(hidden, 3072, dtype=dtype, device="cuda")
        g = torch.Generator(device="cuda").manual_seed(11)
        for p in self.parameters():
            p.data.copy_((torch.randn(p.shape, device="cuda", generator=g) * 0.02).to(dtype))

    def forward(self, x):
        q, k, v = self.qkv_proj.split(self.qkv_proj(x))
        h = self.o_proj(q) + self.text_proj_fc1(x)
        gate, up = self.gate_up_proj.split(self.gate_up_proj(h))
        return self.down_proj(torch.nn.functional.silu(gate) * up), self.codec_head(h)


def _expected_int8(layer, x):
    """Dequantize-then-matmul in fp32 of the packed buffers (the oracle formula on the GPU)."""
    from qtts_amd.quant.int8 import int8_weight_rowmajor
    w = int8_weight_rowmajor(layer).float() * layer.int8_scale.float()[:, None]
    y = x.float() @ w.t()
    if layer.bias is not None:
        y = y + layer.bias.float()
    return y.double().cpu().numpy()


@pytest.mark.parametrize("calibrate", [False, True])
def test_int8_weight_only_hook(calibrate):
    from qtts_amd import QuantConfig, apply_quantization
    from qtts_amd.quant import calibrate as cal
    cal.clear_cache()
    model = TalkerLayer()
    report = apply_quantization(QuantConfig(method="int8_weight_only", calibrate=calibrate), talker=model,
                                calibration_batch=8)
    r = report["talker"]
    assert r["excluded"] == 1 and r["converted"] + r["declined"] == 5
    from qtts_amd.quant.calibrate import ALGO_REFERENCE_GEMM
    from qtts_amd.quant.int8 import layer_algo
    if not calibrate:
        assert r["converted"] == 5 and r["bytes_after"] < r["bytes_before"] and r["kept_weight"] == 0
    else:
        # calibrated per row bucket: every converted layer's shape has a kernel choice for every
        # bucket the callers produce (decode rows, code-predictor rows up to 128, prefill)
        from qtts_amd.quant.int8 import M_BUCKETS
        for name in ("qkv_proj", "o_proj", "gate_up_proj", "down_proj", "text_proj_fc1"):
            layer = getattr(model, name)
            if layer.quant_method is not None:
                assert sorted(layer.quant_algos) == list(M_BUCKETS), name
    assert model.codec_head.quant_method is None and model.codec_head.weight.numel() > 0
    ms = (1, 2, 3, 4, 8, 16, 17, 32, 48, 64, 100, 128) if calibrate else (1, 4, 8, 17)
    for m in ms:
        x = torch.randn(m, 1, 2048, device="cuda").to(torch.bfloat16)
        for name in ("qkv_proj", "o_proj", "text_proj_fc1", "gate_up_proj", "down_proj"):
            layer = getattr(model, name)
            if layer.quant_method is None:
                continue
            xin = x if layer.in_features == 2048 else torch.randn(m, 1, layer.in_features, device="cuda").to(x.dtype)
            y = layer(xin)
            assert y.shape == (m, 1, layer.out_features) and y.dtype == torch.bfloat16
            if layer_algo(layer, m) == ALGO_REFERENCE_GEMM:  # F.linear beat every kernel at this bucket
                assert torch.equal(y, F.linear(xin, layer.weight, layer.bias)), f"{name} m={m}"
                continue
            assert_close(y.reshape(m, -1), _expected_int8(layer, xin.reshape(m, -1)), f"{name} m={m}")


def test_int8_hook_graph_capture_matches_eager():
    from qtts_amd import QuantConfig, apply_quantization
    model = TalkerLayer()
    apply_quantization(QuantConfig(method="int8_weight_only", calibrate=False), talker=model)
    x = torch.randn(4, 2048, device="cuda").to(torch.bfloat16)
    eager = model(x)
    static_x = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model(static_x)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = model(static_x)
    for i in range(4):
        model(x * 0.5)  # eager work in between
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a, b), f"replay {i}"


def test_fp8_hook():
    from qtts_amd import QuantConfig, apply_quantization, ops
    import oracle as O
    model = TalkerLayer()
    report = apply_quantization(QuantConfig(method="fp8"), talker=model)
    assert report["talker"]["converted"] == 5
    from qtts_amd.quant.fp8 import fp8_weight_rowmajor
    layer = model.text_proj_fc1
    qw = fp8_weight_rowmajor(layer)
    assert qw.shape == (2048, 2048) and layer.fp8_weight.numel() == 2048 * 2048
    for m in (1, 8, 256):
        x = torch.randn(m, 2048, device="cuda").to(torch.bfloat16)
        y = layer(x)
        qx, sx = ops.quant_act_fp8(x)
        ref = O.w8a8_ref(qx.view(torch.uint8).cpu().numpy(), sx.cpu().numpy(),
                         qw.view(torch.uint8).cpu().numpy(), layer.fp8_scale.reshape(-1).cpu().numpy())
        # the reference rounds the scaled product to bf16, then adds the bias in bf16
        assert_close(y, ref + layer.bias.double().cpu().numpy(), f"fp8 m={m}", inter=ref)


def test_fp8_weight_only_builds():
    """The reference raises NotImplementedError here (qtts/quant/fp8.py:115-123); this backend has
    the fused kernel the stub asks for (tests/test_gpu_fp8w.py checks its numerics)."""
    from qtts_amd import QuantConfig, build_method
    method = build_method(QuantConfig(method="fp8_weight_only", calibrate=False))
    assert method.name == "fp8_weight_only" and not method.calibrate
