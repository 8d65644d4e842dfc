"""The quantized linears as torch custom ops (qtts_amd/torch_ops.py), without a GPU: every op is
registered under ``torch.ops.qtts``, its fake implementation gives the output shape and dtype the
real one returns, and dynamo traces a quantized code-predictor-style forward through the quant
methods' ``apply`` with no graph break (the reference compiles that forward with
``torch.compile(dynamic=True)``, qtts/models/code_predictor.py:186-192)."""

from __future__ import annotations

import torch
import torch._dynamo
import torch.nn.functional as F
from torch import nn
from torch._subclasses.fake_tensor import FakeTensorMode

from qtts_amd import ops, torch_ops
from qtts_amd.layers.linear import LinearBase, MergedLinear
from qtts_amd.quant import int8 as I
from qtts_amd.quant import fp8 as P


def test_every_op_is_registered():
    for name in torch_ops.OPS:
        assert hasattr(torch.ops.qtts, name), name


def test_fake_shapes():
    bf = torch.bfloat16
    with FakeTensorMode():
        x = torch.empty(3, 5, 1024, dtype=bf, device="cuda")
        qs = torch.empty(4096 * 1024, dtype=torch.int8, device="cuda")
        s = torch.empty(4096, dtype=bf, device="cuda")
        sf = torch.empty(4096, dtype=torch.float32, device="cuda")
        q8 = torch.empty(4096, 1024, dtype=torch.int8, device="cuda")
        f8 = torch.empty(4096, 1024, dtype=torch.float8_e4m3fn, device="cuda")
        w = torch.empty(1024, dtype=bf, device="cuda")
        gu = torch.empty(3, 5, 2048, dtype=bf, device="cuda")
        res = torch.empty(3, 5, 4096, dtype=bf, device="cuda")
        q = torch.ops.qtts
        for y, want in ((q.w8a16_gemm_strips(x, qs, 4096, s, None, 0), 4096),
                        (q.w8a16_gemm(x, q8, s, None, 0), 4096),
                        (q.fp8_linear(x, f8, sf, None, 0, 0), 4096),
                        (q.fp8_linear_strips(x, qs, 4096, sf, None, 0, 0), 4096),
                        (q.int8_linear(x, q8, sf, None, 0, 0), 4096),
                        (q.int8_linear_strips(x, qs, 4096, sf, None, 0, 0), 4096),
                        (q.fp8w_gemm_strips(x, qs, 4096, sf, None, 0), 4096),
                        (q.dequant_linear(x, qs, 0, 4096, 1024, s, None), 4096),
                        (q.rms_norm(x, w, 1e-6), 1024),
                        (q.silu_mul(gu), 1024),
                        (q.w8a16_silu_mul_gemm_strips(gu, qs, 4096, s, None, 0), 4096),
                        (q.w8a16_fused_gemm_strips(x, qs, 4096, s, None, ops.PRO_RMS_NORM, w, 1e-6, res, 0), 4096),
                        (q.w8a16_gate_up_silu_strips(x, qs, 4096, s, None, ops.PRO_NONE, None, 1e-6, 0), 2048)):
            assert y.shape == (3, 5, want) and y.dtype == bf


def _meta_int8_layer(layer: nn.Module) -> nn.Module:
    """What Int8WeightOnlyMethod.process_weights leaves on a layer, as meta tensors."""
    n, k = layer.out_features, layer.in_features
    layer.register_buffer("int8_weight", torch.empty(n * k, dtype=torch.int8, device="meta"), persistent=False)
    layer.register_buffer("int8_scale", torch.empty(n, dtype=torch.bfloat16, device="meta"), persistent=False)
    layer.int8_layout = "strips"
    layer.weight = nn.Parameter(torch.empty(0, dtype=torch.bfloat16, device="meta"), requires_grad=False)
    method = I.Int8WeightOnlyMethod.__new__(I.Int8WeightOnlyMethod)  # apply needs no GPU state
    layer.quant_method = method
    return layer


class PredictorLayer(nn.Module):
    """The code predictor's four linears (hidden 1024, 16 q / 8 kv heads of 128, intermediate 3072)
    around torch norms and activations, attention left out."""

    def __init__(self):
        super().__init__()
        kw = dict(dtype=torch.bfloat16, device="meta")
        self.qkv_proj = _meta_int8_layer(MergedLinear(1024, [2048, 1024, 1024], **kw))
        self.o_proj = _meta_int8_layer(LinearBase(2048, 1024, **kw))
        self.gate_up_proj = _meta_int8_layer(MergedLinear(1024, [3072, 3072], **kw))
        self.down_proj = _meta_int8_layer(LinearBase(3072, 1024, **kw))

    def forward(self, h):
        q, k, v = self.qkv_proj.split(self.qkv_proj(F.rms_norm(h, (1024,))))
        h = h + self.o_proj(q)
        gate, up = self.gate_up_proj.split(self.gate_up_proj(F.rms_norm(h, (1024,))))
        return h + self.down_proj(F.silu(gate) * up)


def test_dynamo_traces_quantized_layers_without_breaks():
    torch._dynamo.reset()
    stack = nn.Sequential(PredictorLayer(), PredictorLayer())
    for rows in (2, 16):  # prefix rows b * p vary from call to call
        x = torch.empty(1, rows, 1024, dtype=torch.bfloat16, device="meta")
        ex = torch._dynamo.explain(stack)(x)
        assert ex.graph_break_count == 0, ex.break_reasons
        assert ex.graph_count == 1
        names = [str(n.target) for g in ex.graphs for n in g.graph.nodes if n.op == "call_function"]
        assert sum("qtts.w8a16_gemm_strips" in t for t in names) == 8, names


def test_fp8_and_int8_methods_trace():
    torch._dynamo.reset()
    lin = LinearBase(1024, 2048, bias=True, dtype=torch.bfloat16, device="meta")
    lin.register_buffer("fp8_weight", torch.empty(2048 * 1024, dtype=torch.float8_e4m3fn, device="meta"),
                        persistent=False)
    lin.register_buffer("fp8_scale", torch.empty(1, 2048, dtype=torch.float32, device="meta"), persistent=False)
    lin.fp8_layout = "strips"
    m = P.Fp8Method.__new__(P.Fp8Method)
    m.div_mode = 0
    lin.quant_method = m
    lin2 = LinearBase(2048, 1024, dtype=torch.bfloat16, device="meta")
    lin2.register_buffer("int8_weight", torch.empty(2048 * 1024, dtype=torch.int8, device="meta"), persistent=False)
    lin2.register_buffer("int8_scale", torch.empty(1024, dtype=torch.float32, device="meta"), persistent=False)
    lin2.int8_layout = "strips"
    m2 = I.Int8Method.__new__(I.Int8Method)
    m2.div_mode = 0
    lin2.quant_method = m2
    f = lambda x: lin2(F.silu(lin(x)))  # noqa: E731
    ex = torch._dynamo.explain(f)(torch.empty(3, 1024, dtype=torch.bfloat16, device="meta"))
    assert ex.graph_break_count == 0, ex.break_reasons
