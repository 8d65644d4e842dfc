"""torch.compile over quantized layers on the GPU: the code predictor's prefix forward is compiled
with ``dynamic=True`` in the reference (qtts/models/code_predictor.py:186-192), and its quantized
linears must not break the graph.  A predictor-shaped stack (hidden 1024, qkv 1024 -> 4096,
o 2048 -> 1024, gate_up 1024 -> 6144, down 3072 -> 1024) is quantized, traced with zero graph
breaks, and the compiled forward (aot_eager: the same kernels, so equal bits) equals eager at
the prefix row counts the predictor runs."""

from __future__ import annotations

import pytest
import torch
import torch._dynamo
import torch.nn.functional as F
from torch import nn

pytestmark = pytest.mark.gpu


class PredictorLayer(nn.Module):
    def __init__(self, seed):
        super().__init__()
        from qtts_amd.layers.linear import LinearBase, MergedLinear
        kw = dict(dtype=torch.bfloat16, device="cuda")
        self.qkv_proj = MergedLinear(1024, [2048, 1024, 1024], **kw)
        self.o_proj = LinearBase(2048, 1024, **kw)
        self.gate_up_proj = MergedLinear(1024, [3072, 3072], **kw)
        self.down_proj = LinearBase(3072, 1024, **kw)
        g = torch.Generator(device="cuda").manual_seed(seed)
        for p in self.parameters():
            p.data.copy_((torch.randn(p.shape, device="cuda", generator=g) * 0.02).to(p.dtype))

    def forward(self, h):
        q, k, v = self.qkv_proj.split(self.qkv_proj(F.rms_norm(h, (1024,))))
        h = h + self.o_proj(q)
        gate, up = self.gate_up_proj.split(self.gate_up_proj(F.rms_norm(h, (1024,))))
        return h + self.down_proj(F.silu(gate) * up)


@pytest.mark.parametrize("method", ["int8_weight_only", "fp8", "int8"])
def test_compiled_predictor_stack_matches_eager(method):
    from qtts_amd import QuantConfig, apply_quantization
    torch._dynamo.reset()
    stack = nn.Sequential(PredictorLayer(1), PredictorLayer(2))
    report = apply_quantization(QuantConfig(method=method, calibrate=False), talker=stack)
    assert report["talker"]["converted"] == 8
    x = torch.randn(1, 16, 1024, device="cuda").to(torch.bfloat16)
    ex = torch._dynamo.explain(stack)(x)
    assert ex.graph_break_count == 0, ex.break_reasons
    compiled = torch.compile(stack, dynamic=True, backend="aot_eager")
    for b, p in ((1, 2), (1, 9), (1, 16), (4, 7), (8, 16)):  # batch x prefix length: M = b * p up to 128
        print(f"{method} b={b} p={p}", flush=True)
        x = torch.randn(b, p, 1024, device="cuda").to(torch.bfloat16)
        with torch.no_grad():
            assert torch.equal(compiled(x), stack(x)), (b, p)
