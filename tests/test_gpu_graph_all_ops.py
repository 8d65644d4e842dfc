"""Every quantized path of the library in ONE captured HIP graph, per row count.

Four layers, one per method (int8 weight-only with the decoder-layer fusions, fp8 W8A8,
int8 W8A8, fp8 weight-only), each a predictor-sized decoder block (qkv, o + residual,
gate_up + SiLU, down + residual), run eagerly once and then captured together with
torch's default (global) capture mode, under which any allocation or synchronizing call
the library made during capture would fail the capture.  Workspaces are reserved when
the weights are processed, so a row count first seen under capture must not need more.
Every replay, with eager work in between, equals the eager outputs bit for bit."""

from __future__ import annotations

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 1024, 3072


class Norm(nn.Module):
    """The reference RMSNorm's attributes (qtts/layers/norm.py:82-93) and eager formula."""

    def __init__(self, n: int, eps: float = 1e-6) -> None:
        super().__init__()
        g = torch.Generator(device="cuda").manual_seed(n)
        self.weight = nn.Parameter((1 + 0.1 * torch.randn(n, device="cuda", generator=g)).to(torch.bfloat16),
                                   requires_grad=False)
        self.eps = eps

    def forward(self, x):
        v = x.float().pow(2).mean(-1, keepdim=True)
        return (x.float() * torch.rsqrt(v + self.eps) * self.weight.float()).to(x.dtype)


class Block(nn.Module):
    def __init__(self, seed: int) -> None:
        super().__init__()
        from qtts_amd.layers import GatedMLP, LinearBase, MergedLinear
        self.norm1, self.norm2 = Norm(HIDDEN), Norm(HIDDEN)
        self.qkv = MergedLinear(HIDDEN, [HIDDEN, HIDDEN // 2, HIDDEN // 2], dtype=torch.bfloat16, device="cuda")
        self.o = LinearBase(HIDDEN, HIDDEN, bias=True, dtype=torch.bfloat16, device="cuda")
        self.mlp = GatedMLP(HIDDEN, INTER, fuse=True, dtype=torch.bfloat16, device="cuda")
        g = torch.Generator(device="cuda").manual_seed(seed)
        for name, p in self.named_parameters():
            if "norm" not in name:
                p.data.copy_((torch.randn(p.shape, device="cuda", generator=g) * 0.02).to(p.dtype))

    def forward(self, x):
        from qtts_amd.layers.decoder import linear_residual, norm_linear, norm_mlp_residual
        q, _, _ = self.qkv.split(norm_linear(self.norm1, self.qkv, x))
        h = linear_residual(self.o, q, x)
        return norm_mlp_residual(self.norm2, self.mlp, h)


def _blocks():
    from qtts_amd import QuantConfig, apply_quantization
    from qtts_amd.layers.activation import fuse_gated_mlps
    blocks = {}
    for i, method in enumerate(("int8_weight_only", "fp8", "int8", "fp8_weight_only")):
        b = Block(seed=100 + i)
        report = apply_quantization(QuantConfig(method=method, calibrate=False), talker=b)
        assert report["talker"]["converted"] == 4, (method, report)
        fuse_gated_mlps(b)
        blocks[method] = b
    return blocks


def test_every_method_in_one_graph():
    blocks = _blocks()
    for m in (1, 3, 8, 16, 64, 300):
        g = torch.Generator(device="cuda").manual_seed(m)
        x = torch.randn(m, HIDDEN, device="cuda", generator=g).to(torch.bfloat16)
        eager = {k: b(x) for k, b in blocks.items()}
        static_x = x.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for b in blocks.values():
                b(static_x)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        print(f"capture m={m}", flush=True)
        with torch.cuda.graph(graph):
            outs = {k: b(static_x) for k, b in blocks.items()}
        for rep in range(3):
            for b in blocks.values():  # eager work between replays
                b(x * 0.5)
            graph.replay()
            torch.cuda.synchronize()
            for k in blocks:
                assert torch.equal(outs[k], eager[k]), f"{k} m={m} replay {rep}"
        del graph
