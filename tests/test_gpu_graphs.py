"""The callers' capture rules over the quantized linears (qtts_amd/graphs.py), on the GPU.

* The talker's decode step (qtts/compilation.py:60-186): rows padded up to a captured size
  in {1, 2, 4, 8, 16, 32, 64} (padding at 101-105), one graph per size, static inputs shared
  by all graphs.  The step here is two talker layers' linears through the decoder-layer
  helpers (layers/decoder.py: RMSNorm + qkv, o + residual, RMSNorm + gate_up + SiLU, down +
  residual), attention replaced by a fixed projection of q, on int8 weight-only layers.
* The code predictor's walk (compilation.py:189-273; code_predictor.py:200-243): 15 exact-
  prefix forwards of a 5-layer predictor-shaped stack per frame, prefix length 2..16, so each
  linear runs at M = batch x prefix; one graph per padded batch.

Each replay must equal an eager run on the same padded input bit for bit (several replays, with
eager work and synchronisation in between, each on fresh inputs), and every quantized linear's
output must be within the GEMM bar of the oracle's dequantize-then-matmul of its own input."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from test_gpu_gemm import assert_close

pytestmark = pytest.mark.gpu


def _init(module: nn.Module, seed: int) -> nn.Module:
    g = torch.Generator(device="cuda").manual_seed(seed)
    for p in module.parameters():
        p.data.copy_((torch.randn(p.shape, device="cuda", generator=g) * 0.02).to(p.dtype))
    return module


class RMSNorm(nn.Module):
    def __init__(self, dim):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.bfloat16, device="cuda"))
        self.eps = 1e-6

    def forward(self, x):
        return F.rms_norm(x, (x.shape[-1],), self.weight, self.eps)


class TalkerLayerLinears(nn.Module):
    """A talker decoder layer's linears and norms (hidden 2048, intermediate 6144)."""

    def __init__(self, seed):
        super().__init__()
        from qtts_amd.layers import GatedMLP
        from qtts_amd.layers.linear import LinearBase, MergedLinear
        kw = dict(dtype=torch.bfloat16, device="cuda")
        self.input_layernorm = RMSNorm(2048)
        self.post_attention_layernorm = RMSNorm(2048)
        self.qkv_proj = MergedLinear(2048, [2048, 1024, 1024], **kw)
        self.o_proj = LinearBase(2048, 2048, **kw)
        self.mlp = GatedMLP(2048, 6144, **kw)
        _init(self, seed)
        with torch.no_grad():
            self.input_layernorm.weight.fill_(1.0)
            self.post_attention_layernorm.weight.normal_(1.0, 0.1)

    def step(self, hidden, trace):
        from qtts_amd.layers.decoder import linear_residual, norm_linear, norm_mlp_residual
        qkv = norm_linear(self.input_layernorm, self.qkv_proj, hidden)
        trace.append(qkv)
        attn = qkv[..., :2048] * 0.5  # attention stands in as a fixed function of q
        hidden = linear_residual(self.o_proj, attn, hidden)
        trace.append(hidden)
        hidden = norm_mlp_residual(self.post_attention_layernorm, self.mlp, hidden)
        trace.append(hidden)
        return hidden


def _quantize(module):
    from qtts_amd import QuantConfig, apply_quantization
    report = apply_quantization(QuantConfig(method="int8_weight_only", calibrate=False), talker=module)
    assert report["talker"]["declined"] == 0
    return module


def _oracle_linear(layer, x):
    """fp64 dequantize-then-matmul of the layer's packed bytes (qtts/quant/kernels.py:113-135)."""
    import oracle as O
    from qtts_amd.quant.int8 import int8_weight_rowmajor
    q = int8_weight_rowmajor(layer).cpu().numpy()
    s = layer.int8_scale.float().cpu().numpy()
    b = None if layer.bias is None else layer.bias.float().cpu().numpy()
    return O.w8a16_ref(x.float().reshape(-1, x.shape[-1]).cpu().numpy(), q, s, b)


def test_talker_decode_graphs_pad_and_replay():
    from qtts_amd.graphs import DECODE_BATCH_SIZES, PaddedGraphs
    layers = nn.ModuleList([_quantize(TalkerLayerLinears(seed)) for seed in (1, 2)])

    def step(hidden):
        trace = []
        for layer in layers:
            hidden = layer.step(hidden, trace)
        return (hidden, *trace)

    graphs = PaddedGraphs(step, (2048,), torch.bfloat16, batch_sizes=DECODE_BATCH_SIZES)
    for rows in (1, 3, 5, 8, 13, 16, 21, 64, 3):
        padded = graphs.padded_rows(rows)
        assert padded == min(b for b in DECODE_BATCH_SIZES if b >= rows)
        for rep in range(2):
            print(f"talker decode rows={rows} padded={padded} replay {rep}", flush=True)
            g = torch.Generator(device="cuda").manual_seed(100 * rows + rep)
            x = torch.randn(rows, 2048, device="cuda", generator=g).to(torch.bfloat16)
            out = graphs.run(x)
            torch.cuda.synchronize()
            # eager on the same padded input (the padded rows are zero, as the graph sees them)
            xp = torch.zeros(padded, 2048, dtype=torch.bfloat16, device="cuda")
            xp[:rows] = x
            want = step(xp)
            torch.cuda.synchronize()
            for a, b in zip(out, want):
                assert torch.equal(a, b[:rows]), (rows, rep)
    assert sorted(graphs.graphs) == [1, 4, 8, 16, 32, 64]
    # each quantized linear's output (eager, equal to the graph's) against the oracle on its input
    _oracle_checks(layers[0])


@torch.no_grad()
def _oracle_checks(layer):
    rows = 5
    x = torch.randn(rows, 2048, device="cuda").to(torch.bfloat16)
    h_norm = layer.input_layernorm(x)
    assert_close(layer.qkv_proj(h_norm), _oracle_linear(layer.qkv_proj, h_norm), "qkv_proj")
    for name in ("o_proj",):
        lin = getattr(layer, name)
        assert_close(lin(x), _oracle_linear(lin, x), name)
    gu = layer.mlp.gate_up_proj
    assert_close(gu(x), _oracle_linear(gu, x), "gate_up_proj")
    act = torch.randn(rows, 6144, device="cuda").to(torch.bfloat16)
    assert_close(layer.mlp.down_proj(act), _oracle_linear(layer.mlp.down_proj, act), "down_proj")


class PredictorStack(nn.Module):
    """A 5-layer code-predictor-shaped stack (hidden 1024; qkv 1024 -> 4096, o 2048 -> 1024,
    gate_up 1024 -> 6144, down 3072 -> 1024) and its walk over the codebook axis: 15 forwards of
    the exact prefix (length 2..16), each appending a function of its last position."""

    groups = 16

    def __init__(self):
        super().__init__()
        from qtts_amd.layers.linear import LinearBase, MergedLinear
        kw = dict(dtype=torch.bfloat16, device="cuda")
        self.layers = nn.ModuleList()
        for i in range(5):
            layer = nn.Module()
            layer.qkv_proj = MergedLinear(1024, [2048, 1024, 1024], **kw)
            layer.o_proj = LinearBase(2048, 1024, **kw)
            layer.gate_up_proj = MergedLinear(1024, [3072, 3072], **kw)
            layer.down_proj = LinearBase(3072, 1024, **kw)
            self.layers.append(_init(layer, 10 + i))

    def prefix(self, h):
        for layer in self.layers:
            q, _, _ = layer.qkv_proj.split(layer.qkv_proj(F.rms_norm(h, (1024,))))
            h = h + layer.o_proj(q)
            gate, up = layer.gate_up_proj.split(layer.gate_up_proj(F.rms_norm(h, (1024,))))
            h = h + layer.down_proj(F.silu(gate) * up)
        return h

    def walk(self, start):
        """start [batch, 2, 1024] -> the last position of every prefix forward [batch, 15, 1024]."""
        batch = start.shape[0]
        seq = torch.zeros(batch, self.groups, 1024, dtype=start.dtype, device=start.device)
        seq[:, :2] = start
        outs = []
        for step in range(1, self.groups):
            hidden = self.prefix(seq[:, :step + 1])
            last = hidden[:, step]
            outs.append(last)
            if step < self.groups - 1:
                seq[:, step + 1] = torch.tanh(last)  # the next codebook's embedding stands in
        return torch.stack(outs, dim=1)


def test_code_predictor_walk_graphs():
    from qtts_amd.graphs import PaddedGraphs
    stack = _quantize(PredictorStack())
    graphs = PaddedGraphs(stack.walk, (2, 1024), torch.bfloat16, batch_sizes=(1, 2, 4, 8))
    for batch in (1, 3, 8, 5, 1):
        padded = graphs.padded_rows(batch)
        for rep in range(2):
            print(f"predictor walk batch={batch} padded={padded} replay {rep}", flush=True)
            g = torch.Generator(device="cuda").manual_seed(7 * batch + rep)
            x = torch.randn(batch, 2, 1024, device="cuda", generator=g).to(torch.bfloat16)
            out = graphs.run(x)
            torch.cuda.synchronize()
            xp = torch.zeros(padded, 2, 1024, dtype=torch.bfloat16, device="cuda")
            xp[:batch] = x
            want = stack.walk(xp)
            torch.cuda.synchronize()
            assert torch.equal(out, want[:batch]), (batch, rep)
    assert sorted(graphs.graphs) == [1, 4, 8]
    # the linears at the walk's row counts, M = batch x prefix, against the oracle
    _walk_oracle_checks(stack.layers[0])


@torch.no_grad()
def _walk_oracle_checks(layer):
    for m in (2, 16, 24, 64, 128):
        x = torch.randn(m, 1024, device="cuda").to(torch.bfloat16)
        assert_close(layer.qkv_proj(x), _oracle_linear(layer.qkv_proj, x), f"qkv m={m}")
        assert_close(layer.gate_up_proj(x), _oracle_linear(layer.gate_up_proj, x), f"gate_up m={m}")
        a = torch.randn(m, 2048, device="cuda").to(torch.bfloat16)
        assert_close(layer.o_proj(a), _oracle_linear(layer.o_proj, a), f"o m={m}")
        d = torch.randn(m, 3072, device="cuda").to(torch.bfloat16)
        assert_close(layer.down_proj(d), _oracle_linear(layer.down_proj, d), f"down m={m}")
