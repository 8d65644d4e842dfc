"""The decoder-layer helpers (qtts_amd.layers.decoder) on layers that are not int8 weight-only:
each returns the reference's composition (qtts/models/talker.py:249-271) unchanged.  CPU only."""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from qtts_amd.layers import GatedMLP, LinearBase
from qtts_amd.layers.decoder import linear_residual, norm_linear, norm_mlp_residual


class Norm(nn.Module):
    """The reference RMSNorm's attributes (qtts/layers/norm.py:82-93) and eager formula."""

    def __init__(self, n: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(1 + 0.1 * torch.randn(n), requires_grad=False)
        self.eps = eps

    def forward(self, x):
        v = x.float().pow(2).mean(-1, keepdim=True)
        return (x.float() * torch.rsqrt(v + self.eps) * self.weight.float()).to(x.dtype)


def test_fallbacks_are_the_reference_composition():
    torch.manual_seed(0)
    norm = Norm(64)
    lin = LinearBase(64, 96)
    with torch.no_grad():
        lin.weight.normal_(0, 0.05)
    x = torch.randn(3, 1, 64)
    assert torch.equal(norm_linear(norm, lin, x), lin(norm(x)))
    o = LinearBase(64, 64, bias=True)
    with torch.no_grad():
        o.weight.normal_(0, 0.05)
        o.bias.normal_(0, 0.1)
    r = torch.randn(3, 1, 64)
    assert torch.equal(linear_residual(o, x, r), r + o(x))
    for fuse in (True, False):
        mlp = GatedMLP(64, 128, fuse=fuse)
        with torch.no_grad():
            for p in mlp.parameters():
                p.normal_(0, 0.05)
        h = norm(x)
        if fuse:
            gate, up = mlp.gate_up_proj.split(mlp.gate_up_proj(h))
        else:
            gate, up = mlp.gate_proj(h), mlp.up_proj(h)
        want = x + mlp.down_proj(F.silu(gate) * up)
        assert torch.equal(norm_mlp_residual(norm, mlp, x), want)
