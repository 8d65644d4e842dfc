"""Layers carrying the quantization hook."""

from .activation import GatedMLP, fuse_gated_mlps, gated_mlp_forward
from .linear import LinearBase, MergedLinear, QuantMethod, iter_linears

__all__ = ["GatedMLP", "LinearBase", "MergedLinear", "QuantMethod", "fuse_gated_mlps", "gated_mlp_forward",
           "iter_linears"]
