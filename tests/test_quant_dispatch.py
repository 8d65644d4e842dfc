"""Host logic of the quantization hook, on the CPU with fake methods and timers.

Mirrors the semantics of qtts/quant/base.py:74-183, qtts/quant/calibrate.py:77-114,
qtts/layers/linear.py:25-104 and qtts/config.py:50-98.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from qtts_amd import QuantConfig, apply_quantization, build_method, quantize_module
from qtts_amd.layers.linear import LinearBase, MergedLinear, iter_linears
from qtts_amd.quant import calibrate
from qtts_amd.quant.base import QuantMethodBase
from qtts_amd.quant.int8 import bucket_of


class FakeMethod(QuantMethodBase):
    """Halves the weight bytes of every layer whose out_features is even; declines odd ones."""

    name = "fake"

    def process_weights(self, layer):
        if layer.out_features % 2:
            layer.register_buffer("fake_q", None, persistent=False)
            return
        layer.register_buffer("fake_q", layer.weight.detach().to(torch.float16), persistent=False)
        layer.weight = nn.Parameter(torch.empty(0), requires_grad=False)

    def applies_to(self, layer):
        return getattr(layer, "fake_q", None) is not None

    def apply(self, layer, x, bias):
        return F.linear(x, layer.fake_q.float(), bias)


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.qkv_proj = MergedLinear(8, [8, 4, 4])
        self.o_proj = LinearBase(8, 8)
        self.text_proj_fc1 = LinearBase(8, 8, bias=True)   # not matched by "text_projection"
        self.codec_head = LinearBase(8, 7)
        self.odd = LinearBase(8, 5)


def _init(m: nn.Module):
    g = torch.Generator().manual_seed(0)
    for p in m.parameters():
        p.data.copy_(torch.randn(p.shape, generator=g))
    return m


def test_quant_config_semantics():
    c = QuantConfig()
    assert not c.enabled and not c.targets_submodel("talker")
    c = QuantConfig(method="int8_weight_only")
    assert c.enabled and c.weight_only and c.targets_submodel("talker") and not c.targets_submodel("code2wav")
    assert c.excludes("model.codec_head") and c.excludes("lm_head.0") and c.excludes("small_to_mtp_projection")
    assert not c.excludes("layers.0.text_proj_fc1")
    assert not QuantConfig(method="fp8").weight_only


def test_quantize_module_counts_and_bytes():
    m = _init(Block())
    x = torch.randn(3, 8)
    before = {n: l(x) for n, l in iter_linears(m)}
    report = quantize_module(m, FakeMethod(), QuantConfig(method="int8_weight_only"), "talker")
    assert report["excluded"] == 1                      # codec_head
    assert report["declined"] == 1                      # odd
    assert report["converted"] == 3                     # qkv, o, text_proj_fc1
    assert report["bytes_after"] < report["bytes_before"]
    assert m.codec_head.quant_method is None and m.odd.quant_method is None
    assert m.o_proj.quant_method is not None
    for name, layer in iter_linears(m):
        torch.testing.assert_close(layer(x), before[name], rtol=1e-2, atol=1e-2)
    assert len(m.qkv_proj.split(m.qkv_proj(x))) == 3


def test_apply_quantization_routing():
    assert apply_quantization(QuantConfig(), talker=Block()) == {}
    with pytest.raises(ValueError, match="unknown quant targets"):
        apply_quantization(QuantConfig(method="int8_weight_only", targets=("vocoder",)), talker=Block())


def test_build_method_errors_without_gpu():
    with pytest.raises(ValueError, match="unknown quantization method"):
        build_method(QuantConfig(method="int4"))  # type: ignore[arg-type]
    if torch.cuda.is_available():
        pytest.skip("checks the no-GPU error path")
    with pytest.raises(RuntimeError):
        build_method(QuantConfig(method="int8_weight_only"))
    with pytest.raises(RuntimeError):
        build_method(QuantConfig(method="fp8"))
    with pytest.raises(RuntimeError):
        build_method(QuantConfig(method="fp8_weight_only"))


def test_linear_base_matches_f_linear_and_merged_partitions():
    lin = _init(LinearBase(6, 4, bias=True))
    x = torch.randn(2, 3, 6)
    torch.testing.assert_close(lin(x), F.linear(x, lin.weight, lin.bias))
    assert "quant=none" in lin.extra_repr()
    ml = MergedLinear(6, [2, 3])
    ml.load_partition(1, torch.ones(3, 6))
    assert torch.equal(ml.weight[2:], torch.ones(3, 6))
    with pytest.raises(ValueError):
        ml.load_partition(0, torch.ones(3, 6))
    with pytest.raises(ValueError):
        ml.load_bias_partition(0, torch.ones(2))


def test_iter_linears_finds_duck_typed_layers():
    class RefStyle(nn.Module):  # the reference's LinearBase exposes these attributes
        def __init__(self):
            super().__init__()
            self.in_features, self.out_features = 4, 4
            self.weight = nn.Parameter(torch.zeros(4, 4))
            self.quant_method = None

    root = nn.Sequential(RefStyle(), LinearBase(4, 4), nn.Linear(4, 4))
    names = [n for n, _ in iter_linears(root)]
    assert names == ["0", "1"]


def _fake_timer(table):
    def timer(fn):
        return table[fn()]
    return timer


def test_pick_fastest_margin_and_cache():
    calibrate.clear_cache()
    t = _fake_timer({"ref": 1.00, "a": 0.96, "b": 0.90, "c": 0.97})
    assert calibrate.pick_fastest({"a": lambda: "a"}, lambda: "ref", key=("k1",), timer=t) is None  # 4% is noise
    assert calibrate.pick_fastest({"a": lambda: "a", "b": lambda: "b", "c": lambda: "c"}, lambda: "ref",
                                  key=("k2",), timer=t) == "b"
    # cached per key: the first verdict stands
    t2 = _fake_timer({"ref": 9.0, "a": 0.1})
    assert calibrate.pick_fastest({"a": lambda: "a"}, lambda: "ref", key=("k1",), timer=t2) is None


def test_calibration_failures_are_never_fatal():
    calibrate.clear_cache()

    def boom():
        raise RuntimeError("capture failed")

    t = _fake_timer({"ref": 1.0, "a": 0.5})
    # a failing candidate is dropped, the others still compete
    assert calibrate.pick_fastest({"bad": boom, "a": lambda: "a"}, lambda: "ref", key=("f1",), timer=t) == "a"
    # a failing reference declines the layer, and that verdict is cached
    assert calibrate.pick_fastest({"a": lambda: "a"}, boom, key=("f2",), timer=t) is None
    assert calibrate.worth_quantizing(lambda: "a", boom, key=("f3",), timer=t) is False
    assert calibrate.worth_quantizing(lambda: "a", lambda: "ref", key=("f4",), timer=t) is True
    calibrate.clear_cache()
    assert not calibrate._CACHE


def test_m_buckets():
    assert [bucket_of(m) for m in (1, 2, 3, 5, 9, 16, 17, 64, 65, 300, 1500, 5000)] == \
        [1, 2, 4, 8, 16, 16, 32, 64, 128, 1024, 2048, 2048]
