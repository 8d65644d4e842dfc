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


class PolicyRecorder(FakeMethod):
    """FakeMethod that records the weight policy each process_weights call saw."""

    def __init__(self):
        self.seen = []

    def process_weights(self, layer):
        self.seen.append(self.stream_weights)
        super().process_weights(layer)


def test_weight_policy_follows_the_submodel_size(monkeypatch):
    """A submodel whose eligible codes exceed the Infinity Cache streams its weights (ALGO_STREAM on
    every converted layer, seen by process_weights for calibration); one that fits keeps them cached."""
    from qtts_amd import _lib
    from qtts_amd.quant import base

    cfg = QuantConfig(method="int8_weight_only")
    m = _init(Block())
    eligible = sum(l.weight.numel() for n, l in iter_linears(m) if not cfg.excludes(n))
    assert eligible == 16 * 8 + 8 * 8 + 8 * 8 + 5 * 8  # codec_head excluded, the declined layer counted
    for limit, stream in ((eligible, False), (eligible - 1, True)):
        monkeypatch.setattr(base, "CACHE_RESIDENT_BYTES", limit)
        m = _init(Block())
        method = PolicyRecorder()
        report = quantize_module(m, method, cfg, "talker")
        assert report["stream_weights"] == int(stream) and method.seen == [stream] * 4
        for name in ("qkv_proj", "o_proj", "text_proj_fc1"):
            layer = getattr(m, name)
            assert layer.quant_stream is stream
            assert base.weight_flags(layer) == (_lib.ALGO_STREAM if stream else 0)
        assert base.weight_flags(m.odd) == 0 and base.weight_flags(m.codec_head) == 0  # not converted


def test_apply_quantization_routing():
    assert apply_quantization(QuantConfig(), talker=Block()) == {}
    with pytest.raises(ValueError, match="name no submodel"):
        apply_quantization(QuantConfig(method="int8_weight_only", targets=("vocoder",)), talker=Block())


def test_build_method_errors_without_gpu():
    with pytest.raises(ValueError, match="no quantization method named"):
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
    assert "quant_method=none" in lin.extra_repr()
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


def _bucket_fixture(times, fail_ref_at=()):
    """Fake per-bucket calibration inputs: labels instead of GPU work, times from ``times(label)``."""
    calls = []

    def kernel(x, algo):
        return ("kernel", algo, x.shape[0])

    def reference(x):
        if x.shape[0] in fail_ref_at:
            raise RuntimeError("capture failed")
        return ("ref", None, x.shape[0])

    def timer(fn):
        label = fn()
        calls.append(label)
        return times(label)

    def candidates(rows):
        c = {"skinny": 1, "skinny_w8": 1 | (8 << 16)} if rows <= 64 else {}
        if rows > 16:
            c["tile"] = 2
        return c

    return kernel, reference, timer, candidates, calls


def test_calibrate_buckets_decides_every_bucket():
    """Every bucket gets its fastest route (skinny, tile or the prefill route); the layer verdict
    is the decode buckets' sum against the reference's (qtts/quant/calibrate.py:77-114 asks the same
    question at one row count)."""
    calibrate.clear_cache()
    buckets = (1, 2, 4, 8, 16, 32, 64, 128, 256, 1024, 2048)

    def times(label):
        kind, algo, rows = label
        if kind == "ref":
            return 10.0 + rows
        if kind == "route":
            return 5.0 + rows * 0.1   # beats the tile kernel at the prefill buckets
        base = {1: 3.0, 1 | (8 << 16): 2.0, 2: 4.0}[algo]
        return base + rows * (0.2 if algo == 2 else 1.0)  # skinny grows fast with rows, tile slowly

    kernel, reference, timer, candidates, calls = _bucket_fixture(times)
    routes = {r: {"dequant": (-1, lambda x: ("route", -1, x.shape[0]))} for r in (256, 1024, 2048)}
    accept, table, report = calibrate.calibrate_buckets("t", 64, 128, torch.float32, torch.device("cpu"), buckets, 16,
                                                        candidates, kernel, reference, routes, timer=timer)
    assert accept
    assert sorted(table) == list(buckets), "every bucket decided"
    for rows in buckets:
        t = report[rows]["timings"]
        assert table[rows] == {"skinny": 1, "skinny_w8": 1 | (8 << 16), "tile": 2, "dequant": -1}[report[rows]["best"]]
        assert t[report[rows]["best"]] == min(t.values())
    assert table[1] == 1 | (8 << 16) and table[16] == 1 | (8 << 16)   # skinny_w8 at decode rows
    assert table[64] == 2 and table[128] == 2                         # tile past the crossover
    assert table[256] == -1 and table[2048] == -1                      # the prefill route wins there
    # cached per (tag, n, k, rows, dtype): a second calibration times nothing
    n_calls = len(calls)
    assert calibrate.calibrate_buckets("t", 64, 128, torch.float32, torch.device("cpu"), buckets, 16, candidates,
                                       kernel, reference, routes, timer=timer)[1] == table
    assert len(calls) == n_calls


def test_calibrate_buckets_verdict_from_decode_rows():
    """The verdict sums the decode buckets: losing one bucket does not decline a layer that wins
    the sum; losing the sum does (and records nothing); the 1.05 margin holds."""
    calibrate.clear_cache()

    def times(label):
        kind, algo, rows = label
        if kind == "ref":
            return 10.0
        return {1: 12.0, 2: 6.0, 4: 9.0, 8: 9.0}[rows] if rows <= 8 else 9.0

    kernel, reference, timer, candidates, _ = _bucket_fixture(times)
    accept, table, _ = calibrate.calibrate_buckets("v1", 8, 8, torch.float32, torch.device("cpu"), (1, 2, 4, 8, 64),
                                                   8, candidates, kernel, reference, timer=timer)
    assert accept and table[1] in (1, 1 | (8 << 16)) and 64 in table   # 36 * 1.05 < 40
    calibrate.clear_cache()

    def close(label):  # 4% better: inside the margin
        return 10.0 if label[0] == "ref" else 9.6

    kernel, reference, timer, candidates, _ = _bucket_fixture(close)
    accept, table, report = calibrate.calibrate_buckets("v2", 8, 8, torch.float32, torch.device("cpu"), (1, 2, 64),
                                                        2, candidates, kernel, reference, timer=timer)
    assert not accept and table == {} and report[1]["best"] is not None


def test_calibrate_buckets_failures_are_never_fatal():
    calibrate.clear_cache()
    kernel, reference, timer, candidates, _ = _bucket_fixture(lambda label: 1.0 if label[0] == "ref" else 0.5,
                                                              fail_ref_at=(4,))
    accept, table, _ = calibrate.calibrate_buckets("f", 8, 8, torch.float32, torch.device("cpu"), (1, 4, 256), 16,
                                                   candidates, kernel, reference, timer=timer)
    assert not accept and table == {}   # the reference failed at a decode bucket: decline
    calibrate.clear_cache()
    kernel, reference, timer, candidates, _ = _bucket_fixture(lambda label: 1.0 if label[0] == "ref" else 0.5,
                                                              fail_ref_at=(256,))
    accept, table, _ = calibrate.calibrate_buckets("g", 8, 8, torch.float32, torch.device("cpu"), (1, 4, 256), 16,
                                                   candidates, kernel, reference, timer=timer)
    assert accept and sorted(table) == [1, 4]   # a prefill bucket that cannot be timed stays automatic


def test_calibrate_buckets_routes_losing_buckets_to_reference():
    """A converted layer that loses to F.linear at some bucket: with keep_reference that bucket
    goes to F.linear on the kept weight (no bucket slower than the layer it replaced); without,
    it keeps its fastest quantized route.  The layer verdict is unchanged."""
    calibrate.clear_cache()

    def times(label):
        kind, algo, rows = label
        if kind == "ref":
            return 10.0
        return {16: 12.0, 256: 20.0}.get(rows, 5.0)

    kernel, reference, timer, candidates, _ = _bucket_fixture(times)
    buckets = (1, 2, 16, 64, 256)
    accept, table, report = calibrate.calibrate_buckets("r1", 8, 8, torch.float32, torch.device("cpu"), buckets, 16,
                                                        candidates, kernel, reference, timer=timer,
                                                        keep_reference=True)
    assert accept   # decode rows: (5 + 5 + 12) * 1.05 < 30
    assert table[16] == calibrate.ALGO_REFERENCE_GEMM and table[256] == calibrate.ALGO_REFERENCE_GEMM
    assert table[1] >= 0 and table[2] >= 0 and table[64] >= 0
    calibrate.clear_cache()
    accept, table, _ = calibrate.calibrate_buckets("r1", 8, 8, torch.float32, torch.device("cpu"), buckets, 16,
                                                   candidates, kernel, reference, timer=timer)
    assert accept and all(a >= 0 for a in table.values())
    assert table[256] == 2   # the tile kernel, the only candidate past 64 rows


def test_reference_route_dispatch():
    """The weight-only method's per-layer table: a bucket routed to F.linear computes F.linear on the
    layer's weight exactly; routes_to_kernel and the fused activation entry say so; another
    layer's table (same shape) is not consulted."""
    from qtts_amd.quant.int8 import Int8WeightOnlyMethod, layer_algo
    from qtts_amd import _lib
    method = object.__new__(Int8WeightOnlyMethod)   # no GPU here: only the host-side routing runs
    lin = _init(LinearBase(8, 4, bias=True, dtype=torch.bfloat16))
    lin.int8_layout = "strips"
    lin.quant_algos = {1: calibrate.ALGO_REFERENCE_GEMM, 256: calibrate.ALGO_REFERENCE_GEMM, 2: 1}
    other = _init(LinearBase(8, 4, bias=True, dtype=torch.bfloat16))
    other.quant_algos = {}
    x = torch.randn(1, 8).to(torch.bfloat16)
    assert torch.equal(method.apply(lin, x, lin.bias), F.linear(x, lin.weight, lin.bias))
    x200 = torch.randn(200, 8).to(torch.bfloat16)
    assert torch.equal(method.apply(lin, x200, lin.bias), F.linear(x200, lin.weight, lin.bias))
    assert layer_algo(lin, 200) == calibrate.ALGO_REFERENCE_GEMM and layer_algo(lin, 2) == 1
    assert layer_algo(other, 1) == _lib.ALGO_AUTO
    assert not method.routes_to_kernel(lin, x) and method.routes_to_kernel(lin, torch.randn(2, 8))
    assert method.apply_gate_up_silu(lin, x, None) is None   # the plain path then calls apply


def test_weight_rotation_for_timing():
    """The calibration rotates through copies of a weight that together pass the L2s: the copy count
    follows the weight size (at least 1, at most 64), and the rotating callable runs the copies in
    turn, one per call, so a graph of as many calls reads each copy once."""
    assert calibrate.rotation(calibrate.ROTATE_BYTES) == 1
    assert calibrate.rotation(calibrate.ROTATE_BYTES * 4) == 1
    assert calibrate.rotation(2 << 20) == 32 and calibrate.rotation(25 << 20) == 3
    assert calibrate.rotation(1) == 64 and calibrate.rotation(1, limit=8) == 8
    seen = []
    run = calibrate.rotating([lambda a, i=i: seen.append((i, a)) for i in range(3)])
    for a in range(7):
        run(a)
    assert seen == [(0, 0), (1, 1), (2, 2), (0, 3), (1, 4), (2, 5), (0, 6)]


def test_calibrate_buckets_inner_calls_reach_the_timer_key():
    """A calibration that rotates over more than 10 weight copies caches its timings apart from one
    that times 10 calls of one weight (the reference's harness)."""
    calibrate.clear_cache()
    kernel, reference, timer, candidates, calls = _bucket_fixture(lambda label: 1.0 if label[0] == "ref" else 0.5)
    calibrate.calibrate_buckets("k", 8, 8, torch.float32, torch.device("cpu"), (1,), 1, candidates, kernel, reference,
                                timer=timer)
    n = len(calls)
    calibrate.calibrate_buckets("k", 8, 8, torch.float32, torch.device("cpu"), (1,), 1, candidates, kernel, reference,
                                timer=timer, inner=32)
    assert len(calls) > n   # timed again: another key


def test_decode_candidates_include_the_automatic_choice_and_half_strips():
    """Every bucket times the automatic choice (which takes row-split strips where whole strips leave
    compute units idle); buckets of up to 64 rows on strip weights with K a multiple of 128 also
    half strips."""
    from qtts_amd import _lib
    from qtts_amd.quant.fp8 import _fp8w_candidates
    from qtts_amd.quant.int8 import _candidates
    for rows in (1, 2, 4, 8, 16, 32, 64):
        c = _candidates(rows, 6144)
        assert c["auto"] == _lib.ALGO_AUTO and c["skinny_half"] == _lib.algo_code(_lib.ALGO_SKINNY_HALF)
        assert "skinny_half" not in _candidates(rows, 6144 + 64) and "skinny_half" not in _candidates(rows)
        assert _fp8w_candidates(rows)["auto"] == _lib.ALGO_AUTO
    for rows in (128, 256):
        assert _candidates(rows, 6144)["auto"] == _lib.ALGO_AUTO and "skinny_half" not in _candidates(rows, 6144)
        assert _fp8w_candidates(rows)["auto"] == _lib.ALGO_AUTO
    # two chunks a tile stage: tile buckets (past 16 rows) with an even chunk count, in one and two splits
    two = _lib.TILE_READ_AHEAD | _lib.TILE_TWO_CHUNKS
    for rows in (32, 128):
        c = _candidates(rows, 6144)
        assert c["tile_bm32_bn64_c2_s2"] == _lib.algo_code(_lib.ALGO_TILE, 2, 4 | two, _lib.tile_shape(32, 64))
        assert "tile_bm32_bn64_c2_s1" in c and "tile_bm32_bn64_c2_s1" not in _candidates(rows, 6144 + 64)
    assert not any("_c2_" in name for name in _candidates(16, 6144))


def test_calibrate_buckets_keeps_the_automatic_choice_on_near_ties():
    """A pinned configuration replaces "auto" only when it is AUTO_MARGIN faster."""
    calibrate.clear_cache()
    pin = 1 | (8 << 16)

    def times(label):
        kind, algo, rows = label
        if kind == "ref":
            return 10.0
        return {0: 2.0, pin: 2.0 / (1.03 if rows == 1 else 1.10)}[algo]  # 3% faster at 1 row, 10% at 2

    def kernel(x, a):
        return ("k", a, x.shape[0])

    def reference(x):
        return ("ref", None, x.shape[0])

    def timer(fn):
        return times(fn())

    accept, table, report = calibrate.calibrate_buckets("near", 8, 8, torch.float32, torch.device("cpu"), (1, 2), 2,
                                                        lambda rows: {"auto": 0, "pin": pin}, kernel, reference,
                                                        timer=timer)
    assert accept and table[1] == 0 and report[1]["best"] == "auto"   # 3%: a near-tie, auto stays
    assert table[2] == pin and report[2]["best"] == "pin"             # 10%: the pin wins
