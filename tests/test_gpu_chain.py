"""GPU parity of the decoder-layer chain (``qtts_w8a16_chain_strips``), through the C ABI.

The chain runs, in one persistent launch, the linears of a talker decoder layer between
two attention calls (qtts/models/talker.py:246-271):

    h1  = h + o_proj(attn)                                          residual epilogue
    act = silu(gate) * up,  gate|up = gate_up(rmsnorm(h1, w_post))  norm prologue, SiLU epilogue
    h2  = h1 + down_proj(act)                                       residual epilogue
    qkv = qkv_proj(rmsnorm(h2, w_in))                               norm prologue

Every stage is checked against the fp64 oracle evaluated on the chain's own input of
that stage, so errors do not compound:

* GEMM outputs (qkv): |y - ref| <= 1e-2 RMS(ref) + ulp/2 (the W8A16 bar).
* Residual stages (h1, h2): the same bound on the linear's part, plus half an ulp of the
  sum (the output rounds once more after the add).
* The SiLU stage: the GEMM bar on gate and up carried through silu(g) * u to first order,
  |d act| <= |silu'(g) u| tol_g + |silu(g)| tol_u, plus an ulp of act for its two
  roundings.  A wrong pairing of gate and up rows, a dropped strip or a missing scale is
  O(RMS) and fails.

The same stages computed by this library's separate kernels (rms_norm, the skinny
GEMM, silu_mul, torch's residual add) must agree to the same bounds; graph replays
with fresh inputs, every grid size down to one workgroup (the ticket order alone then
orders the links), ragged strips and independent links give bit-identical results.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from test_gpu_gemm import half_ulp

pytestmark = pytest.mark.gpu

EPS = 1e-6
# (o: n, k), (gate_up: n, k), (down: n, k), (qkv: n, k)
TALKER_LAYER = ((2048, 2048), (12288, 2048), (2048, 6144), (4096, 2048))
PREDICTOR_LAYER = ((1024, 2048), (6144, 1024), (1024, 3072), (4096, 1024))


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    _ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    return _ops


def _np(t: torch.Tensor) -> np.ndarray:
    return t.double().cpu().numpy()


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


class Layer:
    """Seeded int8 weights of one decoder layer (canonical bytes for the oracle, strips for the kernels)."""

    def __init__(self, ops, shapes, seed, bias=False):
        self.shapes = shapes
        self.q, self.s, self.qs, self.b = [], [], [], []
        g = torch.Generator(device="cuda").manual_seed(seed)
        for n, k in shapes:
            w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
            q, s = ops.pack_int8(w, torch.bfloat16)
            self.q.append(q)
            self.s.append(s)
            self.qs.append(ops.to_strips(q))
            self.b.append((torch.randn(n, device="cuda", generator=g) * 0.1).to(torch.bfloat16) if bias else None)
        hidden = shapes[0][0]
        self.w_post = (1 + 0.1 * torch.randn(hidden, device="cuda", generator=g)).to(torch.bfloat16)
        self.w_in = (1 + 0.1 * torch.randn(hidden, device="cuda", generator=g)).to(torch.bfloat16)

    def buffers(self, m, seed):
        (n_o, k_o), (n_gu, _), (n_d, _), (n_qkv, _) = self.shapes
        g = torch.Generator(device="cuda").manual_seed(seed)
        attn = torch.randn(m, k_o, device="cuda", generator=g).to(torch.bfloat16)
        h = (torch.randn(m, n_o, device="cuda", generator=g) * 2).to(torch.bfloat16)
        out = {"h1": torch.empty(m, n_o, dtype=torch.bfloat16, device="cuda"),
               "act": torch.empty(m, n_gu // 2, dtype=torch.bfloat16, device="cuda"),
               "h2": torch.empty(m, n_d, dtype=torch.bfloat16, device="cuda"),
               "qkv": torch.empty(m, n_qkv, dtype=torch.bfloat16, device="cuda")}
        return attn, h, out

    def links(self, ops, attn, h, out):
        L = ops.ChainLink
        n_o, n_gu, n_d, n_qkv = (s[0] for s in self.shapes)
        return [
            L(attn, self.qs[0], n_o, self.s[0], out["h1"], bias=self.b[0], epilogue=ops.EPI_RESIDUAL, residual=h),
            L(out["h1"], self.qs[1], n_gu, self.s[1], out["act"], bias=self.b[1], prologue=ops.PRO_RMS_NORM,
              norm_weight=self.w_post, eps=EPS, epilogue=ops.EPI_SILU_MUL, after=0),
            L(out["act"], self.qs[2], n_d, self.s[2], out["h2"], bias=self.b[2], epilogue=ops.EPI_RESIDUAL,
              residual=out["h1"], after=1),
            L(out["h2"], self.qs[3], n_qkv, self.s[3], out["qkv"], bias=self.b[3], prologue=ops.PRO_RMS_NORM,
              norm_weight=self.w_in, eps=EPS, after=2),
        ]

    def separate(self, ops, attn, h):
        """The same layer through this library's separate kernels."""
        n_o, n_gu, n_d, n_qkv = (s[0] for s in self.shapes)
        h1 = h + ops.w8a16_gemm_strips(attn, self.qs[0], n_o, self.s[0], self.b[0])
        gu = ops.w8a16_gemm_strips(ops.rms_norm(h1, self.w_post, EPS), self.qs[1], n_gu, self.s[1], self.b[1])
        act = ops.silu_mul(gu)
        h2 = h1 + ops.w8a16_gemm_strips(act, self.qs[2], n_d, self.s[2], self.b[2])
        qkv = ops.w8a16_gemm_strips(ops.rms_norm(h2, self.w_in, EPS), self.qs[3], n_qkv, self.s[3], self.b[3])
        return {"h1": h1, "act": act, "h2": h2, "qkv": qkv}


def _gemm_ref(layer, i, x_np):
    b = layer.b[i]
    return O.w8a16_ref(x_np.astype(np.float32), layer.q[i].cpu().numpy(), layer.s[i].float().cpu().numpy(),
                       None if b is None else b.float().cpu().numpy())


def _bound(ref):
    rms = float(np.sqrt(np.mean(ref * ref)))
    return 1e-2 * rms + half_ulp(ref, torch.bfloat16)


def _check(what, got, ref, bound):
    err = np.abs(got - ref)
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} out of tolerance; max err {err.max():.4g}, "
                           f"worst at {np.unravel_index(np.argmax(err - bound), err.shape)}")


def _normed(x: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    """The oracle's RMSNorm rounded to bf16, as the chain stages it before the MFMAs."""
    ref = O.rms_norm(_bits(x), _bits(w), EPS, O.DT_BF16)
    return torch.from_numpy(ref).to(torch.bfloat16).double().numpy()


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _act_bound(g, u):
    """The GEMM bar on gate and up carried through silu(g) * u to first order (x1.25 for the
    second-order terms), plus act's own two roundings."""
    sg = _silu(g)
    sig = 1.0 / (1.0 + np.exp(-g))
    dsg = sig * (1.0 + g * (1.0 - sig))
    act = sg * u
    return (1.25 * (np.abs(dsg * u) * _bound(g) + np.abs(sg) * _bound(u)) + 2 * half_ulp(act, torch.bfloat16)
            + np.abs(u) * half_ulp(sg, torch.bfloat16))


def check_layer(layer, attn, h, out, what):
    """Each stage of the chain against the fp64 oracle, fed the chain's own inputs of that stage."""
    # h1 = h + o(attn)
    o_ref = _gemm_ref(layer, 0, _np(attn))
    _check(f"{what} h1", _np(out["h1"]), _np(h) + o_ref, _bound(o_ref) + half_ulp(_np(h) + o_ref, torch.bfloat16))
    # act = silu(gate) * up of gate_up(norm(h1))
    gu = _gemm_ref(layer, 1, _normed(out["h1"], layer.w_post))
    half = gu.shape[1] // 2
    g, u = gu[:, :half], gu[:, half:]
    _check(f"{what} act", _np(out["act"]), _silu(g) * u, _act_bound(g, u))
    # h2 = h1 + down(act)
    d_ref = _gemm_ref(layer, 2, _np(out["act"]))
    h2_ref = _np(out["h1"]) + d_ref
    _check(f"{what} h2", _np(out["h2"]), h2_ref, _bound(d_ref) + half_ulp(h2_ref, torch.bfloat16))
    # qkv = qkv(norm(h2))
    q_ref = _gemm_ref(layer, 3, _normed(out["h2"], layer.w_in))
    _check(f"{what} qkv", _np(out["qkv"]), q_ref, _bound(q_ref))


def check_against_separate(layer, ops, attn, h, out, what):
    """Stage by stage against this library's separate kernels, each fed the chain's own input."""
    n_o, n_gu, n_d, n_qkv = (s[0] for s in layer.shapes)
    sep_o = ops.w8a16_gemm_strips(attn, layer.qs[0], n_o, layer.s[0], layer.b[0])
    _check(f"{what} h1 vs separate", _np(out["h1"]), _np(h + sep_o),
           _bound(_np(sep_o)) + half_ulp(_np(h + sep_o), torch.bfloat16))
    sep_q = ops.w8a16_gemm_strips(ops.rms_norm(out["h2"], layer.w_in, EPS), layer.qs[3], n_qkv, layer.s[3],
                                  layer.b[3])
    _check(f"{what} qkv vs separate", _np(out["qkv"]), _np(sep_q), 2 * _bound(_np(sep_q)))
    full = layer.separate(ops, attn, h)
    for key in ("h1", "act", "h2", "qkv"):  # the whole layer: loose, errors compound over four stages
        ref = _np(full[key])
        rms = float(np.sqrt(np.mean(ref * ref)))
        err = float(np.abs(_np(out[key]) - ref).max())
        assert err <= 0.1 * rms + 0.05 * float(np.abs(ref).max()), f"{what} {key}: {err:.4g} vs rms {rms:.4g}"


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_talker_layer_chain(ops, m):
    layer = Layer(ops, TALKER_LAYER, seed=11)
    attn, h, out = layer.buffers(m, seed=100 + m)
    plan = ops.w8a16_chain(layer.links(ops, attn, h, out))
    torch.cuda.synchronize()
    assert not plan.timed_out()
    check_layer(layer, attn, h, out, f"talker m={m}")
    check_against_separate(layer, ops, attn, h, out, f"talker m={m}")


@pytest.mark.parametrize("m", [1, 3, 8])
def test_predictor_layer_chain_with_bias(ops, m):
    """Code-predictor shapes (K = 1024: four strips, two gate/up pairs an item; K = 3072 down),
    every linear with a bias (both halves of gate_up)."""
    layer = Layer(ops, PREDICTOR_LAYER, seed=12, bias=True)
    attn, h, out = layer.buffers(m, seed=200 + m)
    plan = ops.w8a16_chain(layer.links(ops, attn, h, out))
    torch.cuda.synchronize()
    assert not plan.timed_out()
    check_layer(layer, attn, h, out, f"predictor m={m}")
    check_against_separate(layer, ops, attn, h, out, f"predictor m={m}")


def test_grid_sizes_give_identical_bits(ops):
    """Any number of workgroups, down to one (which then runs every item in order and waits
    only on its own earlier items), computes every item the same way; a plan relaunched
    (later epochs of its control block) too."""
    layer = Layer(ops, TALKER_LAYER, seed=13)
    attn, h, ref = layer.buffers(2, seed=300)
    ops.w8a16_chain(layer.links(ops, attn, h, ref))
    for grid in (1, 2, 7, 64, 300, 4096):
        _, _, out = layer.buffers(2, seed=300)
        plan = ops.ChainPlan(layer.links(ops, attn, h, out), algo=grid << 8)
        for rep in range(3):
            for v in out.values():
                v.zero_()
            plan()
            torch.cuda.synchronize()
            for key in ref:
                assert torch.equal(out[key], ref[key]), f"grid={grid} launch {rep} {key}"
        assert not plan.timed_out()


def test_graph_replays_with_fresh_inputs(ops):
    """Captured once, replayed with new attention outputs and hidden states written into the
    same buffers between replays: every replay matches an eager run on the same inputs bit
    for bit (stale activations in some XCD's L2, or a flag of an earlier replay taken for
    this one's, would not)."""
    layer = Layer(ops, TALKER_LAYER, seed=14)
    m = 4
    attn, h, out = layer.buffers(m, seed=400)
    plan = ops.ChainPlan(layer.links(ops, attn, h, out))
    plan()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan()
        plan()  # twice per replay: the second launch must not take the first one's flags
    for rep in range(4):
        a2, h2, _ = layer.buffers(m, seed=401 + rep)
        attn.copy_(a2)
        h.copy_(h2)
        graph.replay()
        torch.cuda.synchronize()
        got = {k: v.clone() for k, v in out.items()}
        _, _, eager = layer.buffers(m, seed=0)
        ops.w8a16_chain(layer.links(ops, attn, h, eager))
        torch.cuda.synchronize()
        for key in got:
            assert torch.equal(got[key], eager[key]), f"replay {rep} {key}"
        if rep == 0:
            check_layer(layer, attn, h, got, "graph replay")
    assert not plan.timed_out()


def test_ragged_strips_and_independent_links(ops):
    """Items with strips past N (4 strips where an item holds 8; 3 where it holds 2), a SiLU link whose last
    item holds one pair of two, a K range whose last wave runs short (31 chunks), links with no
    dependency, an in-place residual, and a link that waits on a link two back."""
    g = torch.Generator(device="cuda").manual_seed(5)
    m = 3

    def lin(n, k):
        w = (torch.randn(n, k, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        q, s = ops.pack_int8(w, torch.bfloat16)
        return q, s, ops.to_strips(q)

    def ref(x, w):
        return O.w8a16_ref(x.float().cpu().numpy(), w[0].cpu().numpy(), w[1].float().cpu().numpy())

    def rows(k):
        return torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)

    def empty(n):
        return torch.empty(m, n, dtype=torch.bfloat16, device="cuda")

    x0, x1, x2, x3 = rows(128), rows(1024), rows(2048), rows(1984)
    r2 = rows(48)
    r2_before = r2.clone()
    w0, w1, w2, w3 = lin(64, 128), lin(96, 1024), lin(48, 2048), lin(80, 1984)
    y0, y1, y3 = empty(64), empty(48), empty(80)
    L = ops.ChainLink
    plan = ops.w8a16_chain([
        L(x0, w0[2], 64, w0[1], y0),                                          # k=128: 8 strips an item, 4 valid
        L(x1, w1[2], 96, w1[1], y1, epilogue=ops.EPI_SILU_MUL),               # 2 pairs an item, 3 pairs
        L(x2, w2[2], 48, w2[1], r2, epilogue=ops.EPI_RESIDUAL, residual=r2),  # in place
        L(x3, w3[2], 80, w3[1], y3),                                          # 31 chunks: 4 waves of 8
    ])
    torch.cuda.synchronize()
    assert not plan.timed_out()
    r0 = ref(x0, w0)
    _check("k=128", _np(y0), r0, _bound(r0))
    gu = ref(x1, w1)
    _check("silu n=96", _np(y1), _silu(gu[:, :48]) * gu[:, 48:], _act_bound(gu[:, :48], gu[:, 48:]))
    rr = ref(x2, w2)
    _check("in-place residual", _np(r2), _np(r2_before) + rr,
           _bound(rr) + half_ulp(_np(r2_before) + rr, torch.bfloat16))
    r3 = ref(x3, w3)
    _check("k=1984", _np(y3), r3, _bound(r3))

    # link 2 reads link 0's output and waits on it directly; link 1 in between is independent
    w4, w5 = lin(32, 64), lin(64, 64)
    x5 = rows(64)
    y0b, y4, y5 = empty(64), empty(32), empty(64)
    plan = ops.w8a16_chain([L(x0, w0[2], 64, w0[1], y0b), L(x5, w5[2], 64, w5[1], y5),
                            L(y0b, w4[2], 32, w4[1], y4, after=0)])
    torch.cuda.synchronize()
    assert torch.equal(y0b, y0)
    r4 = ref(y0b, w4)
    _check("after link 0", _np(y4), r4, _bound(r4))
    r5 = ref(x5, w5)
    _check("independent k=64", _np(y5), r5, _bound(r5))
    assert not plan.timed_out()


def test_empty_and_argument_errors(ops):
    layer = Layer(ops, PREDICTOR_LAYER, seed=15)
    attn, h, out = layer.buffers(1, seed=500)
    links = layer.links(ops, attn, h, out)
    with pytest.raises(ValueError):
        ops.w8a16_chain([])
    bad = list(links)
    bad[1] = ops.ChainLink(out["h1"], layer.qs[1], 6144, layer.s[1],
                           torch.empty(1, 6144, dtype=torch.bfloat16, device="cuda"), after=1)
    with pytest.raises(ValueError, match="earlier link"):
        ops.w8a16_chain(bad)
    with pytest.raises(ValueError):  # the SiLU output is [m, n / 2]
        ops.w8a16_chain([ops.ChainLink(out["h1"], layer.qs[1], 6144, layer.s[1], out["h2"],
                                       epilogue=ops.EPI_SILU_MUL)])
    e = torch.empty(0, 1024, dtype=torch.bfloat16, device="cuda")
    ops.w8a16_chain([ops.ChainLink(e, layer.qs[3], 4096, layer.s[3], torch.empty(0, 4096, dtype=torch.bfloat16,
                                                                                    device="cuda"))])
    torch.cuda.synchronize()
