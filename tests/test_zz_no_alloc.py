"""qtts_fp8_linear_strips_static (the fp8 W8A8 linear on the library's own device workspace, for
callers that cannot allocate) against qtts_fp8_linear_strips on a caller-owned workspace, through
the C ABI: bit for bit, on calls in a row that reuse the shared array (each later call smaller
than the one before), on the two-kernel path (rows past the decode cut-off: activation codes and
split-K counters in the workspace) and the one-kernel decode path, plus the size limit."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    from qtts_amd import _lib, ops
    assert ops.device_supported(), "GPU is not a gfx950"
    return _lib, ops


def _operands(ops, m, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(n, k, device="cuda", generator=g) * 0.02
    x = torch.randn(m, k, device="cuda", generator=g)
    x = torch.where(torch.rand(m, k, device="cuda", generator=g) < 0.01, torch.sign(x) * 20.0, x).to(torch.bfloat16)
    b = (torch.randn(n, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    qw, sw = ops.pack_fp8(w)
    return x, ops.to_strips(qw), sw, b


def _static_call(_lib, x, qws, n, sw, b, algo=0):
    m, k = x.shape
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rc = _lib.load().qtts_fp8_linear_strips_static(x.data_ptr(), _lib.BF16, m, k, k, qws.data_ptr(), n,
                                                   sw.data_ptr(), b.data_ptr(), y.data_ptr(), n, _lib.DIV_DEVICE,
                                                   algo, ctypes.c_void_p(st))
    return rc, y


def test_static_entry_first_called_under_graph_capture(env):
    """The entry point's first call in the process is made inside a HIP graph capture (torch's
    global capture mode, where an allocating or synchronizing call fails the capture): the scratch
    address is resolved and the counter block cleared there.  Two-kernel rows, with and without a
    forced split; every replay, with eager work between them, equals the caller-workspace entry
    point bit for bit."""
    _lib, ops = env
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    m, n, k = 64, 2048, 2048
    x, qws, sw, b = _operands(ops, m, n, k, seed=7)
    split = _lib.algo_code(_lib.ALGO_TILE, splits=2)
    static_x = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the caller-workspace path only
        ops.fp8_linear_strips(static_x, qws, n, sw, b)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc0, y0 = _static_call(_lib, static_x, qws, n, sw, b)
        rc1, y1 = _static_call(_lib, static_x, qws, n, sw, b, split)
    assert rc0 == 0 and rc1 == 0, _lib.last_error()
    g = torch.Generator(device="cuda").manual_seed(8)
    for i in range(3):
        fresh = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        static_x.copy_(fresh)
        ops.fp8_linear_strips(fresh * 0.5, qws, n, sw, b)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y0, ops.fp8_linear_strips(fresh, qws, n, sw, b)), f"replay {i}"
        assert torch.equal(y1, ops.fp8_linear_strips(fresh, qws, n, sw, b, ops.DIV_DEVICE, split)), f"replay {i} split"


def test_static_workspace_matches_caller_workspace(env):
    _lib, ops = env
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    # two-kernel rows (activation codes and split counters in the workspace), each call smaller
    # than the one before it, then decode rows (one kernel, no workspace), then two-kernel again
    for i, (m, n, k) in enumerate([(256, 4096, 2048), (64, 2048, 6144), (17, 12288, 2048), (4, 2048, 2048),
                                   (40, 2048, 2048)]):
        print(f"static fp8 linear m={m} n={n} k={k}", flush=True)
        x, qws, sw, b = _operands(ops, m, n, k, seed=100 + i)
        ref = ops.fp8_linear_strips(x, qws, n, sw, b)
        rc, y = _static_call(_lib, x, qws, n, sw, b)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), (m, n, k)
        # and again with a forced split count: the counters it uses start at zero and are left at zero
        split = _lib.algo_code(_lib.ALGO_TILE if m > 16 else _lib.ALGO_SKINNY, splits=2)
        ref2 = ops.fp8_linear_strips(x, qws, n, sw, b, ops.DIV_DEVICE, split)
        rc, y2 = _static_call(_lib, x, qws, n, sw, b, split)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y2, ref2), (m, n, k, "split")


def test_static_workspace_limit(env):
    _lib, ops = env
    # 32 MiB hold 64 KiB of counters plus the codes of at most ~33.4 M activations
    k = 8192
    m = (_lib.STATIC_SCRATCH_BYTES // k) + 1
    x = torch.zeros(m, k, dtype=torch.bfloat16, device="cuda")
    qws = torch.zeros(16 * k, dtype=torch.uint8, device="cuda")
    sw = torch.ones(16, dtype=torch.float32, device="cuda")
    y = torch.empty(m, 16, dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rc = _lib.load().qtts_fp8_linear_strips_static(x.data_ptr(), _lib.BF16, m, k, k, qws.data_ptr(), 16,
                                                   sw.data_ptr(), None, y.data_ptr(), 16, _lib.DIV_DEVICE, 0,
                                                   ctypes.c_void_p(st))
    assert rc == _lib.ERR_WORKSPACE and "static scratch" in _lib.last_error()
