"""The measurement kernels behind ``bench.py --floor`` (their own library, probe/probe.hip):
the streaming probe reads every byte of its slice exactly once, in the blocks its comment
promises (each wave's xor against numpy), and the empty kernel runs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


class _Probes:
    """bench.py's wrappers of the probe library, bound to torch."""

    def __init__(self):
        import bench
        self.bench = bench

    def probe_stream(self, src, nbytes, waves, loads, sink):
        self.bench.probe_stream(torch, src, nbytes, waves, loads, sink)

    def probe_empty(self, workgroups, waves=1):
        self.bench.probe_empty(torch, workgroups, waves)


@pytest.fixture(scope="module")
def ops():
    from qtts_amd import ops as _ops
    assert _ops.device_supported(), "GPU is not a gfx950"
    return _Probes()


@pytest.mark.parametrize("waves,loads", [(1, 1), (4, 8), (16, 2), (2, 16), (8, 4)])
def test_stream_probe_reads_each_block_once(ops, waves, loads):
    nbytes = 3 * waves * loads * 1024
    g = torch.Generator(device="cuda").manual_seed(waves * 100 + loads)
    buf = torch.randint(-2**31, 2**31 - 1, (nbytes // 4 + 64,), dtype=torch.int32, device="cuda", generator=g)
    src = buf[16:16 + nbytes // 4]  # a 64-byte offset slice: the probe honours the slice start
    sink = torch.full((nbytes // (loads * 1024) + 4,), 7, dtype=torch.int32, device="cuda")
    ops.probe_stream(src, nbytes, waves, loads, sink)
    got = sink.cpu().numpy()
    words = src.cpu().numpy().reshape(-1, loads * 256)  # one row per wave: loads KiB of 32-bit words
    want = np.bitwise_xor.reduce(words, axis=1)
    assert np.array_equal(got[:len(want)], want)
    assert (got[len(want):] == 7).all(), "the probe wrote past its last wave"


def test_empty_probe_and_graph_capture(ops):
    ops.probe_empty(768, 4)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.probe_empty(1, 1)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        for _ in range(8):
            ops.probe_empty(128, 4)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()


def test_probe_wrapper_checks(ops):
    src = torch.zeros(4096, dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError):
        ops.probe_stream(src, 8192, 4, 1, torch.zeros(8, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError):
        ops.probe_stream(src, 4096, 4, 1, torch.zeros(2, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError):  # a strided view would be read past its storage
        ops.probe_stream(torch.zeros(4096, 2, dtype=torch.int8, device="cuda")[:, 0], 4096, 4, 1,
                         torch.zeros(8, dtype=torch.int32, device="cuda"))
