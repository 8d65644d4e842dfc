"""HIP-graph capture of the decode callers' steps, the way qtts captures them.

The reference runs its quantized linears inside two kinds of captured graphs
(qtts/compilation.py): the talker's decode step, with the batch padded up to the next
captured size and one graph per size (TalkerDecodeGraphs, compilation.py:60-186, padding
at 101-105), and the code predictor's whole walk over the codebook axis, 15 exact-prefix
forwards with M = batch x prefix rows, one graph per padded batch (CodePredictorGraphs,
compilation.py:189-273; the walk is code_predictor.py:200-243).  Those classes belong to
the model code, which this package does not rebuild; the harness here reproduces their
capture rules around any step function, so a caller (or a test) can run the quantized
linears exactly as the engine would: static input buffers shared by every graph (views of
the largest), padded rows zeroed, a warm-up on a side stream before each capture, one
memory pool for all graphs, and outputs that stay valid until the next replay
(:class:`PaddedGraphs`).

Nothing here allocates on replay; the quant methods reserve their workspaces at load time
(``ops.WORKSPACE_ROWS``), so capture needs no allocation inside the ops either.
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch

#: The talker's captured decode batch sizes (qtts/config.py:122).
DECODE_BATCH_SIZES = (1, 2, 4, 8, 16, 32, 64)


def _sizes(batch_sizes: Sequence[int]) -> tuple[int, ...]:
    sizes = tuple(sorted({int(b) for b in batch_sizes if int(b) >= 1}))
    if not sizes:
        raise ValueError("at least one batch size >= 1 is needed")
    return sizes


def _padded(sizes: tuple[int, ...], rows: int) -> int:
    for size in sizes:
        if size >= rows:
            return size
    raise ValueError(f"{rows} rows is more than the largest captured batch size {sizes[-1]}")


def _capture(fn: Callable[[], object], pool) -> tuple[torch.cuda.CUDAGraph, object]:
    """Warm ``fn`` up on a side stream (first calls may load kernels or reserve memory, which a
    capture cannot), then capture one call of it into a graph in ``pool``."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, pool=pool):
        out = fn()
    return graph, out


class PaddedGraphs:
    """One captured graph per padded row count around ``step(x) -> outputs``.

    ``x`` is ``[rows, *row_shape]``; ``run`` copies it into a static buffer, zeroes the rows up
    to the next captured batch size, replays (capturing on first use of a size) and returns the
    step's outputs cut to ``rows`` (a tensor or a tuple of tensors with rows first).  As in the
    reference, the outputs are the graph's own buffers, overwritten by the next replay.

    For the talker's rule ``step`` is one decode step over the layers and ``batch_sizes`` the
    decode sizes; for the code predictor's, ``step`` is the whole walk over the codebook axis
    (each of its prefix forwards runs at M = batch x prefix rows) and ``batch_sizes`` the
    predictor's captured batches."""

    def __init__(self, step: Callable[[torch.Tensor], object], row_shape: Sequence[int], dtype: torch.dtype,
                 device: torch.device | str = "cuda", batch_sizes: Sequence[int] = DECODE_BATCH_SIZES) -> None:
        self.step = step
        self.batch_sizes = _sizes(batch_sizes)
        self.inputs = torch.zeros((self.batch_sizes[-1], *row_shape), dtype=dtype, device=device)
        self.pool = None
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, object]] = {}
        self.replays = 0

    def padded_rows(self, rows: int) -> int:
        return _padded(self.batch_sizes, rows)

    def run(self, x: torch.Tensor):
        rows = x.shape[0]
        padded = self.padded_rows(rows)
        self.inputs[:rows].copy_(x)
        if padded > rows:
            self.inputs[rows:padded].zero_()
        entry = self.graphs.get(padded)
        if entry is None:
            view = self.inputs[:padded]
            entry = _capture(lambda: self.step(view), self.pool)
            if self.pool is None:
                self.pool = entry[0].pool()
            self.graphs[padded] = entry
        graph, out = entry
        graph.replay()
        self.replays += 1
        if isinstance(out, torch.Tensor):
            return out[:rows]
        return tuple(o[:rows] for o in out)
