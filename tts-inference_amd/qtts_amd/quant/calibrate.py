"""Per-shape kernel choice, measured on the GPU inside a HIP graph.

Replaces qtts/quant/calibrate.py:40-118.  The reference answers one question per
(N, K, rows, dtype): is the quantized GEMM faster than F.linear by a 1.05 margin?
This module keeps that contract (``worth_quantizing``, same signature and cache
semantics) and adds ``pick_fastest``, which times several quantized candidates
(the skinny and tile HIP kernels and their split variants) against the bf16
reference and keeps the fastest one that beats the reference by the margin.

Timing runs ``inner`` calls captured in one graph and replays it ``iters`` times
(qtts/quant/calibrate.py:40-63), so launch overhead is amortised the way the
engine's decode graph amortises it.  Any exception while timing a candidate drops
that candidate; an exception while timing the reference declines the layer.  A
calibration failure is never fatal (qtts/quant/calibrate.py:96-103).
"""

from __future__ import annotations

import logging
import time
from typing import Callable

import torch

logger = logging.getLogger("qtts_amd.quant.calibrate")

_CACHE: dict[tuple, object] = {}


def graph_time(fn: Callable[[], object], inner: int = 10, iters: int = 50) -> float:
    """Seconds per call of ``fn``, replayed from a captured graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    started = time.perf_counter()
    for _ in range(iters):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - started
    del graph
    return elapsed / (iters * inner)


def eager_time(fn: Callable[[], object], iters: int = 200) -> float:
    for _ in range(20):
        fn()
    torch.cuda.synchronize()
    started = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - started) / iters


def pick_fastest(candidates: dict[str, Callable[[], object]], reference_call: Callable[[], object], *,
                 key: tuple, margin: float = 1.05, use_graph: bool = True,
                 timer: Callable[[Callable[[], object]], float] | None = None) -> str | None:
    """Name of the fastest candidate that beats ``reference_call`` by ``margin``, else None.

    Cached per ``key``: the first verdict for a key is the verdict for the process.
    """
    if key in _CACHE:
        return _CACHE[key]  # type: ignore[return-value]
    t = timer or (graph_time if use_graph else eager_time)
    try:
        reference = t(reference_call)
    except Exception as exc:  # capture can fail for reasons unrelated to the layer
        logger.warning("calibration of the reference failed for %s (%s); leaving it unquantized", key, exc)
        _CACHE[key] = None
        return None
    timings: dict[str, float] = {}
    for name, call in candidates.items():
        try:
            timings[name] = t(call)
        except Exception as exc:
            logger.warning("calibration of %s failed for %s (%s); dropping that candidate", name, key, exc)
    best = min(timings, key=timings.get) if timings else None
    verdict = best if best is not None and timings[best] * margin < reference else None
    _CACHE[key] = verdict
    logger.debug("%s: reference %.2f us, %s -> %s", key, reference * 1e6,
                 ", ".join(f"{n} {v * 1e6:.2f} us" for n, v in timings.items()), verdict or "keep")
    return verdict


def worth_quantizing(quantized_call: Callable[[], object], reference_call: Callable[[], object], *, key: tuple,
                     margin: float = 1.05, use_graph: bool = True,
                     timer: Callable[[Callable[[], object]], float] | None = None) -> bool:
    """Whether ``quantized_call`` beats ``reference_call`` by ``margin`` (qtts/quant/calibrate.py:77-114)."""
    if key in _CACHE:
        return bool(_CACHE[key])
    verdict = pick_fastest({"quantized": quantized_call}, reference_call, key=key, margin=margin,
                           use_graph=use_graph, timer=timer)
    _CACHE[key] = verdict is not None
    return verdict is not None


def clear_cache() -> None:
    _CACHE.clear()
