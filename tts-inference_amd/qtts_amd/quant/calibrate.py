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

``calibrate_buckets`` asks the reference's question at every row bucket the callers
produce.  The reference times one weight's repeated calls, which keeps a small weight in
the L2 caches and times it as if it never streamed; here the callers may hand in several
copies of the weight (``rotate``) that together exceed the L2s, each call of a graph reading
the next one, so both the kernels and F.linear are timed with their weights streaming as
they do in a decode step (each layer's weight read once).  A layer the reference would keep (slower over the decode rows) is declined
here too; a layer it would convert can still lose to F.linear at some bucket (a
prefill row count, say), and with ``keep_reference`` that bucket is routed to F.linear
on the layer's retained weight (``ALGO_REFERENCE_GEMM``), so no bucket runs slower than
the layer it replaced -- the reference's rule that a layer measured slower keeps its
original GEMM (qtts/quant/int8.py:59-67), applied per bucket.
"""

from __future__ import annotations

import logging
import time
from typing import Callable

import torch

logger = logging.getLogger("qtts_amd.quant.calibrate")

_CACHE: dict[tuple, object] = {}

#: Algo value (Python side only) that sends a bucket's calls to F.linear on the layer's own
#: retained weight: the bucket where every quantized route lost to that GEMM.
ALGO_REFERENCE_GEMM = -2


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


#: Bytes of weight copies the weight-only methods rotate through when timing a shape: well past
#: the 8 x 4 MiB of L2, within the 256 MiB Infinity Cache (as the code predictor's 78 MB of int8
#: weights are during its 15 prefix passes).
ROTATE_BYTES = 64 << 20


def rotation(weight_bytes: int, limit: int = 64) -> int:
    """How many copies of a weight of ``weight_bytes`` the calibration rotates through."""
    return max(1, min(limit, -(-ROTATE_BYTES // max(1, weight_bytes))))


def rotating(calls: list[Callable[..., object]]) -> Callable[..., object]:
    """One callable that runs the next of ``calls`` each time it is called (in capture too, so a
    graph of len(calls) calls reads every copy once)."""
    state = [0]

    def run(*args):
        i = state[0]
        state[0] = (i + 1) % len(calls)
        return calls[i](*args)

    return run


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


def time_candidates(candidates: dict[str, Callable[[], object]], reference_call: Callable[[], object], *,
                    key: tuple, use_graph: bool = True,
                    timer: Callable[[Callable[[], object]], float] | None = None
                    ) -> tuple[float | None, dict[str, float]]:
    """Seconds per call of the reference and of every candidate that times without an exception.

    Cached per ``key`` like pick_fastest's verdicts.  A reference that fails gives ``None`` (the
    caller then keeps the layer unquantized); a failing candidate is left out."""
    ck = ("timings",) + tuple(key)
    if ck in _CACHE:
        return _CACHE[ck]  # type: ignore[return-value]
    t = timer or (graph_time if use_graph else eager_time)
    try:
        reference = t(reference_call)
    except Exception as exc:
        logger.warning("calibration of the reference failed for %s (%s); leaving it unquantized", key, exc)
        _CACHE[ck] = (None, {})
        return None, {}
    timings: dict[str, float] = {}
    for name, call in candidates.items():
        try:
            timings[name] = t(call)
        except Exception as exc:
            logger.warning("calibration of %s failed for %s (%s); dropping that candidate", name, key, exc)
    _CACHE[ck] = (reference, timings)
    logger.debug("%s: reference %.2f us, %s", key, reference * 1e6,
                 ", ".join(f"{n} {v * 1e6:.2f} us" for n, v in timings.items()))
    return reference, timings


#: A pinned kernel configuration replaces the automatic choice (the candidate named "auto") at a
#: bucket only when it is this much faster, the margin the accept/decline verdict asks of a
#: quantized layer: candidates within a few percent of each other trade places from run to run, and
#: a pin that won by 2-3% in the calibration's timing (one shape's calls back to back, weights
#: rotated past the L2s) lost by about 1% in the code predictor's frame, where the shapes interleave.
AUTO_MARGIN = 1.05


def calibrate_buckets(tag: str, n: int, k: int, dtype: torch.dtype, device: torch.device,
                      buckets: tuple[int, ...], decode_rows: int,
                      candidates: Callable[[int], dict[str, int]],
                      kernel_call: Callable[[torch.Tensor, int], object],
                      reference_call: Callable[[torch.Tensor], object],
                      route_calls: dict[int, dict[str, tuple[int, Callable[[torch.Tensor], object]]]] | None = None,
                      margin: float = 1.05, use_graph: bool = True,
                      timer: Callable[[Callable[[], object]], float] | None = None,
                      keep_reference: bool = False, inner: int = 10,
                      ) -> tuple[bool, dict[int, int], dict[int, dict]]:
    """Per-bucket kernel choice for one ``[n, k]`` weight (qtts/quant/calibrate.py:77-114 asks one
    question at one row count; this asks it at every row bucket the callers produce).

    At each row count in ``buckets`` it times every candidate algo (``candidates(rows)``, run as
    ``kernel_call(x, algo)``; ``inner`` calls a graph, at least 10) and any extra routes for that
    bucket (``route_calls[rows]``: name ->
    (algo marker, call)) against ``reference_call(x)`` (F.linear on the bf16 weight), on seeded
    random activations.  The layer is worth quantizing when, summed over the decode buckets (rows
    <= ``decode_rows``: the rows a decode step runs), the fastest candidate of each bucket beats
    the reference by ``margin`` -- one verdict per layer, as in the reference, but taken over the
    decode rows instead of at one row count.  A reference that cannot be timed at a decode bucket
    declines the layer; a calibration failure is never fatal.

    Returns ``(accept, {rows: algo}, {rows: {"reference": s, "best": name, "timings": {...}}})``;
    the table holds the fastest candidate of every bucket that timed.  Where that candidate is
    slower than the reference, the bucket gets ``ALGO_REFERENCE_GEMM`` with ``keep_reference``
    (the caller keeps the weight for F.linear there), else the fastest quantized route anyway."""
    table: dict[int, int] = {}
    report: dict[int, dict] = {}
    decode_ref = decode_best = 0.0
    decode_seen = 0
    for rows in buckets:
        gen = torch.Generator(device=device).manual_seed(rows)
        x = torch.randn(rows, k, device=device, dtype=dtype, generator=gen)
        algos = dict(candidates(rows))
        calls = {name: (lambda a=a, x=x: kernel_call(x, a)) for name, a in algos.items()}
        for name, (marker, call) in (route_calls or {}).get(rows, {}).items():
            algos[name] = marker
            calls[name] = (lambda c=call, x=x: c(x))
        t = timer
        if t is None and use_graph:  # ``inner`` calls a graph (one per weight copy the calls rotate over)
            # prefill-sized calls: fewer replays suffice
            t = lambda fn, r=rows: graph_time(fn, inner=max(10, inner), iters=10 if r > 128 else 50)  # noqa: E731
        key = (tag, n, k, rows, str(dtype)) + ((("calls_per_graph", inner),) if inner > 10 else ())
        reference, timings = time_candidates(calls, lambda x=x: reference_call(x), key=key, use_graph=use_graph,
                                             timer=t)
        best = min(timings, key=timings.get) if timings else None
        if best is not None and "auto" in timings and timings[best] * AUTO_MARGIN > timings["auto"]:
            best = "auto"
        report[rows] = {"reference": reference, "best": best, "timings": timings}
        if best is not None:
            loses = reference is not None and timings[best] > reference
            table[rows] = ALGO_REFERENCE_GEMM if keep_reference and loses else algos[best]
        if rows <= decode_rows:
            if reference is None or best is None:
                return False, {}, report
            decode_ref += reference
            decode_best += timings[best]
            decode_seen += 1
    accept = decode_seen > 0 and decode_best * margin < decode_ref
    logger.debug("%s (%d, %d): decode buckets %.2f us quantized vs %.2f us reference -> %s", tag, n, k,
                 decode_best * 1e6, decode_ref * 1e6, "quantize" if accept else "keep")
    return accept, (table if accept else {}), report


def clear_cache() -> None:
    _CACHE.clear()
