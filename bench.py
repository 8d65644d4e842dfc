#!/usr/bin/env python
"""Benchmark of the quantized-linear hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config C]
    python bench.py --summarize-rocprof DIR     # digest a rocprofv3 --kernel-trace run

Default workload: BASELINE.json configs[1], the talker decode linear stack.  28
layers x {qkv 2048->4096, o 2048->2048, gate_up 2048->12288, down 6144->2048},
each layer with its own seeded int8 weights (1.41 GB, > 5x the 256 MB Infinity
Cache), bf16 activations, M in {1, 2, 4, 8}.  The 112 GEMMs of one M are captured
into one HIP graph.  One step = one replay of the stack at each of the four M.

Printed: one JSON line with the whole-step HBM throughput (algorithmic bytes /
time), the per-M stack time next to the bf16 hipBLASLt baseline of the same
stack, a roofline entry for the dominant kernel (gate_up: device duration of each
launch from HIP events bound to its dispatch, the launches running back to back on a
busy GPU as in the graphs) and the reference's CPU path timed on a bounded
sample on this host.

Other configs (--config 0..4) print their own JSON line with the same keys;
--int8-w8a8 times the int8 W8A8 linear (Int8Method) on the talker shapes; --fp8w the
configs[1] decode stack with fp8 weight-only weights (Fp8WeightOnlyMethod); --mlp the
talker MLP with its activation fused into the down projection.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tts-inference_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E, published
ROOFLINE_REPS = 3               # passes over the 28 gate_up weights per M in the roofline timing
COLD_REPS = 2                   # passes of the same launched one by one onto an idle GPU, first
BF16_PEAK_TFLOPS = 2500.0       # dense bf16 MFMA, published
FP8_PEAK_TFLOPS = 5000.0        # dense fp8 MFMA, published
INT8_PEAK_TOPS = 5000.0         # dense int8 MFMA, published

TALKER = [("qkv", 4096, 2048), ("o", 2048, 2048), ("gate_up", 12288, 2048), ("down", 2048, 6144)]
PREDICTOR = [("qkv", 4096, 1024), ("o", 1024, 2048), ("gate_up", 6144, 1024), ("down", 1024, 3072)]


def w8a16_bytes(m: int, n: int, k: int) -> int:
    """Algorithmic HBM bytes of one W8A16 GEMM: int8 weight, bf16 scale, bf16 x in, bf16 y out."""
    return n * k + 2 * n + 2 * m * k + 2 * m * n


def fp8_bytes(m: int, n: int, k: int) -> int:
    """fp8 W8A8: e4m3 weight, fp32 scale, bf16 x in (quantized once), bf16 y out."""
    return n * k + 4 * n + 2 * m * k + 2 * m * n


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------------------
# weights and inputs
# ---------------------------------------------------------------------------------------

def make_stack(torch, ops, shapes, layers: int, keep_bf16: bool, fp8: bool = False, keep_rowmajor: int = 0,
               f32_scale: bool = False):
    """Distinct seeded weights per (layer, linear): W ~ N(0, 0.02) fp32, seed 1000 + 16*layer + idx.

    Each entry holds the packed weight in the strip layout the quant methods store
    (``qs``) and its scale; the row-major packed bytes (``q``) are kept for the first
    ``keep_rowmajor`` layers only (the CPU baseline's sample)."""
    stack = []
    for layer in range(layers):
        for idx, (name, n, k) in enumerate(shapes):
            g = torch.Generator(device="cuda").manual_seed(1000 + 16 * layer + idx)
            w = torch.randn(n, k, device="cuda", generator=g) * 0.02
            if fp8:
                q, s = ops.pack_fp8(w)
            else:
                q, s = ops.pack_int8(w, torch.float32 if f32_scale else torch.bfloat16)
            qs = ops.to_strips(q)
            wb = w.to(torch.bfloat16) if keep_bf16 else None
            stack.append({"layer": layer, "name": name, "n": n, "k": k, "qs": qs, "s": s, "w_bf16": wb,
                          "q": q if layer < keep_rowmajor else None})
            del w, q
    torch.cuda.synchronize()
    return stack


def make_inputs(torch, ks, ms, outliers: bool = False):
    """bf16 activations ~ N(0, 1), seed 7 (+ 1% of entries at +/-20 with ``outliers``)."""
    xs = {}
    for m in ms:
        for k in sorted(set(ks)):
            g = torch.Generator(device="cuda").manual_seed(7 + 131 * m + k)
            x = torch.randn(m, k, device="cuda", generator=g)
            if outliers:
                mask = torch.rand(m, k, device="cuda", generator=g) < 0.01
                x = torch.where(mask, torch.sign(x) * 20.0, x)
            xs[(m, k)] = x.to(torch.bfloat16)
    return xs


def capture(torch, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, graph, steps: int, warmup: int) -> float:
    """Mean ms per replay over ``steps`` replays, bracketed by synchronize, events on the replay stream."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_rounds(torch, graphs: dict, steps: int, warmup: int, rounds: int = 3) -> dict:
    """Median ms per replay of each graph over ``rounds`` rounds, the graphs timed in a rotating
    order.  The first timing of a freshly captured short graph runs up to 20% slow (measured on
    the prefill shapes, for our kernels more than for hipBLASLt), so every path gets the same
    repeated, order-balanced measurement."""
    names = list(graphs)
    times = {nm: [] for nm in names}
    for r in range(rounds):
        for nm in names[r % len(names):] + names[:r % len(names)]:
            times[nm].append(time_graph(torch, graphs[nm], steps, warmup))
    return {nm: statistics.median(ts) for nm, ts in times.items()}


def committed_figure(name: str, key: str) -> tuple[float | None, str | None]:
    """A figure a committed profile summary under profiles/ states on a ``key: value`` line: the
    HBM bytes per launch of a rocprofv3 --pmc run (FETCH_SIZE and WRITE_SIZE, each scaled by what
    the counter reads for a copy of known size), or a kernel's mean duration in a kernel trace."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1]), f"profiles/{name}"
    except OSError:
        pass
    return None, None


def kernel_ms(ops, launches, reps: int) -> float:
    """Mean device duration of the kernels ``launches`` start (callables of one kernel each), over
    ``reps`` passes: each kernel's own start/stop timestamps, taken by HIP events that
    hipExtLaunchKernel binds to its dispatch on the stream it is launched on.  Launched from the
    host one by one, so the GPU idles between them (the cold figure)."""
    with ops.KernelTimer(max_launches=len(launches) * reps + 16) as t:
        for _ in range(reps):
            for fn in launches:
                fn()
    if t.launches != len(launches) * reps or t.untimed:
        raise RuntimeError(f"kernel timer saw {t.launches} kernels (+{t.untimed} untimed), "
                           f"expected {len(launches) * reps}")
    return t.mean_ms


def busy_cycles(torch, busy_ms: float) -> int:
    """Spin-kernel cycles (torch.cuda._sleep) that keep the GPU busy for about ``busy_ms``."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 2_000_000
    torch.cuda.synchronize()
    start.record()
    torch.cuda._sleep(n)
    end.record()
    torch.cuda.synchronize()
    return max(1, int(n * busy_ms / max(start.elapsed_time(end), 1e-3)))


def kernel_ms_busy(torch, ops, groups: dict, reps: int, busy_ms: float = 5.0) -> dict:
    """Mean device duration per group of kernels (``groups``: key -> callables of one kernel each),
    each kernel timed by HIP events bound to its own dispatch (as kernel_ms), with every pass of a
    group queued behind a spin kernel of ``busy_ms``: the host enqueues the whole pass while the GPU
    is busy, so the group's kernels run back to back on a busy GPU, as they do inside the decode
    step's HIP graph.  (Launched one by one onto an idle GPU, the same kernels read 15-20% longer:
    kernel_ms.)  The spin kernel is torch's and is not timed."""
    cycles = busy_cycles(torch, busy_ms)
    out = {}
    for key, launches in groups.items():
        with ops.KernelTimer(max_launches=len(launches) * reps + 16) as t:
            for _ in range(reps):
                torch.cuda._sleep(cycles)
                for fn in launches:
                    fn()
        if t.launches != len(launches) * reps or t.untimed:
            raise RuntimeError(f"kernel timer saw {t.launches} kernels (+{t.untimed} untimed), "
                               f"expected {len(launches) * reps}")
        out[key] = t.mean_ms
    torch.cuda.synchronize()
    return out


# ---------------------------------------------------------------------------------------
# CPU baseline: the reference's CPU path, timed on this host
# ---------------------------------------------------------------------------------------

def cpu_baseline_w8a16(torch, stack, xs, ms, budget_s: float, layers_sample: int):
    from oracle import cpu_path
    # One thread per core this process may run on, capped by OMP_NUM_THREADS where the host
    # sets it (a GPU box's CPU share can be smaller than its affinity mask).
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = max(1, min(threads, int(os.environ["OMP_NUM_THREADS"])))
    saved_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    sample = [e for e in stack if e["layer"] < layers_sample]
    cpu = [(e, e["q"].cpu(), e["s"].cpu()) for e in sample]
    xcpu = {key: v.cpu() for key, v in xs.items()}
    total_bytes = 0
    total_s = 0.0
    started = time.perf_counter()
    for m in ms:
        for e, q, s in cpu:
            x = xcpu[(m, e["k"])]
            for _ in range(3):
                cpu_path.naive_dequant_linear(x, q, s)
            ts = []
            for _ in range(10):
                t0 = time.perf_counter()
                cpu_path.naive_dequant_linear(x, q, s)
                ts.append(time.perf_counter() - t0)
                if time.perf_counter() - started > budget_s and len(ts) >= 3:
                    break
            total_s += statistics.median(ts)
            total_bytes += w8a16_bytes(m, e["n"], e["k"])
    torch.set_num_threads(saved_threads)
    return {
        "value": round(total_bytes / total_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"reference CPU path F.linear(x_bf16, q.to(bf16)*scale[:,None]) (oracle/cpu_path.py) on "
                   f"{layers_sample} of 28 talker layers x 4 linears x M in {list(ms)}, median of up to 10 "
                   f"after 3 warm-ups, torch CPU with {threads} threads (len(os.sched_getaffinity(0)) "
                   f"= {len(os.sched_getaffinity(0))}, OMP_NUM_THREADS = {os.environ.get('OMP_NUM_THREADS')}); "
                   f"{total_s * 1e3:.1f} ms for {total_bytes / 1e6:.1f} MB"),
    }


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------------------
# configs
# ---------------------------------------------------------------------------------------

def run_talker_stack(args, torch, ops):
    """the 28-layer talker decode stack, int8 weight-only, M in {1, 2, 4, 8}."""
    ms = (1, 2, 4, 8)
    layers = 28
    log(f"[bench] packing {layers}x4 talker weights (int8 + bf16 baseline copy)")
    stack = make_stack(torch, ops, TALKER, layers, keep_bf16=True, keep_rowmajor=2)
    ops.reserve_workspace(torch.device("cuda"), max(
        ops.workspace_bytes(ops.OP_W8A16, m, e["n"], e["k"]) for m in ms for e in stack[:4]))
    xs = make_inputs(torch, [k for _, _, k in TALKER], ms)
    int8_bytes = sum(e["n"] * e["k"] for e in stack)

    # Dominant kernel: gate_up, the largest share of the stack; its roofline entry.  Its first
    # launches: COLD_REPS cold passes over the 28 weights at each M (which also take the weights'
    # first-touch costs), then ROOFLINE_REPS busy passes, so that under rocprofv3 --kernel-trace
    # the dispatches COLD_REPS x 28 + 1 .. + ROOFLINE_REPS x 28 of each M are exactly the timed ones
    # (bench.py --summarize-skip / --summarize-first).
    gate = [e for e in stack if e["name"] == "gate_up"]
    st = ops.ALGO_STREAM  # the stack's weight policy: 1.41 GB is past the Infinity Cache
    cold_ms = kernel_ms(ops, [lambda e=e, m=m: ops.w8a16_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"], None, st)
                              for m in ms for e in gate], reps=COLD_REPS)
    busy = kernel_ms_busy(torch, ops, {m: [lambda e=e, m=m: ops.w8a16_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"],
                                                                                   e["s"], None, st) for e in gate]
                                       for m in ms}, reps=ROOFLINE_REPS)
    flows, _ = layer_flows(torch, ops, stack, layers)

    per_m = {}
    total_bytes = 0
    total_ms = 0.0
    for m in ms:
        log(f"[bench] M={m}: capture + time int8 stack and bf16 stack")
        g_q = capture(torch, lambda m=m: [ops.w8a16_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"], None, st)
                                          for e in stack])
        g_b = capture(torch, lambda m=m: [torch.nn.functional.linear(xs[(m, e["k"])], e["w_bf16"]) for e in stack])
        t_q = time_graph(torch, g_q, args.steps, args.warmup)
        t_b = time_graph(torch, g_b, max(5, args.steps // 2), args.warmup)
        nbytes = sum(w8a16_bytes(m, e["n"], e["k"]) for e in stack)
        total_bytes += nbytes
        total_ms += t_q
        per_m[str(m)] = {
            "stack_us": round(t_q * 1e3, 2),
            "GBps": round(nbytes / (t_q * 1e-3) / 1e9, 1),
            "pct_of_hbm_peak": round(100 * nbytes / (t_q * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1),
            "bf16_hipblaslt_stack_us": round(t_b * 1e3, 2),
            "speedup_vs_bf16": round(t_b / t_q, 3),
        }
        # The same weights in the decode step's data flow: norms, SiLU and residual adds fused
        # into the GEMMs, against bf16 torch doing the same.
        attn = xs[(m, 2048)]
        h_in = make_inputs(torch, [2048], [m])[(m, 2048)] * 2
        g_f = capture(torch, lambda: flows["fused"](h_in, attn))
        g_fb = capture(torch, lambda: flows["bf16"](h_in, attn))
        t_f = time_graph(torch, g_f, args.steps, args.warmup)
        t_fb = time_graph(torch, g_fb, max(5, args.steps // 2), args.warmup)
        per_m[str(m)]["layer_flow_fused_us"] = round(t_f * 1e3, 2)
        per_m[str(m)]["layer_flow_bf16_torch_us"] = round(t_fb * 1e3, 2)
        per_m[str(m)]["layer_flow_speedup_vs_bf16"] = round(t_fb / t_f, 3)
        del g_q, g_b, g_f, g_fb
        log(f"[bench] M={m}: {per_m[str(m)]}")

    # The layer flow at 16 rows, outside the line's M = 1..8 (a decode step padded to 9-16 rows): the
    # fused forms run there in two row parts of 8.
    m16 = 16
    attn16 = make_inputs(torch, [2048], [m16])[(m16, 2048)]
    h16 = attn16 * 2
    g_f = capture(torch, lambda: flows["fused"](h16, attn16))
    g_fb = capture(torch, lambda: flows["bf16"](h16, attn16))
    t_f = time_graph(torch, g_f, args.steps, args.warmup)
    t_fb = time_graph(torch, g_fb, max(5, args.steps // 2), args.warmup)
    flow16 = {"fused_us": round(t_f * 1e3, 2), "bf16_torch_us": round(t_fb * 1e3, 2),
              "speedup_vs_bf16": round(t_fb / t_f, 3)}
    del g_f, g_fb
    log(f"[bench] layer flow at M={m16}: {flow16}")

    # The roofline entry: the mean device duration of gate_up over its 28 distinct weights at each
    # M of the step (the mix the graphs replay), each launch timed by HIP events bound to its
    # dispatch while the GPU is busy (kernel_ms_busy); algorithmic bytes averaged over the mix.
    dur_ms = statistics.mean(busy.values())
    g_bytes = statistics.mean(w8a16_bytes(m, 12288, 2048) for m in ms)
    achieved = g_bytes / (dur_ms * 1e-3) / 1e9
    traffic, traffic_src = committed_figure("w8a16_skinny_talker_stack_pmc.md", "traffic_bytes_per_launch")
    prof_us, prof_src = committed_figure("w8a16_skinny_roofline_kernel_trace.md", "avg_launch_us_profile")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": None if traffic is None else int(traffic), "traffic_source": traffic_src,
                "kernel": "w8a16_skinny_kernel (gate_up 12288x2048, M in 1,2,4,8)",
                "avg_launch_us": round(dur_ms * 1e3, 3), "bytes_per_launch": round(g_bytes),
                "avg_launch_us_per_m": {str(m): round(v * 1e3, 3) for m, v in busy.items()},
                "timing": (f"HIP events bound to each dispatch, {ROOFLINE_REPS} passes x 28 distinct weights per M, "
                           "each pass queued behind a spin kernel so the launches run back to back on a busy GPU"),
                # the same launches launched one by one onto an idle GPU
                "cold_avg_launch_us": round(cold_ms * 1e3, 3),
                # this run under rocprofv3 --kernel-trace: dispatches skip + 1 .. skip + take of each M
                "trace_window": {"skip": COLD_REPS * 28, "take": ROOFLINE_REPS * 28},
                "profile_avg_launch_us": prof_us, "profile_source": prof_src,
                "profile_frac": None if prof_us is None else round(g_bytes / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}

    result = {
        "metric": "int8 W-only decode GEMM HBM GB/s (% of peak) + linear-stack us/step, M=1..8",
        "value": round(total_bytes / (total_ms * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "pct_of_hbm_peak": round(100 * total_bytes / (total_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights per layer, N(0,1) bf16 activations)",
        "config": {"workload": "configs[1]: talker decode linear stack, 28 layers x {qkv,o,gate_up,down}, "
                               "int8 weight-only, one HIP graph per M", "layers": layers, "M": list(ms),
                   "int8_weight_bytes": int8_bytes, "parallelism": "none (1 GPU)",
                   "weight_policy": "stream (QTTS_ALGO_STREAM: non-temporal weight loads, as quantize_module picks "
                                    "for a submodel whose codes exceed the 256 MiB Infinity Cache)",
                   "layer_flow": "per_m.layer_flow_*: the same 28 layers in the decode step's data flow "
                                 "(RMSNorm+qkv, o+residual, RMSNorm+gate_up+SiLU, down+residual fused into the "
                                 "int8 GEMMs) against bf16 torch (hipBLASLt F.linear, F.rms_norm, F.silu, adds); "
                                 "o_proj reads a fixed synthetic attention output; layer_flow_m16: the same at "
                                 "16 rows (not part of the value)"},
        "per_m": per_m,
        "layer_flow_m16": flow16,
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (reference CPU path on a 2-layer sample)")
        result["cpu_baseline"] = cpu_baseline_w8a16(torch, stack, xs, ms, args.cpu_seconds, layers_sample=2)
        result["cpu_baseline"]["cpu_model"] = cpu_model()
    return result


def run_single_linear(args, torch, ops):
    """one gate_up linear, M=1, rotated over >= 512 MB of distinct weight copies."""
    copies = 24
    stack = make_stack(torch, ops, [("gate_up", 12288, 2048)], copies, keep_bf16=False)
    xs = make_inputs(torch, [2048], [1])
    st = ops.ALGO_STREAM  # 24 copies, 604 MB: past the Infinity Cache
    g = capture(torch, lambda: [ops.w8a16_gemm_strips(xs[(1, 2048)], e["qs"], e["n"], e["s"], None, st) for e in stack])
    t = time_graph(torch, g, args.steps, args.warmup)
    nbytes = copies * w8a16_bytes(1, 12288, 2048)
    dur_ms = kernel_ms(ops, [lambda e=e: ops.w8a16_gemm_strips(xs[(1, 2048)], e["qs"], e["n"], e["s"], None, st)
                             for e in stack], 2)
    per = w8a16_bytes(1, 12288, 2048)
    return {"metric": "int8 W-only GEMM HBM GB/s, single gate_up linear", "value": round(nbytes / (t * 1e-3) / 1e9, 1),
            "unit": "GB/s", "ms_per_step": round(t, 4), "steps": args.steps, "warmup": args.warmup, "n_gpus": 1,
            "config": {"workload": f"configs[0]: gate_up 12288x2048 M=1 x {copies} distinct copies per step"},
            "roofline": {"bound": "hbm", "achieved": round(per / (dur_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(per / (dur_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                         "traffic": None, "avg_launch_us": round(dur_ms * 1e3, 3)}}


def run_predictor(args, torch, ops):
    """code-predictor stack, 5 layers, 15 prefix passes (prefix 2..16) per frame, batch 1..8."""
    layers = 5
    stack = make_stack(torch, ops, PREDICTOR, layers, keep_bf16=True)
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    out = {}
    for b in (1, 8):
        ms = [b * p for p in range(2, 17)]
        xs = make_inputs(torch, [k for _, _, k in PREDICTOR], ms)
        g_q = capture(torch, lambda: [ops.w8a16_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"])
                                      for m in ms for e in stack])
        g_b = capture(torch, lambda: [torch.nn.functional.linear(xs[(m, e["k"])], e["w_bf16"])
                                      for m in ms for e in stack])
        t_q = time_graph(torch, g_q, args.steps, args.warmup)
        t_b = time_graph(torch, g_b, args.steps, args.warmup)
        out[f"batch{b}"] = {"frame_us": round(t_q * 1e3, 2), "pass_us": round(t_q * 1e3 / 15, 2),
                            "bf16_frame_us": round(t_b * 1e3, 2), "speedup_vs_bf16": round(t_b / t_q, 3),
                            "launches_per_frame": len(ms) * len(stack)}
        del g_q, g_b
    if args.calibrated:
        # The same frames through LinearBase layers converted by the calibrated int8 weight-only method
        # (per-bucket kernel choice; F.linear on the kept weight at the buckets where it won).
        from qtts_amd.layers.linear import LinearBase
        from qtts_amd.quant import calibrate
        from qtts_amd.quant.int8 import Int8WeightOnlyMethod
        calibrate.clear_cache()
        method = Int8WeightOnlyMethod(calibrate=True, calibration_batch=16,
                                      calibration_rows=(1, 2, 4, 8, 16, 32, 64, 128))
        layers_q = []
        for e in stack:
            lin = LinearBase(e["k"], e["n"], dtype=torch.bfloat16, device="cuda")
            lin.weight.data.copy_(e["w_bf16"])
            method.process_weights(lin)
            if method.applies_to(lin):
                lin.quant_method = method
            layers_q.append(lin)
        routed = sorted({f"{PREDICTOR[i % 4][0]}@{r}" for i, lin in enumerate(layers_q)
                         for r, a in getattr(lin, "quant_algos", {}).items() if a == calibrate.ALGO_REFERENCE_GEMM})
        for b in (1, 8):
            ms = [b * p for p in range(2, 17)]
            xs = make_inputs(torch, [k for _, _, k in PREDICTOR], ms)
            g_c = capture(torch, lambda: [lin(xs[(m, lin.in_features)]) for m in ms for lin in layers_q])
            t_c = time_graph(torch, g_c, args.steps, args.warmup)
            del g_c
            r = out[f"batch{b}"]
            r["calibrated_frame_us"] = round(t_c * 1e3, 2)
            r["calibrated_speedup_vs_bf16"] = round(r["bf16_frame_us"] / (t_c * 1e3), 3)
        out["calibrated_routes_to_f_linear"] = routed
        out["calibrated_converted"] = sum(method.applies_to(lin) for lin in layers_q)
    return {"metric": "code-predictor linear stack us/frame", "value": out["batch1"]["frame_us"], "unit": "us",
            "higher_is_better": False, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "config": {"workload": "configs[2]: 5 layers x 4 linears x 15 prefix passes, int8 weight-only"},
            "per_batch": out}


def run_prefill(args, torch, ops):
    """talker shapes at M in {64, 256, 1024, 2048}: the MFMA tile path and the prefill
    route (dequantize the int8 codes into a scratch buffer, then hipBLASLt) against hipBLASLt bf16
    on the resident bf16 weight; ``calibrated`` is the faster of the two int8 routes, the choice the
    calibration makes per prefill bucket.  ``streamed``: the tile kernel and hipBLASLt over the 28
    talker layers' distinct weights, one call each in a graph, as a prefill pass through the talker
    reads them (per call)."""
    from qtts_amd.quant import prefill
    layers = 28
    stack = make_stack(torch, ops, TALKER, layers, keep_bf16=True)
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    for e in stack[:4]:
        prefill.reserve(torch.device("cuda"), e["n"], e["k"], torch.bfloat16)
    res = {}
    for m in (64, 256, 1024, 2048):
        xs = make_inputs(torch, [2048, 6144], [m])
        for e in stack[:4]:
            x = xs[(m, e["k"])]
            fq = lambda e=e, x=x: ops.w8a16_gemm_strips(x, e["qs"], e["n"], e["s"])
            fd = lambda e=e, x=x: prefill.dequant_linear(e["qs"], ops.CODE_INT8, e["n"], e["k"], e["s"], x, None)
            fb = lambda e=e, x=x: torch.nn.functional.linear(x, e["w_bf16"])
            gs = {nm: capture(torch, lambda f=f: [f() for _ in range(10)]) for nm, f in (("q", fq), ("d", fd), ("b", fb))}
            tm = time_rounds(torch, gs, args.steps, args.warmup)
            del gs
            tq, td, tb = tm["q"] / 10, tm["d"] / 10, tm["b"] / 10
            same = [d for d in stack if d["name"] == e["name"]]
            ts = streamed_times(torch, args, {
                "q": [lambda d=d, x=x: ops.w8a16_gemm_strips(x, d["qs"], d["n"], d["s"]) for d in same],
                "b": [lambda d=d, x=x: torch.nn.functional.linear(x, d["w_bf16"]) for d in same]})
            fl = 2 * m * e["n"] * e["k"]
            tc = min(tq, td)
            key = f"M{m}_{e['name']}"
            res[key] = {"us": round(tq * 1e3, 2), "dequant_gemm_us": round(td * 1e3, 2),
                        "bf16_us": round(tb * 1e3, 2), "speedup": round(tb / tq, 3),
                        "calibrated": "tile" if tq <= td else "dequant_gemm",
                        "calibrated_speedup": round(tb / tc, 3),
                        "TFLOPs": round(fl / (tq * 1e-3) / 1e12, 1),
                        "mfma_util": round(fl / (tq * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                        "streamed_us": round(ts["q"] * 1e3, 2), "streamed_bf16_us": round(ts["b"] * 1e3, 2),
                        "streamed_speedup": round(ts["b"] / ts["q"], 3),
                        "streamed_mfma_util": round(fl / (ts["q"] * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}
            log(f"[bench] prefill {key}: {res[key]}")
    return {"metric": "prefill W8A16 MFMA utilisation / speedup vs bf16", "value": None, "unit": "TFLOP/s",
            "n_gpus": 1, "config": {"workload": "configs[3]: talker shapes, M in {64, 256, 1024, 2048}"},
            "shapes": res}


def streamed_times(torch, args, calls: dict) -> dict:
    """ms per call of each entry of ``calls`` (name -> list of callables, one per layer's distinct
    weight): one graph per name over the whole list, median of rotating rounds."""
    gs = {nm: capture(torch, lambda fs=fs: [f() for f in fs]) for nm, fs in calls.items()}
    tm = time_rounds(torch, gs, args.steps, args.warmup)
    del gs
    return {nm: tm[nm] / len(calls[nm]) for nm in calls}


def run_fp8(args, torch, ops):
    """fp8 W8A8 on the talker shapes, M in {1, 8, 256}, x with 1% outliers at 20 sigma.
    Each shape two ways: 10 calls on one weight in a graph (the weight resident in the caches, for
    every path), and ``streamed``: one call on each of the 28 talker layers' distinct weights in a
    graph, as a decode step streams them (per call; 28 x the weight is past the L2s and, but for qkv
    and o, past the Infinity Cache)."""
    layers = 28
    stack = make_stack(torch, ops, TALKER, layers, keep_bf16=True, fp8=True)
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    res = {}
    for m in (1, 8, 256):
        xs = make_inputs(torch, [2048, 6144], [m], outliers=True)
        for e in stack[:4]:
            fq = lambda e=e: ops.fp8_linear_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"])
            fb = lambda e=e: torch.nn.functional.linear(xs[(m, e["k"])], e["w_bf16"])
            tm = time_rounds(torch, {"q": capture(torch, lambda: [fq() for _ in range(10)]),
                                     "b": capture(torch, lambda: [fb() for _ in range(10)])}, args.steps, args.warmup)
            tq, tb = tm["q"] / 10, tm["b"] / 10
            same = [d for d in stack if d["name"] == e["name"]]
            ts = streamed_times(torch, args, {
                "q": [lambda d=d: ops.fp8_linear_strips(xs[(m, d["k"])], d["qs"], d["n"], d["s"], None, ops.DIV_DEVICE,
                                                        ops.ALGO_STREAM) for d in same],
                "b": [lambda d=d: torch.nn.functional.linear(xs[(m, d["k"])], d["w_bf16"]) for d in same]})
            nb = fp8_bytes(m, e["n"], e["k"])
            key = f"M{m}_{e['name']}"
            res[key] = {"us": round(tq * 1e3, 2), "bf16_us": round(tb * 1e3, 2), "speedup": round(tb / tq, 3),
                        "GBps": round(nb / (tq * 1e-3) / 1e9, 1), "streamed_us": round(ts["q"] * 1e3, 2),
                        "streamed_bf16_us": round(ts["b"] * 1e3, 2), "streamed_speedup": round(ts["b"] / ts["q"], 3),
                        "streamed_GBps": round(nb / (ts["q"] * 1e-3) / 1e9, 1)}
            log(f"[bench] fp8 {key}: {res[key]}")
    return {"metric": "fp8 W8A8 linear us and GB/s", "value": None, "unit": "GB/s", "n_gpus": 1,
            "config": {"workload": "configs[4]: talker shapes, fp8 W8A8, M in {1, 8, 256}; resident weights and "
                                   "the 28 layers' distinct weights streamed"}, "shapes": res}


def run_int8_w8a8(args, torch, ops):
    """int8 W8A8 (Int8Method) on the talker shapes, M in {1, 2, 4, 8, 64, 256, 1024}: the one-call
    linear (per-token quantization + int8 MFMA GEMM, one fused kernel for small decode batches)
    against hipBLASLt bf16 and the W8A16 kernel on the same int8 codes; each shape with its weight
    resident (10 calls on one weight) and ``streamed`` (one call on each of the 28 talker layers'
    distinct weights, as a decode step reads them)."""
    layers = 28
    stack = make_stack(torch, ops, TALKER, layers, keep_bf16=True, f32_scale=True)
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    res = {}
    for m in (1, 2, 4, 8, 64, 256, 1024):
        xs = make_inputs(torch, [2048, 6144], [m], outliers=True)
        for e in stack[:4]:
            x = xs[(m, e["k"])]
            s_b = e["s"].to(torch.bfloat16)
            fq = lambda e=e, x=x: ops.int8_linear_strips(x, e["qs"], e["n"], e["s"])
            fw = lambda e=e, x=x, s_b=s_b: ops.w8a16_gemm_strips(x, e["qs"], e["n"], s_b)
            fb = lambda e=e, x=x: torch.nn.functional.linear(x, e["w_bf16"])
            gs = {nm: capture(torch, lambda f=f: [f() for _ in range(10)]) for nm, f in (("q", fq), ("w", fw), ("b", fb))}
            tm = time_rounds(torch, gs, args.steps, args.warmup)
            del gs
            tq, tw, tb = tm["q"] / 10, tm["w"] / 10, tm["b"] / 10
            same = [d for d in stack if d["name"] == e["name"]]
            ts = streamed_times(torch, args, {
                "q": [lambda d=d: ops.int8_linear_strips(x, d["qs"], d["n"], d["s"], None, ops.DIV_DEVICE,
                                                         ops.ALGO_STREAM) for d in same],
                "b": [lambda d=d: torch.nn.functional.linear(x, d["w_bf16"]) for d in same]})
            fl = 2 * m * e["n"] * e["k"]
            nb = fp8_bytes(m, e["n"], e["k"])
            key = f"M{m}_{e['name']}"
            res[key] = {"us": round(tq * 1e3, 2), "w8a16_us": round(tw * 1e3, 2),
                        "bf16_us": round(tb * 1e3, 2), "speedup": round(tb / tq, 3),
                        "GBps": round(nb / (tq * 1e-3) / 1e9, 1),
                        "TOPs": round(fl / (tq * 1e-3) / 1e12, 1),
                        "int8_mfma_util": round(fl / (tq * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                        "streamed_us": round(ts["q"] * 1e3, 2), "streamed_bf16_us": round(ts["b"] * 1e3, 2),
                        "streamed_speedup": round(ts["b"] / ts["q"], 3)}
            log(f"[bench] int8 W8A8 {key}: {res[key]}")
    return {"metric": "int8 W8A8 linear us, GB/s and int8 MFMA utilisation", "value": None, "unit": "us",
            "n_gpus": 1, "config": {"workload": "talker shapes, int8 W8A8 (Int8Method), M in {1, 2, 4, 8, 64, 256, 1024}"},
            "shapes": res}


def run_fp8w_stack(args, torch, ops):
    """The configs[1] talker decode stack with fp8 (e4m3) weight-only weights (Fp8WeightOnlyMethod):
    the same 1.41 GB of 8-bit codes, converted with v_cvt_scalef32_pk_bf16_fp8 instead of from int8."""
    ms = (1, 2, 4, 8)
    layers = 28
    stack = []
    for layer in range(layers):
        for idx, (name, n, k) in enumerate(TALKER):
            g = torch.Generator(device="cuda").manual_seed(1000 + 16 * layer + idx)
            w = torch.randn(n, k, device="cuda", generator=g) * 0.02
            q, s = ops.pack_fp8(w)
            stack.append({"name": name, "n": n, "k": k, "qs": ops.fp8w_strips(q), "s": s})
            del w, q
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    xs = make_inputs(torch, [k for _, _, k in TALKER], ms)
    per_m = {}
    for m in ms:
        g_q = capture(torch, lambda m=m: [ops.fp8w_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"], None,
                                                               ops.ALGO_STREAM) for e in stack])
        t_q = time_graph(torch, g_q, args.steps, args.warmup)
        nbytes = sum(fp8_bytes(m, e["n"], e["k"]) for e in stack)
        per_m[str(m)] = {"stack_us": round(t_q * 1e3, 2), "GBps": round(nbytes / (t_q * 1e-3) / 1e9, 1),
                         "pct_of_hbm_peak": round(100 * nbytes / (t_q * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1)}
        del g_q
        log(f"[bench] fp8 weight-only M={m}: {per_m[str(m)]}")
    return {"metric": "fp8 weight-only decode linear-stack us/step and HBM GB/s", "value": None, "unit": "GB/s",
            "n_gpus": 1, "config": {"workload": "configs[1] shapes with e4m3 weight-only weights, 28 layers, "
                                                "one HIP graph per M", "M": list(ms)}, "per_m": per_m}


def run_mlp(args, torch, ops):
    """The talker MLP at decode (GatedMLP.forward, qtts/layers/activation.py:142-147): 28 layers of
    gate_up -> silu(gate) * up -> down, int8 weight-only, one HIP graph per M.  Three versions:
    torch's activation between the two int8 GEMMs (the reference's composition), the activation
    handed to the down projection (fused into its kernel at M <= 2, one activation kernel above),
    and bf16 hipBLASLt throughout."""
    import torch.nn.functional as F
    ms = (1, 2, 4, 8)
    layers = 28
    shapes = [s_ for s_ in TALKER if s_[0] in ("gate_up", "down")]
    stack = make_stack(torch, ops, shapes, layers, keep_bf16=True)
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    xs = make_inputs(torch, [2048], ms)
    pairs = [(stack[2 * i], stack[2 * i + 1]) for i in range(layers)]

    def act(gu):
        gate, up = gu.split([6144, 6144], dim=-1)
        return F.silu(gate) * up

    per_m = {}
    for m in ms:
        x = xs[(m, 2048)]
        st = ops.ALGO_STREAM  # 28 layers' MLPs, 1.06 GB: past the Infinity Cache
        composed = lambda: [ops.w8a16_gemm_strips(act(ops.w8a16_gemm_strips(x, g["qs"], g["n"], g["s"], None, st)),
                                                  d["qs"], d["n"], d["s"], None, st) for g, d in pairs]
        fused = lambda: [ops.w8a16_silu_mul_gemm_strips(ops.w8a16_gemm_strips(x, g["qs"], g["n"], g["s"], None, st),
                                                        d["qs"], d["n"], d["s"], None, st) for g, d in pairs]
        bf16 = lambda: [F.linear(act(F.linear(x, g["w_bf16"])), d["w_bf16"]) for g, d in pairs]
        t = {}
        for name, fn in (("composed", composed), ("fused", fused), ("bf16", bf16)):
            graph = capture(torch, fn)
            t[name] = time_graph(torch, graph, args.steps, args.warmup)
            del graph
        per_m[str(m)] = {"int8_torch_activation_us": round(t["composed"] * 1e3, 2),
                         "int8_fused_activation_us": round(t["fused"] * 1e3, 2),
                         "bf16_hipblaslt_us": round(t["bf16"] * 1e3, 2),
                         "fused_vs_composed": round(t["composed"] / t["fused"], 3),
                         "fused_vs_bf16": round(t["bf16"] / t["fused"], 3)}
        log(f"[bench] MLP M={m}: {per_m[str(m)]}")
    return {"metric": "talker MLP decode us/step (gate_up, silu*up, down; 28 layers)", "value": None, "unit": "us",
            "n_gpus": 1, "config": {"workload": "talker GatedMLP x 28 layers, int8 weight-only, one HIP graph per M",
                                    "M": list(ms)}, "per_m": per_m}


def layer_flows(torch, ops, stack, layers, eps=1e-6):
    """The talker decode step's linears with their data flow (qtts/models/talker.py:246-271) as
    callables of (h_in, attn): one fused kernel per linear (input_layernorm + qkv_proj, o_proj +
    residual, post_attention_layernorm + gate_up_proj + SiLU * mul, down_proj + residual), and
    bf16 torch (hipBLASLt F.linear, F.rms_norm, F.silu, adds).  Returns (flows, norm weights)."""
    import torch.nn.functional as F
    g = torch.Generator(device="cuda").manual_seed(5)
    w_in = [(1 + 0.1 * torch.randn(2048, generator=g, device="cuda")).to(torch.bfloat16) for _ in range(layers)]
    w_post = [(1 + 0.1 * torch.randn(2048, generator=g, device="cuda")).to(torch.bfloat16) for _ in range(layers)]
    ent = lambda layer, i: stack[4 * layer + i]  # noqa: E731  (qkv, o, gate_up, down)

    st = ops.ALGO_STREAM  # the talker's weight policy

    def fused(h_in, attn):
        qkv = ops.w8a16_fused_gemm_strips(h_in, ent(0, 0)["qs"], 4096, ent(0, 0)["s"], prologue=ops.PRO_RMS_NORM,
                                          norm_weight=w_in[0], eps=eps, algo=st)
        h = h_in
        for layer in range(layers):
            h1 = ops.w8a16_fused_gemm_strips(attn, ent(layer, 1)["qs"], 2048, ent(layer, 1)["s"], residual=h,
                                             algo=st)
            act = ops.w8a16_gate_up_silu_strips(h1, ent(layer, 2)["qs"], 12288, ent(layer, 2)["s"],
                                                prologue=ops.PRO_RMS_NORM, norm_weight=w_post[layer], eps=eps,
                                                algo=st)
            h = ops.w8a16_fused_gemm_strips(act, ent(layer, 3)["qs"], 2048, ent(layer, 3)["s"], residual=h1,
                                            algo=st)
            if layer + 1 < layers:
                qkv = ops.w8a16_fused_gemm_strips(h, ent(layer + 1, 0)["qs"], 4096, ent(layer + 1, 0)["s"],
                                                  prologue=ops.PRO_RMS_NORM, norm_weight=w_in[layer + 1], eps=eps,
                                                  algo=st)
        return h, qkv

    def bf16(h_in, attn):
        qkv = F.linear(F.rms_norm(h_in, (2048,), w_in[0], eps), ent(0, 0)["w_bf16"])
        h = h_in
        for layer in range(layers):
            h1 = h + F.linear(attn, ent(layer, 1)["w_bf16"])
            gu = F.linear(F.rms_norm(h1, (2048,), w_post[layer], eps), ent(layer, 2)["w_bf16"])
            gate, up = gu.split([6144, 6144], dim=-1)
            h = h1 + F.linear(F.silu(gate) * up, ent(layer, 3)["w_bf16"])
            if layer + 1 < layers:
                qkv = F.linear(F.rms_norm(h, (2048,), w_in[layer + 1], eps), ent(layer + 1, 0)["w_bf16"])
        return h, qkv

    return {"fused": fused, "bf16": bf16}, (w_in, w_post)


def run_traffic_probe(args, torch, ops):
    """Kernels for a rocprofv3 --pmc pass: a 256 MiB device copy (known bytes, the counters' scale),
    then the configs[1] stack's kernels, linear by linear (qkv, o, gate_up, down, each over its 28
    distinct weights at M = 1, 2, 4, 8, automatic kernel choice, the stack's streaming weight policy),
    launched eagerly so each dispatch carries its own counters."""
    ms = (1, 2, 4, 8)
    stack = make_stack(torch, ops, TALKER, 28, keep_bf16=False)
    ops.reserve_workspace(torch.device("cuda"), max(
        ops.workspace_bytes(ops.OP_W8A16, m, e["n"], e["k"]) for m in ms for e in stack[:4]))
    xs = make_inputs(torch, [k for _, _, k in TALKER], ms)
    src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    launches = {}
    for name, _, _ in TALKER:
        for m in ms:
            for e in stack:
                if e["name"] == name:
                    ops.w8a16_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"], None, ops.ALGO_STREAM)
                    launches[name] = launches.get(name, 0) + 1
    torch.cuda.synchronize()
    return {"probe": "traffic", "copy_bytes_each_way": src.numel() * 2, "launches": launches,
            "algorithmic_bytes_mean": {name: round(statistics.mean(w8a16_bytes(m, n, k) for m in ms))
                                       for name, n, k in TALKER}}


def run_prefill_probe(args, torch, ops):
    """Kernels for a rocprofv3 --pmc pass over the prefill tile kernel: configs[3]'s gate_up
    (12288 x 2048) at M = 1024, launched eagerly 8 times each (after 3 warm-up launches) as the automatic tile
    (8 waves, 128 x 256), as the 4-wave 128 x 128 tile (3 stages, no read-ahead, no split), and as F.linear on the
    bf16 weight (hipBLASLt)."""
    from qtts_amd import _lib
    ops.reserve_workspace(torch.device("cuda"), 64 << 20)
    n, k, m = 12288, 2048, 1024
    g = torch.Generator(device="cuda").manual_seed(1)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    q, s = ops.pack_int8(w, torch.bfloat16)
    qs = ops.to_strips(q)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    wide = _lib.algo_code(_lib.ALGO_TILE, 1, 3, _lib.tile_shape(128, 128))
    for fn in (lambda: ops.w8a16_gemm_strips(x, qs, n, s), lambda: ops.w8a16_gemm_strips(x, qs, n, s, None, wide),
               lambda: torch.nn.functional.linear(x, w)):
        for _ in range(3):  # warm-up: code objects loaded, weights resident
            fn()
        torch.cuda.synchronize()
        for _ in range(8):
            fn()
    torch.cuda.synchronize()
    return {"probe": "prefill", "shape": [m, n, k], "launches_each": 8}


def run_calibration(args, torch, ops):
    """The per-bucket calibration of the int8 weight-only method on the 8 talker and code-predictor
    shapes: at every row bucket the callers produce, the fastest quantized route (skinny / tile
    kernel configuration, or the prefill route) against F.linear on the bf16 weight (hipBLASLt),
    each timed as 10 calls in a HIP graph (qtts/quant/calibrate.py:40-63), and the layer verdict
    taken over the decode buckets.  A bucket where F.linear beat every quantized route is routed
    to F.linear on the kept weight: its served speedup is 1.0 (``route: "F.linear"``), and
    ``worst_served_speedup`` is the lowest over the buckets of converted layers as they run."""
    from qtts_amd.quant import calibrate
    from qtts_amd.quant.int8 import Int8WeightOnlyMethod, M_BUCKETS
    from qtts_amd.layers.linear import LinearBase
    calibrate.clear_cache()
    method = Int8WeightOnlyMethod(calibrate=True, calibration_batch=16)
    shapes = [("talker_" + nm, n, k) for nm, n, k in TALKER] + [("predictor_" + nm, n, k) for nm, n, k in PREDICTOR]
    out = {}
    worst = worst_served = None
    for name, n, k in shapes:
        lin = LinearBase(k, n, dtype=torch.bfloat16, device="cuda")
        g = torch.Generator(device="cuda").manual_seed(n + k)
        lin.weight.data.copy_((torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16))
        # the weight policy quantize_module picks: the talker's 1.41 GB streams, the predictor's 79 MB stays cached
        method.stream_weights = name.startswith("talker_")
        method.process_weights(lin)
        converted = method.applies_to(lin)
        algos = getattr(lin, "quant_algos", {})
        rep = method.calibration_report[(n, k)]
        rows = {}
        for b in M_BUCKETS:
            r = rep[b]
            if r["reference"] is None or r["best"] is None:
                rows[str(b)] = None
                continue
            t = r["timings"][r["best"]]
            ratio = r["reference"] / t
            routed_ref = algos.get(b) == calibrate.ALGO_REFERENCE_GEMM
            served = 1.0 if routed_ref or not converted else ratio
            rows[str(b)] = {"best": r["best"], "us": round(t * 1e6, 2), "bf16_us": round(r["reference"] * 1e6, 2),
                            "speedup": round(ratio, 3), "route": "F.linear" if routed_ref else r["best"],
                            "served_speedup": round(served, 3)}
            if worst is None or ratio < worst[0]:
                worst = (ratio, name, b)
            if converted and (worst_served is None or served < worst_served[0]):
                worst_served = (served, name, b)
        out[name] = {"converted": converted, "kept_weight": converted and lin.weight.numel() > 0, "buckets": rows}
        log(f"[bench] calibration {name}: " + ", ".join(
            f"{b}:{v['speedup'] if v else None}{'->F.linear' if v and v['route'] == 'F.linear' else ''}"
            for b, v in rows.items()))
    return {"probe": "calibration", "config": {"workload": "int8 weight-only per-bucket calibration, talker and "
                                                           "code-predictor shapes, buckets " + str(list(M_BUCKETS))},
            "worst_speedup": {"speedup": round(worst[0], 3), "shape": worst[1], "rows": worst[2]} if worst else None,
            "worst_served_speedup": ({"speedup": round(worst_served[0], 3), "shape": worst_served[1],
                                      "rows": worst_served[2]} if worst_served else None),
            "shapes": out}


def run_floor(args, torch, ops):
    """The floor of one kernel per linear on this GPU, next to the GEMM stack it bounds.

    * empty: 112 empty launches in one HIP graph (1, 128 and 768 workgroups of 4 waves):
      the cost of a launch boundary alone.
    * stream: the configs[1] stack's memory traffic without its arithmetic -- 28 layers x
      {qkv 8 MiB, o 4 MiB, gate_up 24 MiB, down 12 MiB} streamed by qtts_probe_stream from
      distinct slices of one 1.31 GiB buffer (5x the 256 MB Infinity Cache, so every byte
      comes from HBM), one HIP graph of 112 launches, for several (waves a workgroup, 1 KiB
      loads a wave) shapes; `best` takes the fastest shape per linear.
    * gemm: the configs[1] int8 W8A16 stack itself (automatic kernel choice) at M = 1 and 8.
    Per-launch durations by linear come from a rocprofv3 kernel trace of this mode."""
    sizes = [(name, n * k) for name, n, k in TALKER]
    layers = 28
    layer_bytes = sum(b for _, b in sizes)
    buf = torch.randint(-128, 128, (layers * layer_bytes,), dtype=torch.int8, device="cuda")
    sink = torch.empty(max(b for _, b in sizes) // 1024, dtype=torch.int32, device="cuda")
    offs = []
    for layer in range(layers):
        o = layer * layer_bytes
        for name, b in sizes:
            offs.append((name, o, b))
            o += b
    steps = max(5, args.steps)
    out = {"empty_us_per_launch": {}, "stream_stack_us": {}}
    for wgs in (1, 128, 768):
        g = capture(torch, lambda: [probe_empty(torch, wgs, 4) for _ in range(112)])
        out["empty_us_per_launch"][str(wgs)] = round(time_graph(torch, g, steps, args.warmup) * 1e3 / 112, 3)
        del g
    shapes = [(1, 16), (2, 8), (2, 16), (4, 4), (4, 8), (4, 16), (8, 2), (8, 4), (8, 8), (16, 1), (16, 2), (16, 4)]
    per_kind = {}
    for waves, loads in shapes:
        key = f"w{waves}_l{loads}"
        g = capture(torch, lambda: [probe_stream(torch, buf[o:o + b], b, waves, loads, sink) for _, o, b in offs])
        t = time_graph(torch, g, steps, args.warmup)
        out["stream_stack_us"][key] = round(t * 1e3, 2)
        del g
        # each linear's size alone: consecutive slices of that size over the whole buffer (28
        # slices of o would be only 112 MiB, resident in the Infinity Cache after one replay)
        for name, b in sizes:
            mine = [(o, b) for o in range(0, buf.numel() - b + 1, b)]
            g = capture(torch, lambda: [probe_stream(torch, buf[o:o + b], b, waves, loads, sink) for o, b in mine])
            t_k = time_graph(torch, g, steps, args.warmup) * 1e3 / len(mine)
            del g
            per_kind.setdefault(name, {})[key] = round(t_k, 3)
    out["stream_us_per_launch"] = per_kind
    best = {name: min(v.items(), key=lambda kv: kv[1]) for name, v in per_kind.items()}
    out["stream_best_shape"] = {name: kv[0] for name, kv in best.items()}
    plan = {name: tuple(int(t[1:]) for t in kv[0].split("_")) for name, kv in best.items()}
    g = capture(torch, lambda: [probe_stream(torch, buf[o:o + b], b, *plan[n_], sink) for n_, o, b in offs])
    out["stream_stack_best_us"] = round(time_graph(torch, g, steps, args.warmup) * 1e3, 2)
    del g, buf
    torch.cuda.empty_cache()

    stack = make_stack(torch, ops, TALKER, layers, keep_bf16=False)
    ops.reserve_workspace(torch.device("cuda"), max(
        ops.workspace_bytes(ops.OP_W8A16, m, e["n"], e["k"]) for m in (1, 8) for e in stack[:4]))
    xs = make_inputs(torch, [k for _, _, k in TALKER], (1, 8))
    out["gemm_stack_us"] = {}
    for m in (1, 8):
        g = capture(torch, lambda: [ops.w8a16_gemm_strips(xs[(m, e["k"])], e["qs"], e["n"], e["s"]) for e in stack])
        out["gemm_stack_us"][str(m)] = round(time_graph(torch, g, steps, args.warmup) * 1e3, 2)
        del g
    nbytes = sum(e["n"] * e["k"] for e in stack)
    out["weight_bytes"] = nbytes
    out["stream_best_GBps"] = round(nbytes / (out["stream_stack_best_us"] * 1e-6) / 1e9, 1)
    return {"probe": "floor", "config": {"workload": "configs[1] talker stack memory traffic (28 x 4 linears, "
                                                     "1.41 GB int8), streamed without arithmetic"}, **out}


PROBE_LIB = os.path.join(ROOT, "tts-inference_amd", "probe", "libqtts_probe.so")
_probe = None


def probe_lib():
    """The floor probes' own library (tts-inference_amd/probe/probe.hip), loaded once."""
    global _probe
    if _probe is None:
        import ctypes
        if not os.path.exists(PROBE_LIB):
            raise RuntimeError(f"{PROBE_LIB} is not built (python tts-inference_amd/build.py --probe)")
        lib = ctypes.CDLL(PROBE_LIB)
        p, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        lib.qtts_probe_stream.restype = i32
        lib.qtts_probe_stream.argtypes = [p, i64, i32, i32, p, p]
        lib.qtts_probe_empty.restype = i32
        lib.qtts_probe_empty.argtypes = [i64, i32, p]
        lib.qtts_probe_last_error.restype = ctypes.c_char_p
        _probe = lib
    return _probe


def _probe_check(status: int, what: str) -> None:
    if status != 0:
        msg = probe_lib().qtts_probe_last_error().decode()
        raise (ValueError if status == -1 else RuntimeError)(f"{what}: {msg}")


def probe_stream(torch, src, nbytes: int, waves: int, loads: int, sink) -> None:
    """Stream ``nbytes`` of ``src`` with the measurement kernel: ``waves`` waves a workgroup,
    ``loads`` 1 KiB loads a wave issued before any is used; each wave stores the xor of what it
    read to ``sink`` (int32, one word a wave)."""
    if not (src.is_cuda and sink.is_cuda and src.is_contiguous() and sink.is_contiguous()):
        raise ValueError("probe_stream takes contiguous device tensors")
    if sink.dtype != torch.int32 or sink.numel() * loads * 1024 < nbytes:
        raise ValueError("sink must be int32 with one word per wave")
    if src.numel() * src.element_size() < nbytes:
        raise ValueError("src is smaller than nbytes")
    st = torch.cuda.current_stream(src.device).cuda_stream
    _probe_check(probe_lib().qtts_probe_stream(src.data_ptr(), int(nbytes), int(waves), int(loads),
                                               sink.data_ptr(), st), "probe_stream")


def probe_empty(torch, workgroups: int, waves: int = 1) -> None:
    """Launch an empty kernel of ``workgroups`` x ``waves`` waves on the current stream."""
    _probe_check(probe_lib().qtts_probe_empty(int(workgroups), int(waves), torch.cuda.current_stream().cuda_stream),
                 "probe_empty")


def summarize_pmc(path: str) -> None:
    """Mean counter value per (kernel, grid, counter) from rocprofv3 --pmc CSV output under ``path``."""
    files = glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {path}")
    groups: dict[tuple[str, str, str], list[float]] = {}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                key = ((row.get("Kernel_Name") or "?")[:110], row.get("Grid_Size", "?"), row.get("Counter_Name", "?"))
                groups.setdefault(key, []).append(float(row.get("Counter_Value") or 0))
    print(f"{'dispatches':>10} {'mean':>14} {'min':>14} {'max':>14}  counter  grid  kernel")
    for (name, grid, ctr), v in sorted(groups.items(), key=lambda kv: (kv[0][2], -statistics.mean(kv[1]))):
        print(f"{len(v):10d} {statistics.mean(v):14.1f} {min(v):14.1f} {max(v):14.1f}  {ctr}  {grid}  {name}")


# ---------------------------------------------------------------------------------------
# rocprofv3 digest
# ---------------------------------------------------------------------------------------

def summarize_rocprof(path: str, match: str | None = None, first: int = 0, skip: int = 0) -> None:
    """Average duration per (kernel, grid) from rocprofv3 --kernel-trace CSV output under ``path``:
    the 40 heaviest rows, or with ``match`` (comma-separated name substrings) every matching row.
    With ``skip`` / ``first``, only dispatches skip + 1 .. skip + first of each (kernel, grid) in
    time order (the bench's roofline timing is the first thing to launch its kernel)."""
    files = glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {path}")
    groups: dict[tuple[str, str], list[tuple[float, float]]] = {}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                name = row.get("Kernel_Name") or row.get("KernelName") or "?"
                grid = "x".join(row.get(c, "") for c in ("Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z") if row.get(c))
                if not grid:
                    grid = row.get("Grid_Size", "?")
                start = float(row.get("Start_Timestamp") or row.get("BeginNs") or 0)
                end = float(row.get("End_Timestamp") or row.get("EndNs") or 0)
                groups.setdefault((name[:110], grid), []).append((start, (end - start) / 1e3))
    groups = {key: [d for _, d in (sorted(v)[skip:skip + first] if first else sorted(v)[skip:])]
              for key, v in groups.items()}
    groups = {key: v for key, v in groups.items() if v}
    rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))
    total = sum(sum(v) for _, v in rows)
    if match:
        keys = [t for t in match.split(",") if t]
        rows = [r for r in rows if any(t in r[0][0] for t in keys)]
    else:
        rows = rows[:40]
    print(f"{'calls':>7} {'avg_us':>9} {'min_us':>9} {'total_us':>11} {'pct':>6}  grid  kernel")
    for (name, grid), v in rows:
        print(f"{len(v):7d} {sum(v) / len(v):9.3f} {min(v):9.3f} {sum(v):11.1f} {100 * sum(v) / total:5.1f}%  "
              f"{grid}  {name}")


# ---------------------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=1, choices=range(5), help="index into BASELINE.json configs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="time budget of the CPU baseline sample")
    ap.add_argument("--summarize-rocprof", metavar="DIR")
    ap.add_argument("--summarize-match", metavar="NAMES", help="with --summarize-rocprof: every kernel whose "
                    "name holds one of these comma-separated substrings")
    ap.add_argument("--summarize-first", type=int, default=0, metavar="N",
                    help="with --summarize-rocprof: only the first N dispatches of each kernel (after the skipped)")
    ap.add_argument("--summarize-skip", type=int, default=0, metavar="S",
                    help="with --summarize-rocprof: leave out the first S dispatches of each kernel")
    ap.add_argument("--summarize-pmc", metavar="DIR", help="digest a rocprofv3 --pmc run")
    ap.add_argument("--int8-w8a8", action="store_true",
                    help="time the int8 W8A8 linear (Int8Method) on the talker shapes instead of a config")
    ap.add_argument("--fp8w", action="store_true",
                    help="time the configs[1] decode stack with fp8 weight-only weights instead of a config")
    ap.add_argument("--mlp", action="store_true",
                    help="time the talker MLP (gate_up, silu*up, down) with the activation fused into down")
    ap.add_argument("--calibrated", action="store_true",
                    help="with --config 2: also time the frames through layers converted by the calibrated method")
    ap.add_argument("--calibration", action="store_true",
                    help="print the int8 weight-only per-bucket calibration against hipBLASLt on the model shapes")
    ap.add_argument("--floor", action="store_true",
                    help="time the launch and streaming floor of one kernel per linear next to the configs[1] stack")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="launch only the kernels a rocprofv3 --pmc pass measures (a copy, then the stack's linears)")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="launch only the prefill kernels a rocprofv3 --pmc pass compares (tile kernel, hipBLASLt)")
    args = ap.parse_args()

    if args.summarize_rocprof:
        summarize_rocprof(args.summarize_rocprof, args.summarize_match, args.summarize_first, args.summarize_skip)
        return 0
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc)
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this path runs on one GPU: each GPU box has one MI355X and the quantized "
                                   "linear has no collective; run with --gpus 1 (multi-GPU sharding is "
                                   "described, not built)", "n_gpus": args.gpus}), flush=True)
        return 2

    import torch
    from qtts_amd import ops

    if not torch.cuda.is_available() or not ops.device_supported():
        raise SystemExit("bench.py needs a gfx950 GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    runner = {0: run_single_linear, 1: run_talker_stack, 2: run_predictor, 3: run_prefill, 4: run_fp8}[args.config]
    if args.traffic_probe:
        runner = run_traffic_probe
    if args.prefill_probe:
        runner = run_prefill_probe
    if args.floor:
        runner = run_floor
    if args.calibration:
        runner = run_calibration
    if args.int8_w8a8:
        runner = run_int8_w8a8
    if args.fp8w:
        runner = run_fp8w_stack
    if args.mlp:
        runner = run_mlp
    with torch.inference_mode():
        result = runner(args, torch, ops)
    result["device"] = torch.cuda.get_device_name()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
