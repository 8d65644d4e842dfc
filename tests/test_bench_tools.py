"""bench.py's measurement plumbing without a GPU: the rocprofv3 summarizer's dispatch window (the
roofline profile's average is taken over the same launches the line times), the figures the line
reads from the committed profiles, and the refusal of more than one GPU."""

from __future__ import annotations

import csv
import json
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _trace(path, rows):
    """A rocprofv3 --kernel-trace CSV with the columns the summarizer reads."""
    cols = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
    with open(os.path.join(path, "run_kernel_trace.csv"), "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(cols)
        for name, start_ns, dur_us, grid in rows:
            w.writerow(["KERNEL_DISPATCH", name, start_ns, start_ns + int(dur_us * 1000), grid, 1, 1])


def _table(capsys):
    out = capsys.readouterr().out.splitlines()
    assert out[0].split()[:2] == ["calls", "avg_us"]
    return [line.split() for line in out[1:]]


def test_summarizer_takes_the_dispatch_window_in_time_order(tmp_path, capsys):
    # kernel A: 10 dispatches of 1..10 us, written out of time order; kernel B and a second grid of A
    rows = [("kernA", 1000 * (10 - i), float(10 - i), 4096) for i in range(10)]
    rows += [("kernB", 50_000 + 1000 * i, 100.0, 64) for i in range(3)]
    rows += [("kernA", 90_000 + 1000 * i, 50.0, 8192) for i in range(2)]
    _trace(tmp_path, rows)
    bench.summarize_rocprof(str(tmp_path), match="kernA", skip=2, first=3)
    table = _table(capsys)
    by_grid = {r[5]: r for r in table}
    a = by_grid["4096x1x1"]
    assert int(a[0]) == 3 and float(a[1]) == 4.0 and float(a[2]) == 3.0  # dispatches 3, 4, 5
    assert "64x1x1" not in by_grid  # kernB filtered out by the match
    assert "8192x1x1" not in by_grid  # two dispatches of that grid, none past the skip of 2
    bench.summarize_rocprof(str(tmp_path))
    table = _table(capsys)
    assert table[0][-1] == "kernB" and int(table[0][0]) == 3  # heaviest first (300 us)


def test_line_reads_the_committed_profiles():
    us, src = bench.committed_figure("w8a16_skinny_roofline_kernel_trace.md", "avg_launch_us_profile")
    assert src == "profiles/w8a16_skinny_roofline_kernel_trace.md" and 3.0 < us < 20.0
    traffic, src = bench.committed_figure("w8a16_skinny_talker_stack_pmc.md", "traffic_bytes_per_launch")
    # gate_up's algorithmic bytes a launch, mean over M = 1, 2, 4, 8; the counted traffic is within a few %
    algo = sum(bench.w8a16_bytes(m, 12288, 2048) for m in (1, 2, 4, 8)) / 4
    assert src is not None and 0.95 < traffic / algo < 1.10
    assert bench.committed_figure("no_such_profile.md", "avg_launch_us_profile") == (None, None)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
