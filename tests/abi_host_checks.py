"""Host-side ABI checks run against libqtts_amd_san.so (ASan + UBSan) by test_abi_sanitized.py.

Run in a child process with the ASan runtime preloaded and without torch: the ctypes
binding is loaded straight from its file, so nothing but the library is instrumented.
Every call here stays on the host: argument validation before any device use, the
workspace sizing and launch configuration of every op over a grid of shapes and algo
words, the strip layout's sizes, and the calls that reach the device query on a machine
without a GPU (they must fail cleanly).  Prints OK at the end; a sanitizer report aborts
the process first."""

import ctypes
import importlib.util
import itertools
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "tts-inference_amd", "qtts_amd")
spec = importlib.util.spec_from_file_location("qtts_lib_host", os.path.join(PKG, "_lib.py"))
lib = importlib.util.module_from_spec(spec)
spec.loader.exec_module(lib)
lib.LIB_PATH = os.path.join(PKG, "libqtts_amd_san.so")
L = lib.load()


def err() -> str:
    return L.qtts_last_error().decode()


# ---- argument validation (no device touched) ------------------------------------------
assert L.qtts_abi_version() == lib.ABI_VERSION
assert L.qtts_w8a16_gemm(None, 1, -1, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
assert "negative size" in err()
assert L.qtts_w8a16_gemm(None, 7, 1, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
assert L.qtts_w8a16_gemm(None, 1, 1, 16, 8, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
assert L.qtts_w8a16_gemm(None, 1, 1, 16, 16, None, 8, 16, None, 1, None, None, 8, 9, None, 0, None) == -1
assert L.qtts_w8a16_gemm(None, 1, 1 << 40, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
assert L.qtts_pack_int8_rowwise(None, 1, 4, 16, 16, None, None, 1, None, 5, None) == -1
assert L.qtts_pack_fp8_e4m3_rowwise(None, 1, 0, 16, 16, None, None, 0, None) == 0
assert L.qtts_quant_act_fp8_rows(None, 1, 2, 16, 8, None, None, 0, None) == -1
assert L.qtts_w8a8_fp8_gemm(None, None, 2, 32, 32, None, 4, 32, None, None, None, 9, 4, 0, None, 0, None) == -1
assert L.qtts_dequant_strips(None, 0, 16, 64, None, 1, None, 1, 32, None) == -1
assert L.qtts_dequant_strips(None, 5, 16, 64, None, 1, None, 1, 64, None) == -1
assert L.qtts_dequant_strips(None, 0, 0, 64, None, 1, None, 1, 64, None) == 0
long_name_errors = 0
for status in range(-8, 2):  # every status code's message path, including unknown ones
    L.qtts_w8a16_gemm(None, status, 1, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None)
    long_name_errors += len(err()) > 0
assert long_name_errors > 0

# ---- workspace sizing and launch configuration -----------------------------------------
A = lib.algo_code
ra = lib.TILE_READ_AHEAD
algos = [0, A(lib.ALGO_SKINNY), A(lib.ALGO_TILE), A(lib.ALGO_SKINNY_HALF), A(lib.ALGO_SKINNY_QUARTER)]
algos += [A(lib.ALGO_SKINNY, s, w, c) for s in (0, 1, 3, 8) for w in (0, 1, 4, 16) for c in (0, 4, 8, 12)]
algos += [A(lib.ALGO_TILE, s, p, shape) for s in (0, 1, 2, 5) for p in (0, 2, 3, 4, 6, 8, 3 | ra, 4 | ra, 8 | ra, 0x80, 0xC3, 0xC4, 0xC8)
          for shape in (0, 0x11, 0x12, 0x13, 0x21, 0x22, 0x23, 0x31, 0x32, 0x33, 0x15, 0x26, 0x37)]
algos += [255, 1 << 30, -1]  # malformed words: rejected, never crash
shapes = [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144), (4096, 1024), (1024, 2048), (6144, 1024),
          (1024, 3072), (40, 256), (1000, 512), (72, 768), (1, 64), (17, 4096), (16, 128), (100, 192)]
ms = [0, 1, 2, 3, 4, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 1000, 1024, 2048,
      4096, 65535, 1 << 20]
count = 0
for op in range(-1, 9):
    for (n, k), m, algo in itertools.product(shapes, ms, algos):
        ws = L.qtts_workspace_bytes(op, m, n, k, algo)
        assert ws >= -5, (op, m, n, k, algo, ws)
        count += 1
for op in range(8):
    for big in (1 << 31, 1 << 40, (1 << 62)):
        L.qtts_workspace_bytes(op, big, 4096, 2048, 0)
        L.qtts_workspace_bytes(op, 8, big, 2048, 0)
        L.qtts_workspace_bytes(op, 8, 4096, big, 0)

# ---- the strip layout's sizes ------------------------------------------------------------
for kind in (lib.STRIP_INT8, lib.STRIP_FP8, 2, -1):
    for n, k in itertools.product((0, 1, 15, 16, 17, 12288, 1 << 20), (0, 1, 16, 63, 64, 65, 128, 6144, 1 << 20)):
        v = L.qtts_strip_bytes(n, k, kind)
        assert v >= -5, (kind, n, k, v)
    for big in (1 << 31, 1 << 40, 1 << 62):
        L.qtts_strip_bytes(big, 4096, kind)
        L.qtts_strip_bytes(4096, big, kind)

# ---- calls that reach the device query with no GPU present: clean errors -------------------
assert L.qtts_device_supported(0) in (0, 1)
assert L.qtts_device_supported(-1) == 0 and L.qtts_device_supported(1 << 20) == 0
print(f"OK {count} workspace queries", flush=True)
