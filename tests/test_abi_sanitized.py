"""The host side of the C ABI under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

libqtts_amd_san.so is the library with its host code instrumented (build.py --sanitize;
rebuilt here when a source is newer, about two minutes).  tests/abi_host_checks.py drives
its host-only paths -- argument validation, the workspace sizing and launch configuration
of every op over a grid of shapes and algo words, the strip sizes, the device query with
no GPU -- in a child process with the ASan runtime preloaded (python itself is not
instrumented) and without torch.  Any sanitizer report fails the test."""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(ROOT, "tts-inference_amd"))
import build as B  # noqa: E402


def _asan_runtime() -> str:
    clang = "/opt/rocm/llvm/bin/clang" if os.path.exists("/opt/rocm/llvm/bin/clang") else shutil.which("clang")
    if not clang:
        pytest.skip("no clang to locate the ASan runtime")
    path = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                          text=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip("the clang ASan runtime is not installed")
    return path


def test_host_abi_under_sanitizers():
    asan = _asan_runtime()
    try:
        B.hipcc()
    except RuntimeError:
        pytest.skip("no hipcc to build the sanitized library")
    if B.sanitized_stale():
        B.build(sanitize=True)
    env = dict(os.environ, LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([sys.executable, os.path.join(HERE, "abi_host_checks.py")], env=env, capture_output=True,
                       text=True, timeout=600)
    report = r.stdout[-2000:] + r.stderr[-6000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, report
    assert r.returncode == 0 and r.stdout.startswith("OK"), report
