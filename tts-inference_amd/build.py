"""Build libqtts_amd.so (gfx950) in-tree.

    python tts-inference_amd/build.py            # build
    python tts-inference_amd/build.py --verbose  # echo the hipcc lines
    python tts-inference_amd/build.py --sanitize # libqtts_amd_san.so: host code under ASan + UBSan
    python tts-inference_amd/build.py --probe    # probe/libqtts_probe.so: bench.py --floor's kernels

Each csrc/*.hip compiles to an object under _build/ (parallel), then one link
produces qtts_amd/libqtts_amd.so next to the Python package that loads it.
The shared library is the drop-in boundary (include/qtts_amd.h); nothing else
is built.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "qtts_amd", "libqtts_amd.so")
BUILD_DIR = os.path.join(HERE, "_build")
# The host-side checking build: argument validation, workspace sizing and launch
# configuration under AddressSanitizer and UndefinedBehaviorSanitizer (device code as
# usual; it never runs there).  tests/test_abi_sanitized.py loads it with the ASan runtime
# preloaded, in a process without torch.
SAN_OUT = os.path.join(HERE, "qtts_amd", "libqtts_amd_san.so")
SAN_BUILD_DIR = os.path.join(HERE, "_build_san")
SAN_FLAGS = [f for flag in ("-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
                            "-fno-omit-frame-pointer") for f in ("-Xarch_host", flag)]
SAN_LINK = ["-fsanitize=address,undefined", "-shared-libsan"]
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from forming v_pk_{add,mul,fma}_f32.  The host pass
# does not know the feature and says so; that warning is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The first 14 dwords of every kernel's arguments arrive in SGPRs at wave launch
    # (gfx950 kernarg preloading; the kernels order their parameters so what the first
    # loads need is among them), instead of a scalar load's round trip per workgroup.
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


# Per-file additions to the flags above (none at present).
FILE_FLAGS: dict[str, list[str]] = {}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False, sanitize: bool = False) -> str:
    cc = hipcc()
    out, build_dir = (SAN_OUT, SAN_BUILD_DIR) if sanitize else (OUT, BUILD_DIR)
    extra, link = (SAN_FLAGS, SAN_LINK) if sanitize else ([], [])
    os.makedirs(build_dir, exist_ok=True)
    sources = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = []
    cmds = []
    for src in sources:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    workers = min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = out + ".tmp"
    # -z defs: an entry point declared but not defined fails the link here, not the first import
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *link, "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


PROBE_SRC = os.path.join(HERE, "probe", "probe.hip")
PROBE_OUT = os.path.join(HERE, "probe", "libqtts_probe.so")


def build_probe(verbose: bool = False) -> str:
    """libqtts_probe.so: bench.py --floor's measurement kernels (probe/probe.hip), a library of
    their own so that nothing but the quantized linear is in libqtts_amd.so."""
    cc = hipcc()
    tmp = PROBE_OUT + ".tmp"
    _run([cc, *HIPCC_FLAGS, "-shared", "-Wl,-z,defs", PROBE_SRC, "-o", tmp], verbose)
    os.replace(tmp, PROBE_OUT)
    return PROBE_OUT


def sanitized_stale() -> bool:
    """True when libqtts_amd_san.so is missing or older than a source it is built from."""
    if not os.path.exists(SAN_OUT):
        return True
    built = os.path.getmtime(SAN_OUT)
    srcs = [os.path.join(CSRC, f) for f in os.listdir(CSRC)] + [os.path.join(ROOT, "include", "qtts_amd.h")]
    return any(os.path.getmtime(f) > built for f in srcs)


if __name__ == "__main__":
    if "--probe" in sys.argv:
        print(build_probe(verbose="--verbose" in sys.argv))
    else:
        print(build(verbose="--verbose" in sys.argv, sanitize="--sanitize" in sys.argv))
