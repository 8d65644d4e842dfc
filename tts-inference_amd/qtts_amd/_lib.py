"""ctypes binding of libqtts_amd.so (the C ABI declared in include/qtts_amd.h).

The library is loaded from this package directory.  There is no fallback: if the
library is missing or the device is not a gfx950, calls raise.  Status codes map
to the exceptions the reference raises for the same conditions
(qtts/quant/kernels.py:159-160 ValueError on a shape mismatch; qtts/quant/int8.py:71-73
and qtts/quant/base.py:122-124 RuntimeError when the kernel or device is missing;
qtts/quant/fp8.py:115-123 NotImplementedError).
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
#: QTTS_AMD_LIB names another build of the same library to load instead (e.g. the
#: sanitized one of build.py --sanitize, run with the ASan runtime preloaded)
LIB_PATH = os.environ.get("QTTS_AMD_LIB") or os.path.join(HERE, "libqtts_amd.so")

ABI_VERSION = 1

# qtts_status
OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED = -2
ERR_NOT_IMPLEMENTED = -3
ERR_HIP = -4
ERR_WORKSPACE = -5
#: bytes of the library-owned workspace of qtts_fp8_linear_strips_static (QTTS_STATIC_SCRATCH_BYTES)
STATIC_SCRATCH_BYTES = 32 << 20

# qtts_dtype
F32, BF16, F16 = 0, 1, 2
# qtts_div_mode
DIV_DEVICE, DIV_IEEE = 0, 1
# qtts_algo (bits 0-7); bits 8-15 split count, bits 16-23 waves per workgroup,
# bits 24-31 chunks per wave of the skinny kernels (0 = automatic); for the tile
# kernels bits 16-21 the stage count, bit 22 read-ahead, bit 23 two chunks a stage, bits 24-30 the tile shape
#: read-ahead flag of a tile kernel's stage field (the `waves` argument of algo_code)
TILE_READ_AHEAD = 64
#: two 64-column chunks a stage (W8A16 / fp8 weight-only 32 x 64 tiles of 4 waves, 3 or 4 stages with read-ahead)
TILE_TWO_CHUNKS = 128


def tile_shape(bm: int, bn: int, waves: int = 4, grid2: bool = False) -> int:
    """A tile kernel's shape code (the `cpw` argument of algo_code): BM x BN output tiles, 4 or
    8 waves a workgroup on a 1 x waves grid (or 2 x waves/2 with ``grid2``).  BM = 256 and
    BN = 384 only with 8 waves."""
    if (bm not in (32, 64, 128, 256) or bn not in (64, 128, 256, 384) or waves not in (4, 8)
            or (bm == 256 and waves != 8) or (bn == 384 and waves != 8)):
        raise ValueError(f"no tile shape {bm}x{bn} with {waves} waves")
    return {32: 1, 64: 2, 128: 3, 256: 0}[bm] | (4 if grid2 else 0) | (8 if waves == 8 else 0) | (
        {64: 1, 128: 2, 256: 3, 384: 4}[bn] << 4)
ALGO_AUTO, ALGO_SKINNY, ALGO_TILE = 0, 1, 2
#: the skinny kernel over row-split strips: 2 (HALF) or 4 (QUARTER) workgroups per 16-row strip
ALGO_SKINNY_HALF, ALGO_SKINNY_QUARTER = 3, 4
#: QTTS_ALGO_STREAM: OR-ed into any algo, the decode kernels load the weight non-temporally
#: (for weights read once a step and too large to stay cached between steps); same bits out.
ALGO_STREAM = 0x80
# qtts_op
OP_W8A16, OP_W8A8_FP8, OP_FP8_LINEAR, OP_W8A8_INT8, OP_INT8_LINEAR, OP_FP8W, OP_W8A16_SILU, OP_W8A16_FUSED = range(8)
# qtts_prologue
PRO_NONE, PRO_SILU_MUL, PRO_RMS_NORM = 0, 1, 2
# qtts_strip_kind
STRIP_INT8, STRIP_FP8 = 0, 1
# qtts_code_kind
CODE_INT8, CODE_E4M3 = 0, 1

EXPORTS = (
    "qtts_abi_version",
    "qtts_last_error",
    "qtts_device_supported",
    "qtts_workspace_bytes",
    "qtts_pack_int8_rowwise",
    "qtts_pack_fp8_e4m3_rowwise",
    "qtts_w8a16_gemm",
    "qtts_quant_act_fp8_rows",
    "qtts_w8a8_fp8_gemm",
    "qtts_fp8_linear",
    "qtts_strip_bytes",
    "qtts_to_strips",
    "qtts_from_strips",
    "qtts_dequant_strips",
    "qtts_w8a16_gemm_strips",
    "qtts_w8a8_fp8_gemm_strips",
    "qtts_fp8_linear_strips",
    "qtts_fp8_linear_strips_static",
    "qtts_quant_act_int8_rows",
    "qtts_w8a8_int8_gemm",
    "qtts_int8_linear",
    "qtts_w8a8_int8_gemm_strips",
    "qtts_int8_linear_strips",
    "qtts_fp8w_gemm_strips",
    "qtts_silu_mul",
    "qtts_w8a16_silu_mul_gemm_strips",
    "qtts_rms_norm",
    "qtts_w8a16_fused_gemm_strips",
    "qtts_w8a16_gate_up_silu_strips",
    "qtts_kernel_timer_begin",
    "qtts_kernel_timer_end",
)


def algo_code(family: int = ALGO_AUTO, splits: int = 0, waves: int = 0, cpw: int = 0) -> int:
    if not (0 <= splits < 256 and 0 <= waves < 256 and 0 <= cpw < 128):
        raise ValueError("splits and waves must be in [0, 255], cpw in [0, 127]")
    return family | (splits << 8) | (waves << 16) | (cpw << 24)


class QttsError(RuntimeError):
    pass


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and type the shared library (once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python tts-inference_amd/build.py` "
                "(hipcc, --offload-arch=gfx950)"
            )
        L = ctypes.CDLL(LIB_PATH)
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.qtts_abi_version.restype = i32
        L.qtts_abi_version.argtypes = []
        L.qtts_last_error.restype = ctypes.c_char_p
        L.qtts_last_error.argtypes = []
        L.qtts_device_supported.restype = i32
        L.qtts_device_supported.argtypes = [i32]
        L.qtts_workspace_bytes.restype = i64
        L.qtts_workspace_bytes.argtypes = [i32, i64, i64, i64, i32]
        L.qtts_pack_int8_rowwise.restype = i32
        L.qtts_pack_int8_rowwise.argtypes = [p, i32, i64, i64, i64, p, p, i32, p, i32, p]
        L.qtts_pack_fp8_e4m3_rowwise.restype = i32
        L.qtts_pack_fp8_e4m3_rowwise.argtypes = [p, i32, i64, i64, i64, p, p, i32, p]
        L.qtts_w8a16_gemm.restype = i32
        L.qtts_w8a16_gemm.argtypes = [p, i32, i64, i64, i64, p, i64, i64, p, i32, p, p, i64, i32, p, i64, p]
        L.qtts_quant_act_fp8_rows.restype = i32
        L.qtts_quant_act_fp8_rows.argtypes = [p, i32, i64, i64, i64, p, p, i32, p]
        L.qtts_w8a8_fp8_gemm.restype = i32
        L.qtts_w8a8_fp8_gemm.argtypes = [p, p, i64, i64, i64, p, i64, i64, p, p, p, i32, i64, i32, p, i64, p]
        L.qtts_fp8_linear.restype = i32
        L.qtts_fp8_linear.argtypes = [p, i32, i64, i64, i64, p, i64, i64, p, p, p, i64, i32, i32, p, i64, p]
        L.qtts_strip_bytes.restype = i64
        L.qtts_strip_bytes.argtypes = [i64, i64, i32]
        L.qtts_to_strips.restype = i32
        L.qtts_to_strips.argtypes = [p, i64, i64, i64, i32, p, p]
        L.qtts_from_strips.restype = i32
        L.qtts_from_strips.argtypes = [p, i64, i64, i32, p, i64, p]
        L.qtts_dequant_strips.restype = i32
        L.qtts_dequant_strips.argtypes = [p, i32, i64, i64, p, i32, p, i32, i64, p]
        L.qtts_w8a16_gemm_strips.restype = i32
        L.qtts_w8a16_gemm_strips.argtypes = [p, i32, i64, i64, i64, p, i64, p, i32, p, p, i64, i32, p, i64, p]
        L.qtts_w8a8_fp8_gemm_strips.restype = i32
        L.qtts_w8a8_fp8_gemm_strips.argtypes = [p, p, i64, i64, i64, p, i64, p, p, p, i32, i64, i32, p, i64, p]
        L.qtts_fp8_linear_strips.restype = i32
        L.qtts_fp8_linear_strips.argtypes = [p, i32, i64, i64, i64, p, i64, p, p, p, i64, i32, i32, p, i64, p]
        L.qtts_fp8_linear_strips_static.restype = i32
        L.qtts_fp8_linear_strips_static.argtypes = [p, i32, i64, i64, i64, p, i64, p, p, p, i64, i32, i32, p]
        L.qtts_quant_act_int8_rows.restype = i32
        L.qtts_quant_act_int8_rows.argtypes = [p, i32, i64, i64, i64, p, p, i32, p]
        L.qtts_w8a8_int8_gemm.restype = i32
        L.qtts_w8a8_int8_gemm.argtypes = [p, p, i64, i64, i64, p, i64, i64, p, p, p, i32, i64, i32, p, i64, p]
        L.qtts_int8_linear.restype = i32
        L.qtts_int8_linear.argtypes = [p, i32, i64, i64, i64, p, i64, i64, p, p, p, i64, i32, i32, p, i64, p]
        L.qtts_w8a8_int8_gemm_strips.restype = i32
        L.qtts_w8a8_int8_gemm_strips.argtypes = [p, p, i64, i64, i64, p, i64, p, p, p, i32, i64, i32, p, i64, p]
        L.qtts_int8_linear_strips.restype = i32
        L.qtts_int8_linear_strips.argtypes = [p, i32, i64, i64, i64, p, i64, p, p, p, i64, i32, i32, p, i64, p]
        L.qtts_fp8w_gemm_strips.restype = i32
        L.qtts_fp8w_gemm_strips.argtypes = [p, i32, i64, i64, i64, p, i64, p, p, p, i64, i32, p, i64, p]
        L.qtts_silu_mul.restype = i32
        L.qtts_silu_mul.argtypes = [p, i32, i64, i64, i64, p, i64, p]
        L.qtts_w8a16_silu_mul_gemm_strips.restype = i32
        L.qtts_w8a16_silu_mul_gemm_strips.argtypes = [p, i32, i64, i64, i64, p, i64, p, i32, p, p, i64, i32, p, i64, p]
        L.qtts_rms_norm.restype = i32
        L.qtts_rms_norm.argtypes = [p, i32, i64, i64, i64, p, ctypes.c_float, p, i64, p]
        L.qtts_w8a16_fused_gemm_strips.restype = i32
        L.qtts_w8a16_fused_gemm_strips.argtypes = [p, i32, i64, i64, i64, i32, p, ctypes.c_float, p, i64, p, i32, p,
                                                   p, i64, p, i64, i32, p, i64, p]
        L.qtts_w8a16_gate_up_silu_strips.restype = i32
        L.qtts_w8a16_gate_up_silu_strips.argtypes = [p, i32, i64, i64, i64, i32, p, ctypes.c_float, p, i64, p, i32,
                                                     p, p, i64, i32, p, i64, p]
        L.qtts_kernel_timer_begin.restype = i32
        L.qtts_kernel_timer_begin.argtypes = [i32]
        L.qtts_kernel_timer_end.restype = i32
        L.qtts_kernel_timer_end.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(i64),
                                            ctypes.POINTER(i64)]
        version = L.qtts_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libqtts_amd ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = L
    return _lib


def last_error() -> str:
    return load().qtts_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    """Raise the exception the reference raises for the same condition."""
    if status == OK:
        return
    msg = f"{what}: {last_error()}"
    if status in (ERR_INVALID_ARGUMENT, ERR_WORKSPACE):
        raise ValueError(msg)
    if status == ERR_NOT_IMPLEMENTED:
        raise NotImplementedError(msg)
    raise QttsError(msg)


def device_supported(device: int) -> bool:
    return load().qtts_device_supported(int(device)) == 1
