"""numpy front end of the CPU oracle (oracle/qtts_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product package
(tts-inference_amd/qtts_amd) never imports it.

Arrays are numpy; bf16 and fp16 tensors travel as their uint16 bit patterns.
Each function names the reference file:line it restates (see the C source for
the arithmetic).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

DT_F32, DT_BF16, DT_F16 = 0, 1, 2
DIV_DEVICE, DIV_IEEE = 0, 1

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_e4m3_encode.restype = ctypes.c_uint8
        L.oracle_e4m3_encode.argtypes = [ctypes.c_float]
        L.oracle_e4m3_decode.restype = ctypes.c_float
        L.oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.oracle_pack_int8_rowwise.restype = None
        L.oracle_pack_int8_rowwise.argtypes = [p, i32, i64, i64, i64, p, p, p, i32, i32]
        L.oracle_pack_fp8_rowwise.restype = None
        L.oracle_pack_fp8_rowwise.argtypes = [p, i32, i64, i64, i64, p, p, i32]
        L.oracle_quant_act_fp8.restype = None
        L.oracle_quant_act_fp8.argtypes = [p, i32, i64, i64, i64, p, p, i32]
        L.oracle_w8a16_ref_f64.restype = None
        L.oracle_w8a16_ref_f64.argtypes = [p, i64, i64, p, i64, p, p, p]
        L.oracle_w8a8_ref_f64.restype = None
        L.oracle_w8a8_ref_f64.argtypes = [p, p, i64, i64, p, i64, p, p, p]
        L.oracle_fp8w_ref_f64.restype = None
        L.oracle_fp8w_ref_f64.argtypes = [p, i64, i64, p, i64, p, p, p]
        L.oracle_silu_mul.restype = None
        L.oracle_silu_mul.argtypes = [p, i32, i64, i64, i64, p]
        L.oracle_rms_norm_f64.restype = None
        L.oracle_rms_norm_f64.argtypes = [p, i32, i64, i64, i64, p, ctypes.c_double, p]
        L.oracle_quant_act_int8.restype = None
        L.oracle_quant_act_int8.argtypes = [p, i32, i64, i64, i64, p, p, i32]
        L.oracle_int8_linear_out.restype = None
        L.oracle_int8_linear_out.argtypes = [p, p, i64, i64, p, i64, p, p, i32, p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _src(a: np.ndarray, dtype: int) -> np.ndarray:
    want = np.float32 if dtype == DT_F32 else np.uint16
    if a.dtype != want:
        raise TypeError(f"expected {want} array for dtype code {dtype}, got {a.dtype}")
    return np.ascontiguousarray(a)


# ---- scalar formats -------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (vectorised restatement of the C routine)."""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.ascontiguousarray(v, np.float32).ravel()
    out = np.fromiter((L.oracle_e4m3_encode(float(x)) for x in flat), np.uint8, flat.size)
    return out.reshape(np.shape(v))


def e4m3_decode_table() -> np.ndarray:
    L = lib()
    return np.array([L.oracle_e4m3_decode(c) for c in range(256)], np.float32)


# ---- packers (qtts/quant/int8.py:45-56, 105; qtts/quant/fp8.py:45-49) ----------

def pack_int8(w: np.ndarray, src_dtype: int = DT_F32, store_dtype: int = DT_BF16,
              div_mode: int = DIV_DEVICE):
    """Returns (q int8 [n,k], scale fp32 [n], stored scale [n] in store_dtype)."""
    w = _src(w, src_dtype)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s32 = np.empty(n, np.float32)
    store = np.empty(n, np.float32 if store_dtype == DT_F32 else np.uint16)
    lib().oracle_pack_int8_rowwise(_ptr(w), src_dtype, n, k, k, _ptr(q), _ptr(s32), _ptr(store),
                                   store_dtype, div_mode)
    return q, s32, store


def pack_fp8(w: np.ndarray, src_dtype: int = DT_F32, div_mode: int = DIV_DEVICE):
    """Returns (q e4m3 bits uint8 [n,k], scale fp32 [n])."""
    w = _src(w, src_dtype)
    n, k = w.shape
    q = np.empty((n, k), np.uint8)
    s = np.empty(n, np.float32)
    lib().oracle_pack_fp8_rowwise(_ptr(w), src_dtype, n, k, k, _ptr(q), _ptr(s), div_mode)
    return q, s


def quant_act_fp8(x: np.ndarray, x_dtype: int = DT_BF16, div_mode: int = DIV_DEVICE):
    """Per-token e4m3 activation quantization (qtts/quant/fp8.py:77-78)."""
    x = _src(x, x_dtype)
    m, k = x.shape
    qx = np.empty((m, k), np.uint8)
    sx = np.empty(m, np.float32)
    lib().oracle_quant_act_fp8(_ptr(x), x_dtype, m, k, k, _ptr(qx), _ptr(sx), div_mode)
    return qx, sx


# ---- GEMM oracles ---------------------------------------------------------------

def w8a16_ref(x_f32: np.ndarray, q: np.ndarray, scale_f32: np.ndarray,
              bias_f32: np.ndarray | None = None) -> np.ndarray:
    """fp64 dequantize-then-matmul: x @ (q * scale)^T + bias (qtts/quant/kernels.py:113-132)."""
    x = np.ascontiguousarray(x_f32, np.float32)
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(scale_f32, np.float32)
    b = None if bias_f32 is None else np.ascontiguousarray(bias_f32, np.float32)
    m, k = x.shape
    n = q.shape[0]
    y = np.empty((m, n), np.float64)
    lib().oracle_w8a16_ref_f64(_ptr(x), m, k, _ptr(q), n, _ptr(s), _ptr(b), _ptr(y))
    return y


def w8a8_ref(qx: np.ndarray, sx: np.ndarray, qw: np.ndarray, sw: np.ndarray,
             bias_f32: np.ndarray | None = None) -> np.ndarray:
    """fp64 (qx*sx) @ (qw*sw)^T + bias (qtts/quant/fp8.py:79-89)."""
    qx = np.ascontiguousarray(qx, np.uint8)
    qw = np.ascontiguousarray(qw, np.uint8)
    sx = np.ascontiguousarray(sx, np.float32)
    sw = np.ascontiguousarray(sw, np.float32)
    b = None if bias_f32 is None else np.ascontiguousarray(bias_f32, np.float32)
    m, k = qx.shape
    n = qw.shape[0]
    y = np.empty((m, n), np.float64)
    lib().oracle_w8a8_ref_f64(_ptr(qx), _ptr(sx), m, k, _ptr(qw), n, _ptr(sw), _ptr(b), _ptr(y))
    return y


def fp8w_ref(x_f32: np.ndarray, q: np.ndarray, scale_f32: np.ndarray,
             bias_f32: np.ndarray | None = None) -> np.ndarray:
    """fp64 x @ (e4m3(q) * scale)^T + bias: the fp8 weight-only formula (qtts/quant/fp8.py:92-123
    with qtts/quant/kernels.py:113-135).  q: e4m3 codes as uint8."""
    x = np.ascontiguousarray(x_f32, np.float32)
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(scale_f32, np.float32)
    b = None if bias_f32 is None else np.ascontiguousarray(bias_f32, np.float32)
    m, k = x.shape
    n = q.shape[0]
    y = np.empty((m, n), np.float64)
    lib().oracle_fp8w_ref_f64(_ptr(x), m, k, _ptr(q), n, _ptr(s), _ptr(b), _ptr(y))
    return y


def silu_mul(gate_up: np.ndarray, dtype: int = DT_BF16) -> np.ndarray:
    """``F.silu(gate) * up`` of a fused [m, 2k] gate_up (qtts/layers/activation.py:147)."""
    gu = _src(gate_up, dtype)
    m, k2 = gu.shape
    k = k2 // 2
    h = np.empty((m, k), np.float32 if dtype == DT_F32 else np.uint16)
    lib().oracle_silu_mul(_ptr(gu), dtype, m, k, k2, _ptr(h))
    return h


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float, dtype: int = DT_BF16) -> np.ndarray:
    """RMSNorm in fp64 (qtts/layers/norm.py:50-76): x * inv_rms * w, unrounded.  x and w in
    dtype's encoding (uint16 bits for bf16 / fp16)."""
    xs = _src(x, dtype)
    ws = np.ascontiguousarray(_src(np.atleast_2d(w), dtype)[0])
    m, k = xs.shape
    y = np.empty((m, k), np.float64)
    lib().oracle_rms_norm_f64(_ptr(xs), dtype, m, k, k, _ptr(ws), float(eps), _ptr(y))
    return y


def quant_act_int8(x: np.ndarray, x_dtype: int = DT_BF16, div_mode: int = DIV_DEVICE):
    """Per-token int8 activation quantization (qtts/quant/int8.py:147-149): (qx int8, sx fp32)."""
    x = _src(x, x_dtype)
    m, k = x.shape
    qx = np.empty((m, k), np.int8)
    sx = np.empty(m, np.float32)
    lib().oracle_quant_act_int8(_ptr(x), x_dtype, m, k, k, _ptr(qx), _ptr(sx), div_mode)
    return qx, sx


def int8_linear_out(qx: np.ndarray, sx: np.ndarray, qw: np.ndarray, sw: np.ndarray,
                    bias: np.ndarray | None = None, out_dtype: int = DT_BF16) -> np.ndarray:
    """torch._int_mm + the fp32 epilogue of Int8Method.apply (qtts/quant/int8.py:151-160).

    Exact: returns out_dtype bits (uint16) or fp32 values.  bias in out_dtype's encoding."""
    qx = np.ascontiguousarray(qx, np.int8)
    qw = np.ascontiguousarray(qw, np.int8)
    sx = np.ascontiguousarray(sx, np.float32)
    sw = np.ascontiguousarray(sw, np.float32)
    b = None if bias is None else _src(bias, out_dtype)
    m, k = qx.shape
    n = qw.shape[0]
    y = np.empty((m, n), np.float32 if out_dtype == DT_F32 else np.uint16)
    lib().oracle_int8_linear_out(_ptr(qx), _ptr(sx), m, k, _ptr(qw), n, _ptr(sw), _ptr(b), out_dtype, _ptr(y))
    return y


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / RMS(ref): the north-star tolerance measure (bar: <= 1e-2)."""
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    if rms == 0.0:
        return float(np.max(np.abs(np.asarray(y, np.float64) - ref))) if ref.size else 0.0
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / rms)
