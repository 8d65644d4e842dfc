"""The C ABI without a GPU: the library loads, exports every symbol the header
declares, validates arguments before touching a device, and maps status codes to
the reference's exception types."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from qtts_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qtts_amd.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(qtts_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_exported_set():
    declared = _declared()
    assert declared == sorted(_lib.EXPORTS), declared


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(L, name), f"{name} declared in include/qtts_amd.h but not exported"


def test_abi_version_and_enums_match_header():
    L = _lib.load()
    assert L.qtts_abi_version() == _lib.ABI_VERSION
    text = open(HEADER).read()
    assert f"#define QTTS_ABI_VERSION {_lib.ABI_VERSION}" in text
    for name, value in (("QTTS_ERR_INVALID_ARGUMENT", -1), ("QTTS_ERR_UNSUPPORTED", -2),
                        ("QTTS_ERR_NOT_IMPLEMENTED", -3), ("QTTS_ERR_HIP", -4), ("QTTS_ERR_WORKSPACE", -5),
                        ("QTTS_F32", 0), ("QTTS_BF16", 1), ("QTTS_F16", 2), ("QTTS_DIV_DEVICE", 0),
                        ("QTTS_DIV_IEEE", 1), ("QTTS_ALGO_AUTO", 0), ("QTTS_ALGO_SKINNY", 1), ("QTTS_ALGO_TILE", 2)):
        assert re.search(rf"\b{name}\s*=\s*{value}\b", text), name


def test_argument_validation_precedes_device_use():
    """Bad arguments are rejected with INVALID_ARGUMENT before any HIP call (works with no GPU)."""
    L = _lib.load()
    assert L.qtts_w8a16_gemm(None, 1, -1, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
    assert "negative size" in _lib.last_error()
    assert L.qtts_w8a16_gemm(None, 7, 1, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
    assert L.qtts_w8a16_gemm(None, 1, 1, 16, 8, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
    assert "leading dimension" in _lib.last_error()
    assert L.qtts_w8a16_gemm(None, 1, 1, 16, 16, None, 8, 16, None, 1, None, None, 8, 9, None, 0, None) == -1
    assert L.qtts_pack_int8_rowwise(None, 1, 4, 16, 16, None, None, 1, None, 5, None) == -1
    assert L.qtts_quant_act_fp8_rows(None, 1, 2, 16, 8, None, None, 0, None) == -1
    assert L.qtts_w8a8_fp8_gemm(None, None, 2, 32, 32, None, 4, 32, None, None, None, 9, 4, 0, None, 0, None) == -1
    # empty problems are a no-op success, with no device needed
    assert L.qtts_w8a16_gemm(None, 1, 0, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == 0
    assert L.qtts_pack_fp8_e4m3_rowwise(None, 1, 0, 16, 16, None, None, 0, None) == 0


def test_dequant_strips_argument_checks():
    """qtts_dequant_strips validates sizes, code kind, dtypes and pointers before any device use."""
    L = _lib.load()
    assert L.qtts_dequant_strips(None, 0, 16, 64, None, 1, None, 1, 32, None) == -1  # ldw < k
    assert "bad sizes" in _lib.last_error()
    assert L.qtts_dequant_strips(None, 5, 16, 64, None, 1, None, 1, 64, None) == -1
    assert "code kind" in _lib.last_error()
    assert L.qtts_dequant_strips(None, 1, 16, 64, None, 1, None, 7, 64, None) == -1
    assert "dtype" in _lib.last_error()
    assert L.qtts_dequant_strips(None, 0, 16, 64, None, 1, None, 1, 64, None) == -1
    assert "null pointer" in _lib.last_error()
    assert L.qtts_dequant_strips(None, 0, 0, 64, None, 1, None, 1, 64, None) == 0  # empty: no device needed
    assert re.search(r"\bQTTS_CODE_E4M3\s*=\s*1\b", open(HEADER).read())
    assert (_lib.CODE_INT8, _lib.CODE_E4M3) == (0, 1)


def test_null_pointers_rejected():
    L = _lib.load()
    assert L.qtts_w8a16_gemm(None, 1, 2, 16, 16, None, 8, 16, None, 1, None, None, 8, 0, None, 0, None) == -1
    assert "null pointer" in _lib.last_error()


def test_workspace_query():
    L = _lib.load()
    # one split needs no workspace; forced splits need the counter block plus partials
    assert L.qtts_workspace_bytes(_lib.OP_W8A16, 4, 2048, 2048, _lib.algo_code(_lib.ALGO_SKINNY, 1)) == 0
    n = L.qtts_workspace_bytes(_lib.OP_W8A16, 4, 2048, 2048, _lib.algo_code(_lib.ALGO_SKINNY, 4))
    assert n == 65536 + (2048 // 16) * 4 * 64 * 16
    assert L.qtts_workspace_bytes(_lib.OP_W8A16, 0, 2048, 2048, 0) == 0
    assert L.qtts_workspace_bytes(9, 4, 2048, 2048, 0) == -1
    assert L.qtts_workspace_bytes(_lib.OP_FP8_LINEAR, 8, 2048, 2048, 0) >= 8 * 2048 + 32
    assert L.qtts_workspace_bytes(_lib.OP_W8A16, 4, 2048, 0, 0) >= 0  # K = 0 is a valid query


def test_weight_policy_flag_is_outside_the_kernel_choice():
    """QTTS_ALGO_STREAM changes how weights are loaded, never what runs or what it needs."""
    L = _lib.load()
    assert re.search(r"#define QTTS_ALGO_STREAM 0x80\b", open(HEADER).read())
    assert _lib.ALGO_STREAM == 0x80
    for op in (_lib.OP_W8A16, _lib.OP_W8A16_FUSED, _lib.OP_W8A16_SILU, _lib.OP_FP8W, _lib.OP_FP8_LINEAR,
               _lib.OP_INT8_LINEAR, _lib.OP_W8A8_FP8, _lib.OP_W8A8_INT8):
        for m in (1, 8, 16, 64):
            for algo in (0, _lib.algo_code(_lib.ALGO_SKINNY, 4), _lib.algo_code(_lib.ALGO_TILE, 2)):
                assert (L.qtts_workspace_bytes(op, m, 4096, 2048, algo | _lib.ALGO_STREAM) ==
                        L.qtts_workspace_bytes(op, m, 4096, 2048, algo)), (op, m, algo)


def test_strip_bytes():
    L = _lib.load()
    assert L.qtts_strip_bytes(2048, 2048, _lib.STRIP_INT8) == 2048 * 2048
    assert L.qtts_strip_bytes(17, 100, _lib.STRIP_INT8) == 2 * 2 * 1024
    assert L.qtts_strip_bytes(17, 100, _lib.STRIP_FP8) == 2 * 1 * 2048
    assert L.qtts_strip_bytes(0, 100, _lib.STRIP_FP8) == 0
    assert L.qtts_strip_bytes(16, 16, 7) == -1


def test_device_supported_without_gpu_is_false():
    L = _lib.load()
    assert L.qtts_device_supported(-1) == 0
    assert L.qtts_device_supported(10_000) == 0


def test_status_mapping():
    _lib.check(_lib.OK, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_WORKSPACE, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.ERR_NOT_IMPLEMENTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_HIP, "x")


def test_algo_code_packing():
    assert _lib.algo_code(_lib.ALGO_SKINNY, 4, 8) == 1 | (4 << 8) | (8 << 16)
    with pytest.raises(ValueError):
        _lib.algo_code(_lib.ALGO_TILE, 300)


def test_kernel_timer_argument_checks():
    L = _lib.load()
    assert L.qtts_kernel_timer_begin(0) == _lib.ERR_INVALID_ARGUMENT
    assert L.qtts_kernel_timer_begin((1 << 20) + 1) == _lib.ERR_INVALID_ARGUMENT
    ms, n, u = ctypes.c_double(), ctypes.c_int64(), ctypes.c_int64()
    assert L.qtts_kernel_timer_end(ctypes.byref(ms), ctypes.byref(n), ctypes.byref(u)) == _lib.ERR_INVALID_ARGUMENT
    assert "not armed" in _lib.last_error()
    assert L.qtts_kernel_timer_end(None, ctypes.byref(n), ctypes.byref(u)) == _lib.ERR_INVALID_ARGUMENT


def test_probe_library_is_separate():
    """The floor probes live in their own library (bench.py --floor), not in libqtts_amd.so, and
    reject bad shapes before any device use."""
    L = ctypes.CDLL(_lib.LIB_PATH)
    assert not hasattr(L, "qtts_probe_stream") and not hasattr(L, "qtts_probe_empty")
    import bench
    if not os.path.exists(bench.PROBE_LIB):
        pytest.skip("libqtts_probe.so not built")
    P = bench.probe_lib()
    src, sink = 1 << 20, 1 << 21  # aligned stand-in addresses: never dereferenced on a rejected call
    assert P.qtts_probe_stream(None, 4096, 4, 1, sink, None) == -1
    assert P.qtts_probe_stream(src + 8, 4096, 4, 1, sink, None) == -1
    assert b"aligned" in P.qtts_probe_last_error()
    assert P.qtts_probe_stream(src, 4096, 0, 1, sink, None) == -1
    assert P.qtts_probe_stream(src, 4096, 17, 1, sink, None) == -1
    assert P.qtts_probe_stream(src, 4096, 4, 3, sink, None) == -1
    assert P.qtts_probe_stream(src, 4096 + 1024, 4, 1, sink, None) == -1
    assert b"multiple" in P.qtts_probe_last_error()
    assert P.qtts_probe_stream(src, 0, 4, 1, sink, None) == -1
    assert P.qtts_probe_empty(0, 4, None) == -1
    assert P.qtts_probe_empty(1, 17, None) == -1


def _no_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("calls that pass validation would launch on stand-in addresses")


def _alias_calls(L, x, ldx, y, ldy, m=4, k=64, n=64):
    """Every entry point whose kernels read the activations while others write the output, called
    with x at ``x`` (row stride ldx) and the output at ``y`` (row stride ldy), bf16, stand-in
    addresses for everything else (16-byte aligned, never dereferenced)."""
    q, s, ws, nw = 1 << 30, 1 << 31, 1 << 32, 1 << 33
    BF = _lib.BF16
    return {
        "w8a16_gemm": L.qtts_w8a16_gemm(x, BF, m, k, ldx, q, n, k, s, BF, None, y, ldy, 0, ws, 1 << 20, None),
        "w8a16_gemm_strips": L.qtts_w8a16_gemm_strips(x, BF, m, k, ldx, q, n, s, BF, None, y, ldy, 0, ws, 1 << 20,
                                                      None),
        "fp8w_gemm_strips": L.qtts_fp8w_gemm_strips(x, BF, m, k, ldx, q, n, s, None, y, ldy, 0, ws, 1 << 20, None),
        "w8a16_fused_gemm_strips": L.qtts_w8a16_fused_gemm_strips(x, BF, m, k, ldx, _lib.PRO_RMS_NORM, nw, 1e-6, q,
                                                                  n, s, BF, None, None, 0, y, ldy, 0, ws, 1 << 20,
                                                                  None),
        "w8a16_gate_up_silu_strips": L.qtts_w8a16_gate_up_silu_strips(x, BF, m, k, ldx, _lib.PRO_NONE, None, 1e-6,
                                                                      q, 2 * n, s, BF, None, y, ldy, 0, ws, 1 << 20,
                                                                      None),
        "w8a16_silu_mul_gemm_strips": L.qtts_w8a16_silu_mul_gemm_strips(x, BF, m, k // 2, ldx, q, n, s, BF, None,
                                                                        y, ldy, 0, ws, 1 << 20, None),
        "fp8_linear_strips": L.qtts_fp8_linear_strips(x, BF, m, k, ldx, q, n, s, None, y, ldy, 0, 0, ws, 1 << 20,
                                                      None),
        "int8_linear_strips": L.qtts_int8_linear_strips(x, BF, m, k, ldx, q, n, s, None, y, ldy, 0, 0, ws, 1 << 20,
                                                        None),
    }


def test_output_overlapping_activations_is_rejected():
    """y sharing bytes with x races (every workgroup reads all x rows of its K range while others
    write y): each entry point rejects it before any device use, the W8A16 family included."""
    L = _lib.load()
    x = 1 << 24
    for y, ldy in ((x, 64), (x + 64, 64), (x + 3 * 128 + 32, 64)):   # the same rows; a shifted span
        for name, st in _alias_calls(L, x, 64, y, ldy).items():
            assert st == _lib.ERR_INVALID_ARGUMENT, (name, y - x, st)
            assert "overlaps" in _lib.last_error(), (name, _lib.last_error())
    # x's and y's row blocks of one buffer that share bytes in the first row; and y on another
    # row stride whose second row lands on x's second row
    for y, ldy in ((x + 100, 256), (x + 128, 192)):
        for name, st in _alias_calls(L, x, 256, y, ldy).items():
            assert st == _lib.ERR_INVALID_ARGUMENT and "overlaps" in _lib.last_error(), (name, y - x, ldy)
    # the residual may be y itself, but x may not
    st = L.qtts_w8a16_fused_gemm_strips(x, _lib.BF16, 4, 64, 64, _lib.PRO_NONE, None, 1e-6, 1 << 30, 64, 1 << 31,
                                        _lib.BF16, None, x, 64, x, 64, 0, 1 << 32, 1 << 20, None)
    assert st == _lib.ERR_INVALID_ARGUMENT and "overlaps x" in _lib.last_error()


def test_interleaved_column_blocks_pass_validation():
    """x = buf[:, :k] and y = buf[:, k:k + n] of one buffer interleave their rows without sharing a
    byte: the overlap check lets them through (F.linear accepts that layout), so the call reaches
    the device check, which fails here with no GPU."""
    _no_gpu()
    L = _lib.load()
    base = 1 << 24
    # bf16 rows of 256 elements: x columns [0, 64), y columns [64, 128) (128 bytes in)
    for name, st in _alias_calls(L, base, 256, base + 128, 256).items():
        assert st == _lib.ERR_UNSUPPORTED, (name, st, _lib.last_error())
    # y's block before x's in each row; and y on another row stride (256 bytes against x's 512)
    # whose rows fall in the gaps between x's
    for name, st in _alias_calls(L, base + 256, 256, base, 256).items():
        assert st == _lib.ERR_UNSUPPORTED, (name, st, _lib.last_error())
    for name, st in _alias_calls(L, base, 256, base + 128, 128).items():
        assert st == _lib.ERR_UNSUPPORTED, (name, st, _lib.last_error())


def test_size_queries_reject_sizes_past_2_31():
    """The workspace query and the strip sizes reject sizes past 2^31, as the GEMM entry points
    do (m * k and the padded strip bytes would overflow 64 bits for the largest)."""
    L = _lib.load()
    for big in (1 << 31, 1 << 40, 1 << 62):
        assert L.qtts_workspace_bytes(_lib.OP_FP8_LINEAR, big, 4096, 2048, 0) == -1
        assert L.qtts_workspace_bytes(_lib.OP_W8A16, 8, big, 2048, 0) == -1
        assert L.qtts_workspace_bytes(_lib.OP_INT8_LINEAR, 8, 4096, big, 0) == -1
        assert L.qtts_strip_bytes(big, 4096, _lib.STRIP_INT8) == -1
        assert L.qtts_strip_bytes(4096, big, _lib.STRIP_FP8) == -1
    assert L.qtts_workspace_bytes(_lib.OP_FP8_LINEAR, 8, 4096, 2048, 0) > 0
    assert L.qtts_strip_bytes(16, 64, _lib.STRIP_INT8) == 1024
