"""torch-facing wrappers over the C ABI.

Every function takes and returns torch tensors on a gfx950 device, launches on
torch's current stream, allocates outputs through torch's caching allocator and
never synchronises, so each one can be captured into a HIP graph.  There is no
CPU or eager-PyTorch fallback: a missing library or an unsupported device raises.
"""

from __future__ import annotations

import threading

import torch

from . import _lib
from ._lib import (ALGO_AUTO, ALGO_SKINNY_HALF, ALGO_SKINNY_QUARTER, ALGO_STREAM, DIV_DEVICE, DIV_IEEE,  # noqa: F401
                   OP_FP8_LINEAR, OP_FP8W, OP_INT8_LINEAR, OP_W8A16, OP_W8A16_FUSED, OP_W8A16_SILU, OP_W8A8_FP8, OP_W8A8_INT8, PRO_NONE,
                   PRO_RMS_NORM, PRO_SILU_MUL, STRIP_FP8, STRIP_INT8, CODE_E4M3, CODE_INT8, TILE_READ_AHEAD, TILE_TWO_CHUNKS, algo_code,
                   tile_shape)

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    assert dev is not None
    return dev


def device_supported(device: torch.device | int | None = None) -> bool:
    """Whether ``device`` (default: the current one) is a gfx950 this library runs on."""
    if not torch.cuda.is_available():
        return False
    if device is None:
        idx = torch.cuda.current_device()
    elif isinstance(device, int):
        idx = device
    else:
        idx = device.index if device.index is not None else torch.cuda.current_device()
    return _lib.device_supported(idx)


# ---- workspace ---------------------------------------------------------------------------
# One zero-filled byte buffer per device.  The kernels that use it (split-K meeting
# points) leave it zero-filled again, so it is allocated and cleared once, outside
# any graph capture, and then shared by every call on that device.  Calls that
# share it must be stream-ordered, which holds for one engine thread on one stream.

_ws_lock = threading.Lock()
_workspaces: dict[int, torch.Tensor] = {}
# Outgrown workspaces are never freed: a HIP graph captured earlier still holds
# their address and keeps using them on every replay.
_retired: list[torch.Tensor] = []


def reserve_workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Grow the device's workspace to at least ``nbytes`` (call outside capture)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        ws = _workspaces.get(idx)
        if nbytes <= 0:
            return ws
        if ws is None or ws.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                return ws
            size = max(nbytes, 0 if ws is None else ws.numel())
            size = (size + (1 << 20) - 1) & ~((1 << 20) - 1)
            if ws is not None:
                _retired.append(ws)
            ws = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", idx))
            _workspaces[idx] = ws
        return ws


#: Rows the quant methods reserve workspace for at ``process_weights`` time, so that calls up
#: to this many rows never allocate (decode and prefill buckets up to 2048 rows).
WORKSPACE_ROWS = 2048


def reserve_for_rows(device: torch.device, op: int, n: int, k: int, max_rows: int = WORKSPACE_ROWS) -> None:
    """Reserve what ``op`` needs for an ``[N, K]`` weight at every row count up to ``max_rows``
    (the automatic kernel choice), outside capture: load time, not the hot path."""
    rows = sorted({r for r in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192) if r <= max_rows}
                  | {max(1, int(max_rows))})
    reserve_workspace(device, max(workspace_bytes(op, r, n, k) for r in rows))


def _ensure_workspace(device: torch.device, nbytes: int, what: str) -> None:
    """Make sure the device's workspace holds ``nbytes`` before a call that needs them.  Under
    graph capture nothing can be allocated, so a workspace that is too small raises here (the
    method reserves for ``WORKSPACE_ROWS`` rows at load time; reserve_workspace grows it).
    In eager mode a call past the reservation grows it once."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _workspaces.get(idx)
    if nbytes <= 0 or (ws is not None and ws.numel() >= nbytes):
        return
    if torch.cuda.is_current_stream_capturing():
        have = 0 if ws is None else ws.numel()
        raise ValueError(f"{what}: needs {nbytes} workspace bytes and {have} are reserved; call "
                         f"ops.reserve_workspace(device, {nbytes}) before capturing")
    reserve_workspace(device, nbytes)


def workspace_bytes(op: int, m: int, n: int, k: int, algo: int = ALGO_AUTO) -> int:
    v = _lib.load().qtts_workspace_bytes(op, m, n, k, algo)
    if v < 0:
        _lib.check(int(v), "workspace_bytes")
    return int(v)


def _ws_for(device: torch.device) -> tuple[int | None, int]:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _workspaces.get(idx)
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


# ---- packers -----------------------------------------------------------------------------

def pack_int8(weight: torch.Tensor, scale_dtype: torch.dtype | None = None, div_mode: int = DIV_DEVICE,
              want_f32_scale: bool = False):
    """Per-output-channel symmetric int8 (qtts/quant/int8.py:45-56).

    Returns ``(q [N,K] int8, scale [N] scale_dtype)`` and, with ``want_f32_scale``,
    the unrounded fp32 scale as a third element.  ``scale_dtype`` defaults to fp32
    (the return of quantize_weight_per_channel); Int8WeightOnlyMethod stores it in
    the weight dtype (qtts/quant/int8.py:105).
    """
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    dev = _require_cuda(weight)
    w = weight.detach()
    if w.stride(1) != 1:
        w = w.contiguous()
    n, k = w.shape
    sdt = torch.float32 if scale_dtype is None else scale_dtype
    q = torch.empty((n, k), dtype=torch.int8, device=dev)
    scale = torch.empty(n, dtype=sdt, device=dev)
    s32 = torch.empty(n, dtype=torch.float32, device=dev) if want_f32_scale else None
    st = _lib.load().qtts_pack_int8_rowwise(
        _ptr(w), dtype_code(w.dtype), n, k, w.stride(0), _ptr(q), _ptr(scale), dtype_code(sdt), _ptr(s32),
        div_mode, _stream(dev))
    _lib.check(st, "pack_int8_rowwise")
    return (q, scale, s32) if want_f32_scale else (q, scale)


def pack_fp8(weight: torch.Tensor, div_mode: int = DIV_DEVICE):
    """Per-output-channel e4m3 (qtts/quant/fp8.py:45-49): ``(q [N,K] float8_e4m3fn, scale [N] fp32)``."""
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    dev = _require_cuda(weight)
    w = weight.detach()
    if w.stride(1) != 1:
        w = w.contiguous()
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=dev)
    scale = torch.empty(n, dtype=torch.float32, device=dev)
    st = _lib.load().qtts_pack_fp8_e4m3_rowwise(_ptr(w), dtype_code(w.dtype), n, k, w.stride(0), _ptr(q), _ptr(scale),
                                               div_mode, _stream(dev))
    _lib.check(st, "pack_fp8_e4m3_rowwise")
    return q, scale


# ---- GEMMs --------------------------------------------------------------------------------

def _flatten(x: torch.Tensor) -> torch.Tensor:
    rows = 1
    for d in x.shape[:-1]:
        rows *= d
    a = x.reshape(rows, x.shape[-1])
    if a.stride(-1) != 1 or (a.shape[0] > 1 and a.stride(0) < a.shape[1]):
        a = a.contiguous()
    return a


def w8a16_gemm(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None = None,
               algo: int = ALGO_AUTO) -> torch.Tensor:
    """``x @ (q * scale)^T + bias`` with q dequantized in registers (qtts/quant/kernels.py:138-178).

    x ``[..., K]`` float (bf16/fp16/fp32), q ``[N, K]`` int8, scale ``[N]``, bias ``[N]`` in
    x's dtype or None.  Returns a fresh ``[..., N]`` tensor in x's dtype.
    """
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if q.dim() != 2 or q.dtype != torch.int8:
        raise ValueError(f"weight must be a 2-D int8 tensor, got {q.dtype} {tuple(q.shape)}")
    n = q.shape[0]
    if q.shape[1] != k:
        raise ValueError(f"weight is [{n}, {q.shape[1]}] but x has K={k}")
    if q.stride(1) != 1:
        q = q.contiguous()
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        if bias.dtype != a.dtype:
            bias = bias.to(a.dtype)
        bias = bias.contiguous()
    dev = _require_cuda(a, q, scale, bias)
    scale = scale.contiguous()
    out = torch.empty((rows, n), dtype=a.dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a16_gemm(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(q), n, q.stride(0),
        _ptr(scale), dtype_code(scale.dtype), _ptr(bias), _ptr(out), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a16_gemm")
    return out.reshape(*shape[:-1], n)


def quant_act_fp8(x: torch.Tensor, div_mode: int = DIV_DEVICE):
    """Per-token e4m3 activations (qtts/quant/fp8.py:77-78): ``(qx [M,K] e4m3, sx [M] fp32)``."""
    a = _flatten(x)
    m, k = a.shape
    dev = _require_cuda(a)
    qx = torch.empty((m, k), dtype=torch.float8_e4m3fn, device=dev)
    sx = torch.empty(m, dtype=torch.float32, device=dev)
    st = _lib.load().qtts_quant_act_fp8_rows(_ptr(a), dtype_code(a.dtype), m, k, a.stride(0) if m > 1 else k,
                                             _ptr(qx), _ptr(sx), div_mode, _stream(dev))
    _lib.check(st, "quant_act_fp8_rows")
    return qx, sx


def w8a8_fp8_gemm(qx: torch.Tensor, sx: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor,
                  bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                  algo: int = ALGO_AUTO) -> torch.Tensor:
    """``(qx*sx) @ (qw*sw)^T`` rounded to out_dtype, then ``+ bias`` in out_dtype (qtts/quant/fp8.py:79-89).

    qx ``[M, K]`` e4m3, sx ``[M]`` fp32, qw ``[N, K]`` e4m3 (row-major), sw ``[N]`` fp32.
    """
    if qx.dim() != 2 or qw.dim() != 2:
        raise ValueError("qx and qw must be 2-D")
    m, k = qx.shape
    n = qw.shape[0]
    if qw.shape[1] != k:
        raise ValueError(f"weight is [{n}, {qw.shape[1]}] but x has K={k}")
    if qx.stride(1) != 1:
        qx = qx.contiguous()
    if qw.stride(1) != 1:
        qw = qw.contiguous()
    if sx.numel() != m or sw.numel() != n:
        raise ValueError("scale sizes do not match the operands")
    sx = sx.reshape(-1).to(torch.float32).contiguous()
    sw = sw.reshape(-1).to(torch.float32).contiguous()
    if bias is not None:
        bias = bias.to(out_dtype).contiguous()
    dev = _require_cuda(qx, sx, qw, sw, bias)
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a8_fp8_gemm(
        _ptr(qx), _ptr(sx), m, k, qx.stride(0) if m > 1 else k, _ptr(qw), n, qw.stride(0), _ptr(sw), _ptr(bias),
        _ptr(out), dtype_code(out_dtype), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a8_fp8_gemm")
    return out


def fp8_linear(x: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor, bias: torch.Tensor | None = None,
               div_mode: int = DIV_DEVICE, algo: int = ALGO_AUTO) -> torch.Tensor:
    """The whole of Fp8Method.apply (qtts/quant/fp8.py:72-89): quantize x per token, fp8 GEMM."""
    shape = x.shape
    qx, sx = quant_act_fp8(x, div_mode)
    out = w8a8_fp8_gemm(qx, sx, qw, sw, bias, x.dtype, algo)
    return out.reshape(*shape[:-1], qw.shape[0])


# ---- strip layout ----------------------------------------------------------------------
# The GEMM kernels read weights fastest in the strip layout (include/qtts_amd.h): a
# permutation of the packer's row-major bytes in which every wavefront load is one
# contiguous 1 KiB.  The quant methods keep only this copy; from_strips recovers
# the row-major bytes bit for bit.

def strip_bytes(n: int, k: int, kind: int) -> int:
    v = _lib.load().qtts_strip_bytes(n, k, kind)
    if v < 0:
        _lib.check(int(v), "strip_bytes")
    return int(v)


def to_strips(q: torch.Tensor, kind: int | None = None) -> torch.Tensor:
    """Row-major ``[N, K]`` int8 / e4m3 weight -> strip layout (same dtype; ``[N, K]`` when no padding
    is needed, else 1-D)."""
    if q.dim() != 2:
        raise ValueError("expected a 2-D weight")
    if kind is None:
        kind = STRIP_FP8 if q.dtype == torch.float8_e4m3fn else STRIP_INT8
    dev = _require_cuda(q)
    if q.stride(1) != 1:
        q = q.contiguous()
    n, k = q.shape
    nbytes = strip_bytes(n, k, kind)
    out = torch.empty(nbytes, dtype=q.dtype, device=dev)
    st = _lib.load().qtts_to_strips(_ptr(q), n, k, q.stride(0), kind, _ptr(out), _stream(dev))
    _lib.check(st, "to_strips")
    return out.view(n, k) if nbytes == n * k else out


def from_strips(qs: torch.Tensor, n: int, k: int, kind: int | None = None) -> torch.Tensor:
    """Strip layout -> row-major ``[N, K]`` (the packer's bytes)."""
    if kind is None:
        kind = STRIP_FP8 if qs.dtype == torch.float8_e4m3fn else STRIP_INT8
    dev = _require_cuda(qs)
    out = torch.empty((n, k), dtype=qs.dtype, device=dev)
    st = _lib.load().qtts_from_strips(_ptr(qs), n, k, kind, _ptr(out), k, _stream(dev))
    _lib.check(st, "from_strips")
    return out


def dequant_strips(qs: torch.Tensor, n: int, k: int, scale: torch.Tensor, dtype: torch.dtype,
                   codes: int = CODE_INT8, out: torch.Tensor | None = None) -> torch.Tensor:
    """``dtype(code * scale[:, None])`` as a row-major ``[N, K]`` matrix from 64-column strips of
    int8 (``CODE_INT8``) or e4m3 (``CODE_E4M3``) codes: the reference's dequantized weight,
    ``q.to(dtype) * scale[:, None]`` (qtts/quant/kernels.py:144-148).  ``out``: an ``[N, K]``
    (row-contiguous) tensor of ``dtype`` to write into, e.g. a view of :func:`dequant_scratch`."""
    if qs.dtype not in (torch.int8, torch.uint8) or qs.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"codes are not a 64-column strip [{n}, {k}] buffer")
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    dev = _require_cuda(qs, scale)
    scale = scale.contiguous()
    if out is None:
        out = torch.empty((n, k), dtype=dtype, device=dev)
    elif out.dtype != dtype or tuple(out.shape) != (n, k) or (k > 1 and out.stride(1) != 1):
        raise ValueError(f"out must be an [{n}, {k}] {dtype} tensor with unit column stride")
    st = _lib.load().qtts_dequant_strips(_ptr(qs), codes, n, k, _ptr(scale), dtype_code(scale.dtype), _ptr(out),
                                         dtype_code(dtype), out.stride(0) if n > 1 else k, _stream(dev))
    _lib.check(st, "dequant_strips")
    return out


# One scratch buffer per device for dequantized weights (the int8 weight-only method's
# prefill route: dequantize, then a library GEMM).  Grown outside capture only; an
# outgrown buffer stays alive for the graphs that captured its address.  Calls that
# share it must be stream-ordered, as for the workspace.
_dq_scratch: dict[int, torch.Tensor] = {}


def reserve_dequant_scratch(device: torch.device, nbytes: int) -> None:
    """Grow the device's dequantization scratch to at least ``nbytes`` (call outside capture)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        buf = _dq_scratch.get(idx)
        if nbytes <= 0 or (buf is not None and buf.numel() >= nbytes) or torch.cuda.is_current_stream_capturing():
            return
        if buf is not None:
            _retired.append(buf)
        size = (nbytes + (1 << 20) - 1) & ~((1 << 20) - 1)
        _dq_scratch[idx] = torch.empty(size, dtype=torch.uint8, device=torch.device("cuda", idx))


def dequant_scratch(device: torch.device, n: int, k: int, dtype: torch.dtype) -> torch.Tensor:
    """An ``[N, K]`` ``dtype`` view of the device's dequantization scratch (reserved beforehand)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    need = n * k * torch.empty((), dtype=dtype).element_size()
    buf = _dq_scratch.get(idx)
    if buf is None or buf.numel() < need:
        raise ValueError(f"dequantization scratch holds {0 if buf is None else buf.numel()} bytes, {need} needed "
                         f"(reserve_dequant_scratch before capture)")
    return buf[:need].view(dtype).view(n, k)


def w8a16_gemm_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                      bias: torch.Tensor | None = None, algo: int = ALGO_AUTO) -> torch.Tensor:
    """``w8a16_gemm`` with the int8 weight in the strip layout (``n`` output channels)."""
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if qs.dtype != torch.int8 or qs.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not an int8 strip-layout [{n}, {k}] buffer")
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    dev = _require_cuda(a, qs, scale, bias)
    scale = scale.contiguous()
    out = torch.empty((rows, n), dtype=a.dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a16_gemm_strips(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(qs), n, _ptr(scale),
        dtype_code(scale.dtype), _ptr(bias), _ptr(out), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a16_gemm_strips")
    return out.reshape(*shape[:-1], n)


def w8a8_fp8_gemm_strips(qx: torch.Tensor, sx: torch.Tensor, qws: torch.Tensor, n: int, sw: torch.Tensor,
                         bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                         algo: int = ALGO_AUTO) -> torch.Tensor:
    """``w8a8_fp8_gemm`` with the e4m3 weight in the strip layout."""
    m, k = qx.shape
    if qws.numel() != strip_bytes(n, k, STRIP_FP8):
        raise ValueError(f"weight is not an e4m3 strip-layout [{n}, {k}] buffer")
    if qx.stride(1) != 1:
        qx = qx.contiguous()
    sx = sx.reshape(-1).to(torch.float32).contiguous()
    sw = sw.reshape(-1).to(torch.float32).contiguous()
    if bias is not None:
        bias = bias.to(out_dtype).contiguous()
    dev = _require_cuda(qx, sx, qws, sw, bias)
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a8_fp8_gemm_strips(
        _ptr(qx), _ptr(sx), m, k, qx.stride(0) if m > 1 else k, _ptr(qws), n, _ptr(sw), _ptr(bias), _ptr(out),
        dtype_code(out_dtype), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a8_fp8_gemm_strips")
    return out


def fp8_linear_strips(x: torch.Tensor, qws: torch.Tensor, n: int, sw: torch.Tensor,
                      bias: torch.Tensor | None = None, div_mode: int = DIV_DEVICE,
                      algo: int = ALGO_AUTO) -> torch.Tensor:
    """Fp8Method.apply (qtts/quant/fp8.py:72-89) with the e4m3 weight in the strip layout.

    One C call.  A single kernel quantizes x per token inside the GEMM for decode rows
    (M <= 3, or M <= 8 when K <= 2048) with K % 128 == 0, K <= 6144 and 16-byte aligned
    rows of 16-bit activations (``qtts_fp8_fused_ok``); every other call quantizes into the
    workspace first and runs the fp8 GEMM (two kernels).
    """
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if qws.numel() != strip_bytes(n, k, STRIP_FP8):
        raise ValueError(f"weight is not an e4m3 strip-layout [{n}, {k}] buffer")
    if sw.numel() != n:
        raise ValueError(f"scale has {sw.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    sw = sw.reshape(-1).to(torch.float32).contiguous()
    dev = _require_cuda(a, qws, sw, bias)
    out = torch.empty((rows, n), dtype=a.dtype, device=dev)
    _ensure_workspace(dev, workspace_bytes(OP_FP8_LINEAR, rows, n, k, algo), "fp8_linear")
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_fp8_linear_strips(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(qws), n, _ptr(sw), _ptr(bias),
        _ptr(out), n, div_mode, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "fp8_linear_strips")
    return out.reshape(*shape[:-1], n)


# ---- int8 W8A8 (Int8Method, qtts/quant/int8.py:129-160) --------------------------------

def quant_act_int8(x: torch.Tensor, div_mode: int = DIV_DEVICE):
    """Per-token int8 activations (qtts/quant/int8.py:146-149): ``(qx [M,K] int8, sx [M] fp32)``.

    The scale is computed in x's dtype as the reference does and returned widened to
    fp32 (exactly)."""
    a = _flatten(x)
    m, k = a.shape
    dev = _require_cuda(a)
    qx = torch.empty((m, k), dtype=torch.int8, device=dev)
    sx = torch.empty(m, dtype=torch.float32, device=dev)
    st = _lib.load().qtts_quant_act_int8_rows(_ptr(a), dtype_code(a.dtype), m, k, a.stride(0) if m > 1 else k,
                                              _ptr(qx), _ptr(sx), div_mode, _stream(dev))
    _lib.check(st, "quant_act_int8_rows")
    return qx, sx


def _int8_gemm_args(qx, sx, sw, bias, m, n, out_dtype):
    if qx.dtype != torch.int8:
        raise ValueError(f"activations must be int8, got {qx.dtype}")
    if qx.stride(1) != 1:
        qx = qx.contiguous()
    if sx.numel() != m or sw.numel() != n:
        raise ValueError("scale sizes do not match the operands")
    sx = sx.reshape(-1).to(torch.float32).contiguous()
    sw = sw.reshape(-1).to(torch.float32).contiguous()
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(out_dtype).contiguous()
    return qx, sx, sw, bias


def w8a8_int8_gemm(qx: torch.Tensor, sx: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor,
                   bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                   algo: int = ALGO_AUTO) -> torch.Tensor:
    """``((f32(qx @ qw^T) * sx) * sw + bias)`` rounded once to out_dtype (qtts/quant/int8.py:151-160).

    qx ``[M, K]`` int8, sx ``[M]`` fp32, qw ``[N, K]`` int8 (row-major; the reference keeps
    the transpose), sw ``[N]`` fp32.  The int32 accumulation is exact.
    """
    if qx.dim() != 2 or qw.dim() != 2 or qw.dtype != torch.int8:
        raise ValueError("qx and qw must be 2-D int8 tensors")
    m, k = qx.shape
    n = qw.shape[0]
    if qw.shape[1] != k:
        raise ValueError(f"weight is [{n}, {qw.shape[1]}] but x has K={k}")
    if qw.stride(1) != 1:
        qw = qw.contiguous()
    qx, sx, sw, bias = _int8_gemm_args(qx, sx, sw, bias, m, n, out_dtype)
    dev = _require_cuda(qx, sx, qw, sw, bias)
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a8_int8_gemm(
        _ptr(qx), _ptr(sx), m, k, qx.stride(0) if m > 1 else k, _ptr(qw), n, qw.stride(0), _ptr(sw), _ptr(bias),
        _ptr(out), dtype_code(out_dtype), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a8_int8_gemm")
    return out


def w8a8_int8_gemm_strips(qx: torch.Tensor, sx: torch.Tensor, qws: torch.Tensor, n: int, sw: torch.Tensor,
                          bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                          algo: int = ALGO_AUTO) -> torch.Tensor:
    """``w8a8_int8_gemm`` with the int8 weight in the strip layout."""
    if qx.dim() != 2:
        raise ValueError("qx must be 2-D")
    m, k = qx.shape
    if qws.dtype != torch.int8 or qws.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not an int8 strip-layout [{n}, {k}] buffer")
    qx, sx, sw, bias = _int8_gemm_args(qx, sx, sw, bias, m, n, out_dtype)
    dev = _require_cuda(qx, sx, qws, sw, bias)
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a8_int8_gemm_strips(
        _ptr(qx), _ptr(sx), m, k, qx.stride(0) if m > 1 else k, _ptr(qws), n, _ptr(sw), _ptr(bias), _ptr(out),
        dtype_code(out_dtype), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a8_int8_gemm_strips")
    return out


def _int8_linear(x, qw, n, ldqw, sw, bias, div_mode, algo, strips):
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if sw.numel() != n:
        raise ValueError(f"scale has {sw.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    sw = sw.reshape(-1).to(torch.float32).contiguous()
    dev = _require_cuda(a, qw, sw, bias)
    out = torch.empty((rows, n), dtype=a.dtype, device=dev)
    _ensure_workspace(dev, workspace_bytes(OP_INT8_LINEAR, rows, n, k, algo), "int8_linear")
    ws, ws_n = _ws_for(dev)
    lib = _lib.load()
    if strips:
        st = lib.qtts_int8_linear_strips(
            _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(qw), n, _ptr(sw), _ptr(bias),
            _ptr(out), n, div_mode, algo, ws, ws_n, _stream(dev))
    else:
        st = lib.qtts_int8_linear(
            _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(qw), n, ldqw, _ptr(sw),
            _ptr(bias), _ptr(out), n, div_mode, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "int8_linear_strips" if strips else "int8_linear")
    return out.reshape(*shape[:-1], n)


def int8_linear(x: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor, bias: torch.Tensor | None = None,
                div_mode: int = DIV_DEVICE, algo: int = ALGO_AUTO) -> torch.Tensor:
    """The whole of Int8Method.apply (qtts/quant/int8.py:145-160) in one C call: quantize x
    per token into the workspace, then the int8 GEMM.  qw ``[N, K]`` int8 row-major."""
    if qw.dim() != 2 or qw.dtype != torch.int8:
        raise ValueError(f"weight must be a 2-D int8 tensor, got {qw.dtype} {tuple(qw.shape)}")
    if qw.shape[1] != x.shape[-1]:
        raise ValueError(f"weight is [{qw.shape[0]}, {qw.shape[1]}] but x has K={x.shape[-1]}")
    if qw.stride(1) != 1:
        qw = qw.contiguous()
    return _int8_linear(x, qw, qw.shape[0], qw.stride(0), sw, bias, div_mode, algo, strips=False)


def int8_linear_strips(x: torch.Tensor, qws: torch.Tensor, n: int, sw: torch.Tensor,
                       bias: torch.Tensor | None = None, div_mode: int = DIV_DEVICE,
                       algo: int = ALGO_AUTO) -> torch.Tensor:
    """Int8Method.apply (qtts/quant/int8.py:145-160) with the int8 weight in the strip layout."""
    k = x.shape[-1]
    if qws.dtype != torch.int8 or qws.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not an int8 strip-layout [{n}, {k}] buffer")
    return _int8_linear(x, qws, n, 0, sw, bias, div_mode, algo, strips=True)


# ---- fp8 weight-only (Fp8WeightOnlyMethod, qtts/quant/fp8.py:92-123) -------------------

def fp8w_strips(q: torch.Tensor) -> torch.Tensor:
    """e4m3 ``[N, K]`` codes -> the 64-column strip layout the fp8 weight-only kernels read
    (``uint8``; ``[N, K]`` when no padding is needed, else 1-D)."""
    if q.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise ValueError(f"expected e4m3 codes, got {q.dtype}")
    return to_strips(q.view(torch.uint8), STRIP_INT8)


def fp8w_gemm_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                     bias: torch.Tensor | None = None, algo: int = ALGO_AUTO) -> torch.Tensor:
    """``x @ (e4m3(q) * scale)^T + bias`` with the codes converted in registers.

    x ``[..., K]`` bf16 / fp16 (K % 64 == 0), qs from :func:`fp8w_strips`, scale ``[N]``
    fp32, bias ``[N]`` or None.  Returns a fresh ``[..., N]`` tensor in x's dtype."""
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if qs.element_size() != 1 or qs.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not a 64-column strip-layout [{n}, {k}] buffer of e4m3 codes")
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    scale = scale.reshape(-1).to(torch.float32).contiguous()
    dev = _require_cuda(a, qs, scale, bias)
    out = torch.empty((rows, n), dtype=a.dtype, device=dev)
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_fp8w_gemm_strips(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(qs), n, _ptr(scale), _ptr(bias),
        _ptr(out), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "fp8w_gemm_strips")
    return out.reshape(*shape[:-1], n)


# ---- GatedMLP (qtts/layers/activation.py:142-147) ------------------------------------

def _gate_up_rows(gate_up: torch.Tensor) -> torch.Tensor:
    a = _flatten(gate_up)
    if a.shape[1] % 2:
        raise ValueError(f"gate_up has an odd last dimension {a.shape[1]}; expected [..., 2 * intermediate]")
    return a


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate) * up`` of a fused ``[..., 2I]`` gate_up output in one kernel, with torch's
    rounding for the two-kernel expression.  Returns ``[..., I]`` in gate_up's dtype."""
    shape = gate_up.shape
    a = _gate_up_rows(gate_up)
    rows, k = a.shape[0], a.shape[1] // 2
    dev = _require_cuda(a)
    out = torch.empty((rows, k), dtype=a.dtype, device=dev)
    st = _lib.load().qtts_silu_mul(_ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else 2 * k,
                                   _ptr(out), k, _stream(dev))
    _lib.check(st, "silu_mul")
    return out.reshape(*shape[:-1], k)


def w8a16_silu_mul_gemm_strips(gate_up: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                               bias: torch.Tensor | None = None, algo: int = ALGO_AUTO) -> torch.Tensor:
    """``down(F.silu(gate) * up)`` for an int8 strip-layout down projection, one call: a single
    decode row has the activation computed inside the GEMM kernel."""
    shape = gate_up.shape
    a = _gate_up_rows(gate_up)
    rows, k = a.shape[0], a.shape[1] // 2
    if qs.dtype != torch.int8 or qs.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not an int8 strip-layout [{n}, {k}] buffer")
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    dev = _require_cuda(a, qs, scale, bias)
    scale = scale.contiguous()
    out = torch.empty((rows, n), dtype=a.dtype, device=dev)
    _ensure_workspace(dev, workspace_bytes(OP_W8A16_SILU, rows, n, k, algo), "w8a16_silu_mul_gemm")
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a16_silu_mul_gemm_strips(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else 2 * k, _ptr(qs), n, _ptr(scale),
        dtype_code(scale.dtype), _ptr(bias), _ptr(out), n, algo, ws, ws_n, _stream(dev))
    _lib.check(st, "w8a16_silu_mul_gemm_strips")
    return out.reshape(*shape[:-1], n)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dimension (qtts/layers/norm.py:50-76): fp32 sum of squares,
    ``inv = 1 / sqrt(mean + eps)``, ``(x * inv) * weight`` rounded to x's dtype."""
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if weight.numel() != k:
        raise ValueError(f"norm weight has {weight.numel()} entries for rows of {k}")
    dev = _require_cuda(a, weight)
    w = weight.to(a.dtype).contiguous()
    out = torch.empty((rows, k), dtype=a.dtype, device=dev)
    st = _lib.load().qtts_rms_norm(_ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, _ptr(w),
                                   float(eps), _ptr(out), k, _stream(dev))
    _lib.check(st, "rms_norm")
    return out.reshape(shape)


def w8a16_fused_gemm_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                            bias: torch.Tensor | None = None, *, prologue: int = PRO_NONE,
                            norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                            residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
                            algo: int = ALGO_AUTO) -> torch.Tensor:
    """``[residual +] linear(prologue(x))`` for an int8 strip-layout linear in one call
    (qtts/models/talker.py:246-271).  ``prologue``: PRO_NONE, PRO_SILU_MUL (x is the fused
    ``[..., 2K]`` gate_up output) or PRO_RMS_NORM (with ``norm_weight`` and ``eps``).
    ``residual`` is ``[..., n]`` of x's dtype; ``out`` may be the residual itself."""
    shape = x.shape
    a = _gate_up_rows(x) if prologue == PRO_SILU_MUL else _flatten(x)
    rows = a.shape[0]
    k = a.shape[1] // 2 if prologue == PRO_SILU_MUL else a.shape[1]
    if qs.dtype != torch.int8 or qs.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not an int8 strip-layout [{n}, {k}] buffer")
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if prologue == PRO_RMS_NORM:
        if norm_weight is None or norm_weight.numel() != k:
            raise ValueError(f"RMSNorm prologue needs a norm weight of {k} entries")
        norm_weight = norm_weight.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    res = None
    if residual is not None:
        res = _flatten(residual)
        if res.shape != (rows, n) or res.dtype != a.dtype:
            raise ValueError(f"residual must be [{rows}, {n}] of {a.dtype}, got {tuple(res.shape)} {res.dtype}")
    dev = _require_cuda(a, qs, scale, bias, norm_weight, res)
    scale = scale.contiguous()
    if out is None:
        y = torch.empty((rows, n), dtype=a.dtype, device=dev)
    else:
        y = _flatten(out)
        if y.shape != (rows, n) or y.dtype != a.dtype or y.data_ptr() != out.data_ptr():
            raise ValueError(f"out must be a [{rows}, {n}] {a.dtype} tensor")
    _ensure_workspace(dev, workspace_bytes(OP_W8A16_FUSED, rows, n, k, algo), "w8a16_fused_gemm")
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a16_fused_gemm_strips(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else a.shape[1], int(prologue),
        _ptr(norm_weight), float(eps), _ptr(qs), n, _ptr(scale), dtype_code(scale.dtype), _ptr(bias), _ptr(res),
        res.stride(0) if res is not None and rows > 1 else n, _ptr(y), y.stride(0) if rows > 1 else n, algo, ws, ws_n,
        _stream(dev))
    _lib.check(st, "w8a16_fused_gemm_strips")
    if out is not None:
        return out
    return y.reshape(*shape[:-1], n)


def w8a16_gate_up_silu_strips(x: torch.Tensor, qs: torch.Tensor, n: int, scale: torch.Tensor,
                              bias: torch.Tensor | None = None, *, prologue: int = PRO_NONE,
                              norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                              algo: int = ALGO_AUTO) -> torch.Tensor:
    """``F.silu(gate) * up`` of GatedMLP's fused ``gate_up_proj(prologue(x))`` (qtts/layers/activation.py:
    142-147) on an int8 strip-layout ``[n, K]`` gate_up weight; returns ``[..., n // 2]``.  Up to 8
    rows run as one kernel with the activation in the GEMM's epilogue (the gate_up output is never
    stored).  ``prologue``: PRO_NONE or PRO_RMS_NORM (with ``norm_weight`` and ``eps``)."""
    shape = x.shape
    a = _flatten(x)
    rows, k = a.shape
    if n % 2:
        raise ValueError(f"gate_up width {n} is odd")
    if qs.dtype != torch.int8 or qs.numel() != strip_bytes(n, k, STRIP_INT8):
        raise ValueError(f"weight is not an int8 strip-layout [{n}, {k}] buffer")
    if scale.numel() != n:
        raise ValueError(f"scale has {scale.numel()} entries for {n} output channels")
    if bias is not None:
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} entries for {n} output channels")
        bias = bias.to(a.dtype).contiguous()
    if prologue == PRO_RMS_NORM:
        if norm_weight is None or norm_weight.numel() != k:
            raise ValueError(f"RMSNorm prologue needs a norm weight of {k} entries")
        norm_weight = norm_weight.to(a.dtype).contiguous()
    if a.data_ptr() % 16 or (rows > 1 and a.stride(0) % 8):
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    dev = _require_cuda(a, qs, scale, bias, norm_weight)
    scale = scale.contiguous()
    act = torch.empty((rows, n // 2), dtype=a.dtype, device=dev)
    _ensure_workspace(dev, workspace_bytes(OP_W8A16_FUSED, rows, n, k, algo), "w8a16_fused_gemm")
    ws, ws_n = _ws_for(dev)
    st = _lib.load().qtts_w8a16_gate_up_silu_strips(
        _ptr(a), dtype_code(a.dtype), rows, k, a.stride(0) if rows > 1 else k, int(prologue), _ptr(norm_weight),
        float(eps), _ptr(qs), n, _ptr(scale), dtype_code(scale.dtype), _ptr(bias), _ptr(act), n // 2, algo, ws, ws_n,
        _stream(dev))
    _lib.check(st, "w8a16_gate_up_silu_strips")
    return act.reshape(*shape[:-1], n // 2)


class KernelTimer:
    """Summed device durations of the kernels this library launches inside the block.

    Each kernel launched outside graph capture gets a start/stop event pair bound to
    its own dispatch (``hipExtLaunchKernel``), so ``total_ms / launches`` is the mean
    kernel duration with no launch gaps.  ``untimed`` counts launches past the pool.
    """

    def __init__(self, max_launches: int = 4096) -> None:
        self.max_launches = int(max_launches)
        self.total_ms = 0.0
        self.launches = 0
        self.untimed = 0

    def __enter__(self) -> "KernelTimer":
        _lib.check(_lib.load().qtts_kernel_timer_begin(self.max_launches), "kernel_timer_begin")
        return self

    def __exit__(self, *exc) -> None:
        import ctypes
        ms, n, u = ctypes.c_double(), ctypes.c_int64(), ctypes.c_int64()
        _lib.check(_lib.load().qtts_kernel_timer_end(ctypes.byref(ms), ctypes.byref(n), ctypes.byref(u)),
                   "kernel_timer_end")
        self.total_ms, self.launches, self.untimed = ms.value, n.value, u.value

    @property
    def mean_ms(self) -> float:
        return self.total_ms / self.launches if self.launches else float("nan")

