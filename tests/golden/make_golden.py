"""Write the golden fixtures for the quantized-linear path.

    python tests/golden/make_golden.py          # rewrites tests/golden/*.npz

The reference ships no golden vectors for qtts/quant (its tests never touch it),
so these fixtures are produced by torch on the CPU evaluating the reference's
own expressions, character for character where the expression is device-neutral:

* int8 packer:  qtts/quant/int8.py:53-55 and the stored-scale cast at :105
* fp8 packer:   qtts/quant/fp8.py:47-49
* fp8 activations: qtts/quant/fp8.py:77-78
* naive W8A16 formula: examples/kernels/tune_w8_gemm.py:79
* int8 W8A8 (Int8Method.apply): qtts/quant/int8.py:146-160, torch._int_mm included
* GatedMLP's activation: qtts/layers/activation.py:147 (F.silu(gate) * up)

Two division semantics are recorded for every scale (see oracle/qtts_oracle.c):
``ieee`` is the literal CPU evaluation of ``tensor / python_float``; ``device`` is
what torch's GPU kernel computes for the same expression, ``tensor * fl(1/c)``.
The device variant here is an emulation; tests/test_gpu_pack.py pins it against
torch running the literal expression on the GPU.

No reference code is imported or executed.
"""

from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

TALKER = [("qkv", 4096, 2048), ("o", 2048, 2048), ("gate_up", 12288, 2048), ("down", 2048, 6144)]
PREDICTOR = [("p_qkv", 4096, 1024), ("p_o", 1024, 2048), ("p_gate_up", 6144, 1024), ("p_down", 1024, 3072)]


def _scalar_div(t: torch.Tensor, c: float, mode: str) -> torch.Tensor:
    if mode == "ieee":
        return t / c                                   # literal CPU evaluation
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(c, dtype=torch.float32)
    return (t.to(torch.float32) * inv).to(t.dtype)     # torch GPU: multiply by fp32 reciprocal


def ref_int8(weight: torch.Tensor, mode: str):
    w = weight.detach().float()
    scale = _scalar_div(w.abs().amax(dim=1).clamp_min(1e-12), 127.0, mode)
    q = (w / scale[:, None]).round().clamp_(-127.0, 127.0).to(torch.int8)
    return q, scale


def ref_fp8(weight: torch.Tensor, mode: str):
    w = weight.detach().float()
    scale = _scalar_div(w.abs().amax(dim=1).clamp_min(1e-12), 448.0, mode)
    return (w / scale[:, None]).to(torch.float8_e4m3fn), scale


def ref_act_fp8(x: torch.Tensor, mode: str):
    flat = x.reshape(-1, x.shape[-1]).contiguous()
    amax = flat.abs().amax(dim=1, keepdim=True).clamp_min(1e-6).float()
    scale_x = _scalar_div(amax, 448.0, mode)
    return (flat.float() / scale_x).to(torch.float8_e4m3fn), scale_x.reshape(-1)


def ref_act_int8(x: torch.Tensor, mode: str):
    """int8.py:146-149 on an x-dtype tensor; the scale stays in x's dtype."""
    flat = x.reshape(-1, x.shape[-1]).contiguous()
    scale_x = _scalar_div(flat.abs().amax(dim=1, keepdim=True).clamp_min(1e-6), 127.0, mode)
    q = (flat / scale_x).round().clamp_(-127.0, 127.0).to(torch.int8)
    return q, scale_x.reshape(-1)


def ref_int8_linear(x: torch.Tensor, int8_weight_t: torch.Tensor, int8_scale: torch.Tensor,
                    bias: torch.Tensor | None, mode: str) -> torch.Tensor:
    """int8.py:145-160 with the same row padding for torch._int_mm."""
    q, scale_x = ref_act_int8(x, mode)
    scale_x = scale_x.reshape(-1, 1)
    rows = q.shape[0]
    padded = rows < 17
    if padded:
        q = torch.cat([q, q.new_zeros(17 - rows, q.shape[1])], dim=0)
    acc = torch._int_mm(q, int8_weight_t)
    if padded:
        acc = acc[:rows]
    out = acc.float() * scale_x.float() * int8_scale.reshape(1, -1)
    if bias is not None:
        out += bias.float()
    return out.to(x.dtype)


def special_rows(k: int) -> np.ndarray:
    """Rows whose packing a plausible mistake gets wrong (fp32 values)."""
    rows = []
    rows.append(np.zeros(k, np.float32))                              # all zero
    r = np.zeros(k, np.float32); r[0] = 127.0
    r[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]          # half-even ties
    rows.append(r)
    r = np.zeros(k, np.float32); r[k // 2] = -3.0e-3                   # single nonzero
    rows.append(r)
    r = np.full(k, 0.01, np.float32); r[1] = 0.5; r[2] = -0.5          # +absmax and -absmax
    rows.append(r)
    r = (np.arange(k, dtype=np.float32) - k / 2) * np.float32(1e-41)    # fp32 subnormals
    rows.append(r)
    r = np.linspace(-1, 1, k, dtype=np.float32) * np.float32(3.0e-38)  # near the min normal
    rows.append(r)
    r = np.full(k, -7.0, np.float32)                                   # constant negative
    rows.append(r)
    return np.stack(rows)


def weight_cases(rng: np.random.Generator) -> dict[str, np.ndarray]:
    cases = {
        "w16x256": rng.normal(0, 0.02, (16, 256)).astype(np.float32),
        "w33x130": rng.normal(0, 0.02, (33, 130)).astype(np.float32),
        "w64x2048": rng.normal(0, 0.02, (64, 2048)).astype(np.float32),
        "special256": special_rows(256),
        "special130": special_rows(130),
    }
    for label, _n, k in TALKER + PREDICTOR:
        cases[f"slice_{label}"] = rng.normal(0, 0.02, (4, k)).astype(np.float32)
    return cases


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main() -> None:
    rng = np.random.default_rng(20240601)
    out_int8: dict[str, np.ndarray] = {}
    out_fp8: dict[str, np.ndarray] = {}
    for name, w32 in weight_cases(rng).items():
        for src in ("f32", "bf16"):
            w = torch.from_numpy(w32)
            if src == "bf16":
                w = w.to(torch.bfloat16)
            key = f"{name}.{src}"
            out_int8[f"{key}.src"] = w32 if src == "f32" else bf16_bits(w)
            out_fp8[f"{key}.src"] = out_int8[f"{key}.src"]
            for mode in ("ieee", "device"):
                q, s = ref_int8(w, mode)
                out_int8[f"{key}.{mode}.q"] = q.numpy()
                out_int8[f"{key}.{mode}.scale"] = s.numpy()
                out_int8[f"{key}.{mode}.scale_bf16"] = bf16_bits(s.to(torch.bfloat16))
                qf, sf = ref_fp8(w, mode)
                out_fp8[f"{key}.{mode}.q"] = qf.view(torch.uint8).numpy()
                out_fp8[f"{key}.{mode}.scale"] = sf.numpy()
    np.savez_compressed(os.path.join(HERE, "int8_pack.npz"), **out_int8)
    np.savez_compressed(os.path.join(HERE, "fp8_pack.npz"), **out_fp8)

    # fp8 per-token activations: N(0,1) rows, rows with 1% outliers at 20 sigma,
    # an all-zero row and a row below the 1e-6 clamp.
    act: dict[str, np.ndarray] = {}
    for name, (m, k) in {"a1x2048": (1, 2048), "a8x2048": (8, 2048), "a5x130": (5, 130),
                         "a16x6144": (16, 6144)}.items():
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        idx = rng.random((m, k)) < 0.01
        x[idx] = np.where(rng.random(int(idx.sum())) < 0.5, -20.0, 20.0)
        if m >= 4:
            x[1] = 0.0
            x[2] = rng.normal(0, 1, k).astype(np.float32) * np.float32(1e-7)
        xb = torch.from_numpy(x).to(torch.bfloat16)
        act[f"{name}.x"] = bf16_bits(xb)
        for mode in ("ieee", "device"):
            q, s = ref_act_fp8(xb, mode)
            act[f"{name}.{mode}.q"] = q.view(torch.uint8).numpy()
            act[f"{name}.{mode}.scale"] = s.numpy()
    np.savez_compressed(os.path.join(HERE, "act_fp8.npz"), **act)

    # Tiny GEMMs: bf16 x, int8 q, bf16 scale, optional bf16 bias.  Expected values
    # are the fp64 dequantize-then-matmul (torch float64 matmul) and the
    # reference's naive bf16 formula.
    gemm: dict[str, np.ndarray] = {}
    for name, (m, n, k, has_bias) in {"g1x33x257": (1, 33, 257, True), "g3x16x64": (3, 16, 64, False),
                                      "g2x17x130": (2, 17, 130, True), "g4x64x512": (4, 64, 512, False)}.items():
        w = torch.from_numpy(rng.normal(0, 0.02, (n, k)).astype(np.float32)).to(torch.bfloat16)
        q, s = ref_int8(w, "ieee")
        s_b = s.to(torch.bfloat16)
        x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float32)).to(torch.bfloat16)
        bias = torch.from_numpy(rng.normal(0, 0.1, n).astype(np.float32)).to(torch.bfloat16) if has_bias else None
        y64 = x.double() @ (q.double() * s_b.double()[:, None]).t()
        if bias is not None:
            y64 = y64 + bias.double()
        naive = F.linear(x, q.to(torch.bfloat16) * s_b[:, None], bias)
        gemm[f"{name}.x"] = bf16_bits(x)
        gemm[f"{name}.q"] = q.numpy()
        gemm[f"{name}.scale_bf16"] = bf16_bits(s_b)
        if bias is not None:
            gemm[f"{name}.bias"] = bf16_bits(bias)
        gemm[f"{name}.y_f64"] = y64.numpy()
        gemm[f"{name}.y_naive_bf16"] = bf16_bits(naive)
    np.savez_compressed(os.path.join(HERE, "gemm_small.npz"), **gemm)
    int8_w8a8_fixtures()
    silu_mul_fixtures()
    rms_norm_fixtures()
    for f in ("int8_pack", "fp8_pack", "act_fp8", "gemm_small", "int8_w8a8", "silu_mul", "rms_norm"):
        print(f, os.path.getsize(os.path.join(HERE, f + ".npz")), "bytes")


_TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _bits(t: torch.Tensor) -> np.ndarray:
    """bf16 / fp16 tensors as their uint16 bit patterns, fp32 as values."""
    if t.dtype == torch.float32:
        return t.contiguous().numpy().copy()
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def act_int8_rows(rng: np.random.Generator, m: int, k: int) -> np.ndarray:
    """N(0,1) rows with 1% outliers at 20 sigma; from 4 rows on an all-zero row, a row
    below the 1e-6 clamp, and a row of exact half-way quotients (amax 127 makes the
    scale 1 or a hair below it: 0.5, 1.5, ... then sit on rounding ties)."""
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    idx = rng.random((m, k)) < 0.01
    x[idx] = np.where(rng.random(int(idx.sum())) < 0.5, -20.0, 20.0)
    if m >= 4:
        x[1] = 0.0
        x[2] = rng.normal(0, 1, k).astype(np.float32) * np.float32(1e-7)
        x[3] = (np.arange(k, dtype=np.float32) % 16) - np.float32(7.5)
        x[3, 0] = 127.0
    return x


def int8_w8a8_fixtures() -> None:
    """Int8Method.apply: per-token activation codes and scales in each activation
    dtype, and whole linears (x -> y) through torch._int_mm."""
    rng = np.random.default_rng(20240715)
    out: dict[str, np.ndarray] = {}
    for name, (m, k) in {"a1x2048": (1, 2048), "a8x2048": (8, 2048), "a5x130": (5, 130),
                         "a16x1024": (16, 1024)}.items():
        x32 = act_int8_rows(rng, m, k)
        for dt, tdt in _TORCH_DT.items():
            x = torch.from_numpy(x32).to(tdt)
            out[f"act.{name}.{dt}.x"] = _bits(x)
            for mode in ("ieee", "device"):
                q, s = ref_act_int8(x, mode)
                out[f"act.{name}.{dt}.{mode}.q"] = q.numpy()
                out[f"act.{name}.{dt}.{mode}.scale"] = s.float().numpy()
    for name, (m, n, k, has_bias, dt) in {"l1x33x256.bf16": (1, 33, 256, True, "bf16"),
                                          "l3x16x64.bf16": (3, 16, 64, False, "bf16"),
                                          "l20x40x384.bf16": (20, 40, 384, True, "bf16"),
                                          "l2x24x130.f16": (2, 24, 130, True, "f16"),
                                          "l5x48x256.f32": (5, 48, 256, True, "f32")}.items():
        tdt = _TORCH_DT[dt]
        w = torch.from_numpy(rng.normal(0, 0.02, (n, k)).astype(np.float32)).to(tdt)
        x = torch.from_numpy(act_int8_rows(rng, m, k)).to(tdt)
        bias = torch.from_numpy(rng.normal(0, 0.1, n).astype(np.float32)).to(tdt) if has_bias else None
        q, scale = ref_int8(w, "device")
        out[f"lin.{name}.x"] = _bits(x)
        out[f"lin.{name}.qw"] = q.numpy()
        out[f"lin.{name}.sw"] = scale.numpy()
        if bias is not None:
            out[f"lin.{name}.bias"] = _bits(bias)
        for mode in ("ieee", "device"):
            out[f"lin.{name}.{mode}.y"] = _bits(ref_int8_linear(x, q.t().contiguous(), scale, bias, mode))
    np.savez_compressed(os.path.join(HERE, "int8_w8a8.npz"), **out)


def silu_mul_fixtures() -> None:
    """GatedMLP's activation on a fused gate_up output, each dtype: N(0, 3) values, a
    sweep through silu's range, and the extremes (+-0, large magnitudes, the smallest
    normals)."""
    rng = np.random.default_rng(20240801)
    out: dict[str, np.ndarray] = {}
    k = 1024
    gu = rng.normal(0, 3, (6, 2 * k)).astype(np.float32)
    gu[0, :k] = np.linspace(-30, 30, k, dtype=np.float32)
    gu[1, :8] = [0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30, 1e4, -1e4]
    gu[2, k:] = 1.0
    for dt, tdt in _TORCH_DT.items():
        x = torch.from_numpy(gu).to(tdt)
        gate, up = x[:, :k], x[:, k:]
        out[f"{dt}.gate_up"] = _bits(x)
        out[f"{dt}.h"] = _bits(F.silu(gate) * up)
    np.savez_compressed(os.path.join(HERE, "silu_mul.npz"), **out)


def rms_norm_fixtures() -> None:
    """RMSNorm's eager form (qtts/layers/norm.py:120-133, transformers' Qwen3RMSNorm order)
    on torch-CPU, each dtype, for the talker (2048), predictor (1024) and codec (512)
    widths: N(0, 1) rows, a row of 20-sigma outliers, a constant row, a row near zero
    (eps dominates) and a one-hot row."""
    rng = np.random.default_rng(20240901)
    out: dict[str, np.ndarray] = {}
    eps = 1e-6
    for width in (2048, 1024, 512):
        x = rng.normal(0, 1, (6, width)).astype(np.float32)
        x[1, rng.choice(width, 8, replace=False)] *= 20.0
        x[2, :] = 0.75
        x[3, :] *= 1e-4
        x[4, :] = 0.0
        x[4, 7] = -3.0
        w = rng.normal(1.0, 0.2, width).astype(np.float32)
        for dt, tdt in _TORCH_DT.items():
            xt, wt = torch.from_numpy(x).to(tdt), torch.from_numpy(w).to(tdt)
            x32 = xt.to(torch.float32)
            var = x32.pow(2).mean(-1, keepdim=True)
            y = (wt.to(torch.float32) * (x32 * torch.rsqrt(var + eps))).to(tdt)
            out[f"{dt}.{width}.x"] = _bits(xt)
            out[f"{dt}.{width}.w"] = _bits(wt)
            out[f"{dt}.{width}.y"] = _bits(y)
    out["eps"] = np.array(eps, np.float64)
    np.savez_compressed(os.path.join(HERE, "rms_norm.npz"), **out)


if __name__ == "__main__":
    main()
