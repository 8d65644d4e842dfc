/*
 * CPU oracle for the quantized-linear hot path of qtts (danielhua23/tts-inference).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker.  The product
 * path (tts-inference_amd/) never links, loads or calls it.
 *
 * Every function restates one piece of the reference's algorithm in plain C with
 * IEEE fp32 arithmetic (no fast-math, no FMA contraction: see oracle/Makefile).
 *
 * Division semantics.  The reference computes its scales as `tensor / python_float`
 * (qtts/quant/int8.py:54, qtts/quant/fp8.py:48, qtts/quant/fp8.py:77).  torch
 * evaluates that differently by device:
 *   ORACLE_DIV_DEVICE (0): on a GPU tensor the scalar divisor becomes a multiply by
 *       its fp32 reciprocal, `t * fl(1/c)`.  This is the production path: the
 *       reference quantizes after the weights are on the GPU (qtts/quant/int8.py:82).
 *   ORACLE_DIV_IEEE (1):   on a CPU tensor it is an IEEE fp32 division `t / c`.
 * Tensor-by-tensor divisions (`w / scale[:, None]`, `x / scale_x`) are IEEE fp32
 * divisions on both devices.
 *
 * Pins (tests/test_oracle.py): golden fixtures written by torch-CPU executing the
 * reference's expressions (tests/golden/make_golden.py), closed-form special rows
 * (all-zero, +/-absmax, half-even ties), an exhaustive e4m3 check over every bf16
 * input against torch's float8_e4m3fn cast, the OCP e4m3 decode table, and the
 * fp64 GEMM against numpy matmul plus linearity / one-hot invariants.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { ORACLE_DT_F32 = 0, ORACLE_DT_BF16 = 1, ORACLE_DT_F16 = 2 };
enum { ORACLE_DIV_DEVICE = 0, ORACLE_DIV_IEEE = 1 };

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.  This is the rounding
 * torch applies in `tensor.to(torch.bfloat16)` (qtts/quant/int8.py:105). */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* IEEE binary16 <-> fp32 (round to nearest even), written from the format
 * definition: 1 sign, 5 exponent (bias 15), 10 mantissa bits. */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);       /* m * 2^-24, exact */
        return s ? -v : v;
    }
    return u2f(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t u = f2u(f), s = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);   /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                 /* below 2^-14: subnormal */
        float v = u2f(a) * 16777216.0f;                    /* exact scale by 2^24 */
        return (uint16_t)(s | (uint32_t)rintf(v));
    }
    uint32_t mant = (a & 0x7fffffu) | 0x800000u, e = (a >> 23) - 112u;
    uint32_t r = mant >> 13, rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    if (r == 0x800u) { r = 0x400u; e++; }
    return (uint16_t)(s | (e << 10) | (r & 0x3ffu));
}

static float load_elem(const void* base, int dtype, int64_t idx) {
    if (dtype == ORACLE_DT_BF16) return oracle_bf16_to_f32(((const uint16_t*)base)[idx]);
    if (dtype == ORACLE_DT_F16) return oracle_f16_to_f32(((const uint16_t*)base)[idx]);
    return ((const float*)base)[idx];
}

/* Round an fp32 value to the storage dtype and back (identity for fp32). */
static float round_to(float v, int dtype) {
    if (dtype == ORACLE_DT_BF16) return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
    if (dtype == ORACLE_DT_F16) return oracle_f16_to_f32(oracle_f32_to_f16(v));
    return v;
}

/* fp32 -> OCP e4m3fn (bias 7, max finite 448, 0x7f/0xff NaN, no infinities), round
 * to nearest even.  Magnitudes that round past 448, infinities and NaN give NaN
 * (sign kept): torch's float8_e4m3fn cast is non-saturating, and the reference
 * casts with `.to(torch.float8_e4m3fn)` (qtts/quant/fp8.py:49, :78). */
uint8_t oracle_e4m3_encode(float f) {
    uint32_t u = f2u(f), s = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint8_t)(s | 0x7fu);
    if (a < 0x3c800000u) {                       /* below 2^-6: subnormal step 2^-9 */
        float v = u2f(a) * 512.0f;               /* exact scale by 2^9 */
        return (uint8_t)(s | (uint32_t)rintf(v)); /* 8 -> 0x08 = 2^-6, the min normal */
    }
    int32_t e = (int32_t)(a >> 23) - 127 + 7;    /* biased e4m3 exponent, >= 1 here */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t r = mant >> 20, rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r++;
    if (r == 16u) { r = 8u; e++; }
    if (e > 15) return (uint8_t)(s | 0x7fu);
    uint32_t code = ((uint32_t)e << 3) | (r & 7u);
    if (code >= 0x7fu) return (uint8_t)(s | 0x7fu);
    return (uint8_t)(s | code);
}

/* OCP e4m3fn decode (OCP 8-bit floating point specification, E4M3 column). */
float oracle_e4m3_decode(uint8_t c) {
    uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = (float)m * (1.0f / 512.0f);
    else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
    return (c & 0x80u) ? -v : v;
}

static float scalar_div(float num, float den, int div_mode) {
    if (div_mode == ORACLE_DIV_DEVICE) {
        volatile float inv = 1.0f / den;          /* fp32 reciprocal, as torch's GPU kernel */
        return num * inv;
    }
    return num / den;
}

/* Restates quantize_weight_per_channel, qtts/quant/int8.py:45-56:
 *   scale = amax(|w|, dim=1).clamp_min(1e-12) / 127      (fp32)
 *   q     = round_half_even(w / scale).clamp(-127, 127)  (int8)
 * plus the stored-scale cast of qtts/quant/int8.py:105 (scale.to(weight.dtype)),
 * written to scale_store (bf16 or f16 bits, or fp32) when it is not NULL. */
void oracle_pack_int8_rowwise(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld,
                              int8_t* q, float* scale_f32, void* scale_store, int store_dtype,
                              int div_mode) {
    for (int64_t r = 0; r < n; ++r) {
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) {
            float a = fabsf(load_elem(src, src_dtype, r * ld + c));
            if (a > amax) amax = a;
        }
        if (amax < 1e-12f) amax = 1e-12f;
        float scale = scalar_div(amax, 127.0f, div_mode);
        for (int64_t c = 0; c < k; ++c) {
            float v = rintf(load_elem(src, src_dtype, r * ld + c) / scale);
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[r * k + c] = (int8_t)v;
        }
        if (scale_f32) scale_f32[r] = scale;
        if (scale_store) {
            if (store_dtype == ORACLE_DT_BF16) ((uint16_t*)scale_store)[r] = oracle_f32_to_bf16(scale);
            else if (store_dtype == ORACLE_DT_F16) ((uint16_t*)scale_store)[r] = oracle_f32_to_f16(scale);
            else ((float*)scale_store)[r] = scale;
        }
    }
}

/* Restates quantize_weight_fp8, qtts/quant/fp8.py:45-49:
 *   scale = amax(|w|, dim=1).clamp_min(1e-12) / 448 ; q = e4m3(w / scale). */
void oracle_pack_fp8_rowwise(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld,
                             uint8_t* q, float* scale_f32, int div_mode) {
    for (int64_t r = 0; r < n; ++r) {
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) {
            float a = fabsf(load_elem(src, src_dtype, r * ld + c));
            if (a > amax) amax = a;
        }
        if (amax < 1e-12f) amax = 1e-12f;
        float scale = scalar_div(amax, 448.0f, div_mode);
        for (int64_t c = 0; c < k; ++c)
            q[r * k + c] = oracle_e4m3_encode(load_elem(src, src_dtype, r * ld + c) / scale);
        scale_f32[r] = scale;
    }
}

/* Restates the activation quantization inside Fp8Method.apply, qtts/quant/fp8.py:77-78:
 *   scale_x = f32(amax(|x|, dim=1).clamp_min(1e-6)) / 448   (amax and clamp in x's dtype)
 *   qx      = e4m3(f32(x) / scale_x)
 * The clamp compares against 1e-6 rounded to x's dtype, as torch's clamp_min does. */
void oracle_quant_act_fp8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ld,
                          uint8_t* qx, float* sx, int div_mode) {
    float floor_v = round_to(1e-6f, x_dtype);
    for (int64_t r = 0; r < m; ++r) {
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) {
            float a = fabsf(load_elem(x, x_dtype, r * ld + c));
            if (a > amax) amax = a;
        }
        if (amax < floor_v) amax = floor_v;
        float s = scalar_div(amax, 448.0f, div_mode);
        for (int64_t c = 0; c < k; ++c)
            qx[r * k + c] = oracle_e4m3_encode(load_elem(x, x_dtype, r * ld + c) / s);
        sx[r] = s;
    }
}

/* Dequantize-then-matmul in fp64 (the north-star oracle for the W8A16 GEMM,
 * qtts/quant/kernels.py:113-132 computes the same sum in fp32 with bf16 products):
 *   y[i, j] = sum_c x[i, c] * q[j, c] * scale[j] + bias[j]
 * x is fp32 [m, k] (callers widen bf16 first), q int8 [n, k], scale fp32 [n]
 * (the stored scale widened), bias fp32 [n] or NULL. */
void oracle_w8a16_ref_f64(const float* x, int64_t m, int64_t k, const int8_t* q, int64_t n,
                          const float* scale, const float* bias, double* y) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            const float* xr = x + i * k;
            const int8_t* qr = q + j * k;
            for (int64_t c = 0; c < k; ++c) acc += (double)xr[c] * (double)qr[c];
            acc *= (double)scale[j];
            if (bias) acc += (double)bias[j];
            y[i * n + j] = acc;
        }
}

/* fp8 W8A8 oracle: y = (qx * sx) @ (qw * sw)^T (+ bias), in fp64 (qtts/quant/fp8.py:79-89). */
void oracle_w8a8_ref_f64(const uint8_t* qx, const float* sx, int64_t m, int64_t k,
                         const uint8_t* qw, int64_t n, const float* sw, const float* bias,
                         double* y) {
    static double lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = (double)oracle_e4m3_decode((uint8_t)c);
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (int64_t c = 0; c < k; ++c) acc += lut[qx[i * k + c]] * lut[qw[j * k + c]];
            acc *= (double)sx[i] * (double)sw[j];
            if (bias) acc += (double)bias[j];
            y[i * n + j] = acc;
        }
}

/* Restates the activation quantization inside Int8Method.apply, qtts/quant/int8.py:147-149,
 * where every step runs on a tensor of x's dtype and so rounds to it:
 *   scale_x = dtype(dtype(amax(|x|, dim=1)).clamp_min(dtype(1e-6)) / 127)
 *   q       = clamp(round_half_even(dtype(f32(x) / f32(scale_x))), -127, 127)
 * A NaN quotient (0 / 0 once an fp16 scale underflows to zero) becomes code 0, what
 * the float -> int8 conversion of torch's GPU kernels gives it.  sx holds the scale
 * widened to fp32. */
void oracle_quant_act_int8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ld,
                           int8_t* qx, float* sx, int div_mode) {
    float floor_v = round_to(1e-6f, x_dtype);
    for (int64_t r = 0; r < m; ++r) {
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) {
            float a = fabsf(load_elem(x, x_dtype, r * ld + c));
            if (a > amax) amax = a;
        }
        if (amax < floor_v) amax = floor_v;
        float s = round_to(scalar_div(amax, 127.0f, div_mode), x_dtype);
        for (int64_t c = 0; c < k; ++c) {
            float v = rintf(round_to(load_elem(x, x_dtype, r * ld + c) / s, x_dtype));
            if (isnan(v)) v = 0.0f;
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            qx[r * k + c] = (int8_t)v;
        }
        sx[r] = s;
    }
}

/* Restates torch._int_mm and the fp32 epilogue of Int8Method.apply,
 * qtts/quant/int8.py:151-160:
 *   acc = qx @ qw^T                 exact integer sum, taken modulo 2^32 as int32
 *   out = (f32(acc) * sx[i]) * sw[j] [+ f32(bias[j])]   each step one fp32 rounding
 *   y   = out rounded to out_dtype (bits for bf16 / f16, fp32 values otherwise)
 * qw is [n, k] (the reference multiplies by its [k, n] transpose).  bias: [n] in
 * out_dtype or NULL. */
void oracle_int8_linear_out(const int8_t* qx, const float* sx, int64_t m, int64_t k,
                            const int8_t* qw, int64_t n, const float* sw, const void* bias,
                            int out_dtype, void* y) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (int64_t c = 0; c < k; ++c) acc += (int64_t)qx[i * k + c] * (int64_t)qw[j * k + c];
            int32_t a32 = (int32_t)(uint32_t)(uint64_t)acc;
            float v = (float)a32 * sx[i];
            v = v * sw[j];
            if (bias) v = v + load_elem(bias, out_dtype, j);
            if (out_dtype == ORACLE_DT_BF16) ((uint16_t*)y)[i * n + j] = oracle_f32_to_bf16(v);
            else if (out_dtype == ORACLE_DT_F16) ((uint16_t*)y)[i * n + j] = oracle_f32_to_f16(v);
            else ((float*)y)[i * n + j] = v;
        }
}

/* fp8 weight-only oracle (the fused kernel qtts/quant/fp8.py:92-123 calls for, with the
 * W8A16 formula of qtts/quant/kernels.py:113-135): dequantize-then-matmul in fp64,
 *   y[i, j] = sum_c x[i, c] * e4m3(q[j, c]) * scale[j] + bias[j]
 * x fp32 [m, k] (callers widen bf16 first), q e4m3 codes [n, k], scale fp32 [n],
 * bias fp32 [n] or NULL. */
void oracle_fp8w_ref_f64(const float* x, int64_t m, int64_t k, const uint8_t* q, int64_t n,
                         const float* scale, const float* bias, double* y) {
    double lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = (double)oracle_e4m3_decode((uint8_t)c);
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (int64_t c = 0; c < k; ++c) acc += (double)x[i * k + c] * lut[q[j * k + c]];
            acc *= (double)scale[j];
            if (bias) acc += (double)bias[j];
            y[i * n + j] = acc;
        }
}

/* GatedMLP's activation, qtts/layers/activation.py:147 (`F.silu(gate) * up` on tensors
 * of the activation dtype): silu in fp32 with torch's formula g / (1 + exp(-g)) rounded
 * to the dtype, then the product in fp32 rounded to the dtype.  gate_up: [m, 2k] (gate
 * then up), row stride ld; h: [m, k].  Values travel as bf16 / fp16 bits or fp32. */
/* RMSNorm (qtts/layers/norm.py:50-76): y = x * (1 / sqrt(mean(x^2) + eps)) * w, the sum of
 * squares and every product in fp64 (the reference reduces in fp32 in an order of its
 * block's choosing, so its result is this value rounded to the dtype, give or take
 * one unit in the last place).  x: [m, k] of dtype, row stride ld; w: [k] of dtype;
 * y: [m, k] fp64. */
void oracle_rms_norm_f64(const void* x, int dtype, int64_t m, int64_t k, int64_t ld, const void* w, double eps,
                         double* y) {
    for (int64_t r = 0; r < m; ++r) {
        double ss = 0.0;
        for (int64_t c = 0; c < k; ++c) {
            const double v = load_elem(x, dtype, r * ld + c);
            ss += v * v;
        }
        const double inv = 1.0 / sqrt(ss / (double)k + eps);
        for (int64_t c = 0; c < k; ++c)
            y[r * k + c] = (double)load_elem(x, dtype, r * ld + c) * inv * (double)load_elem(w, dtype, c);
    }
}

void oracle_silu_mul(const void* gate_up, int dtype, int64_t m, int64_t k, int64_t ld, void* h) {
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < k; ++c) {
            float g = load_elem(gate_up, dtype, r * ld + c);
            float u = load_elem(gate_up, dtype, r * ld + k + c);
            float s = round_to(g / (1.0f + expf(-g)), dtype);
            float v = s * u;
            if (dtype == ORACLE_DT_BF16) ((uint16_t*)h)[r * k + c] = oracle_f32_to_bf16(v);
            else if (dtype == ORACLE_DT_F16) ((uint16_t*)h)[r * k + c] = oracle_f32_to_f16(v);
            else ((float*)h)[r * k + c] = v;
        }
}
