/*
 * qtts_amd — C ABI of the MI355X (gfx950) quantized-linear hot path.
 *
 * One shared library, libqtts_amd.so, built from tts-inference_amd/csrc.  Every
 * entry point takes plain device pointers, sizes in elements, leading dimensions
 * in elements and a hipStream_t passed as void*.  Nothing here allocates device
 * memory, synchronises the stream or reads device memory on the host, so every
 * call can be captured into a hipGraph.  The caller owns every buffer.
 *
 * Return value: QTTS_OK (0) or a negative qtts_status; qtts_last_error() then
 * holds a message for the calling thread.
 */
#ifndef QTTS_AMD_H
#define QTTS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QTTS_ABI_VERSION 1

typedef enum {
    QTTS_OK = 0,
    QTTS_ERR_INVALID_ARGUMENT = -1, /* shapes, strides, dtypes: the reference raises ValueError */
    QTTS_ERR_UNSUPPORTED = -2,      /* no gfx950 device / unsupported combination: RuntimeError */
    QTTS_ERR_NOT_IMPLEMENTED = -3,  /* NotImplementedError */
    QTTS_ERR_HIP = -4,              /* a HIP runtime call failed: RuntimeError */
    QTTS_ERR_WORKSPACE = -5         /* workspace missing or too small: ValueError */
} qtts_status;

/* Element types.  Activations, outputs, biases and stored scales use these codes. */
typedef enum { QTTS_F32 = 0, QTTS_BF16 = 1, QTTS_F16 = 2 } qtts_dtype;

/* How `tensor / python_float` rounds in the reference's scale computations
 * (qtts/quant/int8.py:54, qtts/quant/fp8.py:48, qtts/quant/fp8.py:77).
 * QTTS_DIV_DEVICE: t * fl(1/c), what torch computes for a GPU tensor — the
 *                  reference's production path, since it quantizes on the GPU.
 * QTTS_DIV_IEEE:   t / c, what torch computes for a CPU tensor. */
typedef enum { QTTS_DIV_DEVICE = 0, QTTS_DIV_IEEE = 1 } qtts_div_mode;

/* Kernel family for the GEMMs.  AUTO picks by shape; the calibrator pins one.
 * SKINNY_HALF and SKINNY_QUARTER (qtts_w8a16_gemm_strips, qtts_w8a16_fused_gemm_strips and
 * qtts_w8a16_silu_mul_gemm_strips only): the skinny kernel with each
 * 16-row weight strip shared by 2 (or 4) workgroups of 8 (or 4) rows, for at most 8 (or 4)
 * activation rows, K a multiple of 128 (or 256) and no split; AUTO takes them where the
 * strips alone would leave compute units idle.  qtts_w8a16_gemm_strips also runs SKINNY_HALF on
 * 9-64 activation rows, and the fused entry points on 9-16, in row parts of 8 (ceil(m / 8)
 * workgroups per half strip, each staging its own rows; AUTO takes them on layers of few strips
 * and small weights). */
typedef enum {
    QTTS_ALGO_AUTO = 0,
    QTTS_ALGO_SKINNY = 1,
    QTTS_ALGO_TILE = 2,
    QTTS_ALGO_SKINNY_HALF = 3,
    QTTS_ALGO_SKINNY_QUARTER = 4
} qtts_algo;

/* Weight policy flag, OR-ed into any `algo` of the GEMM and linear entry points (and of
 * qtts_workspace_bytes, which ignores it).  With it the decode kernels (the skinny and fused
 * W8A16, fp8 weight-only, fp8 and int8 W8A8 kernels, at most 16 activation rows) load the
 * weight non-temporally: for weights that each step reads once and that are too large to
 * stay in the Infinity Cache between steps, so that their stream does not evict the cached
 * activations or the lines of smaller, reused weights.  Results are the same bits either
 * way; the tile kernels ignore it (their tiles re-read the weight). */
#define QTTS_ALGO_STREAM 0x80

/* Strip layouts (see qtts_to_strips). */
typedef enum { QTTS_STRIP_INT8 = 0, QTTS_STRIP_FP8 = 1 } qtts_strip_kind;

/* Workspace owners for qtts_workspace_bytes. */
typedef enum {
    QTTS_OP_W8A16 = 0,
    QTTS_OP_W8A8_FP8 = 1,
    QTTS_OP_FP8_LINEAR = 2,
    QTTS_OP_W8A8_INT8 = 3,
    QTTS_OP_INT8_LINEAR = 4,
    QTTS_OP_FP8W = 5,
    QTTS_OP_W8A16_SILU = 6,
    QTTS_OP_W8A16_FUSED = 7
} qtts_op;

/* What qtts_w8a16_fused_gemm_strips applies to its activations before the GEMM. */
typedef enum { QTTS_PRO_NONE = 0, QTTS_PRO_SILU_MUL = 1, QTTS_PRO_RMS_NORM = 2 } qtts_prologue;

/* --- housekeeping ------------------------------------------------------------ */

int qtts_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* qtts_last_error(void);

/* 1 if `device` is a gfx950 GPU this library can run on, 0 otherwise.
 * Replaces the capability test of fp8_supported (qtts/quant/base.py:133-152)
 * and the Triton check of kernel_available (qtts/quant/kernels.py:83-84). */
int qtts_device_supported(int device);

/* Bytes of workspace `op` needs for an [m, k] x [n, k]^T product with `algo`
 * (QTTS_ALGO_AUTO: the largest any automatic choice uses).  The workspace holds
 * split-K counters and partial sums.  It must be zero-filled before its first use
 * with this library; every call leaves its counters at zero again (partial sums
 * need no clearing), so one buffer serves any number of calls, including graph
 * replays, with no memset.  Calls that share a workspace must be ordered (one
 * stream); concurrent calls on one workspace race.  A buffer smaller than a
 * call's automatic choice needs is not an error: the call then runs without
 * split-K.  An explicit split count (algo bits 8-15) that does not fit is.
 *
 * `algo` for the GEMMs: a qtts_algo in bits 0-7; bits 8-15 set the number of K
 * splits across workgroups (a minimum for the skinny kernels, which add splits
 * until each wave's share fits its in-flight group).  For the skinny kernels, bits
 * 16-23 are the waves per workgroup (1, 2, 4, 8, 16) and bits 24-29 the chunks in
 * flight per wave (4 or 8; 4 or 6 with 16 waves; W8A16 calls of up to 8 rows on
 * strip weights with K % 64 == 0 also take 12 with 8 waves).  Those W8A16 calls, and
 * calls of 9-16 rows with one split on at most 128 strips (two row parts of 8), stage
 * their activation rows through
 * LDS; bit 30 makes them load the MFMA operands straight from memory instead (same
 * bits out, for timing both).  For the tile kernels, bits
 * 16-21 are the LDS pipeline stages (2, 3, 4, 6, 8; the int8 W8A8 tile builds 2-4),
 * bit 22 reads each stage's operands from LDS one stage ahead (3 stages or more), bit
 * 23 (W8A16 and fp8 weight-only) makes a stage two 64-column chunks (4-wave 32 x 64
 * tiles with 3 or 4 stages and read-ahead, an even chunk count per split; same bits as
 * one chunk a stage), and bits 16-23 all zero pick stages, read-ahead and chunks a
 * stage automatically.  Bits 24-30 are a tile shape code c: bits 28-30 (c >> 4) log2(BN / 32) in 1..3;
 * bit 27 (c & 8) 8 waves a workgroup in place of 4 (two a SIMD; 3 or 4 stages);
 * for W8A16 bits 24-25 (c & 3) log2(BM / 16) in 1..3 (0: 256 rows, 8 waves only) and
 * bit 26 (c & 4) a 2 x 2 (2 x 4) wave grid in place of 1 x 4 (1 x 8); for W8A8 (fp8,
 * int8) bits 24-26 (c & 7) log2(BM / 16) in 1..3, 8 waves on BM 64 or 128 and BN 128
 * or 256.  Tiles with 8 waves are built where the grid divides the tile (W8A16:
 * 64 x 128, 64 x 256, 128 x 256 and, with BN code 4, 128 x 384 (3 stages, no read-ahead)
 * on 1 x 8; 32 x 64, 64 x 128, 128 x 128, 128 x 256, 256 x 128 on 2 x 4).  0 = automatic
 * everywhere.  The calibrator uses these to time variants. */
int64_t qtts_workspace_bytes(int op, int64_t m, int64_t n, int64_t k, int algo);

/* --- weight packers ------------------------------------------------------------ */

/* Symmetric per-output-channel int8, replacing quantize_weight_per_channel
 * (qtts/quant/int8.py:45-56) plus the stored-scale cast of
 * Int8WeightOnlyMethod.process_weights (qtts/quant/int8.py:105):
 *   scale[r] = max(amax_c |w[r,c]|, 1e-12) / 127         (fp32, div_mode)
 *   q[r, c]  = clamp(round_half_even(w[r,c] / scale[r]), -127, 127)
 * src: [n, k] of src_dtype with row stride ld_src.  q_out: [n, k] int8, row
 * stride k.  scale_out: [n] of scale_dtype (rounded to nearest even from fp32).
 * scale_f32_out: optional [n] fp32 copy of the unrounded scale (NULL to skip). */
int qtts_pack_int8_rowwise(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld_src,
                           int8_t* q_out, void* scale_out, int scale_dtype, float* scale_f32_out,
                           int div_mode, void* stream);

/* Symmetric per-output-channel OCP e4m3fn, replacing quantize_weight_fp8
 * (qtts/quant/fp8.py:45-49):
 *   scale[r] = max(amax_c |w[r,c]|, 1e-12) / 448 ; q = e4m3_rne(w / scale)
 * q_out: [n, k] e4m3 bytes, row stride k; scale_out: [n] fp32. */
int qtts_pack_fp8_e4m3_rowwise(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld_src,
                               uint8_t* q_out, float* scale_out, int div_mode, void* stream);

/* --- strip layout ------------------------------------------------------------------ */

/* The [n, k] weight bytes re-tiled so that each wavefront load of the GEMM kernels
 * is one contiguous 1 KiB: 16-row strips, CH-column chunks (CH = 64 for
 * QTTS_STRIP_INT8, 128 for QTTS_STRIP_FP8), block (s, c) of 16*CH bytes at
 * (s * ceil(k/CH) + c) * 16 * CH; inside it, half h and lane l (0..63) own the 16
 * bytes at h*1024 + l*16 = row 16s + l%16, columns CH*c + (l/16)*(CH/4) + 16h .. +15.
 * Rows >= n and columns >= k are zero.  A pure permutation of the packer's output:
 * qtts_from_strips recovers the row-major bytes exactly.  No counterpart in the
 * reference, whose Triton kernel reads the row-major buffer (qtts/quant/kernels.py:108-117);
 * the quant methods store this layout in place of it. */
int64_t qtts_strip_bytes(int64_t n, int64_t k, int kind);
int qtts_to_strips(const void* src, int64_t n, int64_t k, int64_t ld_src, int kind, void* dst, void* stream);
int qtts_from_strips(const void* src, int64_t n, int64_t k, int kind, void* dst, int64_t ld_dst, void* stream);

/* Codes a QTTS_STRIP_INT8 matrix can hold: int8 (the int8 weight-only and W8A8
 * methods) or OCP e4m3 (the fp8 weight-only method). */
typedef enum { QTTS_CODE_INT8 = 0, QTTS_CODE_E4M3 = 1 } qtts_code_kind;

/* w[r, c] = w_dtype(f32(code[r, c]) * f32(scale[r])): the dequantized weight of the
 * reference's dequantize-then-matmul form, q.to(dtype) * scale[:, None]
 * (qtts/quant/kernels.py:144-148), from a QTTS_STRIP_INT8 matrix of `codes`.  The int8
 * weight-only method runs it ahead of a plain library GEMM for the prefill row counts
 * its calibration gives to that route (the bf16 baseline the calibration times).
 * qs: qtts_strip_bytes(n, k, QTTS_STRIP_INT8) bytes.  scale: [n] of scale_dtype (bf16,
 * fp16 or fp32).  w: [n, k] of w_dtype (bf16, fp16 or fp32), row stride ldw >= k. */
int qtts_dequant_strips(const void* qs, int codes, int64_t n, int64_t k, const void* scale, int scale_dtype,
                        void* w, int w_dtype, int64_t ldw, void* stream);

/* --- W8A16: int8 weights, bf16/fp16/fp32 activations ----------------------------- */

/* y[m, n] = cast(sum_c x[m,c] * q[n,c] * f32(scale[n]) + f32(bias[n])), fp32
 * accumulation, replacing w8_gemm (qtts/quant/kernels.py:138-178) and its kernel
 * _w8_gemm_kernel (qtts/quant/kernels.py:89-135).
 * x: [m, k] of x_dtype, row stride ldx.  q: [n, k] int8, row stride ldq.
 * scale: [n] of scale_dtype.  bias: [n] of x_dtype, or NULL.  y: [m, n] of x_dtype,
 * row stride ldy.  ws/ws_bytes: workspace (see qtts_workspace_bytes); may be NULL
 * when the chosen kernel needs none. */
int qtts_w8a16_gemm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                    const int8_t* q, int64_t n, int64_t ldq,
                    const void* scale, int scale_dtype, const void* bias,
                    void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream);

/* qtts_w8a16_gemm with the weight in the QTTS_STRIP_INT8 layout (qs, qtts_strip_bytes
 * bytes).  x must be bf16 or fp16 with 16-byte aligned rows and k % 16 == 0. */
int qtts_w8a16_gemm_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                           const int8_t* qs, int64_t n, const void* scale, int scale_dtype,
                           const void* bias, void* y, int64_t ldy, int algo, void* ws,
                           int64_t ws_bytes, void* stream);

/* --- GatedMLP: activation and down projection ----------------------------------- */

/* The activation of GatedMLP.forward (qtts/layers/activation.py:142-147) in one pass:
 *   h[r, c] = dtype(dtype(silu(g)) * u),  g = gate_up[r, c], u = gate_up[r, k + c],
 *   silu(g) = g / (1 + exp(-g)) in fp32
 * with torch's rounding for `F.silu(gate) * up` on x_dtype tensors (two kernels there).
 * gate_up: [m, 2k] of x_dtype, row stride ld_gate_up (the fused gate_up_proj output,
 * gate then up).  h: [m, k], row stride ldh. */
int qtts_silu_mul(const void* gate_up, int x_dtype, int64_t m, int64_t k, int64_t ld_gate_up,
                  void* h, int64_t ldh, void* stream);

/* down_proj(F.silu(gate) * up) with an int8 weight-only down projection on strip
 * weights: qtts_w8a16_gemm_strips of qtts_silu_mul's output, in one call.  A single
 * decode row (m == 1, k % 64 == 0) has the activation computed inside the GEMM kernel
 * while it stages its activation row; other calls run qtts_silu_mul into the workspace
 * first.  Same bits either way.  x_dtype bf16 or fp16; workspace: qtts_workspace_bytes(QTTS_OP_W8A16_SILU). */
int qtts_w8a16_silu_mul_gemm_strips(const void* gate_up, int x_dtype, int64_t m, int64_t k,
                                    int64_t ld_gate_up, const int8_t* qs, int64_t n,
                                    const void* scale, int scale_dtype, const void* bias,
                                    void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes,
                                    void* stream);

/* --- the decoder layer around the W8A16 GEMM -------------------------------------- */

/* RMSNorm._fused_forward (qtts/layers/norm.py:50-76, 103-118), one row per call row:
 *   inv = 1 / sqrt(sum_c f32(x[r,c])^2 / k + eps)   (fp32, correctly rounded)
 *   y[r, c] = dtype((f32(x[r,c]) * inv) * f32(weight[c]))
 * x, y: [m, k] of x_dtype (row strides ldx, ldy); weight: [k] of x_dtype. */
int qtts_rms_norm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* weight,
                  float eps, void* y, int64_t ldy, void* stream);

/* One W8A16 linear of the talker's decoder layer (qtts/models/talker.py:246-271) with
 * its neighbours, on strip weights (k % 64 == 0, bf16 / fp16 activations):
 *   y = [residual +] linear(prologue(x))
 *   prologue QTTS_PRO_NONE:     x [m, k];
 *            QTTS_PRO_SILU_MUL: x is the gate_up output [m, 2k], h = silu(gate) * up
 *                               as qtts_silu_mul (GatedMLP.forward, activation.py:142-147);
 *            QTTS_PRO_RMS_NORM: x [m, k], h = qtts_rms_norm(x, norm_weight, eps)
 *                               (input_layernorm before qkv_proj, post_attention_layernorm
 *                               before gate_up_proj);
 *   residual: [m, n] of x_dtype, row stride ldr, or NULL; y = dtype(f32(residual) +
 *   f32(linear)), the linear rounded to x_dtype first, as `residual + o_proj(...)`
 *   (talker.py:270-271).  residual may be y itself (an in-place hidden-state update).
 * Fused into the GEMM launch (prologue computed while the activation rows are staged,
 * residual added in the epilogue): SiLU for m == 1, RMSNorm for m <= 16 (without a
 * residual and without split-K), the residual for m <= 16 (9-16 rows in two row parts of
 * 8 with one split) and up to 64 on half strips (row parts of 8).  Otherwise the separate kernels run around qtts_w8a16_gemm_strips,
 * through the workspace.  SiLU and the residual give the same bits either way; a fused
 * RMSNorm stages dtype((x * inv) * w) as qtts_rms_norm does, with its sum of squares in
 * another order.  scale_dtype: x_dtype or fp32 for the fused launches (any
 * for the separate ones).  Workspace: qtts_workspace_bytes(QTTS_OP_W8A16_FUSED). */
int qtts_w8a16_fused_gemm_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                                 int prologue, const void* norm_weight, float eps,
                                 const int8_t* qs, int64_t n, const void* scale, int scale_dtype,
                                 const void* bias, const void* residual, int64_t ldr, void* y,
                                 int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream);

/* GatedMLP's gate_up_proj and activation (qtts/layers/activation.py:142-147), optionally
 * after post_attention_layernorm (qtts/models/talker.py:271), on int8 strip weights:
 *   h = x (QTTS_PRO_NONE) or qtts_rms_norm(x, norm_weight, eps) (QTTS_PRO_RMS_NORM),
 *   g | u = w8a16_linear(h) (qs: the fused [n, k] gate_up weight, gate rows first),
 *   act[r, c] = dtype(dtype(silu(g[r, c])) * u[r, c])   for c < n / 2
 * with the rounding of qtts_w8a16_fused_gemm_strips followed by qtts_silu_mul.  Up to 16
 * decode rows with n % 32 == 0 run as ONE launch (a workgroup holds gate strip s and up
 * strip s + n/32 and writes the activation from its epilogue; the gate_up output is
 * never stored); otherwise the prologue, the GEMM and qtts_silu_mul run in turn through
 * the workspace.  No counterpart in the reference, which stores gate_up and runs the
 * activation as two more kernels.  x: [m, k] bf16 / fp16, 16-byte aligned rows, k % 64 == 0.
 * act: [m, n / 2], row stride ldact.  Workspace: qtts_workspace_bytes(QTTS_OP_W8A16_FUSED). */
int qtts_w8a16_gate_up_silu_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                                   int prologue, const void* norm_weight, float eps,
                                   const int8_t* qs, int64_t n, const void* scale, int scale_dtype,
                                   const void* bias, void* act, int64_t ldact, int algo, void* ws,
                                   int64_t ws_bytes, void* stream);

/* --- fp8 W8A8 --------------------------------------------------------------------- */

/* Per-token e4m3 activation quantization, replacing the activation half of
 * Fp8Method.apply (qtts/quant/fp8.py:77-78):
 *   sx[r] = f32(max(amax_c |x[r,c]|, dtype(1e-6))) / 448  (amax and clamp in x_dtype)
 *   qx[r, c] = e4m3_rne(f32(x[r,c]) / sx[r])
 * qx: [m, k] e4m3 bytes, row stride k.  sx: [m] fp32. */
int qtts_quant_act_fp8_rows(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                            uint8_t* qx, float* sx, int div_mode, void* stream);

/* y[m, n] = cast(cast(sum_c qx[m,c] * qw[n,c] * sx[m] * sw[n]) + bias[n]), fp32
 * accumulation on fp8 MFMA, replacing torch._scaled_mm with rowwise scales and the
 * bias add that follows it (qtts/quant/fp8.py:79-89).  The product is rounded to
 * out_dtype before the bias is added in out_dtype, as the reference does.
 * qx: [m, k] e4m3, row stride ldqx.  qw: [n, k] e4m3, row stride ldqw.
 * bias: [n] of out_dtype or NULL.  y: [m, n] of out_dtype (QTTS_BF16/F16/F32). */
int qtts_w8a8_fp8_gemm(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                       const uint8_t* qw, int64_t n, int64_t ldqw, const float* sw,
                       const void* bias, void* y, int out_dtype, int64_t ldy,
                       int algo, void* ws, int64_t ws_bytes, void* stream);

/* The whole of Fp8Method.apply (qtts/quant/fp8.py:72-89) in one call:
 * qtts_quant_act_fp8_rows into the workspace, then qtts_w8a8_fp8_gemm.
 * x: [m, k] of x_dtype; y: [m, n] of x_dtype, not overlapping x; bias: [n] of x_dtype
 * or NULL.  Workspace: qtts_workspace_bytes(QTTS_OP_FP8_LINEAR).
 * Decode rows on strip weights (qtts_fp8_linear_strips) with bf16 / fp16 activations in
 * 16-byte aligned rows, 1 <= m <= 8 and k % 128 == 0, k <= 6144, run ONE kernel that
 * quantizes x inside the GEMM, with the same output bits as the two-kernel path and no
 * workspace (ws may be NULL): automatically for m <= 3, or m <= 8 with k <= 2048; and for
 * any such m when algo is QTTS_ALGO_AUTO or QTTS_ALGO_SKINNY with only bits 16-23 set, which
 * then give that kernel's waves per workgroup (a power of two up to 16 with
 * 3 * waves >= k / 128).  Any split count (bits 8-15) or chunk count (bits 24-29) keeps
 * the two-kernel path. */
int qtts_fp8_linear(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                    const uint8_t* qw, int64_t n, int64_t ldqw, const float* sw,
                    const void* bias, void* y, int64_t ldy, int div_mode,
                    int algo, void* ws, int64_t ws_bytes, void* stream);

/* qtts_w8a8_fp8_gemm and qtts_fp8_linear with the weight in the QTTS_STRIP_FP8
 * layout.  Activation rows must be 16-byte aligned and k % 32 == 0. */
int qtts_w8a8_fp8_gemm_strips(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                              const uint8_t* qws, int64_t n, const float* sw, const void* bias,
                              void* y, int out_dtype, int64_t ldy, int algo, void* ws,
                              int64_t ws_bytes, void* stream);
int qtts_fp8_linear_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                           const uint8_t* qws, int64_t n, const float* sw, const void* bias,
                           void* y, int64_t ldy, int div_mode, int algo, void* ws, int64_t ws_bytes,
                           void* stream);

/* qtts_fp8_linear_strips with no workspace argument and no allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its workspace is a
 * library-owned device array of QTTS_STATIC_SCRATCH_BYTES on each GPU it runs on, held
 * until the process ends; the call itself allocates nothing and synchronises nothing.
 * Every call on one GPU shares that GPU's array and leaves its last contents there, so
 * calls that overlap on one GPU (concurrent streams or threads) race: order them on one
 * stream.  A call whose activation codes do not fit (64 KiB of split-K counters, m * k code
 * bytes and 4 m scale bytes, each rounded up to 256) fails with QTTS_ERR_WORKSPACE; a split-K
 * choice that does not fit in the rest runs without the split.  Arguments and results are
 * those of qtts_fp8_linear_strips (decode rows that take the one-kernel path use no
 * workspace at all). */
#define QTTS_STATIC_SCRATCH_BYTES (32ll << 20)
int qtts_fp8_linear_strips_static(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                                  const uint8_t* qws, int64_t n, const float* sw, const void* bias,
                                  void* y, int64_t ldy, int div_mode, int algo, void* stream);

/* --- int8 W8A8 -------------------------------------------------------------------- */

/* Per-token int8 activation quantization, replacing the activation half of
 * Int8Method.apply (qtts/quant/int8.py:146-149).  Every step is in x_dtype, as the
 * reference computes it on an x_dtype tensor:
 *   s[r]      = dtype(max(amax_c |x[r,c]|, dtype(1e-6)) / 127)           (div_mode)
 *   qx[r, c]  = clamp(round_half_even(dtype(f32(x[r,c]) / s[r])), -127, 127)
 * A NaN quotient (0 / 0 when an fp16 scale underflows to zero) stores code 0.
 * qx: [m, k] int8, row stride k.  sx: [m] fp32 (the x_dtype scale, widened exactly). */
int qtts_quant_act_int8_rows(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                             int8_t* qx, float* sx, int div_mode, void* stream);

/* y[m, n] = cast(((f32(acc) * sx[m]) * sw[n]) + f32(bias[n])), acc = sum_c qx[m,c] * qw[n,c]
 * in exact int32 on int8 MFMA, replacing torch._int_mm and the fp32 epilogue that
 * follows it (qtts/quant/int8.py:151-160).  Each fp32 step rounds on its own and the
 * result is rounded once to out_dtype, so the output is bit-identical to the
 * reference's for the same codes and scales (K <= 133,000 keeps acc from wrapping;
 * torch._int_mm wraps the same way past it).
 * qx: [m, k] int8, row stride ldqx.  qw: [n, k] int8, row stride ldqw (the
 * reference stores the transpose, [k, n]).  sx: [m] fp32.  sw: [n] fp32 (the
 * unrounded per-channel scale, int8.py:140).  bias: [n] of out_dtype or NULL.
 * y: [m, n] of out_dtype.  algo as for the other GEMMs: SKINNY serves any m, TILE
 * needs k % 128 == 0 and 16-byte aligned rows (else the skinny kernel runs).  AUTO
 * takes SKINNY for m <= 16 and, on strip weights, up to m = 128 while
 * ceil(m / 16) * n * k <= 24 MiB; TILE otherwise. */
int qtts_w8a8_int8_gemm(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                        const int8_t* qw, int64_t n, int64_t ldqw, const float* sw,
                        const void* bias, void* y, int out_dtype, int64_t ldy,
                        int algo, void* ws, int64_t ws_bytes, void* stream);

/* The whole of Int8Method.apply (qtts/quant/int8.py:145-160) in one call:
 * qtts_quant_act_int8_rows into the workspace, then qtts_w8a8_int8_gemm.  The
 * reference's padding to 17 rows for torch._int_mm (int8.py:150-155) has no
 * counterpart: every m runs as is.  x: [m, k] of x_dtype; y: [m, n] of x_dtype, not
 * overlapping x; bias: [n] of x_dtype or NULL.  Workspace: qtts_workspace_bytes(QTTS_OP_INT8_LINEAR).
 * With strip weights, bf16 / fp16 activations (16-byte aligned rows), m <= 8 and
 * k % 64 == 0, k <= 8192, one kernel quantizes inside the GEMM, with the same output
 * bits and no workspace (ws may be NULL): automatically while the per-CU quantization work is small
 * (every workgroup quantizes all m x k activations), or always when algo is
 * QTTS_ALGO_SKINNY with only a wave count (a power of two up to 16) set.  Any split
 * count keeps the two-kernel path. */
int qtts_int8_linear(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                     const int8_t* qw, int64_t n, int64_t ldqw, const float* sw,
                     const void* bias, void* y, int64_t ldy, int div_mode,
                     int algo, void* ws, int64_t ws_bytes, void* stream);

/* qtts_w8a8_int8_gemm and qtts_int8_linear with the weight in the QTTS_STRIP_INT8
 * layout.  Activation rows must be 16-byte aligned and k % 16 == 0. */
int qtts_w8a8_int8_gemm_strips(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                               const int8_t* qws, int64_t n, const float* sw, const void* bias,
                               void* y, int out_dtype, int64_t ldy, int algo, void* ws,
                               int64_t ws_bytes, void* stream);
int qtts_int8_linear_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                            const int8_t* qws, int64_t n, const float* sw, const void* bias,
                            void* y, int64_t ldy, int div_mode, int algo, void* ws, int64_t ws_bytes,
                            void* stream);

/* --- fp8 weight-only: e4m3 weights, bf16 / fp16 activations ---------------------- */

/* y[m, n] = cast(sum_c x[m,c] * e4m3(q[n,c]) * scale[n] + f32(bias[n])): the fused
 * kernel Fp8WeightOnlyMethod names as the home for fp8 weights (qtts/quant/fp8.py:92-123;
 * the reference itself raises NotImplementedError), with the W8A16 GEMM's arithmetic
 * (qtts/quant/kernels.py:113-135): fp32 accumulation of exact e4m3 x activation
 * products, times the fp32 scale, plus the bias, one rounding to x_dtype.
 * qs: the e4m3 codes of qtts_pack_fp8_e4m3_rowwise, permuted by qtts_to_strips with
 * kind QTTS_STRIP_INT8 (the 64-column strips the W8A16 kernels read).  x: bf16 or
 * fp16 with 16-byte aligned rows; k % 64 == 0.  scale: [n] fp32.  bias: [n] of x_dtype
 * or NULL.  algo as for qtts_w8a16_gemm_strips (the skinny kernel takes M <= 16).
 * Workspace: qtts_workspace_bytes(QTTS_OP_FP8W). */
int qtts_fp8w_gemm_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                          const uint8_t* qs, int64_t n, const float* scale, const void* bias,
                          void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream);

/* Kernel timer.  No counterpart in the reference: benchmark instrumentation.
 * Between qtts_kernel_timer_begin and qtts_kernel_timer_end, each kernel the
 * library launches on a stream that is not capturing a graph records a start and
 * stop event bound to that kernel's dispatch (hipExtLaunchKernel), up to
 * max_launches kernels.  qtts_kernel_timer_end waits for them and returns the
 * summed kernel durations, the number of kernels timed and the number launched
 * after the pool ran out.  One timer per process; calls that overlap from several
 * threads all land in the same pool. */
int qtts_kernel_timer_begin(int max_launches);
int qtts_kernel_timer_end(double* total_ms, int64_t* launches, int64_t* untimed);

#ifdef __cplusplus
}
#endif

#endif /* QTTS_AMD_H */
