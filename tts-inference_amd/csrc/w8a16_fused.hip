// The W8A16 decode GEMM with its neighbours in the talker's decoder layer
// (qtts/models/talker.py:246-271), gfx950:
//
//   qkv     = qkv_proj(input_layernorm(hidden))            prologue: RMSNorm
//   hidden  = hidden + o_proj(attn)                         epilogue: residual add
//   gate_up = gate_up_proj(post_attention_layernorm(hidden)) prologue: RMSNorm
//   hidden  = hidden + down_proj(silu(gate) * up)           prologue: SiLU * mul,
//                                                           epilogue: residual add
//
//  * rms_norm_*_kernel: RMSNorm on its own (qtts/layers/norm.py:50-76): fp32 sum of
//    squares, inv = 1 / sqrt(sum / K + eps) correctly rounded, (x * inv) * w rounded
//    to the activation dtype.  One wave a row.
//  * silu_mul_*_kernel: `F.silu(gate) * up` in one pass with torch's two roundings
//    (common.h: silu_mul).
//  * residual_add_kernel: y = residual + t, for calls whose GEMM cannot add it (the
//    GEMM writes t into the workspace: y may be the residual itself).
//  * qtts_launch_w8a16_fused: one skinny launch with the prologue computed while the
//    activation row is staged in LDS and the residual added in the epilogue
//    (skinny.h: PRO, RES) when the call allows it, otherwise the separate kernels
//    around the plain W8A16 GEMM.  Fused: SiLU for one row (for two rows it no longer
//    hides under the weight stream: talker down 9.4 us fused against 9.0 us for the
//    two passes at M = 2; 7.0 against 9.1 us at M = 1); RMSNorm for up to 16 rows without
//    a split-K (every workgroup needs the whole row's sum); the residual for up to 16
//    staged rows (9-16 in two row parts of 8, one split).  A fused and a separate RMSNorm
//    sum in different orders: the fused
//    result is within the GEMM tolerance of the separate one, not bit-identical.
#include "skinny_fused.h"

using namespace qtts;

namespace qtts {

constexpr int kEltThreads = 256;

// 8 elements a thread; rows 16-byte aligned, k % 8 == 0.  Grid: (vector blocks, rows).
template <typename XT>
__global__ __launch_bounds__(kEltThreads) void silu_mul_vec_kernel(const XT* __restrict__ gu, int64_t k, int64_t ld,
                                                                   XT* __restrict__ h, int64_t ldh) {
  const int64_t r = blockIdx.y;
  const int64_t v = (int64_t)blockIdx.x * kEltThreads + threadIdx.x;
  if (8 * v >= k) return;
  const XT* g = gu + r * ld + 8 * v;
  const i32x4_t gv = *(const i32x4_t*)g, uv = *(const i32x4_t*)(g + k);
  *(i32x4_t*)(h + r * ldh + 8 * v) = silu_mul8<XT>(gv, uv);
}

template <typename XT>
__global__ __launch_bounds__(kEltThreads) void silu_mul_kernel(const XT* __restrict__ gu, int64_t k, int64_t ld,
                                                               XT* __restrict__ h, int64_t ldh) {
  const int64_t r = blockIdx.y;
  for (int64_t c = (int64_t)blockIdx.x * kEltThreads + threadIdx.x; c < k; c += (int64_t)gridDim.x * kEltThreads)
    h[r * ldh + c] = from_f32<XT>(silu_mul<XT>(to_f32(gu[r * ld + c]), to_f32(gu[r * ld + k + c])));
}

// RMSNorm, one wave a row, 4 rows a workgroup.  Vector form: 16-bit rows, 16-byte
// aligned, k % 8 == 0; lane l owns elements 512 v + 8 l .. + 7.  The row is read
// twice (the second time from cache): once for the sum, once to scale it.
constexpr int kNormRowsPerBlock = 4;

template <typename XT>
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void rms_norm_vec_kernel(const XT* __restrict__ x, int64_t ldx,
                                                                             const XT* __restrict__ w, int k, float eps,
                                                                             XT* __restrict__ y, int64_t ldy, int m) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kNormRowsPerBlock + (threadIdx.x >> 6);
  if (row >= m) return;
  const XT* xr = x + row * ldx;
  float ss = 0.0f;
  for (int e0 = 8 * lane; e0 < k; e0 += 512) {
    const i32x4_t v = *(const i32x4_t*)(xr + e0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = to_f32(XT{(uint16_t)v[i]}), b = to_f32(XT{(uint16_t)((uint32_t)v[i] >> 16)});
      ss = __builtin_fmaf(a, a, ss);
      ss = __builtin_fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)k + eps);
  for (int e0 = 8 * lane; e0 < k; e0 += 512) {
    const i32x4_t v = *(const i32x4_t*)(xr + e0), wv = *(const i32x4_t*)(w + e0);
    i32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t p = (uint32_t)v[i], q = (uint32_t)wv[i];
      const float h0 = (to_f32(XT{(uint16_t)p}) * inv) * to_f32(XT{(uint16_t)q});
      const float h1 = (to_f32(XT{(uint16_t)(p >> 16)}) * inv) * to_f32(XT{(uint16_t)(q >> 16)});
      o[i] = (int)pack2_f32<XT>(h0, h1);
    }
    *(i32x4_t*)(y + row * ldy + e0) = o;
  }
}

template <typename XT>
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void rms_norm_kernel(const XT* __restrict__ x, int64_t ldx,
                                                                         const XT* __restrict__ w, int k, float eps,
                                                                         XT* __restrict__ y, int64_t ldy, int m) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kNormRowsPerBlock + (threadIdx.x >> 6);
  if (row >= m) return;
  float ss = 0.0f;
  for (int c = lane; c < k; c += 64) {
    const float a = to_f32(x[row * ldx + c]);
    ss = __builtin_fmaf(a, a, ss);
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)k + eps);
  for (int c = lane; c < k; c += 64) y[row * ldy + c] = from_f32<XT>((to_f32(x[row * ldx + c]) * inv) * to_f32(w[c]));
}

// y[r, c] = residual[r, c] + t[r, c] in fp32, rounded once: torch's `residual + out`
// on two tensors of the activation dtype (y may be the residual).  Grid: (column
// blocks, rows).
template <typename XT>
__global__ __launch_bounds__(kEltThreads) void residual_add_kernel(const XT* res, int64_t ldr,
                                                                   const XT* __restrict__ t, int64_t ldt, XT* y,
                                                                   int64_t ldy, int64_t n) {
  const int64_t r = blockIdx.y;
  for (int64_t c = (int64_t)blockIdx.x * kEltThreads + threadIdx.x; c < n; c += (int64_t)gridDim.x * kEltThreads)
    y[r * ldy + c] = from_f32<XT>(to_f32(res[r * ldr + c]) + to_f32(t[r * ldt + c]));
}

}  // namespace qtts

namespace {

int64_t al256(int64_t v) { return (v + 255) & ~(int64_t)255; }
int64_t esize(int dt) { return dt == QTTS_F32 ? 4 : 2; }

int launch_residual_add(const void* res, int64_t ldr, const void* t, int64_t ldt, void* y, int64_t ldy, int x_dtype,
                        int64_t m, int64_t n, hipStream_t st) {
  const dim3 grid((unsigned)std::min<int64_t>((n + kEltThreads - 1) / kEltThreads, 65535), (unsigned)m);
#define QTTS_RES(T) \
  qtts::launch(&residual_add_kernel<T>, grid, dim3(kEltThreads), 0, st, (const T*)res, ldr, (const T*)t, ldt, (T*)y, ldy, n)
  if (x_dtype == QTTS_BF16) QTTS_RES(bf16_t);
  else if (x_dtype == QTTS_F16) QTTS_RES(f16_t);
  else QTTS_RES(float);
#undef QTTS_RES
  return qtts_check_launch("residual_add");
}

}  // namespace

int qtts_launch_w8a16(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n,
                      int64_t ldq, int layout, const void* scale, int scale_dtype, const void* bias, void* y,
                      int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st);
int64_t qtts_w8a16_ws_bytes(int64_t m, int64_t n, int64_t k, int algo);
int qtts_w8a16_xrows_built(int waves, int cpw);

int qtts_launch_silu_mul(const void* gu, int x_dtype, int64_t m, int64_t k, int64_t ld, void* h, int64_t ldh,
                         hipStream_t st) {
  const bool vec = x_dtype != QTTS_F32 && k % 8 == 0 && (uintptr_t)gu % 16 == 0 && (uintptr_t)h % 16 == 0 &&
                   ld % 8 == 0 && ldh % 8 == 0 && k <= (int64_t)8 * kEltThreads * 65535;  // one vector a thread
  const int64_t per = vec ? 8 * kEltThreads : kEltThreads;
  const int64_t bx = std::min<int64_t>((k + per - 1) / per, 65535);
  const dim3 grid((unsigned)bx, (unsigned)m), block(kEltThreads);
  if (vec && x_dtype == QTTS_BF16)
    qtts::launch(&silu_mul_vec_kernel<bf16_t>, grid, block, 0, st, (const bf16_t*)gu, k, ld, (bf16_t*)h, ldh);
  else if (vec)
    qtts::launch(&silu_mul_vec_kernel<f16_t>, grid, block, 0, st, (const f16_t*)gu, k, ld, (f16_t*)h, ldh);
  else if (x_dtype == QTTS_BF16)
    qtts::launch(&silu_mul_kernel<bf16_t>, grid, block, 0, st, (const bf16_t*)gu, k, ld, (bf16_t*)h, ldh);
  else if (x_dtype == QTTS_F16)
    qtts::launch(&silu_mul_kernel<f16_t>, grid, block, 0, st, (const f16_t*)gu, k, ld, (f16_t*)h, ldh);
  else
    qtts::launch(&silu_mul_kernel<float>, grid, block, 0, st, (const float*)gu, k, ld, (float*)h, ldh);
  return qtts_check_launch("silu_mul");
}

int qtts_launch_rms_norm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* w, float eps,
                         void* y, int64_t ldy, hipStream_t st) {
  const bool vec = x_dtype != QTTS_F32 && k % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 &&
                   (uintptr_t)y % 16 == 0 && ldx % 8 == 0 && ldy % 8 == 0;
  const dim3 grid((unsigned)((m + kNormRowsPerBlock - 1) / kNormRowsPerBlock)), block(64 * kNormRowsPerBlock);
#define QTTS_NORM(KER, T) \
  qtts::launch(&KER<T>, grid, block, 0, st, (const T*)x, ldx, (const T*)w, (int)k, eps, (T*)y, ldy, (int)m)
  if (vec && x_dtype == QTTS_BF16) QTTS_NORM(rms_norm_vec_kernel, bf16_t);
  else if (vec) QTTS_NORM(rms_norm_vec_kernel, f16_t);
  else if (x_dtype == QTTS_BF16) QTTS_NORM(rms_norm_kernel, bf16_t);
  else if (x_dtype == QTTS_F16) QTTS_NORM(rms_norm_kernel, f16_t);
  else QTTS_NORM(rms_norm_kernel, float);
#undef QTTS_NORM
  return qtts_check_launch("rms_norm");
}

// Workspace of qtts_launch_w8a16_fused: the GEMM's own (its counter block always
// reserved), then, for calls that run them as separate passes, the GEMM's output
// [m, n] before the residual is added and the prologue's output [m, k].
int64_t qtts_w8a16_fused_ws_bytes(int64_t m, int64_t n, int64_t k, int algo, int x_dtype) {
  return al256(std::max<int64_t>(qtts_w8a16_ws_bytes(m, n, k, algo), kCounterBytes)) + al256(m * n * esize(x_dtype)) +
         al256(m * k * esize(x_dtype));
}

namespace {

// One fused skinny launch: QTTS_OK, 1 when this call cannot be fused (the caller then
// runs the separate kernels), or an error status.  pair: the SiLU-pair gate_up launch
// (in.n is the fused gate_up width; one workgroup per gate strip, no split).
int try_fused(int pro, bool res, const FusedArgs& in, int x_dtype, int sdt, int algo, void* ws, int64_t ws_bytes,
              bool pair = false) {
  const int splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff, cpw = (algo >> 24) & 0x3f;
  const int64_t m = in.m, n = in.n, k = in.k;
  if (pair) {
    const int family = algo & 0xff;
    if (splits > 1 || m > 16 || n % 32 || family == QTTS_ALGO_SKINNY_QUARTER) return 1;
    // Half strips: each workgroup's MFMA operand holds 8 gate rows and their 8 up rows, so the
    // grid and the wave configuration are the plain GEMM's (N/16 workgroups); requested by
    // family, and the automatic choice without a prologue or with more than 256 gate strips.
    // Measured over 28 distinct weights (µs a call, two-strip -> half strips, M = 1 / 8): the
    // talker's gate_up 8.10 -> 6.92 / 8.79 -> 7.97, with the RMSNorm prologue 8.20 -> 7.19 /
    // 10.32 -> 9.97; the code predictor's 4.36 -> 4.16 / 4.55 -> 4.41, but with the prologue
    // 4.37 -> 4.42 / 5.50 -> 5.82 (every workgroup repeats the norm's per-row work, and its 192
    // two-strip workgroups leave fewer of it).
    const bool auto_half = family == QTTS_ALGO_AUTO && (pro == kProNone || n / 32 > 256);
    if (family == QTTS_ALGO_SKINNY_HALF || auto_half) {
      const SkinnyCfg c = skinny_cfg(m, n, k, 1, waves, cpw);
      if (c.S == 1 && pair_half_built(c.waves, c.cpw) && in.ldx <= INT32_MAX) {
        FusedArgs a = in;
        a.c = c;
        a.sub = 2;
        a.blocks = (unsigned)(((int64_t)c.strips + 7) / 8 * 8);
        a.counters = nullptr;
        a.part = nullptr;
        const bool f32s = sdt == QTTS_F32;
        const int mx = m <= 2 ? (int)m : (m <= 4 ? 4 : 8);
        int rc;
        if (pro == kProRmsNorm)
          rc = mx == 1 ? launch_fused<kProRmsNorm, false, 1, true>(x_dtype, f32s, a)
                       : mx == 2 ? launch_fused<kProRmsNorm, false, 2, true>(x_dtype, f32s, a)
                       : (mx == 4 ? launch_fused<kProRmsNorm, false, 4, true>(x_dtype, f32s, a)
                                  : launch_fused<kProRmsNorm, false, 8, true>(x_dtype, f32s, a));
        else
          rc = mx == 1 ? launch_fused<kProNone, false, 1, true>(x_dtype, f32s, a)
                       : mx == 2 ? launch_fused<kProNone, false, 2, true>(x_dtype, f32s, a)
                       : (mx == 4 ? launch_fused<kProNone, false, 4, true>(x_dtype, f32s, a)
                                  : launch_fused<kProNone, false, 8, true>(x_dtype, f32s, a));
        if (rc == 0) return qtts_check_launch("w8a16_gate_up_silu_half");
      }
      if (family == QTTS_ALGO_SKINNY_HALF) return 1;  // the separate path runs it
    }
    if (family == QTTS_ALGO_SKINNY_HALF) return 1;
    SkinnyCfg c = skinny_cfg(m, n / 2, k, 1, waves, cpw);  // one workgroup per gate strip
    // Automatic, without a prologue: twice the plain choice's waves with half its chunks
    // each (measured 4% faster on the talker gate_up at M = 1..8).  With the RMSNorm
    // prologue the plain choice, since every wave repeats the norm's per-row work (the
    // doubled grid measured 6-10% slower).
    if (waves == 0 && cpw == 0 && pro == kProNone && c.cpw == 8 && c.waves <= 8)
      c = skinny_cfg(m, n / 2, k, 1, 2 * c.waves, 4);
    if (c.S != 1 || !pair_built(c.waves, c.cpw)) return 1;
    FusedArgs a = in;
    a.c = c;
    if (in.ldx > INT32_MAX) return 1;
    a.blocks = (unsigned)((c.strips + 7) / 8 * 8);
    a.counters = nullptr;
    a.part = nullptr;
    const bool f32s = sdt == QTTS_F32;
    const int mx = m <= 2 ? (int)m : (m <= 4 ? 4 : 8);  // staged rows: the fewest built that cover m
    int rc;
    if (pro == kProRmsNorm)
      rc = mx == 1 ? launch_fused<kProRmsNorm, false, 1, true>(x_dtype, f32s, a)
                   : mx == 2 ? launch_fused<kProRmsNorm, false, 2, true>(x_dtype, f32s, a)
                   : (mx == 4 ? launch_fused<kProRmsNorm, false, 4, true>(x_dtype, f32s, a)
                              : launch_fused<kProRmsNorm, false, 8, true>(x_dtype, f32s, a));
    else
      rc = mx == 1 ? launch_fused<kProNone, false, 1, true>(x_dtype, f32s, a)
                   : mx == 2 ? launch_fused<kProNone, false, 2, true>(x_dtype, f32s, a)
                   : (mx == 4 ? launch_fused<kProNone, false, 4, true>(x_dtype, f32s, a)
                              : launch_fused<kProNone, false, 8, true>(x_dtype, f32s, a));
    if (rc != 0) return 1;
    return qtts_check_launch("w8a16_gate_up_silu");
  }
  // Row-split strips: the plain launch's choice (w8a16.hip launch_fast), so a fused call and the
  // plain GEMM it replaces give the same bits.
  const int family = algo & 0xff;
  int sub = family == QTTS_ALGO_SKINNY_HALF ? 2 : (family == QTTS_ALGO_SKINNY_QUARTER ? 4 : 1);
  if (sub > 1 && (splits != 0 || !skinny_sub_rows_ok(m, k, sub))) return 1;  // the separate path reports it
  if (family == QTTS_ALGO_AUTO && splits == 0 && (algo >> 16) == 0)
    sub = m <= 8 ? skinny_auto_sub(m, n, k) : skinny_row_parts_sub(m, n, k);
  // Up to 16 rows (9-16 in two row parts of 8); past 16 only on half strips in row parts, where
  // the plain GEMM takes them too.
  if (m > 16 && sub != 2) return 1;
  if (sub > 1) {
    const SkinnyCfg c = skinny_cfg_sub(n, k, sub, waves, cpw);
    if (!fused_sub_built(sub, c.waves, c.cpw) || c.waves * c.cpw < c.cps || in.ldx > INT32_MAX) return 1;
    FusedArgs a = in;
    a.c = c;
    a.sub = sub;
    a.blocks = (unsigned)(((int64_t)c.strips * sub + 7) / 8 * 8);
    a.counters = nullptr;
    a.part = nullptr;
    const bool f32s = sdt == QTTS_F32;
    int rc = 1;
    if (pro == kProSiluMul) rc = res ? launch_fused<kProSiluMul, true, 1>(x_dtype, f32s, a)
                                     : launch_fused<kProSiluMul, false, 1>(x_dtype, f32s, a);
    else if (pro == kProNone && res)
      rc = m == 1 ? launch_fused<kProNone, true, 1>(x_dtype, f32s, a)
                  : m == 2 ? launch_fused<kProNone, true, 2>(x_dtype, f32s, a)
                  : (m <= 4 ? launch_fused<kProNone, true, 4>(x_dtype, f32s, a)
                            : launch_fused<kProNone, true, 8>(x_dtype, f32s, a));
    if (rc != 0) return 1;
    return qtts_check_launch("w8a16_fused_skinny_sub");
  }
  SkinnyCfg c = skinny_cfg(m, n, k, splits, waves, cpw);
  // As the plain staged launch: 8 waves of 12 chunks from 2 to 8 rows for long K.
  if (m >= 2 && m <= 8 && waves == 0 && cpw == 0 && c.waves == 16 && c.S == 1 && 8 * 12 >= (k + 63) / 64)
    c = skinny_cfg(m, n, k, splits, 8, 12);
  const int64_t need = skinny_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 fused: %d splits need %lld workspace bytes, got %lld", c.S,
                            (long long)need, (long long)ws_bytes);
    c = skinny_cfg(m, n, k, 1, 16, 6);  // no room for a split: longer runs per wave
    if (c.S > 1) return 1;
  }
  if (!qtts_w8a16_xrows_built(c.waves, c.cpw)) return 1;
  if ((pro == kProRmsNorm || m > 8) && c.S > 1) return 1;  // row parts need one split
  if (c.S > 1 && c.strips > kMaxSplitTiles) return 1;
  if (c.S > 65535) return 1;  // past the grid's y limit
  const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8;  // grid x; grid y: the K splits
  if (blocks >= ((int64_t)1 << 31) || in.ldx > INT32_MAX) return 1;
  FusedArgs a = in;
  a.c = c;
  a.blocks = (unsigned)blocks;
  a.counters = (unsigned*)ws;
  a.part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
  const bool f32s = sdt == QTTS_F32;
  int rc = 1;
  if (pro == kProSiluMul) rc = res ? launch_fused<kProSiluMul, true, 1>(x_dtype, f32s, a)
                                   : launch_fused<kProSiluMul, false, 1>(x_dtype, f32s, a);
  else if (pro == kProRmsNorm && !res)
    rc = m == 1 ? launch_fused<kProRmsNorm, false, 1>(x_dtype, f32s, a)
                : m == 2 ? launch_fused<kProRmsNorm, false, 2>(x_dtype, f32s, a)
                : (m <= 4 ? launch_fused<kProRmsNorm, false, 4>(x_dtype, f32s, a)
                          : launch_fused<kProRmsNorm, false, 8>(x_dtype, f32s, a));
  else if (pro == kProNone && res)
    rc = m == 1 ? launch_fused<kProNone, true, 1>(x_dtype, f32s, a)
                : m == 2 ? launch_fused<kProNone, true, 2>(x_dtype, f32s, a)
                : (m <= 4 ? launch_fused<kProNone, true, 4>(x_dtype, f32s, a) : launch_fused<kProNone, true, 8>(x_dtype, f32s, a));
  if (rc != 0) return 1;
  return qtts_check_launch("w8a16_fused_skinny");
}

}  // namespace

// y = [residual +] w8a16_linear(prologue(x)) on strip weights (K % 64 == 0).
//   pro kProNone:    x [m, k];
//   pro kProSiluMul: x is the gate_up output [m, 2k] (gate then up), row stride ldx;
//   pro kProRmsNorm: x [m, k], normalized with weight nw [k] (x's dtype) and eps.
// residual [m, n] (row stride ldr, x's dtype) or NULL; it may be y itself.
int qtts_launch_w8a16_fused(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int pro, const void* nw,
                            float eps, const int8_t* qs, int64_t n, const void* scale, int sdt, const void* bias,
                            const void* res, int64_t ldr, void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes,
                            hipStream_t st) {
  const int family = algo & 0xff;
  const bool direct_x = (algo >> 24) & 0x40;
  const bool kernel_ok = k % 64 == 0 && x_dtype != QTTS_F32 && (sdt == x_dtype || sdt == QTTS_F32) &&
                         family != QTTS_ALGO_TILE && !direct_x;
  FusedArgs a{};
  a.m = m;
  a.k = k;
  a.qs = qs;
  a.n = n;
  a.scale = scale;
  a.bias = bias;
  a.aux = nw;
  a.eps = eps;
  a.res = res;
  a.ldr = ldr;
  a.y = y;
  a.ldy = ldy;
  a.st = st;
  const bool x_aligned = (uintptr_t)x % 16 == 0 && (m == 1 || ldx % 8 == 0);
  // 1. The prologue inside the GEMM: SiLU * mul for one row, RMSNorm for up to 16.
  if (pro != kProNone && kernel_ok && x_aligned &&
      ((pro == kProSiluMul && m == 1) || (pro == kProRmsNorm && m <= 16 && !res && (uintptr_t)nw % 16 == 0))) {
    a.x = x;
    a.ldx = ldx;
    const int rc = try_fused(pro, res != nullptr, a, x_dtype, sdt, algo, ws, ws_bytes);
    if (rc != 1) return rc;
  }
  // 2. The prologue as its own pass, into the workspace tail.
  const void* xin = x;
  int64_t ldin = ldx, avail = ws_bytes;
  if (pro != kProNone) {
    const int64_t h_bytes = al256(m * k * esize(x_dtype));
    if (!ws || ws_bytes < kCounterBytes + h_bytes)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 fused: workspace of %lld bytes < %lld needed",
                            (long long)ws_bytes, (long long)qtts_w8a16_fused_ws_bytes(m, n, k, algo, x_dtype));
    avail = (ws_bytes - h_bytes) & ~(int64_t)255;
    void* h = (char*)ws + avail;
    const int rc = pro == kProSiluMul ? qtts_launch_silu_mul(x, x_dtype, m, k, ldx, h, k, st)
                                      : qtts_launch_rms_norm(x, x_dtype, m, k, ldx, nw, eps, h, k, st);
    if (rc != QTTS_OK) return rc;
    xin = h;
    ldin = k;
  }
  // 3. The residual in the GEMM's epilogue (up to 16 staged rows, up to 64 on half strips).
  if (res && kernel_ok && m <= kRowPartsMaxM && (uintptr_t)xin % 16 == 0 && (m == 1 || ldin % 8 == 0)) {
    a.x = xin;
    a.ldx = ldin;
    const int rc = try_fused(kProNone, true, a, x_dtype, sdt, algo, ws, avail);
    if (rc != 1) return rc;
  }
  // 4. The plain GEMM, then the residual (the GEMM writes into the workspace: y may be
  // the residual).
  if (!res)
    return qtts_launch_w8a16(xin, x_dtype, m, k, ldin, qs, n, 0, kLayoutStrips, scale, sdt, bias, y, ldy, algo, ws,
                             avail, st);
  const int64_t t_bytes = al256(m * n * esize(x_dtype));
  if (!ws || avail < t_bytes)
    return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 fused: workspace of %lld bytes < %lld needed",
                          (long long)ws_bytes, (long long)qtts_w8a16_fused_ws_bytes(m, n, k, algo, x_dtype));
  avail = (avail - t_bytes) & ~(int64_t)255;
  void* t = (char*)ws + avail;
  const int rc = qtts_launch_w8a16(xin, x_dtype, m, k, ldin, qs, n, 0, kLayoutStrips, scale, sdt, bias, t, n, algo, ws,
                                   avail, st);
  if (rc != QTTS_OK) return rc;
  return launch_residual_add(res, ldr, t, n, y, ldy, x_dtype, m, n, st);
}

int qtts_launch_w8a16_silu(const void* gu, int x_dtype, int64_t m, int64_t k, int64_t ld, const int8_t* qs, int64_t n,
                           const void* scale, int sdt, const void* bias, void* y, int64_t ldy, int algo, void* ws,
                           int64_t ws_bytes, hipStream_t st) {
  return qtts_launch_w8a16_fused(gu, x_dtype, m, k, ld, kProSiluMul, nullptr, 0.0f, qs, n, scale, sdt, bias, nullptr, 0,
                                 y, ldy, algo, ws, ws_bytes, st);
}

int64_t qtts_w8a16_silu_ws_bytes(int64_t m, int64_t n, int64_t k, int algo, int x_dtype) {
  return qtts_w8a16_fused_ws_bytes(m, n, k, algo, x_dtype);
}

// act = silu(gate) * up of GatedMLP's gate_up_proj(prologue(x)) on strip weights
// (qtts/layers/activation.py:142-147): x [m, k]; prologue none or RMSNorm (nw, eps);
// qs the fused [n, k] gate_up weight (gate rows then up rows, n % 2 == 0); act [m, n/2]
// with row stride ldact.  Up to 16 decode rows (n % 32 == 0): one launch, the activation
// in the GEMM's epilogue.  Otherwise the norm, the GEMM into the workspace and
// silu_mul run one after another.
int qtts_launch_w8a16_gate_up_silu(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int pro,
                                   const void* nw, float eps, const int8_t* qs, int64_t n, const void* scale, int sdt,
                                   const void* bias, void* act, int64_t ldact, int algo, void* ws, int64_t ws_bytes,
                                   hipStream_t st) {
  const int family = algo & 0xff;
  const bool direct_x = (algo >> 24) & 0x40;
  const bool kernel_ok = k % 64 == 0 && x_dtype != QTTS_F32 && (sdt == x_dtype || sdt == QTTS_F32) &&
                         family != QTTS_ALGO_TILE && !direct_x;
  const bool x_aligned = (uintptr_t)x % 16 == 0 && (m == 1 || ldx % 8 == 0);
  if (kernel_ok && x_aligned && (pro == kProNone || (uintptr_t)nw % 16 == 0)) {
    FusedArgs a{};
    a.x = x;
    a.m = m;
    a.k = k;
    a.ldx = ldx;
    a.qs = qs;
    a.n = n;
    a.scale = scale;
    a.bias = bias;
    a.aux = nw;
    a.eps = eps;
    a.y = act;
    a.ldy = ldact;
    a.st = st;
    const int rc = try_fused(pro, false, a, x_dtype, sdt, algo, ws, ws_bytes, true);
    if (rc != 1) return rc;
  }
  // Separately: the prologue and the GEMM through the fused entry (output into the
  // workspace tail), then the activation.
  const int64_t g_bytes = al256(m * n * esize(x_dtype));
  if (!ws || ws_bytes < kCounterBytes + g_bytes)
    return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 gate_up silu: workspace of %lld bytes < %lld needed",
                          (long long)ws_bytes, (long long)qtts_w8a16_fused_ws_bytes(m, n, k, algo, x_dtype));
  const int64_t avail = (ws_bytes - g_bytes) & ~(int64_t)255;
  void* gu = (char*)ws + avail;
  int rc = qtts_launch_w8a16_fused(x, x_dtype, m, k, ldx, pro, nw, eps, qs, n, scale, sdt, bias, nullptr, 0, gu, n,
                                   algo, ws, avail, st);
  if (rc != QTTS_OK) return rc;
  return qtts_launch_silu_mul(gu, x_dtype, m, n / 2, n, act, ldact, st);
}
