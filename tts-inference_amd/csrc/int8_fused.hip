// The whole of Int8Method.apply (qtts/quant/int8.py:145-160) for decode rows (M <= 8)
// in one gfx950 kernel: per-token int8 quantization of the activations, the int8 GEMM
// on strip-layout weights (exact int32 accumulation on v_mfma_i32_16x16x64_i8), and
// the reference's fp32 epilogue.  The two-kernel path (quant_act_int8_vec_kernel, then
// int8_skinny_kernel) gives the same bits: the codes, the scale and the int32 sums
// are the same numbers, and the epilogue is the same function (int8_epilogue).
//
// A workgroup owns one 16-row weight strip and all of K; its W waves split K into
// runs of at most C 64-column chunks.  Every load is issued before any is consumed:
// the wave's weight chunks (the MFMA A operand, 16 bytes a lane, as the strip layout
// stores them), its K slice of every activation row, and the epilogue operands.
// Then, with no further global traffic:
//   1. per-row |x| maxima: each lane folds its 8-element vector, a DPP / shuffle max
//      over the lanes of the row, and one LDS atomic max per row and wave (the slices
//      of all waves cover the row);
//   2. s[m] = dtype(max(amax, dtype(1e-6)) / 127) with the reference's scalar
//      division (int8_act_scale, as the stand-alone kernel computes it), and 1/s;
//   3. each wave quantizes its own slice, code = clamp(rint(dtype(x / s)), +-127),
//      the quotient correctly rounded from the reciprocal, into its LDS area laid out
//      as MFMA B operands: lane (m, g) of chunk c holds code[m][64 c + 16 g .. + 15];
//   4. one MFMA per chunk, the waves meet in LDS (int32 sums: any order gives the same
//      bits), and wave 0 writes y = round(((f32(acc) * s[m]) * sw[n]) [+ bias[n]]).
// A row's slice is 8 C vectors of 8 elements, padded to VP = 16, 32 or 64 lanes, so a
// wave holds 64 / VP rows per slot and a lane quantizes one vector per row it holds:
// 8 elements per row for C = 6 or 8, 4 for C = 4, 2 for C = 2.  More waves with fewer
// chunks each spread a call's quantization over more lanes.  RM (1, 4 or 8 rows) sizes
// the slots and the B operand area: rows >= M of it stay unwritten and only feed
// output columns that are never stored.
#include <algorithm>

#include "common.h"
#include "layout.h"

namespace qtts {

// The stand-alone kernel's code (int8_act_code, IEEE x / s) from the reciprocal
// rs = RN(1 / s): q0 = RN(x rs), the residual x - q0 s exact in one FMA, one FMA step
// (Markstein) gives the correctly rounded quotient for a normal s.  |x / s| <= 127.3
// here (s comes from the row's own maximum), so nothing overflows.  The sign of a zero
// quotient may differ from IEEE's; its code does not.
template <typename XT> __device__ __forceinline__ uint32_t act_code_rcp(float x, float s, float rs) {
  const float q0 = x * rs;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, s, x), rs, q0);
  const float v = __builtin_rintf(round_through<XT>(q));
  return (uint32_t)(v != v ? 0 : (int)fminf(fmaxf(v, -127.0f), 127.0f)) & 0xffu;
}

// Slice padding (vectors a row) for C chunks a wave.
template <int C> constexpr int fused_vp() { return C <= 2 ? 16 : (C <= 4 ? 32 : 64); }

template <typename XT, int W, int C, int RM, bool NT = false>
__global__ __launch_bounds__(W * 64) void int8_linear_fused_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ qws, int N,
    const float* sw, const XT* bias, XT* __restrict__ y, int64_t ldy, int strips, int div_mode) {
  constexpr int VP = fused_vp<C>();       // lanes per row in a slot
  constexpr int RPS = 64 / VP;            // rows a slot holds
  constexpr int SLOTS = (RM + RPS - 1) / RPS;
  static_assert(8 * C <= VP, "a row's slice must fit its lanes");
  __shared__ i32x4_t red[W > 1 ? W - 1 : 1][64];
  __shared__ unsigned amax_bits[RM];
  __shared__ float sx_lds[RM], sq_lds[RM], rcp_lds[RM];
  __shared__ __align__(16) uint8_t qxs[W][C][RM * 64];

  // Strip -> workgroup as the other skinny kernels: consecutive strips on different XCDs.
  const int strip = blockIdx.x;
  if (strip >= strips) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int nchunks = K >> 6;
  const int cw = (nchunks + W - 1) / W;  // <= C, guaranteed by the launcher
  const int wc0 = min(wave * cw, nchunks - 1);
  const int nw = max(0, min(cw, nchunks - wave * cw));  // chunks this wave owns
  const int vr = nw * 8;                                  // live vectors per row in its slice
  const int sub = lane / VP, v = lane % VP;               // row within a slot, vector within the row

  if (tid < RM) amax_bits[tid] = 0u;

  // ---- every load first ----------------------------------------------------------
  const int8_t* wp = qws + ((int64_t)strip * nchunks + wc0) * 1024 + lane * 16;
  i32x4_t wv[C];
#pragma unroll
  for (int u = 0; u < C; ++u)  // clamped: inside the strip
    wv[u] = load_weight<NT>(wp + (int64_t)min(u, max(nw - 1, 0)) * 1024);
  // Slot j: row RPS j + sub, columns 64 wc0 + 8 v ..; dead lanes read a clamped address.
  i32x4_t xv[SLOTS];
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    const int row = RPS * j + sub;
    const bool live = row < M && v < vr;
    xv[j] = *(const i32x4_t*)(x + (int64_t)(live ? row : 0) * ldx + (int64_t)wc0 * 64 + (live ? 8 * v : 0));
  }
  uint32_t swb[4], bib[4];
  {
    const XT* bsrc = bias ? bias : y;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int n = min(strip * 16 + 4 * g + t, N - 1);
      swb[t] = __hip_atomic_load((uint32_t*)sw + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      bib[t] = __hip_atomic_load((uint16_t*)bsrc + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // amax_bits cleared

  // ---- 1. per-row |x| maxima -------------------------------------------------------
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    if (RPS * j < M) {  // wave-uniform: every lane takes part in the group max
      const int row = RPS * j + sub;
      float mx = 0.0f;
      if (row < M && v < vr) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t pr = (uint32_t)xv[j][e];
          mx = fmaxf(mx, fmaxf(fabsf(to_f32(XT{(uint16_t)pr})), fabsf(to_f32(XT{(uint16_t)(pr >> 16)}))));
        }
      }
      mx = group_max<VP>(mx);
      if (v == 0 && row < M) atomicMax(&amax_bits[row], __float_as_uint(mx));  // non-negative floats order as bits
    }
  }
  __syncthreads();

  // ---- 2. scales ---------------------------------------------------------------------
  // A zero scale (an fp16 row whose 1e-6 floor / 127 underflows) divides nonzero codes
  // to +-inf (+-127) and zeros to NaN (0); quantizing with 2^-64 instead gives the same
  // codes, since every nonzero fp16 value / 2^-64 is far past 127 and such a row holds
  // no infinity.  The epilogue keeps the true scale.
  if (tid < RM) {
    const float s = int8_act_scale<XT>(__uint_as_float(amax_bits[tid]), div_mode);
    const float sq = s == 0.0f ? 0x1p-64f : s;
    sx_lds[tid] = s;
    sq_lds[tid] = sq;
    rcp_lds[tid] = 1.0f / sq;  // correctly rounded (IEEE division)
  }
  __syncthreads();

  // ---- 3. quantize this wave's slice into its B operands --------------------------------
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    if (RPS * j < M) {
      const int row = RPS * j + sub;
      if (row < M && v < vr) {
        const float s = sq_lds[row], rs = rcp_lds[row];
        uint32_t word[2] = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t pr = (uint32_t)xv[j][e];
          const uint32_t c0 = act_code_rcp<XT>(to_f32(XT{(uint16_t)pr}), s, rs);
          const uint32_t c1 = act_code_rcp<XT>(to_f32(XT{(uint16_t)(pr >> 16)}), s, rs);
          word[e >> 1] |= (c0 | (c1 << 8)) << (16 * (e & 1));
        }
        // chunk v / 8; columns 8 (v % 8) .. + 7 of it: lane group (v % 8) / 2, bytes 8 (v % 2)
        const int c = v >> 3, kk = v & 7;
        *(uint2*)&qxs[wave][c][((kk >> 1) * RM + row) * 16 + (kk & 1) * 8] = make_uint2(word[0], word[1]);
      }
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the LDS writes above precede the reads below

  // ---- 4. MFMAs ------------------------------------------------------------------------
  // B operand of lane (m, g): row min(m, RM - 1) of lane group g; rows >= M are unwritten
  // (any int8 values) and only reach D columns >= M, which are never stored.
  i32x4_t acc = {0, 0, 0, 0};
  const int boff = (g * RM + min(r, RM - 1)) * 16;
#pragma unroll
  for (int u = 0; u < C; ++u) {
    if (u < nw) {
      const i32x4_t b = *(const i32x4_t*)&qxs[wave][u][boff];
      acc = mma_i8_16x16x64(wv[u], b, acc);
    }
  }

  if (W > 1) {
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
      const i32x4_t o = red[w][lane];
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = (int)((unsigned)acc[t] + (unsigned)o[t]);
    }
  }

  // D: lane (r, g) holds rows 4g..4g+3 (weight rows n) of column r (activation row m).
  if (r < M) {
    const float s = sx_lds[r];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int n = strip * 16 + 4 * g + t;
      if (n < N) {
        const float b = bias ? to_f32(XT{(uint16_t)bib[t]}) : 0.0f;
        y[(int64_t)r * ldy + n] = from_f32<XT>(int8_epilogue(acc[t], s, __uint_as_float(swb[t]), b, bias != nullptr));
      }
    }
  }
}

}  // namespace qtts

using namespace qtts;

namespace {

constexpr int kInt8FusedMaxRows = 8;
// Every workgroup quantizes all M x K activations, so the automatic choice takes the
// fused kernel only while a CU's share of that work (its workgroups of the 256-CU
// gfx950 times M x K) stays under this many elements: measured on the talker shapes at
// M = 1..8 (cold weights), the fused kernel wins below it and the two-kernel path above
// (down_proj, K = 6144: M <= 3; gate_up, 768 strips: M <= 3; qkv and o: every M <= 8).
constexpr int64_t kInt8FusedMaxWork = 20480;
constexpr int64_t kGfx950Cus = 256;

// Waves and chunks per wave.  W: the request (a power of two up to 16), else the
// automatic choice (the fewest waves whose runs of at most 8 chunks cover K at M = 1;
// twice that at M = 2 or with several workgroups a CU, four times otherwise, at most 16:
// more waves spread the quantization).  C: the smallest build (2, 4, 6 or 8 chunks)
// that holds a wave's run.
bool int8_fused_cfg(int64_t m, int64_t n, int64_t k, int waves_req, int& W, int& C) {
  if (k <= 0 || k % 64 != 0) return false;
  const int64_t nchunks = k / 64;
  if (nchunks > 16 * 8) return false;
  int wmin = 1;
  while ((int64_t)wmin * 8 < nchunks) wmin *= 2;
  const int64_t wg_per_cu = ((n + 15) / 16 + kGfx950Cus - 1) / kGfx950Cus;
  if (waves_req > 0) {
    if (waves_req > 16 || (waves_req & (waves_req - 1)) || waves_req < wmin) return false;
    W = waves_req;
  } else {
    W = m <= 1 ? wmin : std::min(16, wmin * (m == 2 || wg_per_cu > 1 ? 2 : 4));
  }
  const int cw = (int)((nchunks + W - 1) / W);
  C = cw <= 2 ? 2 : (cw <= 4 ? 4 : (cw <= 6 ? 6 : 8));
  return true;
}

int rows_build(int64_t m) { return m <= 1 ? 1 : (m <= 4 ? 4 : 8); }

}  // namespace

// 1 if the fused kernel takes this call: 1 <= m <= 8, k % 64 == 0, k <= 8192, and
// either a requested wave count that is a power of two, at most 16, and enough for runs
// of at most 8 chunks, or (waves = 0) a CU's share of the quantization within
// kInt8FusedMaxWork.
int qtts_int8_fused_ok(int64_t m, int64_t n, int64_t k, int waves) {
  int W, C;
  if (m < 1 || m > kInt8FusedMaxRows || n < 1 || !int8_fused_cfg(m, n, k, waves, W, C)) return 0;
  if (waves > 0) return 1;
  const int64_t wg_per_cu = ((n + 15) / 16 + kGfx950Cus - 1) / kGfx950Cus;
  return wg_per_cu * m * k <= kInt8FusedMaxWork ? 1 : 0;
}

// x [m, k] bf16/fp16 (16-byte aligned rows), qws int8 strip layout, sw fp32.
int qtts_launch_int8_linear_fused(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qws,
                                  int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode,
                                  int waves, hipStream_t st) {
  int W, C;
  if (!qtts_int8_fused_ok(m, n, k, waves) || !int8_fused_cfg(m, n, k, waves, W, C))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fused int8 linear: unsupported shape m=%lld k=%lld waves=%d",
                          (long long)m, (long long)k, waves);
  const unsigned blocks = (unsigned)((n + 15) / 16);
  const int strips = (int)blocks;
  const int RM = rows_build(m);
#define QTTS_I8F(XT, WV, CV, RMV)                                                                            \
  qtts::launch_by_policy<std::is_same<XT, bf16_t>::value>([&](auto nt) {                                      \
    qtts::launch(&int8_linear_fused_kernel<XT, WV, CV, RMV, decltype(nt)::value>, dim3(blocks), dim3(WV * 64), \
                 0, st, (const XT*)x, (int)m, (int)k, ldx, qws, (int)n, sw, (const XT*)bias, (XT*)y, ldy, strips,  \
                 div_mode);                                                                                    \
  })
#define QTTS_I8F_RM(XT, WV, CV)           \
  do {                                    \
    if (RM == 1) QTTS_I8F(XT, WV, CV, 1); \
    else if (RM == 4) QTTS_I8F(XT, WV, CV, 4); \
    else QTTS_I8F(XT, WV, CV, 8);         \
  } while (0)
#define QTTS_I8F_C(XT, WV)                      \
  do {                                          \
    switch (C) {                                \
      case 2: QTTS_I8F_RM(XT, WV, 2); break;    \
      case 4: QTTS_I8F_RM(XT, WV, 4); break;    \
      case 6: QTTS_I8F_RM(XT, WV, 6); break;    \
      default: QTTS_I8F_RM(XT, WV, 8); break;   \
    }                                           \
  } while (0)
#define QTTS_I8F_W(XT)                     \
  do {                                     \
    switch (W) {                           \
      case 1: QTTS_I8F_C(XT, 1); break;    \
      case 2: QTTS_I8F_C(XT, 2); break;    \
      case 4: QTTS_I8F_C(XT, 4); break;    \
      case 8: QTTS_I8F_C(XT, 8); break;    \
      default: QTTS_I8F_C(XT, 16); break;  \
    }                                      \
  } while (0)
  if (x_dtype == QTTS_BF16) QTTS_I8F_W(bf16_t);
  else QTTS_I8F_W(f16_t);
#undef QTTS_I8F_W
#undef QTTS_I8F_C
#undef QTTS_I8F_RM
#undef QTTS_I8F
  return qtts_check_launch("int8_linear_fused");
}
