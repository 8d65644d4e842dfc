// The whole of Fp8Method.apply (qtts/quant/fp8.py:72-89) for decode rows (M <= 8) in
// one gfx950 kernel: per-token e4m3 quantization of the activations, the fp8 GEMM
// on strip-layout weights, and the reference's epilogue.
//
// A workgroup owns one 16-row weight strip and all of K; its W waves split K into
// runs of at most C 128-column chunks.  Every load is issued before any is consumed
// (one memory round trip per call): the wave's weight chunks (the MFMA A operand,
// 32 bytes a lane), its K slice of every activation row, and the epilogue operands.
// Then, with no further global traffic:
//   1. per-row |x| maxima: each lane folds its 8-element vectors, LDS atomic max
//      across the workgroup (the slices of all waves cover the row);
//   2. sx[m] = f32(max(amax, dtype(1e-6))) / 448 with the reference's scalar
//      division, exactly as the stand-alone activation kernel computes it;
//   3. each wave quantizes its own slice, qx = e4m3_rne(f32(x) / sx[m]) (a correctly
//      rounded quotient from the row's reciprocal, then v_cvt_pk_fp8_f32), into its
//      LDS area laid out as MFMA B operands (lane (m, g) of chunk c:
//      qx[m][128 c + 32 g .. + 31]);
//   4. one v_mfma_scale_f32_16x16x128_f8f6f4 per chunk, waves meet in LDS, and wave 0
//      writes y = round(acc * sx[m] * sw[n]) [+ bias] in the activation dtype.
// A row's slice is 16 C vectors of 8 elements, padded to VP = 16, 32 or 64 lanes, so a
// wave holds 64 / VP rows per slot and a lane quantizes one vector per row it holds; the
// row maxima meet through a DPP / shuffle max per row and one LDS atomic per row and
// wave.  Every workgroup quantizes all M x K activations, so the work grows with M and
// K: past three rows the launcher takes the fused kernel only for K <= 2048.  RM (1, 4
// or 8 rows) sizes the slots.  Rows >= M of a written B operand stay unwritten: they only
// feed output columns that are never stored.
#include <algorithm>

#include "common.h"
#include "layout.h"

namespace qtts {

template <typename XT, int W, int C, int RM, bool NT = false>
__global__ __launch_bounds__(W * 64) void fp8_linear_fused_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const uint8_t* __restrict__ qws, int N,
    const float* sw, const XT* bias, XT* __restrict__ y, int64_t ldy, int strips, int div_mode) {
  constexpr int VP = C <= 1 ? 16 : (C <= 2 ? 32 : 64);  // lanes per row in a slot (16 C vectors, padded)
  constexpr int RPS = 64 / VP;                              // rows a slot holds
  constexpr int SLOTS = (RM + RPS - 1) / RPS;
  static_assert(16 * C <= VP, "a row's slice must fit its lanes");
  __shared__ f32x4_t red[W > 1 ? W - 1 : 1][64];
  __shared__ unsigned amax_bits[16];
  __shared__ float sx_lds[16], rcp_lds[16];
  __shared__ __align__(16) uint8_t qxs[W][C][2048];

  // Strip -> workgroup as the other skinny kernels: consecutive strips on different XCDs.
  const int strip = blockIdx.x;
  if (strip >= strips) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int nchunks = K >> 7;
  const int cw = (nchunks + W - 1) / W;  // <= C, guaranteed by the launcher
  const int wc0 = min(wave * cw, nchunks - 1);
  const int nw = max(0, min(cw, nchunks - wave * cw));  // chunks this wave owns
  const int vr = nw * 16;                                 // live vectors per row in its slice
  const int sub = lane / VP, v = lane % VP;               // row within a slot, vector within the row

  if (tid < 16) amax_bits[tid] = 0u;

  // ---- every load first ----------------------------------------------------------
  const uint8_t* wp = qws + ((int64_t)strip * nchunks + wc0) * 2048 + lane * 16;
  i32x4_t w0[C], w1[C];
#pragma unroll
  for (int u = 0; u < C; ++u) {
    const int64_t off = (int64_t)min(u, max(nw - 1, 0)) * 2048;  // clamped: stays inside the strip
    w0[u] = load_weight<NT>(wp + off);
    w1[u] = load_weight<NT>(wp + off + 1024);
  }
  // Slot j: row RPS j + sub, columns 128 wc0 + 8 v ..; dead lanes read a clamped address.
  i32x4_t xv[SLOTS];
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    const int row = RPS * j + sub;
    const bool live = row < M && v < vr;
    xv[j] = *(const i32x4_t*)(x + (int64_t)(live ? row : 0) * ldx + (int64_t)wc0 * 128 + (live ? 8 * v : 0));
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
  if (tid < 16) {
    const float floor_v = round_through<XT>(1e-6f);
    const float sxv = scalar_div(fmaxf(__uint_as_float(amax_bits[tid]), floor_v), 448.0f, div_mode);
    sx_lds[tid] = sxv;
    rcp_lds[tid] = 1.0f / sxv;  // correctly rounded (IEEE division)
  }
  __syncthreads();

  // ---- 3. quantize this wave's slice into its B operands --------------------------------
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    if (RPS * j < M) {
      const int row = RPS * j + sub;
      if (row < M && v < vr) {
        const float s = sx_lds[row], rs = rcp_lds[row];
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t pr = (uint32_t)xv[j][e];
          const float q0 = div_by(to_f32(XT{(uint16_t)pr}), s, rs);
          const float q1 = div_by(to_f32(XT{(uint16_t)(pr >> 16)}), s, rs);
          const uint32_t pair = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false) & 0xffffu;
          if (e < 2) lo |= pair << (16 * e);
          else hi |= pair << (16 * (e - 2));
        }
        // chunk v / 16; within it columns 8 (v % 16): lane group (v % 16) / 4, byte 8 (v % 4)
        const int c = v >> 4, kk = v & 15;
        *(uint2*)&qxs[wave][c][((kk >> 2) * 16 + row) * 32 + (kk & 3) * 8] = make_uint2(lo, hi);
      }
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the LDS writes above precede the reads below

  // ---- 4. MFMAs ------------------------------------------------------------------------
  // Only chunks this wave quantized: the B operand of any other chunk is unwritten LDS,
  // and a NaN byte there would poison every column even against zero weights.  (Every
  // load has completed by now, so the wave-uniform branch costs no wait.)
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < C; ++u) {
    if (u < nw) {
      const i32x4_t b0 = *(const i32x4_t*)&qxs[wave][u][lane * 32];
      const i32x4_t b1 = *(const i32x4_t*)&qxs[wave][u][lane * 32 + 16];
      const i32x8_t a = {w0[u][0], w0[u][1], w0[u][2], w0[u][3], w1[u][0], w1[u][1], w1[u][2], w1[u][3]};
      const i32x8_t b = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
      acc = mma_fp8_16x16x128(a, b, acc);
    }
  }

  if (W > 1) {
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w) acc += red[w][lane];
  }

  // D: lane (r, g) holds rows 4g..4g+3 (weight rows n) of column r (activation row m).
  if (r < M) {
    const float s = sx_lds[r];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int n = strip * 16 + 4 * g + t;
      if (n < N) {
        float v = round_through<XT>(acc[t] * s * __uint_as_float(swb[t]));
        if (bias) v += to_f32(XT{(uint16_t)bib[t]});
        y[(int64_t)r * ldy + n] = from_f32<XT>(v);
      }
    }
  }
}

}  // namespace qtts

using namespace qtts;

namespace {

constexpr int kFusedMaxChunks = 48;  // 16 waves x 3 chunks: K <= 6144
constexpr int kFusedMaxRows = 8;
// Past three rows the automatic choice takes the fused kernel only for K <= 2048: measured
// with cold weights on the talker shapes at M = 1..8, it beats the two-kernel path at every
// M for K = 2048 (qkv 5.6 against 6.8 us, gate_up 10.8 against 11.7 at M = 8) and up to
// M = 3 for K = 6144 (down_proj: 8.6 against 8.9 us at M = 3, 9.6 against 9.0 at M = 4).
constexpr int64_t kFp8FusedMaxKPast3 = 2048;

// Waves and chunks per wave: 2 chunks a wave up to 32 chunks, 3 above; at least enough
// waves to cover K, and more (up to 16) until the call runs 2048 waves (doubling them from
// two rows on measured slower: gate_up 9.4 against 7.7 us at M = 2).  A requested wave
// count (a power of two up to 16 that covers K in runs of at most 3) replaces them.
// C: the smallest build (1, 2 or 3 chunks) that holds a wave's run.
bool fused_cfg(int64_t m, int64_t n, int64_t k, int waves_req, int& W, int& C) {
  (void)m;
  const int nchunks = (int)(k / 128);
  if (nchunks < 1 || nchunks > kFusedMaxChunks) return false;
  if (waves_req > 0) {
    if (waves_req > 16 || (waves_req & (waves_req - 1)) || waves_req * 3 < nchunks) return false;
    W = waves_req;
  } else {
    const int c0 = nchunks <= 32 ? 2 : 3;
    W = 1;
    while (W * c0 < nchunks) W *= 2;
    const int64_t strips = (n + 15) / 16;
    while (W < 16 && strips * W < 2048) W *= 2;
  }
  C = (nchunks + W - 1) / W;
  return W <= 16 && C <= 3;
}

}  // namespace

// 1 if the fused kernel takes this call: 1 <= m <= 8, k % 128 == 0, k <= 6144, and either
// a requested wave count fused_cfg accepts or (waves = 0) m <= 3 or k <= 2048.
int qtts_fp8_fused_ok(int64_t m, int64_t n, int64_t k, int waves) {
  int W, C;
  if (m < 1 || m > kFusedMaxRows || n < 1 || k % 128 != 0 || !fused_cfg(m, n, k, waves, W, C)) return 0;
  return waves > 0 || m <= 3 || k <= kFp8FusedMaxKPast3 ? 1 : 0;
}

// x [m, k] bf16/fp16 (16-byte aligned rows), qws e4m3 strip layout.
int qtts_launch_fp8_linear_fused(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qws,
                                 int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode,
                                 int waves, hipStream_t st) {
  int W, C;
  if (!qtts_fp8_fused_ok(m, n, k, waves) || !fused_cfg(m, n, k, waves, W, C))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fused fp8 linear: unsupported shape m=%lld k=%lld waves=%d",
                          (long long)m, (long long)k, waves);
  const unsigned blocks = (unsigned)((n + 15) / 16);
  const int strips = (int)blocks;
  const int RM = m <= 1 ? 1 : (m <= 4 ? 4 : 8);
#define QTTS_F8F(XT, WV, CV, RMV)                                                                           \
  qtts::launch_by_policy<std::is_same<XT, bf16_t>::value>([&](auto nt) {                                     \
    qtts::launch(&fp8_linear_fused_kernel<XT, WV, CV, RMV, decltype(nt)::value>, dim3(blocks), dim3(WV * 64), \
                 0, st, (const XT*)x, (int)m, (int)k, ldx, qws, (int)n, sw, (const XT*)bias, (XT*)y, ldy, strips, \
                 div_mode);                                                                                   \
  })
#define QTTS_F8F_RM(XT, WV, CV)                \
  do {                                         \
    if (RM == 1) QTTS_F8F(XT, WV, CV, 1);      \
    else if (RM == 4) QTTS_F8F(XT, WV, CV, 4); \
    else QTTS_F8F(XT, WV, CV, 8);              \
  } while (0)
#define QTTS_F8F_C(XT, WV)                    \
  do {                                        \
    if (C == 1) QTTS_F8F_RM(XT, WV, 1);       \
    else if (C == 2) QTTS_F8F_RM(XT, WV, 2);  \
    else QTTS_F8F_RM(XT, WV, 3);              \
  } while (0)
#define QTTS_F8F_W(XT)                     \
  do {                                     \
    switch (W) {                           \
      case 1: QTTS_F8F_C(XT, 1); break;    \
      case 2: QTTS_F8F_C(XT, 2); break;    \
      case 4: QTTS_F8F_C(XT, 4); break;    \
      case 8: QTTS_F8F_C(XT, 8); break;    \
      default: QTTS_F8F_C(XT, 16); break; \
    }                                      \
  } while (0)
  if (x_dtype == QTTS_BF16) QTTS_F8F_W(bf16_t);
  else QTTS_F8F_W(f16_t);
#undef QTTS_F8F_W
#undef QTTS_F8F_C
#undef QTTS_F8F_RM
#undef QTTS_F8F
  return qtts_check_launch("fp8_linear_fused");
}
