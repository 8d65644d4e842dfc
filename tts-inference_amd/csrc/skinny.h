// The W8A16 skinny kernel (decode rows), shared by w8a16.hip (activation operands
// loaded straight from global memory) and w8a16_xrows.hip (activation rows staged
// through LDS).  See w8a16.hip for the kernel family as a whole.
#pragma once

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "layout.h"
#include "pipe.h"
#include "splitk.h"

// Whether the row-split kernel (w8a16_xrows_sub.hip) is built for (sub, waves, units per wave).
int qtts_w8a16_sub_built(int sub, int waves, int cpw);

namespace qtts {

// Raw element bits, zero-extended to 32: a load whose value is not needed until the
// epilogue, with no conversion the compiler could schedule (and wait for) early.
// The load is a relaxed atomic (workgroup scope: an ordinary cached load in the
// ISA) because compilers do not sink atomic loads towards their use; a plain load
// of an epilogue-only value gets moved to the end of the kernel, where its latency
// becomes a second round trip.
template <typename T> __device__ __forceinline__ uint32_t load_bits(const T* p) {
  if constexpr (sizeof(T) == 2)
    return __hip_atomic_load((uint16_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    return __hip_atomic_load((uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
template <typename T> __device__ __forceinline__ float bits_to_f32(uint32_t b) {
  if constexpr (std::is_same<T, float>::value) return __uint_as_float(b);
  else return to_f32(T{(uint16_t)b});
}

// ------------------------------------------------------------------------------------
// skinny: M <= 16 * MB (MB m-blocks of 16 activation rows; MB > 1 on strip weights
// with K % 64 == 0 only)
// ------------------------------------------------------------------------------------

// MX > 0 (one m-block, full-K strip weights, M <= MX, or up to 2 MX rows in row parts: y0
// below): the activation operands come
// through LDS instead of one 16-byte global load per lane and MFMA.  Each wave loads
// the MX rows of its own K range once, 16 bytes a lane with no duplicates (rows past
// M repeat row M - 1), writes them to a wave-private LDS block and reads its MFMA
// B operands from there.  The MFMA operand layout gives lanes of rows >= M copies of
// row 0's data, so direct loads fetch (16 / M)x the activation bytes through the
// vector memory path the weight stream needs; staged, that path carries M rows once.
// F8W: the weight codes are OCP e4m3 (fp8 weight-only) instead of int8.
// PRO (staged rows only), a prologue computed while the rows are staged:
//   kProSiluMul: x is GatedMLP's fused gate_up output, [M, 2K] with row stride ldx, and
//     the GEMM multiplies silu(gate) * up (gate = columns [0, K), up = [K, 2K);
//     qtts/layers/activation.py:142-147);
//   kProRmsNorm (no split: S == 1): the GEMM multiplies RMSNorm(x) with weight aux
//     and epsilon eps (qtts/layers/norm.py:50-76), row by row, staged as the reference
//     rounds it: XT((x * inv) * aux), inv = 1 / sqrt(sum of x^2 / K + eps) in fp32.  Each
//     wave sums x^2 over its K range, the workgroup meets at one fence-free barrier
//     while the weight loads stay in flight, and every wave adds the W partials in wave
//     order before it stages its range (stage_x).
// RES (staged rows only): y = residual + the linear's output, the output rounded to
// XT first, as `residual + linear(x)` computes it (qtts/models/talker.py:270-271).
// PAIR (staged rows, no split): GatedMLP's gate_up_proj followed by its activation
//   (qtts/layers/activation.py:142-147).  q holds the fused [N, K] gate_up weight
//   (gate rows, then up rows); workgroup s runs gate strip s and up strip s + N/32:
//   each wave loads both strips' chunks of its K range and feeds each staged B operand
//   to two MFMAs, and the workgroup stores y[:, c] = XT(XT(silu(g)) * u) for g, u the
//   linear's outputs of columns c and c + N/2 rounded to XT: y is [M, N/2].  The
//   gate_up output itself is never stored.
// PAIR with SUB = 2 (staged rows, up to 8 of them, no split): the gate_up GEMM on half strips.
//   Workgroup p takes gate rows [8p, 8p + 8) and the matching up rows N/2 + [8p, 8p + 8) as the 16
//   rows of its MFMA A operand (lanes of rows 0-7 load the gate strip's half, rows 8-15 the up
//   strip's), so one accumulator holds both and the grid has the plain GEMM's N/16 workgroups
//   (the two-strip PAIR has N/32, each with twice the bytes).  Each output element sums the
//   same K chunks in the same order as the plain GEMM's, so the result equals the GEMM followed
//   by the activation bit for bit at the same wave configuration; lane (j, g) for g < 2 takes
//   the up value of lane (j, g + 2), i.e. lane ^ 32, in the epilogue.
// SUB > 1 (staged rows, M <= 16 / SUB, no split, no PAIR): row-split strips.  SUB
//   workgroups share each 16-row strip, workgroup p taking weight rows
//   [p * RP, (p + 1) * RP) of it (RP = 16 / SUB), so a layer of few strips still spreads
//   over every compute unit without a split-K meeting.  Each MFMA then covers SUB chunks
//   ("a unit") of those RP rows: A row b * RP + i holds weight row i of chunk b of the unit
//   and B column b * RP + j activation row j of the same chunk, so the SUB diagonal
//   RP x RP blocks of D are the chunks' contributions (the off-diagonal blocks mix chunks
//   and are never read) and the epilogue adds them, in chunk order, across lanes.  Every
//   lane loads weight bytes it needs and every MFMA is useful, as with whole strips.
// Parameters: everything the kernel reads before its first loads (q, x, scale, bias, aux,
// ldx, M and the split count, K, N) comes first, in the 14
// dwords the hardware preloads into SGPRs at wave launch (kernarg preloading, build.py), so
// no kernel-argument load stands between a wave's start and its weight loads.  Measured on the talker linears (cold weights, M = 1): the former order,
// whose early values sat in two 64-byte argument lines fetched one after the other, plus the
// split mapping's division, cost 0.6-1.2 us a launch.
enum : int { kProNone = 0, kProSiluMul = 1, kProRmsNorm = 2 };

template <typename XT, typename ST, int W, int CPW, int LAYOUT, bool FULLK, int MB = 1, int MX = 0, bool F8W = false,
          int PRO = kProNone, bool RES = false, bool PAIR = false, int SUB = 1, bool NT = false>
__global__ __launch_bounds__(W * 64) void w8a16_skinny_kernel(
    const int8_t* __restrict__ q, const XT* __restrict__ x, const ST* scale, const XT* bias,
    const XT* __restrict__ aux, int ldx, int MS, int K, int N, XT* y, int64_t ldy, int64_t ldq,
    float* __restrict__ part, unsigned* __restrict__ counters, float eps, const XT* res, int64_t ldr) {
  typedef mfma16<XT> MM;
  typedef typename MM::vec V;
  static_assert(MB == 1 || (FULLK && LAYOUT == kLayoutStrips), "several m-blocks need full-K strip weights");
  static_assert(MX == 0 || (MB == 1 && FULLK && LAYOUT == kLayoutStrips), "staged rows need one m-block, full K");
  static_assert(PRO == kProNone || MX > 0, "a prologue runs on staged rows");
  static_assert(!RES || MX > 0, "the residual epilogue is built with staged rows");
  static_assert(!PAIR || (MX > 0 && !RES && PRO != kProSiluMul), "the SiLU pair epilogue runs on staged rows");
  static_assert(SUB == 1 || ((SUB == 2 || SUB == 4) && MX > 0 && MX <= 16 / SUB && !PAIR) ||
                    (PAIR && SUB == 2 && MX > 0 && MX <= 8),
                "row-split strips run on staged rows, at most 16 / SUB of them");
  constexpr bool PH = PAIR && SUB == 2;  // the gate_up GEMM on half strips: 8 gate + 8 up rows
  constexpr bool P2 = PAIR && !PH;       // the two-strip pair: a gate strip and its up strip
  constexpr int CS = PH ? 1 : SUB;       // chunks one MFMA covers (a unit)
  constexpr int RP = 16 / SUB;  // weight rows per workgroup (PH: gate rows)
  constexpr bool SILU = PRO == kProSiluMul, NORM = PRO == kProRmsNorm;
  constexpr int NA = P2 ? 2 : 1;  // accumulators a wave carries: gate (and up)
  // DIST: the epilogue shared by the waves (below); every wave, wave 0 included, publishes its sums.
  constexpr bool DIST = W > 1 && MB == 1 && !P2;
  __shared__ f32x4_t red[DIST ? W : (W > 1 ? W - 1 : 1)][MB * NA][64];
  __shared__ float nss[NORM ? W : 1][NORM ? MX : 1];
  __shared__ __align__(16) uint16_t xrow[MX > 0 ? W : 1][MX > 0 ? MX : 1][MX > 0 ? CPW * CS * 64 : 8];

  // Grid: x = output strips (times SUB, rounded up to a multiple of 8), y = K splits.  Workgroups are
  // dealt to the 8 XCDs round-robin in x-fastest order, so with gridDim.x % 8 == 0 every
  // split of a strip runs on one XCD and its split-K meeting stays in one L2.
  // MS = M | S << 8: the rows (at most 64 here) and the split count share one preloaded dword
  // (gridDim.y would be a hidden-argument load).
  // Row parts (staged rows, one split): grid z = p takes the call's rows MX p .. MX p + MX - 1 (of x,
  // the residual and y), so a call of more than MX rows runs as MX-row workgroups, ceil(M / MX) per
  // strip (or half strip).  M is this workgroup's row count, y0 its first row.
  const int y0 = MX > 0 ? (int)blockIdx.z * MX : 0;
  const int M = MX > 0 ? min((MS & 0xff) - y0, MX) : MS & 0xff, S = MS >> 8;
  const int strip = SUB == 1 ? blockIdx.x : blockIdx.x / SUB, split = blockIdx.y;
  const int part_row = SUB == 1 ? 0 : (blockIdx.x % SUB) * RP;  // this workgroup's first strip row
  const int strips = PAIR ? ((N >> 1) + 15) >> 4 : (N + 15) >> 4;  // PAIR: the gate strips
  if (strip >= strips) return;

  // wave index through readfirstlane: provably uniform, so per-wave bounds stay scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int n = strip * 16 + r;
  const bool n_ok = n < N, m_ok = r < M;
  const int nchunks = (K + 63) >> 6;
  // This workgroup's units of SUB chunks (SUB divides nchunks, checked by the host): split
  // `split` of S of ceil(units / S) units each (the host's split size:
  // ceil(n / ceil(n / ceil(n / s))) = ceil(n / s)).
  int c0 = 0, c1 = CS == 1 ? nchunks : nchunks / CS;
  if (SUB == 1 && S > 1) {
    const int cps = (nchunks + S - 1) / S;
    c0 = split * cps;
    c1 = min(c0 + cps, nchunks);
  }
  const int cw = (c1 - c0 + W - 1) / W;  // <= CPW, guaranteed by the launcher
  const int wc0 = c0 + wave * cw, wc1 = min(wc0 + cw, c1);

  const int8_t* wp;
  int64_t wstride;
  // P2: the up strip is strip + strips (strips = the gate strips, N/32).
  const int64_t up_off = P2 ? (int64_t)strips * nchunks * 1024 : 0;
  if constexpr (PH) {
    // lane (r, g): gate row 16 strip + part_row + r % 8 (r < 8) or the up row N/2 above it,
    // bytes 16 g .. + 15 of each chunk (N % 32 == 0: both halves sit in whole strips)
    const int R = strip * 16 + part_row + (r & 7) + (r < 8 ? 0 : (N >> 1));
    wp = q + (int64_t)(R >> 4) * nchunks * 1024 + ((R & 15) + 16 * g) * 16;
    wstride = 1024;
  } else if constexpr (LAYOUT == kLayoutStrips && SUB > 1) {
    // lane (r, g): strip row part_row + r % RP of chunk r / RP of each unit, bytes 16 g .. + 15
    wp = q + (int64_t)strip * nchunks * 1024 + (r / RP) * 1024 + (part_row + r % RP + 16 * g) * 16;
    wstride = SUB * 1024;
  } else if constexpr (LAYOUT == kLayoutStrips) {
    wp = q + (int64_t)strip * nchunks * 1024 + lane * 16;
    wstride = 1024;
  } else {
    wp = q + (int64_t)(n_ok ? n : 0) * ldq + 16 * g;
    wstride = 64;
  }
  // Activation row r + 16 mb of each m-block; rows past M read row 0 (full K) or are
  // zero (ragged K): they only feed D columns that are never stored.
  const XT* xp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) xp[mb] = x + (int64_t)(r + 16 * mb < M ? r + 16 * mb : 0) * ldx + 16 * g;
  const i32x4_t zero = {0, 0, 0, 0};

  // A group of CPW chunks is issued in full before any of it is consumed.  With
  // FULLK (K % 64 == 0, strip layout) the loads are branch-free: chunk indices past
  // the wave's range are clamped to its last chunk (consume zeroes their weights).
  i32x4_t w[CPW], wu[P2 ? CPW : 1], xa[MB][CPW], xb[MB][CPW];
  auto issue = [&](int base) {
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      if constexpr (FULLK) {
        const int c = min(base + u, wc1 - 1);
        w[u] = load_weight<NT>(wp + (int64_t)c * wstride);
        if constexpr (P2) wu[u] = load_weight<NT>(wp + up_off + (int64_t)c * wstride);
        if constexpr (MX == 0) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            xa[mb][u] = *(const i32x4_t*)(xp[mb] + (int64_t)c * 64);
            xb[mb][u] = *(const i32x4_t*)(xp[mb] + (int64_t)c * 64 + 8);
          }
        }
      } else {
        const int c = base + u;
        const bool live = c < wc1;  // wave-uniform
        const bool kin = c * 64 + 16 * g < K;
        if (LAYOUT == kLayoutStrips) w[u] = live ? load_weight<NT>(wp + (int64_t)c * wstride) : zero;
        else w[u] = (live && n_ok && kin) ? load_weight<NT>(wp + (int64_t)c * wstride) : zero;
        xa[0][u] = (live && m_ok && kin) ? *(const i32x4_t*)(xp[0] + (int64_t)c * 64) : zero;
        xb[0][u] = (live && m_ok && kin) ? *(const i32x4_t*)(xp[0] + (int64_t)c * 64 + 8) : zero;
      }
    }
  };
  f32x4_t acc[MB], up[P2 ? MB : 1];  // P2: up holds the up strip's sums
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (P2) up[0] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  auto consume = [&](int base) {
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      if constexpr (FULLK) {
        // Unconditional MFMAs on zeroed weights past the range: a branch here would
        // let the compiler sink the loads into it, one round trip per chunk.
        const bool live = base + u < wc1;
        const i32x4_t wv = live ? w[u] : zero;
        const V wlo = wcvt<F8W, XT>((uint32_t)wv[0], (uint32_t)wv[1]);
        const V whi = wcvt<F8W, XT>((uint32_t)wv[2], (uint32_t)wv[3]);
        if constexpr (P2) {  // the up strip's chunk on the same B operands, in the same order
          const i32x4_t uv = live ? wu[u] : zero;
          const V ulo = wcvt<F8W, XT>((uint32_t)uv[0], (uint32_t)uv[1]);
          const V uhi = wcvt<F8W, XT>((uint32_t)uv[2], (uint32_t)uv[3]);
          acc[0] = MM::mma(wlo, __builtin_bit_cast(V, xa[0][u]), acc[0]);
          up[0] = MM::mma(ulo, __builtin_bit_cast(V, xa[0][u]), up[0]);
          acc[0] = MM::mma(whi, __builtin_bit_cast(V, xb[0][u]), acc[0]);
          up[0] = MM::mma(uhi, __builtin_bit_cast(V, xb[0][u]), up[0]);
          continue;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] = MM::mma(wlo, __builtin_bit_cast(V, xa[mb][u]), acc[mb]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] = MM::mma(whi, __builtin_bit_cast(V, xb[mb][u]), acc[mb]);
      } else if (base + u < wc1) {
        const V wlo = wcvt<F8W, XT>((uint32_t)w[u][0], (uint32_t)w[u][1]);
        const V whi = wcvt<F8W, XT>((uint32_t)w[u][2], (uint32_t)w[u][3]);
        acc[0] = MM::mma(wlo, __builtin_bit_cast(V, xa[0][u]), acc[0]);
        acc[0] = MM::mma(whi, __builtin_bit_cast(V, xb[0][u]), acc[0]);
      }
    }
  };
  // Epilogue operands: raw bits, loaded unconditionally (clamped index; y stands in
  // for a missing bias), so nothing needs their values before the epilogue.  (Loading a
  // strip's scale and bias once per workgroup through the scalar cache instead was measured
  // 0.1-0.2 us a launch slower on the talker linears: the LDS staging of the rows waits on
  // every outstanding scalar load, and those miss to HBM like the weights.)
  uint32_t sc[4] = {0u, 0u, 0u, 0u}, bi[4] = {0u, 0u, 0u, 0u}, rb[RES ? 4 : 1] = {0u};
  uint32_t su[P2 ? 4 : 1] = {0u}, bu[P2 ? 4 : 1] = {0u};  // P2: the up rows' scale and bias
  auto issue_epilogue = [&]() {
    const XT* bsrc = bias ? bias : y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // PH: lane (r, g) holds D rows 4 g .. + 3: gate rows for g < 2, the matching up rows above
      const int nn = PH ? strip * 16 + part_row + 4 * (g & 1) + i + (g < 2 ? 0 : (N >> 1))
                        : min(strip * 16 + part_row + 4 * g + i, N - 1);
      sc[i] = load_bits(scale + nn);
      bi[i] = load_bits(bsrc + nn);
      if constexpr (P2) {
        const int nu = min(nn + (N >> 1), N - 1);
        su[i] = load_bits(scale + nu);
        bu[i] = load_bits(bsrc + nu);
      }
      if constexpr (RES) rb[i] = load_bits(res + (int64_t)(y0 + min(r, M - 1)) * ldr + nn);
    }
  };

  // Staged activation rows (MX > 0): vector v of lane l holds elements
  // 512 v + 8 l .. + 7 of the wave's K range of each row (XV vectors cover CPW
  // units of CS chunks); lanes past the range repeat its last 8 elements.
  constexpr int XV = (CPW * CS * 64 + 511) / 512;
  const int xlen = (wc1 - wc0) * CS * 64, xbeg = wc0 * CS * 64;  // the wave's K range, elements
  // SILU: xu holds the up half; NORM: xu[0] holds the norm weight over the same range.
  i32x4_t xr[MX > 0 ? MX : 1][XV], xu[SILU ? MX : 1][SILU || NORM ? XV : 1];
  auto issue_x = [&]() {
    if constexpr (MX > 0) {
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        const int e = min(512 * v + 8 * lane, xlen - 8);
#pragma unroll
        for (int m = 0; m < MX; ++m) {
          const XT* row = x + (int64_t)(y0 + min(m, M - 1)) * ldx + xbeg + e;
          xr[m][v] = *(const i32x4_t*)row;
          if constexpr (SILU) xu[m][v] = *(const i32x4_t*)(row + K);
          if constexpr (NORM) {
            if (m == 0) xu[0][v] = *(const i32x4_t*)(aux + xbeg + e);
          }
        }
      }
    }
  };
  // Writes the wave's staged rows to LDS and reads the MFMA B operands back.  NORM stages the
  // normalized rows as the reference computes them, XT((x * inv) * weight) with inv = 1 / sqrt(sum
  // of x^2 / K + eps): each wave sums x^2 over its range for each row (fp32, lane partials over
  // its vectors in element order, a pair per v_dot2, then the wave's butterfly) and publishes it; after one barrier
  // (no fence: the weight loads stay in flight) every wave adds the partials in wave order and
  // scales its own elements.
  auto stage_x = [&]() {
    if constexpr (NORM) {
      float ss[MX];
#pragma unroll
      for (int m = 0; m < MX; ++m) ss[m] = 0.0f;
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        const bool in = 512 * v + 8 * lane < xlen;  // lanes past the range repeat its last 8
#pragma unroll
        for (int m = 0; m < MX; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (in) ss[m] = sq2_acc<XT>((uint32_t)xr[m][v][i], ss[m]);
      }
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        const float t = wave_sum_rows(ss[m]);
        if (lane == 0) nss[wave][m] = t;
      }
      wait_lgkmcnt0();
      barrier_only();  // every wave's partials (waves without chunks publish zeros)
      // The raw rows stay in registers across the barrier and are converted after it (an empty
      // asm hides their values from the compiler, which would otherwise keep all MX x 8 converted
      // floats of a lane live across the barrier).
#pragma unroll
      for (int v = 0; v < XV; ++v)
#pragma unroll
        for (int m = 0; m < MX; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            int t = xr[m][v][i];
            asm volatile("" : "+v"(t));
            xr[m][v][i] = t;
          }
      // lane m computes row m's inverse RMS (partials in wave order), read back per row as a scalar
      float tl = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) tl += nss[w][lane < MX ? lane : 0];
      const int invl = __builtin_bit_cast(int, 1.0f / __builtin_sqrtf(tl / (float)K + eps));
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        const float inv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(invl, m));
#pragma unroll
        for (int v = 0; v < XV; ++v) {
          const int e = min(512 * v + 8 * lane, xlen - 8);
          i32x4_t o;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t p = (uint32_t)xr[m][v][i], w2 = (uint32_t)xu[0][v][i];
            const float a = to_f32(XT{(uint16_t)p}), b = to_f32(XT{(uint16_t)(p >> 16)});
            o[i] = (int)pack2_f32<XT>((a * inv) * to_f32(XT{(uint16_t)w2}), (b * inv) * to_f32(XT{(uint16_t)(w2 >> 16)}));
          }
          *(i32x4_t*)&xrow[wave][m][e] = o;
        }
      }
    } else if constexpr (MX > 0) {
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        const int e = min(512 * v + 8 * lane, xlen - 8);
#pragma unroll
        for (int m = 0; m < MX; ++m) {
          if constexpr (SILU) *(i32x4_t*)&xrow[wave][m][e] = silu_mul8<XT>(xr[m][v], xu[m][v]);
          else *(i32x4_t*)&xrow[wave][m][e] = xr[m][v];
        }
      }
    }
    if constexpr (MX > 0) {
      // B operand of lane (r, g): row r (rows >= M read row 0; their D columns are
      // never stored), elements 64 u + 16 g .. + 15 of chunk u of the range.  SUB > 1:
      // row r % RP of chunk r / RP of unit u.
      const int rj = CS == 1 ? r : r % RP;
      const int rr = rj < M ? rj : 0;
#pragma unroll
      for (int u = 0; u < CPW; ++u) {
        const int cu = min(u, wc1 - wc0 - 1);
        const int ch = CS == 1 ? cu : cu * SUB + r / RP;
        xa[0][u] = *(const i32x4_t*)&xrow[wave][rr][64 * ch + 16 * g];
        xb[0][u] = *(const i32x4_t*)&xrow[wave][rr][64 * ch + 16 * g + 8];
      }
    }
  };

  // One group per wave, no loop: the host sizes the grid so a wave's share fits
  // (a loop's back edge would make the compiler wait for every load in flight at
  // its head); the whole call is one round trip.  The epilogue operands are fetched
  // after the weights: a compute unit's vector memory instructions pass its address
  // unit in issue order, and the weight stream is the critical path.  (Every wave
  // fetches them: a branch on the wave index would end in a wait for all loads.)
  if (wc0 < wc1) {  // wave-uniform: waves past the K range only reduce
    issue_x();
    issue(wc0);
    // The epilogue's addresses need kernel arguments past the preloaded ones (bias, y):
    // their scalar load must not be waited for before the last weight load is issued.
    __builtin_amdgcn_sched_barrier(0);
    issue_epilogue();
    // Keep the scheduler from interleaving loads with the MFMAs: every load must
    // be in flight before the first wait.
    __builtin_amdgcn_sched_barrier(0);
    stage_x();  // waits for the activation rows only; the weights stay in flight
    consume(wc0);
  } else {
    // A wave past the K range only adds zeros to the reduction; with the shared epilogue (DIST)
    // it finishes elements too, so it loads their operands, else nothing (wave 0 always has chunks).
    if constexpr (DIST) issue_epilogue();
    if constexpr (NORM) {  // zeros for the norm's partials, then the staging's barrier
      if (lane == 0)
#pragma unroll
        for (int m = 0; m < MX; ++m) nss[wave][m] = 0.0f;
      wait_lgkmcnt0();
      barrier_only();
    }
  }

  // The epilogue shared by the waves (DIST: one m-block, no two-strip pair, no split): wave w
  // finishes element w of each lane's four (fewer than 4 waves: elements w, w + W, ...), so the
  // scale, bias, rounding, residual and the SiLU pair's activation of a workgroup run on up to 4
  // waves at once instead of on wave 0 alone (measured: the SiLU pair's epilogue cost 0.35-0.42
  // us a launch on wave 0).  Each element adds the waves' sums in wave order, as wave 0 does
  // below, so the bits are the same.
  if constexpr (DIST) {
    if (SUB != 1 || S == 1) {
      red[wave][0][lane] = acc[0];
      __syncthreads();
      if (wave >= 4) return;
      // Element I of this lane's four (compile-time, so sc, bi and rb stay in registers).
      auto finish = [&](auto I) {
        constexpr int i = decltype(I)::value;
        float a = red[0][0][lane][i];
#pragma unroll
        for (int w = 1; w < W; ++w) a += red[w][0][lane][i];
        if constexpr (SUB == 2 && !PAIR) {
          a += __shfl_xor(a, 40, 64);  // as below
        } else if constexpr (SUB == 4) {
          a = ((a + __shfl(a, lane + 20, 64)) + __shfl(a, lane + 40, 64)) + __shfl(a, lane + 60, 64);
        }
        float v = a * bits_to_f32<ST>(sc[i]);
        if (bias) v += bits_to_f32<XT>(bi[i]);
        const int nn = strip * 16 + part_row + 4 * g + i;
        if constexpr (PH) {
          v = round_through<XT>(v);
          const float u = __shfl_xor(v, 32, 64);
          if (g < 2 && r < M && nn < (N >> 1)) y[(int64_t)(y0 + r) * ldy + nn] = from_f32<XT>(silu_mul<XT>(v, u));
        } else if (r < M && (SUB == 1 || 4 * g < RP) && nn < (PAIR ? N >> 1 : N)) {
          if constexpr (RES) v = bits_to_f32<XT>(rb[i]) + round_through<XT>(v);
          y[(int64_t)(y0 + r) * ldy + nn] = from_f32<XT>(v);
        }
      };
      // wave w: elements w, w + W, ... (wave-uniform branches)
      if (wave == 0) {
        finish(std::integral_constant<int, 0>{});
        if constexpr (W == 2) finish(std::integral_constant<int, 2>{});
      } else if (wave == 1) {
        finish(std::integral_constant<int, 1>{});
        if constexpr (W == 2) finish(std::integral_constant<int, 3>{});
      } else if (wave == 2) {
        finish(std::integral_constant<int, 2>{});
      } else {
        finish(std::integral_constant<int, 3>{});
      }
      return;
    }
  }

  if (W > 1) {
    if (wave > 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) red[wave - 1][mb][lane] = acc[mb];
      if constexpr (P2) red[wave - 1][1][lane] = up[0];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] += red[w][mb][lane];
      if constexpr (P2) up[0] += red[w][1][lane];
    }
  }

  if constexpr (SUB == 2 && !PAIR) {
    // D rows 8 + i, columns 8 + j (chunk 1 of each unit) onto rows i, columns j (chunk 0):
    // lane (j, g) for g < 2 takes lane (j + 8, g + 2), i.e. lane ^ 40.
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[0][i] += __shfl_xor(acc[0][i], 40, 64);
  } else if constexpr (SUB == 4) {
    // block b (rows and columns 4b .. 4b + 3) of lane (j, 0) sits in lane j + 20 b
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = acc[0][i];
      acc[0][i] = ((v + __shfl(v, lane + 20, 64)) + __shfl(v, lane + 40, 64)) + __shfl(v, lane + 60, 64);
    }
  }

  if (SUB == 1 && S > 1) {
    float a[4 * MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) a[4 * mb + i] = acc[mb][i];
    // Only wave 0 is left: the meeting has 64 participants per workgroup.
    if (!splitk_meet<4 * MB>(a, part + (int64_t)strip * S * 64 * 4 * MB, &counters[strip], S, split, lane, 64,
                             nullptr))
      return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{a[4 * mb], a[4 * mb + 1], a[4 * mb + 2], a[4 * mb + 3]};
  }

  if constexpr (PH) {
    // lanes g < 2: gate rows 8p + 4 g + i; lanes g >= 2 the up rows N/2 above them.  Every lane
    // scales and rounds its own (as the plain GEMM's output), then lane (j, g < 2) takes its up
    // value from lane ^ 32 and writes XT(XT(silu(g)) * u).
    const int m = r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[0][i] * bits_to_f32<ST>(sc[i]);
      if (bias) v += bits_to_f32<XT>(bi[i]);
      v = round_through<XT>(v);
      const float u = __shfl_xor(v, 32, 64);
      const int nn = strip * 16 + part_row + 4 * g + i;
      if (g < 2 && m < M && nn < (N >> 1)) y[(int64_t)(y0 + m) * ldy + nn] = from_f32<XT>(silu_mul<XT>(v, u));
    }
    return;
  }

  // D layout of the 16x16 MFMA: lane (r, g) holds rows 4g..4g+3 (weight rows n) of
  // column r (activation row m = r + 16 mb).
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = r + 16 * mb;
    if (m < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int nn = strip * 16 + part_row + 4 * g + i;
        if ((SUB == 1 || 4 * g < RP) && nn < (PAIR ? N >> 1 : N)) {
          float v = acc[mb][i] * bits_to_f32<ST>(sc[i]);
          if (bias) v += bits_to_f32<XT>(bi[i]);
          if constexpr (RES) v = bits_to_f32<XT>(rb[i]) + round_through<XT>(v);
          if constexpr (P2) {
            float u = up[0][i] * bits_to_f32<ST>(su[i]);
            if (bias) u += bits_to_f32<XT>(bu[i]);
            v = silu_mul<XT>(round_through<XT>(v), round_through<XT>(u));
          }
          y[(int64_t)(y0 + m) * ldy + nn] = from_f32<XT>(v);
        }
      }
    }
  }
}

// ---- host side: the skinny configuration ------------------------------------------

// Launches w8a16_skinny_kernel under the calling entry point's weight policy: the NT
// (streaming) instantiation for bf16 activations on full-K strip weights (the decode layers of a
// bf16 model) when QTTS_ALGO_STREAM is set, plain loads otherwise (the other activation types
// and layouts are built without NT: they give the same bits, with cached weight loads).
template <typename XT, typename ST, int W, int CPW, int LAYOUT, bool FULLK, int MB = 1, int MX = 0, bool F8W = false,
          int PRO = kProNone, bool RES = false, bool PAIR = false, int SUB = 1, typename... Args>
inline void launch_skinny(dim3 grid, dim3 block, hipStream_t st, Args... args) {
  if constexpr (std::is_same<XT, bf16_t>::value && LAYOUT == kLayoutStrips && FULLK) {
    if (weight_policy()) {
      launch(&w8a16_skinny_kernel<XT, ST, W, CPW, LAYOUT, FULLK, MB, MX, F8W, PRO, RES, PAIR, SUB, true>, grid, block,
             0, st, args...);
      return;
    }
  }
  launch(&w8a16_skinny_kernel<XT, ST, W, CPW, LAYOUT, FULLK, MB, MX, F8W, PRO, RES, PAIR, SUB>, grid, block, 0, st,
         args...);
}

struct SkinnyCfg { int mb, waves, cpw, S, cps, strips; };

// The skinny kernels take up to kSkinnyMaxM rows on strip weights.  The automatic
// choice keeps them up to 32 rows (two m-blocks) for weights of at most 9 MiB with
// K <= 2048 and otherwise moves to the tile kernel past 16 rows: measured on the talker
// and code-predictor shapes at M = 16..128, where the tile kernel wins on the 12-25 MB
// weights from 24 rows, on the predictor's down_proj (K = 3072: 8.9 against 9.7 us at
// 24 rows, 9.1 against 11.3 at 32) and everywhere from 48.
constexpr int kSkinnyMaxM = 64, kSkinnyAutoMaxM = 32;
constexpr int64_t kSkinnyAutoMaxBytes = 9 << 20, kSkinnyAutoMaxK = 2048;

// m-blocks of 16 activation rows a skinny call carries.
inline int skinny_mb(int64_t m) { return m <= 16 ? 1 : (m <= 32 ? 2 : 4); }

// Chunks (64 columns, 1 KiB of a strip) a wave keeps in flight at once; a chunk holds
// 4 + 8 MB registers a lane.  Built: MB = 1: 4 or 8 (4 or 6 at 16 waves, whose 1024
// threads leave 128 registers a lane); MB = 2: 4 or 8 (4 at 16 waves); MB = 4: 4, at
// most 8 waves.
inline bool skinny_cpw_ok(int mb, int w, int cpw) {
  if (mb == 1) return w == 16 ? (cpw == 4 || cpw == 6) : (cpw == 4 || cpw == 8);
  if (mb == 2) return w == 16 ? cpw == 4 : (cpw == 4 || cpw == 8);
  return mb == 4 && w <= 8 && cpw == 4;
}
inline int skinny_cpw_max(int mb, int w) { return mb == 1 ? (w == 16 ? 6 : 8) : (mb == 2 ? (w == 16 ? 4 : 8) : 4); }
inline int skinny_waves_max(int mb) { return mb == 4 ? 8 : 16; }

inline SkinnyCfg skinny_cfg(int64_t m, int64_t n, int64_t k, int splits_req, int waves_req, int cpw_req) {
  SkinnyCfg c;
  c.mb = skinny_mb(m);
  c.strips = (int)((n + 15) / 16);
  const int nchunks = std::max(1, (int)((k + 63) / 64));
  int W = waves_req, S = splits_req, C = cpw_req;
  if (W <= 0) {
    // Few, fat waves: the fewest waves (with the most chunks in flight each) that
    // cover a strip's K without a split.  Measured on the talker and code-predictor
    // shapes this beats more, thinner waves at every M in 1..16.
    W = 1;
    while (W < skinny_waves_max(c.mb) && W * skinny_cpw_max(c.mb, W) < nchunks) W *= 2;
  }
  if (C <= 0) C = skinny_cpw_max(c.mb, W);
  c.waves = W;
  c.cpw = C;
  // The kernel runs one group of C chunks per wave: raise S until a wave's share
  // fits (a requested split count is a minimum).
  S = std::max(S, 1);
  S = std::max(S, (nchunks + W * C - 1) / (W * C));
  S = std::min(S, nchunks);
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  return c;
}

// Row-split strips (SUB = 2 or 4 workgroups per strip; staged rows, M <= 16 / SUB, no
// split): W waves of CPW units of SUB chunks; cps holds the units of the full K.  By
// default the fewest waves with at most 6 units each, then the fewest units per wave of a
// built pair that covers K (6 units per wave measured best on the talker's down_proj and
// the predictor's down_proj; 4 on the predictor's o_proj, 16 units in all).
inline SkinnyCfg skinny_cfg_sub(int64_t n, int64_t k, int sub, int waves_req, int cpw_req) {
  SkinnyCfg c;
  c.mb = 1;
  c.strips = (int)((n + 15) / 16);
  c.S = 1;
  c.cps = std::max(1, (int)((k + 63) / 64) / sub);
  int W = waves_req;
  int C = cpw_req;
  if (W <= 0 || C <= 0) {
    bool found = false;
    int w0 = 1;
    if (W <= 0 && C <= 0)
      while (w0 < 16 && (c.cps + w0 - 1) / w0 > 6) w0 *= 2;
    for (int w = W > 0 ? W : w0; w <= (W > 0 ? W : 16) && !found; w *= 2) {
      for (int cpw = C > 0 ? C : 1; cpw <= (C > 0 ? C : 16) && !found; ++cpw) {
        if (w * cpw >= c.cps && qtts_w8a16_sub_built(sub, w, cpw)) {
          W = w;
          C = cpw;
          found = true;
        }
      }
    }
    if (!found) {  // reported as not built by the launcher
      W = W > 0 ? W : 16;
      C = C > 0 ? C : (c.cps + W - 1) / W;
    }
  }
  c.waves = W;
  c.cpw = C;
  return c;
}

// Whether a call can take row-split strips: strip weights, K a multiple of SUB chunks, at
// most 16 / SUB rows.
inline bool skinny_sub_ok(int64_t m, int64_t k, int sub) {
  return sub > 1 && m >= 1 && m <= 16 / sub && m <= 8 && k % 64 == 0 && (k / 64) % sub == 0;
}

// Row parts of the staged W8A16 kernel (grid z; skinny.h kernel, y0): calls of more than 8 rows
// run as 8-row workgroups, ceil(M / 8) per strip or half strip (one split), each staging its own
// rows.  Half strips take them up to 64 rows, whole strips up to 16; the automatic choice takes
// them where they pay (skinny_row_parts_auto, skinny_row_parts_sub).
constexpr int kRowPartsMaxM = 64;
inline int skinny_row_parts(int64_t m) { return m > 8 ? (int)((m + 7) / 8) : 1; }
inline bool skinny_sub_rows_ok(int64_t m, int64_t k, int sub) {
  return m >= 1 && m <= kRowPartsMaxM && (m <= 8 ? skinny_sub_ok(m, k, sub) : sub == 2 && skinny_sub_ok(8, k, sub));
}
// Whether the automatic choice takes row parts at 9-16 rows: on at most 128 strips, where the
// doubled grid fills idle compute units (half strips on at most 64).  Measured per call against
// direct loads in the stack graphs at M = 9 / 12 / 16: the code predictor's down_proj (64 strips,
// half strips) 1.36 / 1.60 / 2.12 us faster, its o_proj 0.63 / 0.75 / 1.06; the talker's down_proj
// (128 strips, whole) 0.85 / 1.54 / 2.53, its o_proj 0.47 / 0.62 / 0.90.  On more strips each
// extra workgroup re-reads its strip's weight: qkv 0.5-1.0 us and gate_up up to 3.4 us slower.
inline bool skinny_row_parts_auto(int64_t m, int64_t n) { return m > 8 && m <= 16 && (n + 15) / 16 <= 128; }
// The automatic choice of half strips in row parts: at 9-16 rows on at most 64 strips (above), and
// at 17-64 rows on at most 128 strips while the parts' weight reads (parts x N x K bytes, the
// re-reads served by the L2s and the Infinity Cache) stay within 20 MiB.  Measured per call against
// the automatic tile or m-block choice in the stack graphs, M = 24 / 32 / 40 / 48 / 64: the code
// predictor's o_proj (2 MiB) 1.85 / 2.49 / 2.42 / 2.38 / 1.81 us faster, its down_proj (3 MiB)
// 2.62 / 2.60 / 0.95 / 0.75 faster and 0.28 slower (24 MiB); the talker's o_proj (4 MiB) 1.07 /
// 1.23 / 1.93 / 1.19 faster and even at 32 MiB; its down_proj (12 MiB) 2.0-17.9 slower.
inline int skinny_row_parts_sub(int64_t m, int64_t n, int64_t k) {
  const int64_t strips = (n + 15) / 16;
  if (!skinny_sub_rows_ok(m, k, 2) || m <= 8) return 1;
  if (m <= 16) return strips <= 64 ? 2 : 1;
  return strips <= 128 && skinny_row_parts(m) * n * k <= (int64_t)20 << 20 ? 2 : 1;
}

// The automatic row split for a decode call: half strips where whole ones leave most compute
// units idle (at most 64 strips) or give each of at most 128 workgroups 64 KiB or more
// (K >= 4096), or at most 128 strips from 2 rows up.  Measured, cold weights, M = 1..8: the
// talker's down_proj (N = 2048, K = 6144) 4.57 against 5.13 us at M = 1 and 5.77 against 6.46
// at M = 8; the code predictor's o_proj (N = 1024, K = 2048) 2.98 against 3.11 and down_proj
// (N = 1024, K = 3072) 3.31 against 3.84; the talker's o_proj (N = 2048, K = 2048, streamed
// over 28 weights) 3.41 against 3.41 at M = 1, but 3.39 against 3.54 at M = 2, 3.53 against
// 3.65 at M = 4 and 3.70 against 3.78 at M = 8.  Quarter strips lost on every talker and
// predictor shape.
inline int skinny_auto_sub(int64_t m, int64_t n, int64_t k) {
  const int64_t strips = (n + 15) / 16;
  if ((strips <= 64 || (strips <= 128 && (k >= 4096 || m >= 2))) && skinny_sub_ok(m, k, 2)) return 2;
  return 1;
}

inline int64_t skinny_ws(const SkinnyCfg& c) {
  return c.S <= 1 ? 0 : kCounterBytes + (int64_t)c.strips * c.S * 64 * 4 * c.mb * 4;
}

}  // namespace qtts
