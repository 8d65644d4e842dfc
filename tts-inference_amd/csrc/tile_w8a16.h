// The W8A16 pipelined tile kernel (M > 16, strip weights, K % 64 == 0) and its host
// configuration, shared by tile.hip (int8 weights) and fp8w.hip (e4m3 weights,
// F8W): the two differ only in the conversion of the weight codes to the MFMA
// operand type.
//
// Replaces _w8_gemm_kernel (qtts/quant/kernels.py:89-135) for M > 16 when K % 64 == 0.
//
// A workgroup of 4 waves owns a BM x BN output tile and a K range; it walks the K
// range in 64-column stages through a P-deep LDS ring.  Stage loads are direct
// global -> LDS transfers (global_load_lds_dwordx4, 16 bytes per lane), so P-1
// stages are in flight while one is consumed, with no registers held for them.  With
// read-ahead (PF, 3 stages or more) a wave reads the next stage's operands from LDS
// into a second register set while the MFMAs of the current one run, so no LDS
// latency sits between a stage's barrier and its first MFMA; P-2 stages of global
// loads are then in flight.  Every load writes one 1 KiB MFMA fragment in lane order:
//   * activation fragment (m-block mb, half h): lane l carries
//     x[m0 + 16 mb + l % 16][k + 16 (l / 16) + 8 h .. + 7]  (8 bf16);
//   * weight fragment (strip sb): the strip layout's 1 KiB block, lane l carries
//     w[n0 + 16 sb + l % 16][k + 16 (l / 16) .. + 15]  (16 int8).
// So every MFMA operand read is one conflict-free ds_read_b128 at lane * 16.  The
// int8 half h of a weight fragment pairs with activation half h: together they
// cover the stage's 64 K columns in two v_mfma_f32_16x16x32 steps.
//
// The 4 waves form a WM x (4/WM) grid over the tile.  With WM = 1 each wave owns
// BN/4 output columns for all BM rows, so each weight fragment is dequantized
// (int8 -> bf16, exact) by exactly one wave, but every wave reads all of the tile's
// activation fragments from LDS; WM = 2 halves those activation reads (LDS
// bandwidth, not the matrix cores, bounds the 1 x 4 grid on the larger tiles) at the
// cost of dequantizing each weight fragment twice.  Rows past M and strips past N are read clamped and
// never stored; K must be a multiple of 64 (the strip layout pads N, not K).
//
// Tiles are numbered n-fastest, and the dispatcher deals consecutive workgroups to
// the 8 XCDs in turn, so each XCD works through its own n-columns of the weight for
// every m-tile: the weight is read once from HBM and its re-reads across m-tiles
// hit that XCD's L2.  Split-K, for shapes with too few tiles to fill the GPU, meets
// through the workspace in the same launch (splitk.h).
#pragma once

#include <algorithm>

#include "common.h"
#include "layout.h"
#include "pipe.h"
#include "splitk.h"

namespace qtts {

// Scale bits with no branch on the dtype: always 16-bit loads (an fp32 scale is read
// as its two halves), so no join waits for the loads before the epilogue needs them.
__device__ __forceinline__ uint32_t load_scale_bits(const void* s, int dt, int n) {
  const bool f32 = dt == QTTS_F32;
  const uint16_t* p = (const uint16_t*)s;
  const uint32_t lo = __hip_atomic_load((uint16_t*)p + (f32 ? 2 * n : n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  const uint32_t hi = __hip_atomic_load((uint16_t*)p + (f32 ? 2 * n + 1 : n), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_WORKGROUP);
  return f32 ? (lo | (hi << 16)) : lo;
}

__device__ __forceinline__ float scale_bits_to_f32(uint32_t b, int dt) {
  if (dt == QTTS_F32) return __uint_as_float(b);
  if (dt == QTTS_BF16) return to_f32(bf16_t{(uint16_t)b});
  return to_f32(f16_t{(uint16_t)b});
}

template <typename XT> __device__ __forceinline__ float xbits_to_f32(uint32_t b) { return to_f32(XT{(uint16_t)b}); }

// CPS: chunks a stage (2: half the stage barriers and load waits of a small-K call; the host
// keeps every split's chunk count a multiple of it).
template <typename XT, int BM, int BN, int P, int WM, bool F8W, bool PF = false, int NW = 4, int CPS = 1>
__global__ __launch_bounds__(NW * 64) void w8a16_pipe_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ qs, int N,
    const void* __restrict__ scale, int sdt, const XT* __restrict__ bias, XT* __restrict__ y, int64_t ldy,
    float* __restrict__ part, unsigned* __restrict__ counters, int mtiles, int ntiles, int S, int cps) {
  typedef mfma16<XT> MM;
  typedef typename MM::vec V;
  constexpr int WN = NW / WM;          // the NW waves form a WM x WN grid over the tile
  constexpr int TMB = BM / 16;         // 16-row m-blocks per tile
  constexpr int MB = TMB / WM;         // 16-row m-blocks per wave
  constexpr int NB = BN / 16 / WN;     // 16-column strips per wave
  constexpr int XF = 2 * TMB;          // activation fragments per stage
  constexpr int WF = BN / 16;          // weight fragments per stage
  constexpr int F = XF + WF;
  constexpr int FPW = F / NW;          // fragments each wave loads per stage
  constexpr int SB = F * 1024 * CPS;   // stage bytes
  static_assert(F % NW == 0 && (NW == 4 || NW == 8), "fragments must split evenly over the waves");
  static_assert(CPS == 1 || CPS == 2, "one or two chunks a stage");
  static_assert((WM == 1 || WM == 2) && MB >= 1 && NB >= 1, "wave grid must cover the tile");
  static_assert(P >= 2 && P * SB + 64 <= kLdsBytes, "stage ring must fit in LDS");
  static_assert((P - 2) * FPW * CPS < 64, "vmcnt is 6 bits");
  __shared__ __align__(1024) uint8_t ring[P * SB];
  __shared__ uint32_t epi_sc[BN], epi_bi[BN];  // the tile's scale and bias bits, column by column
  __shared__ unsigned flag;

  int tile, split;
  decode_wg(blockIdx.x, S, tile, split);
  if (tile >= mtiles * ntiles) return;
  const int nt = tile % ntiles, mt = tile / ntiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;  // this wave's m-blocks wm*MB.., strips wn*NB..
  const int c16 = lane & 15, g = lane >> 4;
  const int nchunks = K >> 6;
  const int strips = (N + 15) >> 4;
  const int kc0 = split * cps;
  const int nk = min(cps, nchunks - kc0) / CPS;  // stages of this split

  // Epilogue operands: thread t < BN loads column t's scale and bias bits first (the oldest
  // loads in flight, so waiting for them costs about what waiting for stage 0 does) and
  // parks them in LDS, where the epilogue reads them; held in registers through the K loop
  // they would cost 8 NB registers a lane, enough to cut the larger tiles' occupancy.
  uint32_t my_sc = 0u, my_bi = 0u;
  if (tid < BN) {
    const int n = min(n0 + tid, N - 1);
    my_sc = load_scale_bits(scale, sdt, n);
    my_bi = __hip_atomic_load((uint16_t*)(bias ? bias : y) + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }

  // This wave's fragments: per-lane source at chunk kc0 and the per-chunk stride.
  const uint8_t* src[FPW];
  int64_t stride[FPW];
#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int f = wave * FPW + j;
    if (f < XF) {
      const int mb = f >> 1, h = f & 1;
      const int m = min(m0 + mb * 16 + c16, M - 1);
      src[j] = (const uint8_t*)(x + (int64_t)m * ldx + (int64_t)kc0 * 64 + 16 * g + 8 * h);
      stride[j] = 64 * (int64_t)sizeof(XT);
    } else {
      const int s = min(n0 / 16 + (f - XF), strips - 1);
      src[j] = (const uint8_t*)qs + ((int64_t)s * nchunks + kc0) * 1024 + lane * 16;
      stride[j] = 1024;
    }
  }

  auto issue = [&](uint8_t* stage, int i) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < CPS; ++c)
#pragma unroll
      for (int j = 0; j < FPW; ++j)
        load_to_lds16(src[j] + (int64_t)(i * CPS + c) * stride[j], stage + c * F * 1024 + (wave * FPW + j) * 1024);
  };

  f32x4_t acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // One stage from registers: strip by strip the MFMAs of strip nb, with the conversion
  // of strip nb+1 issued ahead of them, h = 0 before h = 1 so that consecutive MFMAs
  // never share an accumulator.
  auto mma = [&](const V (&xa)[MB][2], const i32x4_t (&wq)[NB]) __attribute__((always_inline)) {
    V cur[2], nxt[2];
    cur[0] = wcvt<F8W, XT>((uint32_t)wq[0][0], (uint32_t)wq[0][1]);
    cur[1] = wcvt<F8W, XT>((uint32_t)wq[0][2], (uint32_t)wq[0][3]);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (nb + 1 < NB) {
        nxt[0] = wcvt<F8W, XT>((uint32_t)wq[nb + 1][0], (uint32_t)wq[nb + 1][1]);
        nxt[1] = wcvt<F8W, XT>((uint32_t)wq[nb + 1][2], (uint32_t)wq[nb + 1][3]);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = MM::mma(cur[h], xa[mb][h], acc[nb][mb]);
      if (nb + 1 < NB) {
        cur[0] = nxt[0];
        cur[1] = nxt[1];
      }
    }
  };
  auto read = [&](V (&xa)[MB][2], i32x4_t (&wq)[NB], const uint8_t* stage) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int h = 0; h < 2; ++h) xa[mb][h] = *(const V*)(stage + (2 * (wm * MB + mb) + h) * 1024 + lane * 16);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) wq[nb] = *(const i32x4_t*)(stage + (XF + wn * NB + nb) * 1024 + lane * 16);
  };

  for (int p = 0; p < P - 1; ++p)
    if (p < nk) issue(ring + p * SB, p);
  if (tid < BN) {  // visible to the epilogue after the K loop's barriers (every wave's LDS
    epi_sc[tid] = my_sc;  // reads of a stage, waited for before its MFMAs, come after these
    epi_bi[tid] = my_bi;  // writes in program order), or the barrier below
  }
  if (nk <= 0) {
    wait_lgkmcnt0();
    barrier_only();
  }
  if constexpr (!PF) {
    // Stage i: wait for this wave's loads of stage i (up to P-2 later stages may stay
    // in flight), barrier, issue stage i+P-1, read and consume stage i.
    int cur = 0, nxt = P - 1;
    for (int i = 0; i < nk; ++i) {
      wait_stages<FPW * CPS, P - 2>(nk - 1 - i);
      barrier_only();
      if (i + P - 1 < nk) issue(ring + nxt * SB, i + P - 1);
#pragma unroll
      for (int c = 0; c < CPS; ++c) {
        V xa[MB][2];
        i32x4_t wq[NB];
        read(xa, wq, ring + cur * SB + c * F * 1024);
        mma(xa, wq);
      }
      cur = cur + 1 == P ? 0 : cur + 1;
      nxt = nxt + 1 == P ? 0 : nxt + 1;
    }
  } else {
    // Operands read one stage ahead into a second register set: step i waits for stage
    // i+1's loads (up to P-3 later stages may stay in flight), barrier (stage i+1 has
    // landed for every wave, and every wave is done with stage i-1, whose buffer the
    // issue of stage i+P-1 reuses), issues stage i+P-1, reads stage i+1, and runs stage
    // i's MFMAs from the registers read the step before.  The compiler places those reads
    // after the MFMAs; their latency then passes during the next step's wait and barrier
    // instead of between a barrier and the first MFMA of the stage they feed (pinning them
    // ahead of the MFMAs measured slower: the wait-count pass then waits for them there).
    V xa0[CPS][MB][2], xa1[CPS][MB][2];
    i32x4_t wq0[CPS][NB], wq1[CPS][NB];
    auto read_st = [&](V (&xs)[CPS][MB][2], i32x4_t (&ws)[CPS][NB], const uint8_t* stage) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < CPS; ++c) read(xs[c], ws[c], stage + c * F * 1024);
    };
    auto mma_st = [&](const V (&xs)[CPS][MB][2], const i32x4_t (&ws)[CPS][NB]) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < CPS; ++c) mma(xs[c], ws[c]);
    };
    if (nk > 0) {
      wait_stages<FPW * CPS, P - 2>(nk - 1);
      barrier_only();
      read_st(xa0, wq0, ring);
    }
    // Steps i with a next stage: wait for stage i+1, barrier, issue stage i+P-1, read
    // stage i+1 into the other register set, then stage i's MFMAs.  The loop runs the
    // steps in pairs with no branch around the MFMAs (a join there makes the register
    // allocator copy every accumulator); the last one or two stages follow it.
    auto advance = [&](int i, V (&xn)[CPS][MB][2], i32x4_t (&wn_)[CPS][NB]) __attribute__((always_inline)) {
      wait_stages<FPW * CPS, (P >= 3 ? P - 3 : 0)>(nk - 2 - i);
      barrier_only();
      if (i + P - 1 < nk) issue(ring + ((i + P - 1) % P) * SB, i + P - 1);
      read_st(xn, wn_, ring + ((i + 1) % P) * SB);
    };
    int i = 0;
    for (; i + 2 < nk; i += 2) {
      advance(i, xa1, wq1);
      mma_st(xa0, wq0);
      advance(i + 1, xa0, wq0);
      mma_st(xa1, wq1);
    }
    if (i + 1 < nk) {
      advance(i, xa1, wq1);
      mma_st(xa0, wq0);
      mma_st(xa1, wq1);
    } else if (i < nk) {
      mma_st(xa0, wq0);
    }
  }

  if (S > 1) {
    constexpr int NV = NB * MB * 4;
    float a[NV];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t = 0; t < 4; ++t) a[(nb * MB + mb) * 4 + t] = acc[nb][mb][t];
    if (!splitk_meet<NV>(a, part + (int64_t)tile * S * (NW * 64) * NV, &counters[tile], S, split, tid, NW * 64, &flag))
      return;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[nb][mb][t] = a[(nb * MB + mb) * 4 + t];
  }

  // D of each 16x16 MFMA: lane (c16, g) holds rows 4g..4g+3 (weight rows n) of
  // column c16 (activation row m): four consecutive outputs of one row of y.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int nbase = n0 + (wn * NB + nb) * 16 + 4 * g;
    float sc[4], bi[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int col = (wn * NB + nb) * 16 + 4 * g + t;
      sc[t] = scale_bits_to_f32(epi_sc[col], sdt);
      bi[t] = bias ? xbits_to_f32<XT>(epi_bi[col]) : 0.0f;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = m0 + (wm * MB + mb) * 16 + c16;
      if (m >= M) continue;
      XT* yr = y + (int64_t)m * ldy;
      float v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = bias ? acc[nb][mb][t] * sc[t] + bi[t] : acc[nb][mb][t] * sc[t];
      const uint32_t lo = pack2_f32<XT>(v[0], v[1]), hi = pack2_f32<XT>(v[2], v[3]);
      if (nbase + 3 < N && ((uintptr_t)(yr + nbase) & 7) == 0) {
        *(uint2*)(yr + nbase) = make_uint2(lo, hi);
      } else {
        const uint16_t o[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (nbase + t < N) yr[nbase + t] = XT{o[t]};
      }
    }
  }
}


struct PipeCfg { int bm, bn, P, wm, S, cps, mtiles, ntiles, pf, nw, cps2; };

constexpr int pipe_stage_bytes_c(int bm, int bn) { return (bm / 8 + bn / 16) * 1024; }

// Stage counts built per tile shape (read-ahead from 3); a calibrator may pick one through
// algo bits 16-23.
inline bool pipe_p_ok(int bm, int bn, int p, int nw = 4) {
  if (p != 2 && p != 3 && p != 4 && p != 6 && p != 8) return false;
  if (nw == 8 && p != 3 && p != 4) return false;
  const int fpw = (bm / 8 + bn / 16) / nw;
  return p * pipe_stage_bytes_c(bm, bn) + 64 <= kLdsBytes && (p - 2) * fpw < 64;
}

// Automatic choice, from sweeps of tile shape x wave count x stages x read-ahead x splits
// over the talker shapes at M = 64..2048 (configs[3]; µs at M = 256 / 1024 / 2048 below):
//   * 32 x 64 tiles and 4 waves where they number at most 256, up to M = 128, and up to
//     M = 256 for K <= 4096 (o_proj at M = 256: 9.1; the decode-sized shapes), and where
//     they number at most 512 for K <= 1024 up to M = 256 (the code predictor's qkv at
//     M = 256: 8.2 against 10.3 with 8 waves; its gate_up at M = 128: 8.0 against 9.7),
//     and where they number at most 384 up to M = 64 (the talker's gate_up at 40 / 48 rows:
//     -0.7 / -0.4 µs a call against 8 waves on 64 x 128, level at 64);
//   * otherwise 8 waves (two a SIMD) on a 1 x 8 grid, each wave dequantizing only its own
//     weight columns, with 4 stages read one stage ahead:
//       - 128 x 384 tiles (3 stages, no read-ahead: 197 registers, the read-ahead set would
//         spill) where N is a multiple of 384, they number at least 256 and they fill
//         whole rounds of 256 workgroups at least as well as 128 x 256 would (gate_up at
//         M = 1024: 256 tiles, 52.7 against 65.9 us on 384 tiles of 128 x 256; 106.7
//         against 111.7 at M = 2048);
//       - else 128 x 256 tiles where they number at least 192, or at least 128 with K >= 4096
//         (gate_up from M = 512: 39.9 / 74.8 / 124.2, against 51.5 / 78.1 / 142.9 with
//         the former 4-wave 64 x 128 and 128 x 128 tiles; qkv at M = 2048 43.5 against
//         52.3; down_proj at M = 2048 68.4 against 72.0);
//       - else 64 x 256 tiles where they number at least 192 (gate_up at M = 256: 23.3
//         against 25.7; qkv at M = 1024 25.4 against 26.8);
//       - else 64 x 128 (down_proj 17.1 / 37.7 against 18.4 / 39.7, o_proj at M = 1024
//         15.4 against 16.7, gate_up at M = 128 14.9 against 18.5).
//   Splits: with 4 waves, split K while the workgroups stay within 256, keeping >= 8 chunks
//   a split, except for K <= 1024 with at least 128 tiles and for at least 192 tiles (the
//   code predictor's qkv and gate_up at 40-96 rows, cache-resident: 192 tiles 1.0-1.3 µs a
//   call faster unsplit than in two splits, 128 tiles 0.3 µs; the talker's gate_up at 17-32
//   rows and qkv at 72-96, 192 tiles: 0.9-1.6 µs faster unsplit); the former rule split until
//   there were at least 256 workgroups, up to 384 (the talker's o_proj at 72-96 rows, 96
//   tiles, 0.8-1.0 µs faster in two splits than in four; at 160-192 rows 1.7-1.9 µs faster
//   unsplit than in two; the predictor's o_proj and down_proj at 160-192 rows 0.8-1.2);
//   with 8 waves likewise (a split-K meeting costs more than the idle compute units it
//   fills: gate_up at M = 128, 192 tiles, 14.9 unsplit against 18.7 in two splits).
// Two chunks a stage: the 4-wave 32 x 64 tiles with 4 stages and read-ahead where they number
//   at most 256 or K >= 2048, and every split's chunk count is even (half the stage waits and barriers of
//   a latency-bound call; a call minus the same kernel with one chunk a stage, µs, over 5
//   layers: code predictor qkv -0.53 to -0.59 at M = 48-128, down_proj -0.21 to -0.39 at
//   64-128, gate_up -0.51 / -0.58 at 48 / 64; talker qkv -1.0 at 48 / 64 and -3.25 at 128,
//   down_proj -5.48 and o_proj -1.65 at 128; the talker's gate_up at 40-64 rows, 384 tiles,
//   -0.1 to -0.8).  Past 256 tiles with K = 1024 it lost (predictor gate_up +0.3 at 96 / 128
//   rows, 288 / 384 tiles; qkv +0.33 at 256 rows, 512 tiles).
// A workspace too small for the splits drops the automatic choice to one split.
// shape_req (algo bits 24-30): bits 0-1 log2(BM / 16) in 1..3 (0 = 256 rows, 8 waves
// only), bit 2 a 2 x 2 (2 x 4 with 8 waves) wave grid in place of 1 x 4 (1 x 8), bit 3
// 8 waves in place of 4, bits 4-6 log2(BN / 32) in 1..3 (4: 384 columns, 8 waves, 128
// rows); 0 = automatic.  stages_req
// (algo bits 16-23): bits 0-5 the stage count (0 = automatic), bit 6 read-ahead; 0 =
// automatic.
inline PipeCfg pipe_cfg(int64_t m, int64_t n, int64_t k, int splits_req, int stages_req, int shape_req = 0) {
  PipeCfg c;
  const int nchunks = std::max(1, (int)(k / 64));
  auto tiles_of = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
  c.wm = 1;
  c.nw = 4;
  c.cps2 = (stages_req >> 7) & 1;
  if (shape_req != 0) {
    c.nw = (shape_req & 8) ? 8 : 4;
    c.bm = (shape_req & 3) == 0 ? 256 : 16 << (shape_req & 3);
    c.bn = ((shape_req >> 4) & 7) == 4 ? 384 : 32 << ((shape_req >> 4) & 7);
    c.wm = (shape_req >> 2) & 1 ? 2 : 1;
  } else if (m <= 256 && ((tiles_of(32, 64) <= 256 && (m <= 128 || nchunks <= 64)) ||
                          (tiles_of(32, 64) <= 512 && nchunks <= 16) || (tiles_of(32, 64) <= 384 && m <= 64))) {
    c.bm = 32;
    c.bn = 64;
  } else {
    c.nw = 8;
    const int64_t t256 = tiles_of(128, 256);
    // the share of a whole number of rounds (256 compute units, one workgroup each) tiles fill
    auto fill = [](int64_t t) { return (double)t / (double)(((t + 255) / 256) * 256); };
    if (n % 384 == 0 && tiles_of(128, 384) >= 256 && fill(tiles_of(128, 384)) >= fill(t256)) {
      c.bm = 128;
      c.bn = 384;
    } else if (t256 >= 192 || (t256 >= 128 && nchunks >= 64)) {
      c.bm = 128;
      c.bn = 256;
    } else if (tiles_of(64, 256) >= 192) {
      c.bm = 64;
      c.bn = 256;
    } else {
      c.bm = 64;
      c.bn = 128;
    }
  }
  c.mtiles = (int)((m + c.bm - 1) / c.bm);
  c.ntiles = (int)((n + c.bn - 1) / c.bn);
  if (stages_req == 0) {
    c.P = 4 * pipe_stage_bytes_c(c.bm, c.bn) + 64 <= kLdsBytes ? 4 : 3;
    c.pf = c.bn == 384 ? 0 : 1;  // 384 columns: 3 stages, no room for a second register set
  } else {
    c.P = (stages_req & 0x3f) > 0 ? (stages_req & 0x3f) : (c.bm * c.bn <= 32 * 64 ? 4 : 3);
    c.pf = (stages_req >> 6) & 1;
  }
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  int S = splits_req;
  if (S <= 0) {
    S = 1;
    if (c.nw == 8)
      while (tiles * S * 2 <= 256 && nchunks / (S * 2) >= 8) S *= 2;
    else if (!((nchunks <= 16 && tiles >= 128) || tiles >= 192))
      while (tiles * S * 2 <= 256 && nchunks / (S * 2) >= 8) S *= 2;
  }
  S = std::max(1, std::min(S, nchunks));
  if (tiles > kMaxSplitTiles) S = 1;
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  if (stages_req == 0 && c.nw == 4 && c.bm == 32 && c.bn == 64 && c.P == 4 && c.pf && (tiles <= 256 || nchunks >= 32) &&
      c.cps % 2 == 0 && nchunks % 2 == 0)
    c.cps2 = 1;
  return c;
}

inline int64_t pipe_ws(const PipeCfg& c) {
  if (c.S <= 1) return 0;
  // one fp32 partial tile per (tile, split)
  return kCounterBytes + (int64_t)c.mtiles * c.ntiles * c.S * c.bm * c.bn * 4;
}

struct PipeArgs {
  const void* x; int64_t m, k, ldx; const int8_t* qs; int64_t n; const void* scale; int sdt; const void* bias;
  void* y; int64_t ldy; float* part; unsigned* counters;
};

template <bool F8W, typename XT, int BM, int BN, int P, int WM>
inline void launch_pipe_p(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
  if constexpr (P * pipe_stage_bytes_c(BM, BN) + 64 <= kLdsBytes) {
    if constexpr (BM == 32 && BN == 64 && WM == 1 && (P == 3 || P == 4)) {
      if (c.cps2) {
        qtts::launch(&w8a16_pipe_kernel<XT, BM, BN, P, WM, F8W, true, 4, 2>, dim3(blocks), dim3(256), 0, st,
                     (const XT*)a.x, (int)a.m, (int)a.k, a.ldx, a.qs, (int)a.n, a.scale, a.sdt, (const XT*)a.bias,
                     (XT*)a.y, a.ldy, a.part, a.counters, c.mtiles, c.ntiles, c.S, c.cps);
        return;
      }
    }
    if (c.pf)
      qtts::launch(&w8a16_pipe_kernel<XT, BM, BN, P, WM, F8W, true>, dim3(blocks), dim3(256), 0, st, (const XT*)a.x,
                   (int)a.m, (int)a.k, a.ldx, a.qs, (int)a.n, a.scale, a.sdt, (const XT*)a.bias, (XT*)a.y, a.ldy, a.part,
                   a.counters, c.mtiles, c.ntiles, c.S, c.cps);
    else
      qtts::launch(&w8a16_pipe_kernel<XT, BM, BN, P, WM, F8W>, dim3(blocks), dim3(256), 0, st, (const XT*)a.x, (int)a.m,
                   (int)a.k, a.ldx, a.qs, (int)a.n, a.scale, a.sdt, (const XT*)a.bias, (XT*)a.y, a.ldy, a.part,
                   a.counters, c.mtiles, c.ntiles, c.S, c.cps);
  }
}

template <bool F8W, typename XT, int BM, int BN, int WM>
inline void launch_pipe_stages(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
  switch (c.P) {
    case 2: launch_pipe_p<F8W, XT, BM, BN, 2, WM>(c, a, blocks, st); break;
    case 3: launch_pipe_p<F8W, XT, BM, BN, 3, WM>(c, a, blocks, st); break;
    case 4: launch_pipe_p<F8W, XT, BM, BN, 4, WM>(c, a, blocks, st); break;
    case 6: launch_pipe_p<F8W, XT, BM, BN, 6, WM>(c, a, blocks, st); break;
    default: launch_pipe_p<F8W, XT, BM, BN, 8, WM>(c, a, blocks, st); break;
  }
}

template <bool F8W, typename XT, int BM, int BN>
inline void launch_pipe_grid(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
  if (c.wm == 2) launch_pipe_stages<F8W, XT, BM, BN, 2>(c, a, blocks, st);
  else launch_pipe_stages<F8W, XT, BM, BN, 1>(c, a, blocks, st);
}

template <bool F8W, typename XT, int BM>
inline void launch_pipe_bn(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
  if (c.bn == 256) launch_pipe_grid<F8W, XT, BM, 256>(c, a, blocks, st);
  else if (c.bn == 128) launch_pipe_grid<F8W, XT, BM, 128>(c, a, blocks, st);
  else launch_pipe_grid<F8W, XT, BM, 64>(c, a, blocks, st);
}

template <bool F8W, typename XT, int BM, int BN, int WM>
inline void launch_pipe8_p(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
#define QTTS_P8(P, PF)                                                                                             \
  do {                                                                                                             \
    if constexpr (P * pipe_stage_bytes_c(BM, BN) + 64 <= kLdsBytes)                                                \
      qtts::launch(&w8a16_pipe_kernel<XT, BM, BN, P, WM, F8W, PF, 8>, dim3(blocks), dim3(512), 0, st,              \
                   (const XT*)a.x, (int)a.m, (int)a.k, a.ldx, a.qs, (int)a.n, a.scale, a.sdt, (const XT*)a.bias,   \
                   (XT*)a.y, a.ldy, a.part, a.counters, c.mtiles, c.ntiles, c.S, c.cps);                           \
  } while (0)
  if constexpr (BN == 384) {  // built with 3 stages and no read-ahead only (the launcher checks)
    QTTS_P8(3, false);
  } else if (c.P == 3) {
    if (c.pf) QTTS_P8(3, true);
    else QTTS_P8(3, false);
  } else {
    if (c.pf) QTTS_P8(4, true);
    else QTTS_P8(4, false);
  }
#undef QTTS_P8
}

// Eight waves (two a SIMD): 32 x 64, 128 x 128 and 256 x 128 tiles on a 2 x 4 grid,
// 64 x 256 and 128 x 384 (3 stages, no read-ahead) on 1 x 8, 64 x 128 and 128 x 256 on either.
template <bool F8W, typename XT>
inline void launch_pipe8(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
  if (c.bm == 32) launch_pipe8_p<F8W, XT, 32, 64, 2>(c, a, blocks, st);
  else if (c.bm == 64 && c.bn == 256) launch_pipe8_p<F8W, XT, 64, 256, 1>(c, a, blocks, st);
  else if (c.bm == 64 && c.wm == 1) launch_pipe8_p<F8W, XT, 64, 128, 1>(c, a, blocks, st);
  else if (c.bm == 64) launch_pipe8_p<F8W, XT, 64, 128, 2>(c, a, blocks, st);
  else if (c.bm == 128 && c.bn == 128) launch_pipe8_p<F8W, XT, 128, 128, 2>(c, a, blocks, st);
  else if (c.bm == 256 && c.bn == 128) launch_pipe8_p<F8W, XT, 256, 128, 2>(c, a, blocks, st);
  else if (c.bm == 128 && c.bn == 256 && c.wm == 1) launch_pipe8_p<F8W, XT, 128, 256, 1>(c, a, blocks, st);
  else if (c.bn == 384) launch_pipe8_p<F8W, XT, 128, 384, 1>(c, a, blocks, st);
  else launch_pipe8_p<F8W, XT, 128, 256, 2>(c, a, blocks, st);
}

inline bool pipe8_shape_built(int bm, int bn, int wm) {
  return (bm == 32 && bn == 64 && wm == 2) || (bm == 64 && bn == 128) || (bm == 64 && bn == 256 && wm == 1) ||
         (bm == 128 && bn == 384 && wm == 1) || (bm == 128 && bn == 128 && wm == 2) ||
         (bm == 256 && bn == 128 && wm == 2) || (bm == 128 && bn == 256);
}

template <bool F8W, typename XT>
inline void launch_pipe_bm(const PipeCfg& c, const PipeArgs& a, unsigned blocks, hipStream_t st) {
  if (c.nw == 8) launch_pipe8<F8W, XT>(c, a, blocks, st);
  else if (c.bm == 32) launch_pipe_bn<F8W, XT, 32>(c, a, blocks, st);
  else if (c.bm == 64) launch_pipe_bn<F8W, XT, 64>(c, a, blocks, st);
  else launch_pipe_bn<F8W, XT, 128>(c, a, blocks, st);
}

// stages_req: bits 0-5 the count, bit 6 read-ahead, bit 7 two chunks a stage, nothing above.
inline bool pipe_stages_ok(int stages) { return stages >= 0 && (stages >> 8) == 0; }

inline bool pipe_shape_ok(int shape) {
  if (shape == 0) return true;
  const int b = shape & 3, c = (shape >> 4) & 7;
  if (shape & 8) {  // eight waves: the built tiles only (BN code 4: 384 columns)
    const int bm = b == 0 ? 256 : 16 << b, bn = c == 4 ? 384 : 32 << c;
    return (shape >> 7) == 0 && c >= 1 && c <= 4 && pipe8_shape_built(bm, bn, (shape & 4) ? 2 : 1);
  }
  return (shape >> 7) == 0 && b >= 1 && c >= 1 && c <= 3;
}

// x [m, k] (bf16 or fp16, 16-byte aligned rows), qs strip layout, k % 64 == 0, m > 0.
template <bool F8W>
inline int w8a16_pipe_launch(const char* what, const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                              const int8_t* qs, int64_t n, const void* scale, int sdt, const void* bias, void* y,
                              int64_t ldy, int splits, int stages, int shape, void* ws, int64_t ws_bytes,
                              hipStream_t st) {
  if (!pipe_shape_ok(shape))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: bad tile shape code %d", what, shape);
  if (!pipe_stages_ok(stages))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: bad stages code %d", what, stages);
  PipeCfg c = pipe_cfg(m, n, k, splits, stages, shape);
  if (c.pf && c.P < 3)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: read-ahead needs 3 stages", what);
  if (c.bn == 384 && (c.P != 3 || c.pf))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: 128x384 tiles are built with 3 stages and no read-ahead", what);
  if (c.cps2 && !(c.nw == 4 && c.bm == 32 && c.bn == 64 && c.wm == 1 && c.pf && (c.P == 3 || c.P == 4)))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                          "%s: two chunks a stage are built for 32x64 tiles of 4 waves, 3 or 4 stages, read-ahead", what);
  if (!pipe_p_ok(c.bm, c.bn, c.P, c.nw))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: %d stages are not built for a %dx%d tile", what, c.P,
                          c.bm, c.bn);
  const int64_t need = pipe_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "%s with %d splits needs %lld workspace bytes, got %lld", what,
                            c.S, (long long)need, (long long)ws_bytes);
    c = pipe_cfg(m, n, k, 1, stages, shape);
  }
  if (c.cps2 && (c.cps % 2 != 0 || (k / 64) % 2 != 0))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: two chunks a stage need an even chunk count per split (%d)",
                          what, c.cps);
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  const int64_t blocks = (tiles + 7) / 8 * 8 * c.S;
  if (blocks <= 0 || blocks >= ((int64_t)1 << 31))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: problem too large", what);
  unsigned* counters = (unsigned*)ws;
  float* part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
  const PipeArgs a{x, m, k, ldx, qs, n, scale, sdt, bias, y, ldy, part, counters};
  if (x_dtype == QTTS_BF16) launch_pipe_bm<F8W, bf16_t>(c, a, (unsigned)blocks, st);
  else launch_pipe_bm<F8W, f16_t>(c, a, (unsigned)blocks, st);
  return qtts_check_launch(what);
}

}  // namespace qtts
