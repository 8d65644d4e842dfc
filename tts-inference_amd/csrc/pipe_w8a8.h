// W8A8 GEMM for prefill-sized rows (M > 16) on gfx950, shared by the fp8 (OCP e4m3)
// and int8 paths: both operands are 8-bit codes that go from LDS to the matrix cores
// with no conversion, and only the MFMA, the accumulator type and the epilogue differ.
//
//   fp8:  y = round(acc_f32 * sx[m] * sw[n]) [+ bias]     torch._scaled_mm rowwise,
//         qtts/quant/fp8.py:79-89 (bias added in the output dtype after rounding)
//   int8: y = round((f32(acc_i32) * sx[m]) * sw[n] [+ f32(bias)])     torch._int_mm and
//         the fp32 epilogue of qtts/quant/int8.py:151-160 (one rounding at the end)
//
// Same pipeline as the W8A16 tile kernel (tile.hip): 4 waves (8, two a SIMD, on the
// larger tiles) own a BM x BN tile and walk K through a P-deep LDS ring filled by
// direct global -> LDS loads, one barrier per stage.  A stage is 128 K columns, and
// every load writes one 1 KiB half of the stage's MFMA fragments in lane order (lane l:
// row l % 16 of a 16-row block, 16 bytes at stage column Kind::col(l / 16, h)):
//   * fp8: the two halves are the 32-byte operand of one
//     v_mfma_scale_f32_16x16x128_f8f6f4 (unit block scales); col = 32 g + 16 h, the
//     QTTS_STRIP_FP8 block's lane order;
//   * int8: each half is the 16-byte operand of one v_mfma_i32_16x16x64_i8 over one
//     64-column chunk; col = 64 h + 16 g, two consecutive QTTS_STRIP_INT8 blocks.
// With strip weights a weight half is 1 KiB of contiguous memory; with row-major
// weights (int8 only) it is gathered like an activation half, 64 contiguous bytes a
// row.  Of NW waves, wave w owns columns [n0 + w BN/NW, n0 + (w+1) BN/NW) for all BM rows.
#pragma once

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "layout.h"
#include "pipe.h"
#include "splitk.h"

namespace qtts {

template <typename OT> __device__ __forceinline__ uint32_t load_out_bits(const OT* p) {
  if constexpr (sizeof(OT) == 4)
    return __hip_atomic_load((uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    return __hip_atomic_load((uint16_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <typename OT> __device__ __forceinline__ float out_bits_to_f32(uint32_t b) {
  if constexpr (std::is_same<OT, float>::value) return __uint_as_float(b);
  else return to_f32(OT{(uint16_t)b});
}

__device__ __forceinline__ i32x8_t concat8(i32x4_t a, i32x4_t b) {
  return i32x8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

struct PipeFp8 {
  typedef f32x4_t acc_t;
  typedef float part_t;
  typedef uint8_t code_t;
  static __device__ __forceinline__ int col(int g, int h) { return 32 * g + 16 * h; }
  static __device__ __forceinline__ acc_t mma(i32x4_t w0, i32x4_t w1, i32x4_t x0, i32x4_t x1, acc_t c) {
    return mma_fp8_16x16x128(concat8(w0, w1), concat8(x0, x1), c);
  }
  template <typename OT>
  static __device__ __forceinline__ float out(float acc, float sx, float sw, float bias, bool has_bias) {
    const float v = round_through<OT>(acc * sx * sw);
    return has_bias ? v + bias : v;
  }
};

struct PipeI8 {
  typedef i32x4_t acc_t;
  typedef int part_t;
  typedef int8_t code_t;
  static __device__ __forceinline__ int col(int g, int h) { return 64 * h + 16 * g; }
  static __device__ __forceinline__ acc_t mma(i32x4_t w0, i32x4_t w1, i32x4_t x0, i32x4_t x1, acc_t c) {
    return mma_i8_16x16x64(w1, x1, mma_i8_16x16x64(w0, x0, c));
  }
  template <typename OT>
  static __device__ __forceinline__ float out(int acc, float sx, float sw, float bias, bool has_bias) {
    return int8_epilogue(acc, sx, sw, bias, has_bias);
  }
};

template <typename Kind, typename OT, int BM, int BN, int P, int LAYOUT, bool PF = false, int NW = 4>
__global__ __launch_bounds__(NW * 64) void w8a8_pipe_kernel(
    const typename Kind::code_t* __restrict__ qx_, const float* __restrict__ sx, int M, int K, int64_t ldqx,
    const typename Kind::code_t* __restrict__ qw_, int N, int64_t ldqw, const float* __restrict__ sw,
    const OT* __restrict__ bias, OT* __restrict__ y, int64_t ldy, typename Kind::part_t* __restrict__ part,
    unsigned* __restrict__ counters, int mtiles, int ntiles, int S, int cps) {
  typedef typename Kind::acc_t acc_t;
  typedef typename Kind::part_t part_t;
  constexpr int MB = BM / 16;          // 16-row m-blocks per tile
  constexpr int NB = BN / 16 / NW;     // 16-column strips per wave
  constexpr int XF = 2 * MB;           // activation halves per stage
  constexpr int WF = 2 * (BN / 16);    // weight halves per stage
  constexpr int F = XF + WF;
  constexpr int FPW = F / NW;          // halves each wave loads per stage
  constexpr int SB = F * 1024;         // stage bytes
  static_assert(F % NW == 0 && NB >= 1 && (NW == 4 || NW == 8), "fragments must split evenly over the waves");
  static_assert(P >= 2 && P * SB + 64 <= kLdsBytes, "stage ring must fit in LDS");
  static_assert((P - 2) * FPW < 64, "vmcnt is 6 bits");
  __shared__ __align__(1024) uint8_t ring[P * SB];
  __shared__ unsigned flag;
  const uint8_t* qx = (const uint8_t*)qx_;
  const uint8_t* qw = (const uint8_t*)qw_;

  int tile, split;
  decode_wg(blockIdx.x, S, tile, split);
  if (tile >= mtiles * ntiles) return;
  const int nt = tile % ntiles, mt = tile / ntiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int nchunks = K >> 7;
  const int strips = (N + 15) >> 4;
  const int kc0 = split * cps;
  const int nk = min(cps, nchunks - kc0);

  // Epilogue operands first, as raw bits (loads the compiler will not sink).
  uint32_t sxb[MB], swb[NB][4], bib[NB][4];
  {
    const OT* bsrc = bias ? bias : y;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      sxb[mb] = __hip_atomic_load((uint32_t*)sx + min(m0 + mb * 16 + c16, M - 1), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int n = min(n0 + (wave * NB + nb) * 16 + 4 * g + t, N - 1);
        swb[nb][t] = __hip_atomic_load((uint32_t*)sw + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        bib[nb][t] = load_out_bits(bsrc + n);
      }
  }

  const uint8_t* src[FPW];
  int64_t stride[FPW];
#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int f = wave * FPW + j;
    if (f < XF) {
      const int mb = f >> 1, h = f & 1;
      const int m = min(m0 + mb * 16 + c16, M - 1);
      src[j] = qx + (int64_t)m * ldqx + (int64_t)kc0 * 128 + Kind::col(g, h);
      stride[j] = 128;
    } else {
      const int sb = (f - XF) >> 1, h = (f - XF) & 1;
      if constexpr (LAYOUT == kLayoutStrips) {
        const int s = min(n0 / 16 + sb, strips - 1);
        src[j] = qw + ((int64_t)s * nchunks + kc0) * 2048 + h * 1024 + lane * 16;
        stride[j] = 2048;
      } else {
        const int n = min(n0 + sb * 16 + c16, N - 1);
        src[j] = qw + (int64_t)n * ldqw + (int64_t)kc0 * 128 + Kind::col(g, h);
        stride[j] = 128;
      }
    }
  }

  auto issue = [&](uint8_t* stage, int i) {
#pragma unroll
    for (int j = 0; j < FPW; ++j) load_to_lds16(src[j] + (int64_t)i * stride[j], stage + (wave * FPW + j) * 1024);
  };

  acc_t acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = acc_t{0, 0, 0, 0};

  // A stage's operands: every activation half of the tile, and this wave's weight halves.
  struct Ops { i32x4_t x0[MB], x1[MB], w0[NB], w1[NB]; };
  auto read = [&](Ops& o, const uint8_t* stage) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      o.x0[mb] = *(const i32x4_t*)(stage + (2 * mb) * 1024 + lane * 16);
      o.x1[mb] = *(const i32x4_t*)(stage + (2 * mb + 1) * 1024 + lane * 16);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint8_t* wsrc = stage + (XF + 2 * (wave * NB + nb)) * 1024 + lane * 16;
      o.w0[nb] = *(const i32x4_t*)wsrc;
      o.w1[nb] = *(const i32x4_t*)(wsrc + 1024);
    }
  };
  auto mma = [&](const Ops& o) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = Kind::mma(o.w0[nb], o.w1[nb], o.x0[mb], o.x1[mb], acc[nb][mb]);
  };

  for (int p = 0; p < P - 1; ++p)
    if (p < nk) issue(ring + p * SB, p);
  if constexpr (!PF) {
    // Stage i: wait for this wave's loads of stage i (up to P-2 later stages may stay in
    // flight), barrier, issue stage i+P-1, read and consume stage i.
    int cur = 0, nxt = P - 1;
    for (int i = 0; i < nk; ++i) {
      wait_stages<FPW, P - 2>(nk - 1 - i);
      barrier_only();
      if (i + P - 1 < nk) issue(ring + nxt * SB, i + P - 1);
      Ops o;
      read(o, ring + cur * SB);
      mma(o);
      cur = cur + 1 == P ? 0 : cur + 1;
      nxt = nxt + 1 == P ? 0 : nxt + 1;
    }
  } else {
    // Read-ahead, as in the W8A16 tile kernel: step i waits for stage i+1 (up to P-3
    // later stages in flight), barrier (stage i+1 landed for every wave; every wave is
    // done with stage i-1, whose buffer the issue of stage i+P-1 reuses), issues stage
    // i+P-1, reads stage i+1 into the other register set, then runs stage i's MFMAs.
    // Steps go in pairs with no branch around the MFMAs.
    Ops o0, o1;
    if (nk > 0) {
      wait_stages<FPW, P - 2>(nk - 1);
      barrier_only();
      read(o0, ring);
    }
    auto advance = [&](int i, Ops& on) __attribute__((always_inline)) {
      wait_stages<FPW, (P >= 3 ? P - 3 : 0)>(nk - 2 - i);
      barrier_only();
      if (i + P - 1 < nk) issue(ring + ((i + P - 1) % P) * SB, i + P - 1);
      read(on, ring + ((i + 1) % P) * SB);
    };
    int i = 0;
    for (; i + 2 < nk; i += 2) {
      advance(i, o1);
      mma(o0);
      advance(i + 1, o0);
      mma(o1);
    }
    if (i + 1 < nk) {
      advance(i, o1);
      mma(o0);
      mma(o1);
    } else if (i < nk) {
      mma(o0);
    }
  }

  if (S > 1) {
    constexpr int NV = NB * MB * 4;
    part_t a[NV];
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

  // D of each 16x16 MFMA: lane (c16, g) holds rows 4g..4g+3 (weight rows n) of column
  // c16 (activation row m).
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int nbase = n0 + (wave * NB + nb) * 16 + 4 * g;
    float swv[4], biv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      swv[t] = __uint_as_float(swb[nb][t]);
      biv[t] = out_bits_to_f32<OT>(bib[nb][t]);
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = m0 + mb * 16 + c16;
      if (m >= M) continue;
      const float sxv = __uint_as_float(sxb[mb]);
      OT* yr = y + (int64_t)m * ldy;
      float v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = Kind::template out<OT>(acc[nb][mb][t], sxv, swv[t], biv[t], bias != nullptr);
      if constexpr (std::is_same<OT, float>::value) {
        if (nbase + 3 < N && ((uintptr_t)(yr + nbase) & 15) == 0) {
          *(f32x4_t*)(yr + nbase) = f32x4_t{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (nbase + t < N) yr[nbase + t] = v[t];
        }
      } else {
        const uint32_t lo = pack2_f32<OT>(v[0], v[1]), hi = pack2_f32<OT>(v[2], v[3]);
        if (nbase + 3 < N && ((uintptr_t)(yr + nbase) & 7) == 0) {
          *(uint2*)(yr + nbase) = make_uint2(lo, hi);
        } else {
          const uint16_t o[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (nbase + t < N) yr[nbase + t] = OT{o[t]};
        }
      }
    }
  }
}

// ---- host side: configuration and launch --------------------------------------------

struct W8A8PipeCfg { int bm, bn, P, S, cps, mtiles, ntiles, pf, nw; };

constexpr int w8a8_stage_bytes(int bm, int bn) { return (bm / 8 + bn / 8) * 1024; }

inline bool w8a8_p_ok(int bm, int bn, int p, int nw = 4) {
  if (p != 2 && p != 3 && p != 4 && p != 6 && p != 8) return false;
  if (nw == 8 && p != 3 && p != 4) return false;
  const int fpw = (bm / 8 + bn / 8) / nw;
  return p * w8a8_stage_bytes(bm, bn) + 64 <= kLdsBytes && (p - 2) * fpw < 64;
}

// Automatic choice, from sweeps of tile shape x wave count x stages x read-ahead x splits
// over the talker shapes at M = 64..2048 (int8 and fp8 alike; 128-column stages; µs for
// int8, the former choice in brackets):
//   * 32 x 64 tiles, 4 waves, 4 stages up to M = 256 while they number at most 512 (the
//     4-wave kernel stays ahead there: qkv at M = 128 6.3 against 9.0 with 8 waves);
//   * otherwise 8 waves (two a SIMD), each owning BN / 8 columns of all BM rows:
//       - 128 x 256 tiles, 3 stages, where they number at least 192 (gate_up from
//         M = 512: 24.6 / 45.2 / 76.7 at M = 512 / 1024 / 2048 [27.0 / 50.7 / 97.6]; qkv
//         at M = 2048 26.4 [36.6]);
//       - else 64 x 256 tiles, 3 stages, where they number at least 192 (qkv at M = 1024
//         16.2 [18.8], o_proj at M = 2048 16.9 [19.4], gate_up at M = 256 15.6 [18.4]);
//       - else 64 x 128 tiles, 4 stages read one stage ahead (o_proj at M = 512 / 1024
//         9.3 / 9.8 [10.9 / 10.7], down_proj 16.6 / 22.2 [18.9 / 25.3], gate_up at M = 128
//         9.7 [13.2]);
// then split K: with 4 waves while the workgroups stay within 256 and the tiles number fewer
// than 192, keeping >= 4 stages a split (the former rule split until there were at least 256
// workgroups, up to 384, and from 192 tiles into two; a linear with its activation
// quantization, over 5 layers, µs, fp8 / int8: the talker's gate_up at 17-32 rows 11.8-12.3
// -> 10.0-10.3, qkv at 96 rows 11.3 / 11.5 -> 9.5 / 9.7, o_proj at 160-192 rows 11.1-11.5
// -> 9.3-10.0, down_proj at 160-192 rows 17.4-18.5 -> 16.1-17.3; the predictor's gate_up at
// 48-64 rows 9.9-10.2 -> 8.1-8.2 (fp8), its o_proj and down_proj at 160-192 rows 0.7-1.1
// faster; the one loss over 17-256 rows the talker's int8 qkv at 192 rows, +0.18);
// with 8 waves only while the workgroups stay within 256 and each split keeps >= 16
// stages (a split-K meeting costs more than idle compute units on short K: o_proj at
// M = 512, 128 tiles, 9.3 unsplit against 10.2 in two splits).  shape_req: bits 0-2
// log2(BM / 16) in 1..3, bit 3 8 waves (BM 64 or 128, BN 128 or 256), bits 4-6
// log2(BN / 32) in 1..3, 0 = automatic; stages_req: bits 0-5 the stage count, bit 6
// read-ahead, 0 = automatic.
inline W8A8PipeCfg w8a8_cfg(int64_t m, int64_t n, int64_t k, int splits_req, int stages_req, int shape_req) {
  W8A8PipeCfg c;
  const int nchunks = std::max(1, (int)(k / 128));
  auto tiles_of = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
  c.nw = 4;
  if (shape_req != 0) {
    c.bm = 16 << (shape_req & 7);
    c.bn = 32 << ((shape_req >> 4) & 7);
    c.nw = shape_req & 8 ? 8 : 4;
  } else if (m <= 256 && tiles_of(32, 64) <= 512) {
    c.bm = 32;
    c.bn = 64;
  } else {
    c.nw = 8;
    if (tiles_of(128, 256) >= 192) {
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
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  if (stages_req == 0) {
    if (c.nw == 8) {  // read-ahead where 4 stages fit
      c.P = 4 * w8a8_stage_bytes(c.bm, c.bn) + 64 <= kLdsBytes ? 4 : 3;
      c.pf = c.P == 4 ? 1 : 0;
    } else {
      const bool ra = c.bm == 64 && c.bn == 128 && tiles <= 256;
      c.P = c.bm * c.bn <= 32 * 64 || ra ? 4 : 3;
      c.pf = ra ? 1 : 0;
    }
  } else {
    c.pf = (stages_req >> 6) & 1;
    c.P = (stages_req & 0x3f) > 0 ? (stages_req & 0x3f) : (c.bm * c.bn <= 32 * 64 ? 4 : 3);
  }
  int S = splits_req;
  if (S <= 0) {
    S = 1;
    if (c.nw == 8)
      while (tiles * S * 2 <= 256 && nchunks / (S * 2) >= 16) S *= 2;
    else if (tiles < 192)
      while (tiles * S * 2 <= 256 && nchunks / (S * 2) >= 4) S *= 2;
  }
  S = std::max(1, std::min(S, nchunks));
  if (tiles > kMaxSplitTiles) S = 1;
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  return c;
}

// Split-K workspace: the counter block, then 4-byte partials (fp32 or int32).
inline int64_t w8a8_ws(const W8A8PipeCfg& c) {
  if (c.S <= 1) return 0;
  return kCounterBytes + (int64_t)c.mtiles * c.ntiles * c.S * c.bm * c.bn * 4;  // one partial tile a split
}

// 8 waves (bit 3 of the shape code): BM 64 or 128, BN 128 or 256.
inline bool w8a8_shape_ok(int shape) {
  if (shape == 0) return true;
  const int b = shape & 7, c = (shape >> 4) & 7;
  if ((shape >> 7) != 0 || b < 1 || b > 3 || c < 1 || c > 3) return false;
  return !(shape & 8) || (b >= 2 && c >= 2);
}

template <typename Kind> struct W8A8Args {
  const typename Kind::code_t* qx; const float* sx; int64_t m, k, ldqx; const typename Kind::code_t* qw;
  int64_t n, ldqw; const float* sw; const void* bias; void* y; int64_t ldy; typename Kind::part_t* part;
  unsigned* counters;
};

template <typename Kind, typename OT, int LAYOUT, int BM, int BN, int P>
void w8a8_launch_p(const W8A8PipeCfg& c, const W8A8Args<Kind>& a, unsigned blocks, hipStream_t st) {
  if constexpr (P * w8a8_stage_bytes(BM, BN) + 64 <= kLdsBytes) {
    if (c.pf)
      qtts::launch(&w8a8_pipe_kernel<Kind, OT, BM, BN, P, LAYOUT, true>, dim3(blocks), dim3(256), 0, st, a.qx, a.sx,
                   (int)a.m, (int)a.k, a.ldqx, a.qw, (int)a.n, a.ldqw, a.sw, (const OT*)a.bias, (OT*)a.y, a.ldy,
                   a.part, a.counters, c.mtiles, c.ntiles, c.S, c.cps);
    else
      qtts::launch(&w8a8_pipe_kernel<Kind, OT, BM, BN, P, LAYOUT>, dim3(blocks), dim3(256), 0, st, a.qx, a.sx,
                   (int)a.m, (int)a.k, a.ldqx, a.qw, (int)a.n, a.ldqw, a.sw, (const OT*)a.bias, (OT*)a.y, a.ldy,
                   a.part, a.counters, c.mtiles, c.ntiles, c.S, c.cps);
  }
}

// kMaxP: the deepest ring built (2, 3, 4, 6, 8 up to it); deeper requests are rejected
// by the caller.
template <typename Kind, typename OT, int LAYOUT, int kMaxP, int BM, int BN>
void w8a8_launch_stages(const W8A8PipeCfg& c, const W8A8Args<Kind>& a, unsigned blocks, hipStream_t st) {
  switch (c.P) {
    case 2: w8a8_launch_p<Kind, OT, LAYOUT, BM, BN, 2>(c, a, blocks, st); break;
    case 3: w8a8_launch_p<Kind, OT, LAYOUT, BM, BN, 3>(c, a, blocks, st); break;
    case 4: w8a8_launch_p<Kind, OT, LAYOUT, BM, BN, 4>(c, a, blocks, st); break;
    case 6: if constexpr (kMaxP >= 6) w8a8_launch_p<Kind, OT, LAYOUT, BM, BN, 6>(c, a, blocks, st); break;
    default: if constexpr (kMaxP >= 8) w8a8_launch_p<Kind, OT, LAYOUT, BM, BN, 8>(c, a, blocks, st); break;
  }
}

template <typename Kind, typename OT, int LAYOUT, int kMaxP, int BM>
void w8a8_launch_bn(const W8A8PipeCfg& c, const W8A8Args<Kind>& a, unsigned blocks, hipStream_t st) {
  if (c.bn == 256) w8a8_launch_stages<Kind, OT, LAYOUT, kMaxP, BM, 256>(c, a, blocks, st);
  else if (c.bn == 128) w8a8_launch_stages<Kind, OT, LAYOUT, kMaxP, BM, 128>(c, a, blocks, st);
  else w8a8_launch_stages<Kind, OT, LAYOUT, kMaxP, BM, 64>(c, a, blocks, st);
}

template <typename Kind, typename OT, int LAYOUT, int BM, int BN>
void w8a8_launch8_p(const W8A8PipeCfg& c, const W8A8Args<Kind>& a, unsigned blocks, hipStream_t st) {
#define QTTS_W8P8(P, PF)                                                                                             \
  do {                                                                                                               \
    if constexpr (P * w8a8_stage_bytes(BM, BN) + 64 <= kLdsBytes)                                                    \
      qtts::launch(&w8a8_pipe_kernel<Kind, OT, BM, BN, P, LAYOUT, PF, 8>, dim3(blocks), dim3(512), 0, st, a.qx, a.sx, \
                   (int)a.m, (int)a.k, a.ldqx, a.qw, (int)a.n, a.ldqw, a.sw, (const OT*)a.bias, (OT*)a.y, a.ldy,      \
                   a.part, a.counters, c.mtiles, c.ntiles, c.S, c.cps);                                              \
  } while (0)
  if (c.P == 3) {
    if (c.pf) QTTS_W8P8(3, true);
    else QTTS_W8P8(3, false);
  } else {
    if (c.pf) QTTS_W8P8(4, true);
    else QTTS_W8P8(4, false);
  }
#undef QTTS_W8P8
}

// Eight waves (two a SIMD), each owning BN / 8 columns of all BM rows.
template <typename Kind, typename OT, int LAYOUT>
void w8a8_launch8(const W8A8PipeCfg& c, const W8A8Args<Kind>& a, unsigned blocks, hipStream_t st) {
  if (c.bm == 64 && c.bn == 128) w8a8_launch8_p<Kind, OT, LAYOUT, 64, 128>(c, a, blocks, st);
  else if (c.bm == 64) w8a8_launch8_p<Kind, OT, LAYOUT, 64, 256>(c, a, blocks, st);
  else if (c.bn == 128) w8a8_launch8_p<Kind, OT, LAYOUT, 128, 128>(c, a, blocks, st);
  else w8a8_launch8_p<Kind, OT, LAYOUT, 128, 256>(c, a, blocks, st);
}

template <typename Kind, typename OT, int LAYOUT, int kMaxP>
void w8a8_launch_bm(const W8A8PipeCfg& c, const W8A8Args<Kind>& a, unsigned blocks, hipStream_t st) {
  if (c.nw == 8) w8a8_launch8<Kind, OT, LAYOUT>(c, a, blocks, st);
  else if (c.bm == 32) w8a8_launch_bn<Kind, OT, LAYOUT, kMaxP, 32>(c, a, blocks, st);
  else if (c.bm == 64) w8a8_launch_bn<Kind, OT, LAYOUT, kMaxP, 64>(c, a, blocks, st);
  else w8a8_launch_bn<Kind, OT, LAYOUT, kMaxP, 128>(c, a, blocks, st);
}

// Validates the request, falls back to one split when the workspace is too small for
// an automatic split count, and launches.  Returns a qtts_status.
template <typename Kind, int LAYOUT, int kMaxP>
int w8a8_pipe_launch(const char* what, W8A8Args<Kind> a, int out_dtype, int splits, int stages, int shape, void* ws,
                     int64_t ws_bytes, hipStream_t st) {
  if (!w8a8_shape_ok(shape)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: bad tile shape code %d", what, shape);
  if (stages < 0 || (stages >> 7) != 0)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: bad stages code %d", what, stages);
  W8A8PipeCfg c = w8a8_cfg(a.m, a.n, a.k, splits, stages, shape);
  if (c.pf && c.P < 3) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: read-ahead needs 3 stages", what);
  if (!w8a8_p_ok(c.bm, c.bn, c.P, c.nw) || c.P > kMaxP)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: %d stages are not built for a %dx%d tile", what, c.P, c.bm,
                          c.bn);
  const int64_t need = w8a8_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "%s with %d splits needs %lld workspace bytes, got %lld", what, c.S,
                            (long long)need, (long long)ws_bytes);
    c = w8a8_cfg(a.m, a.n, a.k, 1, stages, shape);
  }
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  const int64_t blocks = (tiles + 7) / 8 * 8 * c.S;
  if (blocks <= 0 || blocks >= ((int64_t)1 << 31))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "%s: problem too large", what);
  a.counters = (unsigned*)ws;
  a.part = ws ? (typename Kind::part_t*)((char*)ws + kCounterBytes) : nullptr;
  if (out_dtype == QTTS_BF16) w8a8_launch_bm<Kind, bf16_t, LAYOUT, kMaxP>(c, a, (unsigned)blocks, st);
  else if (out_dtype == QTTS_F16) w8a8_launch_bm<Kind, f16_t, LAYOUT, kMaxP>(c, a, (unsigned)blocks, st);
  else w8a8_launch_bm<Kind, float, LAYOUT, kMaxP>(c, a, (unsigned)blocks, st);
  return qtts_check_launch(what);
}

}  // namespace qtts
