// fp8 (OCP e4m3) W8A8 GEMM for prefill-sized rows (M > 16) on strip-layout weights,
// gfx950: y = round(acc * sx[m] * sw[n]) [+ bias].
//
// Replaces torch._scaled_mm with rowwise scales and the bias add after it
// (qtts/quant/fp8.py:79-89) for M > 16 when K % 128 == 0.
//
// Same pipeline as the W8A16 tile kernel (tile.hip): 4 waves own a BM x BN tile and
// walk K through a P-deep LDS ring filled by direct global -> LDS loads, one barrier
// per stage.  A stage is 128 K columns, and every load writes one 1 KiB half of an
// MFMA fragment in lane order:
//   * activation half (m-block mb, half h): lane l carries
//     qx[m0 + 16 mb + l % 16][k + 32 (l / 16) + 16 h .. + 15];
//   * weight half (strip sb, half h): half h of the strip layout's 2 KiB block, lane l
//     carries w[n0 + 16 sb + l % 16][k + 32 (l / 16) + 16 h .. + 15].
// A lane's two halves are its 32-byte operand of one v_mfma_scale_f32_16x16x128_f8f6f4
// (unit block scales), so the e4m3 bytes go from LDS to the matrix core with no
// conversion.  Wave w owns columns [n0 + w BN/4, n0 + (w+1) BN/4) for all BM rows.
//
// Epilogue order follows the reference: the fp32 accumulator times sx[m] * sw[n] is
// rounded to the output dtype, then the bias is added in the output dtype.
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

template <typename OT, int BM, int BN, int P>
__global__ __launch_bounds__(256) void fp8_pipe_kernel(
    const uint8_t* __restrict__ qx, const float* __restrict__ sx, int M, int K, int64_t ldqx,
    const uint8_t* __restrict__ qs, int N, const float* __restrict__ sw, const OT* __restrict__ bias,
    OT* __restrict__ y, int64_t ldy, float* __restrict__ part, unsigned* __restrict__ counters, int mtiles,
    int ntiles, int S, int cps) {
  constexpr int MB = BM / 16;          // 16-row m-blocks per tile
  constexpr int NB = BN / 64;          // 16-column strips per wave
  constexpr int XF = 2 * MB;           // activation halves per stage
  constexpr int WF = 2 * (BN / 16);    // weight halves per stage
  constexpr int F = XF + WF;
  constexpr int FPW = F / 4;           // halves each wave loads per stage
  constexpr int SB = F * 1024;         // stage bytes
  static_assert(F % 4 == 0, "fragments must split evenly over 4 waves");
  static_assert(P >= 2 && P * SB + 64 <= kLdsBytes, "stage ring must fit in LDS");
  static_assert((P - 2) * FPW < 64, "vmcnt is 6 bits");
  __shared__ __align__(1024) uint8_t ring[P * SB];
  __shared__ unsigned flag;

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
      src[j] = qx + (int64_t)m * ldqx + (int64_t)kc0 * 128 + 32 * g + 16 * h;
      stride[j] = 128;
    } else {
      const int sb = (f - XF) >> 1, h = (f - XF) & 1;
      const int s = min(n0 / 16 + sb, strips - 1);
      src[j] = qs + ((int64_t)s * nchunks + kc0) * 2048 + h * 1024 + lane * 16;
      stride[j] = 2048;
    }
  }

  auto issue = [&](uint8_t* stage, int i) {
#pragma unroll
    for (int j = 0; j < FPW; ++j) load_to_lds16(src[j] + (int64_t)i * stride[j], stage + (wave * FPW + j) * 1024);
  };

  f32x4_t acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const uint8_t* stage) {
    i32x8_t xa[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      xa[mb] = concat8(*(const i32x4_t*)(stage + (2 * mb) * 1024 + lane * 16),
                       *(const i32x4_t*)(stage + (2 * mb + 1) * 1024 + lane * 16));
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint8_t* wsrc = stage + (XF + 2 * (wave * NB + nb)) * 1024 + lane * 16;
      const i32x8_t wf = concat8(*(const i32x4_t*)wsrc, *(const i32x4_t*)(wsrc + 1024));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mma_fp8_16x16x128(wf, xa[mb], acc[nb][mb]);
    }
  };

  for (int p = 0; p < P - 1; ++p)
    if (p < nk) issue(ring + p * SB, p);
  int cur = 0, nxt = P - 1;
  for (int i = 0; i < nk; ++i) {
    wait_stages<FPW, P - 2>(nk - 1 - i);
    barrier_only();
    if (i + P - 1 < nk) issue(ring + nxt * SB, i + P - 1);
    compute(ring + cur * SB);
    cur = cur + 1 == P ? 0 : cur + 1;
    nxt = nxt + 1 == P ? 0 : nxt + 1;
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
    if (!splitk_meet<NV>(a, part + (int64_t)tile * S * 256 * NV, &counters[tile], S, split, tid, 256, &flag))
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
      for (int t = 0; t < 4; ++t) {
        v[t] = round_through<OT>(acc[nb][mb][t] * sxv * swv[t]);
        if (bias) v[t] += biv[t];
      }
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

}  // namespace qtts

using namespace qtts;

namespace {

struct F8PipeCfg { int bm, bn, P, S, cps, mtiles, ntiles; };

constexpr int f8_stage_bytes(int bm, int bn) { return (bm / 8 + bn / 8) * 1024; }

bool f8_p_ok(int bm, int bn, int p) {
  if (p != 2 && p != 3 && p != 4 && p != 6 && p != 8) return false;
  const int fpw = (bm / 8 + bn / 8) / 4;
  return p * f8_stage_bytes(bm, bn) + 64 <= kLdsBytes && (p - 2) * fpw < 64;
}

// The W8A16 tile kernel's measured choice (tile.hip), with 128-column chunks: 32 x 64
// tiles and 4 stages up to M = 128, 64 x 128 and 3 stages above; split K until there
// are 256 workgroups, keeping >= 4 chunks a split.  shape_req as for that kernel.
F8PipeCfg f8_cfg(int64_t m, int64_t n, int64_t k, int splits_req, int stages_req, int shape_req) {
  F8PipeCfg c;
  const int nchunks = std::max(1, (int)(k / 128));
  if (shape_req != 0) {
    c.bm = 16 << (shape_req & 15);
    c.bn = 32 << ((shape_req >> 4) & 7);
  } else if (m <= 128) {
    c.bm = 32;
    c.bn = 64;
  } else {
    c.bm = 64;
    c.bn = 128;
  }
  c.mtiles = (int)((m + c.bm - 1) / c.bm);
  c.ntiles = (int)((n + c.bn - 1) / c.bn);
  c.P = stages_req > 0 ? stages_req : (c.bm * c.bn <= 32 * 64 ? 4 : 3);
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  int S = splits_req;
  if (S <= 0) {
    S = 1;
    while (tiles * S < 256 && nchunks / (S * 2) >= 4) S *= 2;
  }
  S = std::max(1, std::min(S, nchunks));
  if (tiles > kMaxSplitTiles) S = 1;
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  return c;
}

int64_t f8_ws(const F8PipeCfg& c) {
  if (c.S <= 1) return 0;
  const int64_t nv = (int64_t)(c.bn / 64) * (c.bm / 16) * 4;
  return kCounterBytes + (int64_t)c.mtiles * c.ntiles * c.S * 256 * nv * 4;
}

bool f8_shape_ok(int shape) {
  if (shape == 0) return true;
  const int b = shape & 15, c = (shape >> 4) & 7;
  return (shape >> 7) == 0 && b >= 1 && b <= 3 && c >= 1 && c <= 3;
}

struct F8Args {
  const uint8_t* qx; const float* sx; int64_t m, k, ldqx; const uint8_t* qs; int64_t n; const float* sw;
  const void* bias; void* y; int64_t ldy; float* part; unsigned* counters;
};

template <typename OT, int BM, int BN, int P>
void f8_launch_p(const F8PipeCfg& c, const F8Args& a, unsigned blocks, hipStream_t st) {
  if constexpr (P * f8_stage_bytes(BM, BN) + 64 <= kLdsBytes) {
    qtts::launch(&fp8_pipe_kernel<OT, BM, BN, P>, dim3(blocks), dim3(256), 0, st, a.qx, a.sx, (int)a.m, (int)a.k,
                 a.ldqx, a.qs, (int)a.n, a.sw, (const OT*)a.bias, (OT*)a.y, a.ldy, a.part, a.counters, c.mtiles,
                 c.ntiles, c.S, c.cps);
  }
}

template <typename OT, int BM, int BN>
void f8_launch_stages(const F8PipeCfg& c, const F8Args& a, unsigned blocks, hipStream_t st) {
  switch (c.P) {
    case 2: f8_launch_p<OT, BM, BN, 2>(c, a, blocks, st); break;
    case 3: f8_launch_p<OT, BM, BN, 3>(c, a, blocks, st); break;
    case 4: f8_launch_p<OT, BM, BN, 4>(c, a, blocks, st); break;
    case 6: f8_launch_p<OT, BM, BN, 6>(c, a, blocks, st); break;
    default: f8_launch_p<OT, BM, BN, 8>(c, a, blocks, st); break;
  }
}

template <typename OT, int BM>
void f8_launch_bn(const F8PipeCfg& c, const F8Args& a, unsigned blocks, hipStream_t st) {
  if (c.bn == 256) f8_launch_stages<OT, BM, 256>(c, a, blocks, st);
  else if (c.bn == 128) f8_launch_stages<OT, BM, 128>(c, a, blocks, st);
  else f8_launch_stages<OT, BM, 64>(c, a, blocks, st);
}

template <typename OT>
void f8_launch_bm(const F8PipeCfg& c, const F8Args& a, unsigned blocks, hipStream_t st) {
  if (c.bm == 32) f8_launch_bn<OT, 32>(c, a, blocks, st);
  else if (c.bm == 64) f8_launch_bn<OT, 64>(c, a, blocks, st);
  else f8_launch_bn<OT, 128>(c, a, blocks, st);
}

}  // namespace

int64_t qtts_fp8_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int shape) {
  if (!f8_shape_ok(shape)) return 0;
  return f8_ws(f8_cfg(m, n, k, splits, 0, shape));
}

// qx [m, k] e4m3 (16-byte aligned rows), qs e4m3 strip layout, k % 128 == 0, m > 0.
int qtts_launch_fp8_pipe(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qs,
                         int64_t n, const float* sw, const void* bias, void* y, int out_dtype, int64_t ldy, int splits,
                         int stages, int shape, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (!f8_shape_ok(shape))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8 tile: bad tile shape code %d", shape);
  F8PipeCfg c = f8_cfg(m, n, k, splits, stages, shape);
  if (!f8_p_ok(c.bm, c.bn, c.P))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8 tile: %d stages are not built for a %dx%d tile", c.P, c.bm,
                          c.bn);
  const int64_t need = f8_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "fp8 tile with %d splits needs %lld workspace bytes, got %lld", c.S,
                            (long long)need, (long long)ws_bytes);
    c = f8_cfg(m, n, k, 1, stages, shape);
  }
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  const int64_t blocks = (tiles + 7) / 8 * 8 * c.S;
  if (blocks <= 0 || blocks >= ((int64_t)1 << 31))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8 tile: problem too large");
  unsigned* counters = (unsigned*)ws;
  float* part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
  const F8Args a{qx, sx, m, k, ldqx, qs, n, sw, bias, y, ldy, part, counters};
  if (out_dtype == QTTS_BF16) f8_launch_bm<bf16_t>(c, a, (unsigned)blocks, st);
  else if (out_dtype == QTTS_F16) f8_launch_bm<f16_t>(c, a, (unsigned)blocks, st);
  else f8_launch_bm<float>(c, a, (unsigned)blocks, st);
  return qtts_check_launch("w8a8_fp8_tile");
}
