// fp8 (OCP e4m3) W8A8 GEMM for gfx950: y = ((qx*sx) @ (qw*sw)^T) [+ bias].
//
// Replaces torch._scaled_mm with rowwise scales and the bias add after it
// (qtts/quant/fp8.py:79-89).  Both operands are already e4m3, so the weight bytes go
// straight from HBM into v_mfma_scale_f32_16x16x128_f8f6f4 (unit block scales)
// with no conversion at all:
//
//  * skinny (M <= 16): a wave owns a 16-row strip of qw; per 128-byte chunk of K a
//    lane loads 32 weight bytes (two 128-bit loads) and the matching 32 activation
//    bytes, and issues one MFMA.  Waves split K and meet in LDS; workgroups may
//    split K further and meet through the workspace (last arrival reduces).
//  * tile (M > 16): LDS-tiled, BM x 128 x 128, 4 waves in 2x2, double-buffered.
//  * generic: any alignment / K; correctness path.
//
// Weights come row-major [N, K] or in the strip layout of layout.h (128-byte
// chunks: each lane's 32 bytes are two 1 KiB-contiguous wave loads).
//
// Epilogue order follows the reference: the fp32 accumulator is scaled by
// sx[m] * sw[n] and rounded to the output dtype, then the bias is added in the
// output dtype (fp8.py:79-89 add the bias after _scaled_mm returns).
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "layout.h"
#include "skinny.h"
#include "splitk.h"

namespace qtts {

template <typename OT>
__device__ __forceinline__ void fp8_store(OT* __restrict__ y, int64_t ldy, int m, int n, float acc,
                                          const float* __restrict__ sx, const float* __restrict__ sw,
                                          const OT* __restrict__ bias) {
  float v = round_through<OT>(acc * sx[m] * sw[n]);
  if (bias) v += to_f32(bias[n]);
  y[(int64_t)m * ldy + n] = from_f32<OT>(v);
}

// e4m3 decode for the generic path (OCP E4M3: bias 7, subnormal step 2^-9).
__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  const uint32_t e = (c >> 3) & 15u, mnt = c & 7u;
  float v;
  if (e == 15u && mnt == 7u) v = __builtin_nanf("");
  else if (e == 0u) v = (float)mnt * (1.0f / 512.0f);
  else v = __uint_as_float(((e + 120u) << 23) | (mnt << 20));
  return (c & 0x80u) ? -v : v;
}

// ------------------------------------------------------------------------------------

// SUB = 2 (half strips, strip weights, M <= 8, K % 256 == 0, no split): two workgroups
// share each 16-row strip, 8 weight rows each.  One MFMA covers a unit of two chunks:
// A rows 0-7 hold chunk 2u and rows 8-15 chunk 2u + 1 of the workgroup's 8 rows, B
// columns 0-7 the activation rows for chunk 2u and 8-15 the same rows for chunk 2u + 1,
// so D's diagonal 8 x 8 blocks are the two chunks' contributions, added at the end.
template <typename OT, int WAVES, int U, int LAYOUT, int SUB = 1, bool NT = false>
__global__ __launch_bounds__(WAVES * 64) void fp8_skinny_kernel(
    const uint8_t* __restrict__ qx, const float* sx, int M, int K, int64_t ldqx,
    const uint8_t* __restrict__ qw, int N, int64_t ldqw, const float* sw, const OT* bias,
    OT* __restrict__ y, int64_t ldy, float* __restrict__ part, unsigned* __restrict__ counters, int strips, int S,
    int cps) {
  static_assert(SUB == 1 || (SUB == 2 && LAYOUT == kLayoutStrips), "half strips need strip weights");
  constexpr int RP = 16 / SUB;  // weight rows per workgroup
  __shared__ f32x4_t red[WAVES > 1 ? WAVES - 1 : 1][64];
  int strip, split;
  if constexpr (SUB == 1) {
    decode_wg(blockIdx.x, S, strip, split);
  } else {  // no split: the host launches half strips with S == 1
    strip = blockIdx.x / SUB;
    split = 0;
  }
  const int part_row = SUB == 1 ? 0 : (blockIdx.x % SUB) * RP;  // this workgroup's first strip row
  if (strip >= strips) return;

  // wave index through readfirstlane: provably uniform, so per-wave bounds stay scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int n = strip * 16 + r;
  const bool n_ok = n < N, m_ok = r < M;
  const int xrow = SUB == 1 ? r : r % RP;  // the activation row lane r loads (B column r)
  const bool x_ok = xrow < M;
  const int nchunks = (K + 127) >> 7;
  // units of SUB chunks (SUB divides nchunks, checked by the host)
  const int c0 = split * cps, c1 = min(c0 + cps, SUB == 1 ? nchunks : nchunks / SUB);
  const int cw = (c1 - c0 + WAVES - 1) / WAVES;
  const int wc0 = c0 + wave * cw, wc1 = min(wc0 + cw, c1);
  const uint8_t* wp;
  int64_t wstride, whalf;
  if constexpr (LAYOUT == kLayoutStrips && SUB > 1) {
    // lane (r, g): strip row part_row + r % RP of chunk r / RP of each unit
    wp = qw + (int64_t)strip * nchunks * 2048 + (r / RP) * 2048 + (part_row + r % RP + 16 * g) * 16;
    wstride = SUB * 2048;
    whalf = 1024;
  } else if constexpr (LAYOUT == kLayoutStrips) {
    wp = qw + (int64_t)strip * nchunks * 2048 + lane * 16;
    wstride = 2048;
    whalf = 1024;
  } else {
    wp = qw + (int64_t)(n_ok ? n : 0) * ldqw + 32 * g;
    wstride = 128;
    whalf = 16;
  }
  const uint8_t* xp = qx + (int64_t)(x_ok ? xrow : 0) * ldqx + (SUB == 1 ? 0 : (r / RP) * 128) + 32 * g;
  const int64_t xstride = SUB * 128;
  const i32x4_t zero = {0, 0, 0, 0};

  // A group of U chunks is issued in full before any of it is consumed.
  i32x4_t w0[U], w1[U], x0[U], x1[U];
  auto issue = [&](int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + u;
      const bool live = cc < wc1;
      const bool ok = live && (SUB > 1 || cc * 128 + 32 * g < K);  // half strips: K % 256 == 0
      const bool wok = LAYOUT == kLayoutStrips ? live : (ok && n_ok);
      w0[u] = wok ? load_weight<NT>(wp + (int64_t)cc * wstride) : zero;
      w1[u] = wok ? load_weight<NT>(wp + (int64_t)cc * wstride + whalf) : zero;
      x0[u] = (ok && x_ok) ? *(const i32x4_t*)(xp + (int64_t)cc * xstride) : zero;
      x1[u] = (ok && x_ok) ? *(const i32x4_t*)(xp + (int64_t)cc * xstride + 16) : zero;
    }
  };
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto consume = [&](int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c + u < wc1) {
        const i32x8_t a = {w0[u][0], w0[u][1], w0[u][2], w0[u][3], w1[u][0], w1[u][1], w1[u][2], w1[u][3]};
        const i32x8_t b = {x0[u][0], x0[u][1], x0[u][2], x0[u][3], x1[u][0], x1[u][1], x1[u][2], x1[u][3]};
        acc = mma_fp8_16x16x128(a, b, acc);
      }
    }
  };
  // Epilogue operands as raw bits, loaded unconditionally (see w8a16.hip).
  uint32_t sxv, swv[4], bi[4];
  auto issue_epilogue = [&]() {
    sxv = *(const uint32_t*)(sx + min(r, M - 1));
    const OT* bsrc = bias ? bias : y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nn = min(strip * 16 + part_row + 4 * g + i, N - 1);
      swv[i] = *(const uint32_t*)(sw + nn);
      if constexpr (sizeof(OT) == 2) bi[i] = *(const uint16_t*)(bsrc + nn);
      else bi[i] = *(const uint32_t*)(bsrc + nn);
    }
  };
  if (wc1 - wc0 <= U) {
    issue(wc0);
    issue_epilogue();
    __builtin_amdgcn_sched_barrier(0);  // every load in flight before the first wait
    consume(wc0);
  } else {
    for (int c = wc0; c < wc1; c += U) {
      issue(c);
      consume(c);
    }
    issue_epilogue();
  }

  if (WAVES > 1) {
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < WAVES - 1; ++w) acc += red[w][lane];
  }

  if constexpr (SUB == 2) {
    // D rows 8 + i, columns 8 + j (the odd chunk of each unit) onto rows i, columns j: lane
    // (j, g) for g < 2 takes lane (j + 8, g + 2), i.e. lane ^ 40
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += __shfl_xor(acc[i], 40, 64);
  }

  if (SUB == 1 && S > 1) {
    float a[4] = {acc[0], acc[1], acc[2], acc[3]};
    if (!splitk_meet<4>(a, part + (int64_t)strip * S * 64 * 4, &counters[strip], S, split, lane, 64, nullptr))
      return;
    acc = f32x4_t{a[0], a[1], a[2], a[3]};
  }

  if (m_ok && (SUB == 1 || r < RP)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nn = strip * 16 + part_row + 4 * g + i;
      if ((SUB == 1 || 4 * g < RP) && nn < N) {
        float v = round_through<OT>(acc[i] * __uint_as_float(sxv) * __uint_as_float(swv[i]));
        if (bias) {
          if constexpr (sizeof(OT) == 2) v += to_f32(OT{(uint16_t)bi[i]});
          else v += __uint_as_float(bi[i]);
        }
        y[(int64_t)r * ldy + nn] = from_f32<OT>(v);
      }
    }
  }
}

// ------------------------------------------------------------------------------------

constexpr int kF8BN = 128, kF8BK = 128, kF8LdsK = kF8BK + 16;  // bytes

template <typename OT, int BM, int LAYOUT>
__global__ __launch_bounds__(256) void fp8_tile_kernel(
    const uint8_t* __restrict__ qx, const float* __restrict__ sx, int M, int K, int64_t ldqx,
    const uint8_t* __restrict__ qw, int N, int64_t ldqw, const float* __restrict__ sw, const OT* __restrict__ bias,
    OT* __restrict__ y, int64_t ldy, float* __restrict__ part, unsigned* __restrict__ counters, int mtiles,
    int ntiles, int S, int cps) {
  constexpr int BN = kF8BN, BK = kF8BK, LK = kF8LdsK;
  constexpr int TM = BM / 32, TN = 4;
  constexpr int XL = BM * 8 / 256;  // 16-byte x chunks per thread per stage
  constexpr int WL = BN * 8 / 256;  // 16-byte w chunks per thread per stage
  __shared__ __align__(16) uint8_t As[2][BM][LK];
  __shared__ __align__(16) uint8_t Bs[2][BN][LK];
  __shared__ unsigned flag;

  int tile, split;
  decode_wg(blockIdx.x, S, tile, split);
  if (tile >= mtiles * ntiles) return;
  const int strips = (N + 15) / 16;
  const int mt = tile % mtiles, nt = tile / mtiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int c16 = lane & 15, g = lane >> 4;
  const int nchunks = (K + BK - 1) / BK;
  const int k0c = split * cps, k1c = min(k0c + cps, nchunks);
  const i32x4_t zero = {0, 0, 0, 0};

  i32x4_t xr[XL], wr[WL];
  auto load_stage = [&](int kc) {
#pragma unroll
    for (int l = 0; l < XL; ++l) {
      const int id = tid + 256 * l, row = id >> 3, col = (id & 7) * 16;
      const int m = m0 + row, k = kc * BK + col;
      xr[l] = (m < M && k < K) ? *(const i32x4_t*)(qx + (int64_t)m * ldqx + k) : zero;
    }
#pragma unroll
    for (int l = 0; l < WL; ++l) {
      const int id = tid + 256 * l;
      if constexpr (LAYOUT == kLayoutStrips) {
        // 8 strips x one chunk = 8 blocks of 2 KiB; unit (id & 127) of block id / 128
        const int s = n0 / 16 + (id >> 7);
        wr[l] = s < strips ? *(const i32x4_t*)(qw + ((int64_t)s * nchunks + kc) * 2048 + (id & 127) * 16) : zero;
      } else {
        const int row = id >> 3, col = (id & 7) * 16;
        const int n = n0 + row, k = kc * BK + col;
        wr[l] = (n < N && k < K) ? *(const i32x4_t*)(qw + (int64_t)n * ldqw + k) : zero;
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int l = 0; l < XL; ++l) {
      const int id = tid + 256 * l;
      *(i32x4_t*)&As[buf][id >> 3][(id & 7) * 16] = xr[l];
    }
#pragma unroll
    for (int l = 0; l < WL; ++l) {
      const int id = tid + 256 * l;
      if constexpr (LAYOUT == kLayoutStrips) {
        const int slot = id & 63, h = (id >> 6) & 1;
        *(i32x4_t*)&Bs[buf][(id >> 7) * 16 + (slot & 15)][(slot >> 4) * 32 + h * 16] = wr[l];
      } else {
        *(i32x4_t*)&Bs[buf][id >> 3][(id & 7) * 16] = wr[l];
      }
    }
  };

  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  if (k0c < k1c) {
    load_stage(k0c);
    store_stage(0);
  }
  __syncthreads();
  for (int kc = k0c; kc < k1c; ++kc) {
    const int buf = (kc - k0c) & 1;
    if (kc + 1 < k1c) load_stage(kc + 1);
    i32x8_t a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const uint8_t* p = &As[buf][wm * (BM / 2) + i * 16 + c16][g * 32];
      const i32x4_t lo = *(const i32x4_t*)p, hi = *(const i32x4_t*)(p + 16);
      a[i] = i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint8_t* p = &Bs[buf][wn * 64 + j * 16 + c16][g * 32];
      const i32x4_t lo = *(const i32x4_t*)p, hi = *(const i32x4_t*)(p + 16);
      b[j] = i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mma_fp8_16x16x128(a[i], b[j], acc[i][j]);
    if (kc + 1 < k1c) store_stage(buf ^ 1);
    __syncthreads();
  }

  if (S > 1) {
    constexpr int NV = TM * TN * 4;
    float a[NV];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) a[(i * TN + j) * 4 + t] = acc[i][j][t];
    if (!splitk_meet<NV>(a, part + (int64_t)tile * S * 256 * NV, &counters[tile], S, split, tid, 256, &flag))
      return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[i][j][t] = a[(i * TN + j) * 4 + t];
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * 64 + j * 16 + c16;
      if (n >= N) continue;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = m0 + wm * (BM / 2) + i * 16 + 4 * g + t;
        if (m < M) fp8_store(y, ldy, m, n, acc[i][j][t], sx, sw, bias);
      }
    }
}

// ------------------------------------------------------------------------------------

template <typename OT>
__global__ __launch_bounds__(64) void fp8_generic_kernel(
    const uint8_t* __restrict__ qx, const float* __restrict__ sx, int M, int K, int64_t ldqx,
    const uint8_t* __restrict__ qw, int N, int64_t ldqw, const float* __restrict__ sw, const OT* __restrict__ bias,
    OT* __restrict__ y, int64_t ldy) {
  const int n = blockIdx.x, m0 = blockIdx.y * 4, lane = threadIdx.x;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k = lane; k < K; k += 64) {
    const float w = e4m3_decode(qw[(int64_t)n * ldqw + k]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (m0 + i < M) acc[i] += e4m3_decode(qx[(int64_t)(m0 + i) * ldqx + k]) * w;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float s = wave_sum(acc[i]);
    if (lane == 0 && m0 + i < M) fp8_store(y, ldy, m0 + i, n, s, sx, sw, bias);
  }
}

}  // namespace qtts

using namespace qtts;

namespace {

struct F8Cfg { int family, waves, S, cps, strips, bm, mtiles, ntiles; };

constexpr int kF8CPW = 4;  // 128-byte chunks a wave keeps in flight at once

F8Cfg fp8_cfg(int64_t m, int64_t n, int64_t k, int algo) {
  F8Cfg c{};
  c.family = algo & 0xff;
  const int splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  if (c.family == QTTS_ALGO_AUTO) c.family = m <= 16 ? QTTS_ALGO_SKINNY : QTTS_ALGO_TILE;
  if (c.family == QTTS_ALGO_SKINNY) {
    c.strips = (int)((n + 15) / 16);
    const int nchunks = std::max(1, (int)((k + 127) / 128));
    int W = waves, S = splits;
    if (W <= 0) {
      W = 1;
      while (W < 16 && ((nchunks + W - 1) / W > kF8CPW || (int64_t)c.strips * W < 2048)) W *= 2;
    }
    if (S <= 0) {
      S = 1;
      while ((nchunks + S * W - 1) / (S * W) > kF8CPW) S *= 2;
    }
    c.waves = W;
    S = std::max(1, std::min(S, nchunks));
    if (c.strips > kMaxSplitTiles) S = 1;
    c.cps = (nchunks + S - 1) / S;
    c.S = (nchunks + c.cps - 1) / c.cps;
  } else {
    c.bm = m <= 32 ? 32 : (m <= 64 ? 64 : 128);
    c.mtiles = (int)((m + c.bm - 1) / c.bm);
    c.ntiles = (int)((n + kF8BN - 1) / kF8BN);
    const int nchunks = std::max(1, (int)((k + kF8BK - 1) / kF8BK));
    int S = splits;
    if (S <= 0) {
      S = 1;
      while (c.mtiles * c.ntiles * S * 2 <= 512 && nchunks / (S * 2) >= 4) S *= 2;
    }
    S = std::max(1, std::min(S, nchunks));
    if ((int64_t)c.mtiles * c.ntiles > kMaxSplitTiles) S = 1;
    c.cps = (nchunks + S - 1) / S;
    c.S = (nchunks + c.cps - 1) / c.cps;
  }
  return c;
}

int64_t fp8_cfg_ws(const F8Cfg& c) {
  if (c.S <= 1) return 0;
  if (c.family == QTTS_ALGO_SKINNY) return kCounterBytes + (int64_t)c.strips * c.S * 64 * 16;
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  return kCounterBytes + tiles * c.S * 256 * (c.bm / 32) * 4 * 4 * 4;
}

}  // namespace

int64_t qtts_fp8_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int shape);
int qtts_launch_fp8_pipe(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qs,
                         int64_t n, const float* sw, const void* bias, void* y, int out_dtype, int64_t ldy, int splits,
                         int stages, int shape, void* ws, int64_t ws_bytes, hipStream_t st);

int64_t qtts_fp8_gemm_ws_bytes(int64_t m, int64_t n, int64_t k, int algo) {
  int64_t a;
  if ((algo & 0xff) == QTTS_ALGO_AUTO) {
    const int rest = algo & ~0xff;
    a = fp8_cfg_ws(fp8_cfg(std::min<int64_t>(m, 16), n, k, rest | QTTS_ALGO_SKINNY));
    if (m > 16) a = std::max(a, fp8_cfg_ws(fp8_cfg(m, n, k, rest | QTTS_ALGO_TILE)));
  } else {
    a = fp8_cfg_ws(fp8_cfg(m, n, k, algo));
  }
  const int family = algo & 0xff;
  if (k % 128 == 0 && (family == QTTS_ALGO_TILE || (family == QTTS_ALGO_AUTO && m > 16)))
    a = std::max(a, qtts_fp8_pipe_ws_bytes(m, n, k, (algo >> 8) & 0xff, (algo >> 24) & 0xff));
  return a;
}

template <typename OT, int LAYOUT>
static int fp8_launch_fast(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qw,
                           int64_t n, int64_t ldqw, const float* sw, const OT* bias, OT* y, int64_t ldy, int algo,
                           void* ws, int64_t ws_bytes, hipStream_t st) {
  F8Cfg c = fp8_cfg(m, n, k, algo);
  if (c.family == QTTS_ALGO_SKINNY && m > 16)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "skinny fp8 kernel handles M <= 16, got M=%lld", (long long)m);
  if (LAYOUT == kLayoutStrips && c.family == QTTS_ALGO_TILE && k % 128 == 0) {
    constexpr int odt = std::is_same<OT, bf16_t>::value ? QTTS_BF16 : (std::is_same<OT, f16_t>::value ? QTTS_F16 : QTTS_F32);
    return qtts_launch_fp8_pipe(qx, sx, m, k, ldqx, qw, n, sw, bias, y, odt, ldy, (algo >> 8) & 0xff,
                                (algo >> 16) & 0xff, (algo >> 24) & 0xff, ws, ws_bytes, st);
  }
  const int64_t need = fp8_cfg_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if ((algo >> 8) & 0xff)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a8 fp8 GEMM needs %lld workspace bytes, got %lld", (long long)need,
                            (long long)ws_bytes);
    c = fp8_cfg(m, n, k, c.family | (1 << 8) | (algo & 0xff0000));
  }
  unsigned* counters = (unsigned*)ws;
  float* part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
  // Half strips for decode rows where whole strips leave compute units idle (skinny.h's
  // rule: the talker's down_proj from M = 4, below which the fused linear runs);
  // automatic choice only.  Units of two 128-column chunks, so K % 256 == 0.
  if (LAYOUT == kLayoutStrips && c.family == QTTS_ALGO_SKINNY && algo == QTTS_ALGO_AUTO && m <= 8 &&
      k % 256 == 0 && skinny_auto_sub(m, n, k) == 2) {
    const int strips = (int)((n + 15) / 16), units = (int)(k / 256);
    int W = 1;
    while (W < 16 && ((units + W - 1) / W > kF8CPW || (int64_t)strips * 2 * W < 2048)) W *= 2;
    const int64_t blocks = ((int64_t)strips * 2 + 7) / 8 * 8;
    if ((units + W - 1) / W <= kF8CPW && blocks < ((int64_t)1 << 31)) {
#define QTTS_F8H(WV)                                                                                            \
  qtts::launch_by_policy<std::is_same<OT, bf16_t>::value>([&](auto nt) {                                        \
    qtts::launch(&fp8_skinny_kernel<OT, WV, kF8CPW, kLayoutStrips, 2, decltype(nt)::value>, dim3((unsigned)blocks), \
                 dim3(WV * 64), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, bias, y, ldy,          \
                 (float*)nullptr, (unsigned*)nullptr, strips, 1, units);                                           \
  })
      switch (W) {
        case 1: QTTS_F8H(1); break;
        case 2: QTTS_F8H(2); break;
        case 4: QTTS_F8H(4); break;
        case 8: QTTS_F8H(8); break;
        default: QTTS_F8H(16); break;
      }
#undef QTTS_F8H
      return qtts_check_launch("w8a8_fp8_skinny_half");
    }
  }
  if (c.family == QTTS_ALGO_SKINNY) {
    const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8 * c.S;
#define QTTS_F8S(W, U)                                                                                          \
  qtts::launch_by_policy<std::is_same<OT, bf16_t>::value && LAYOUT == kLayoutStrips>([&](auto nt) {             \
    qtts::launch(&fp8_skinny_kernel<OT, W, U, LAYOUT, 1, decltype(nt)::value>, dim3((unsigned)blocks),          \
                 dim3(W * 64), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, bias, y, ldy, part,    \
                 counters, c.strips, c.S, c.cps);                                                               \
  })
    switch (c.waves) {
      case 1: QTTS_F8S(1, kF8CPW); break;
      case 2: QTTS_F8S(2, kF8CPW); break;
      case 4: QTTS_F8S(4, kF8CPW); break;
      case 8: QTTS_F8S(8, kF8CPW); break;
      case 16: QTTS_F8S(16, kF8CPW); break;
      default: return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8 skinny: waves must be 1, 2, 4, 8 or 16");
    }
#undef QTTS_F8S
    return qtts_check_launch("w8a8_fp8_skinny");
  }
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  const int64_t blocks = (tiles + 7) / 8 * 8 * c.S;
#define QTTS_F8T(BM)                                                                                           \
  qtts::launch(&fp8_tile_kernel<OT, BM, LAYOUT>, dim3((unsigned)blocks), dim3(256), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, \
                                                                    bias, y, ldy, part, counters, c.mtiles, c.ntiles,  \
                                                                    c.S, c.cps)
  if (c.bm == 32) QTTS_F8T(32);
  else if (c.bm == 64) QTTS_F8T(64);
  else QTTS_F8T(128);
#undef QTTS_F8T
  return qtts_check_launch("w8a8_fp8_tile");
}

template <typename OT>
static int fp8_launch_typed(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qw,
                            int64_t n, int64_t ldqw, int layout, const float* sw, const OT* bias, OT* y, int64_t ldy,
                            int algo, void* ws, int64_t ws_bytes, hipStream_t st) {
  const bool x_ok = ((uintptr_t)qx % 16 == 0) && (ldqx % 16 == 0) && (k % 32 == 0) && k > 0;
  if (layout == kLayoutStrips) {
    if (!x_ok)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                            "strip-layout fp8 weights need 16-byte aligned activation rows and K %% 32 == 0");
    return fp8_launch_fast<OT, kLayoutStrips>(qx, sx, m, k, ldqx, qw, n, ldqw, sw, bias, y, ldy, algo, ws, ws_bytes,
                                              st);
  }
  if (!x_ok || (uintptr_t)qw % 16 != 0 || ldqw % 16 != 0) {
    dim3 grid((unsigned)n, (unsigned)((m + 3) / 4));
    qtts::launch(&fp8_generic_kernel<OT>, dim3(grid), dim3(64), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, bias, y, ldy);
    return qtts_check_launch("w8a8_fp8_generic");
  }
  return fp8_launch_fast<OT, kLayoutRowMajor>(qx, sx, m, k, ldqx, qw, n, ldqw, sw, bias, y, ldy, algo, ws, ws_bytes,
                                              st);
}

// layout: kLayoutRowMajor (qw [n, k], row stride ldqw) or kLayoutStrips (ldqw ignored).
int qtts_launch_fp8_gemm(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qw,
                         int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias, void* y,
                         int out_dtype, int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (out_dtype == QTTS_BF16)
    return fp8_launch_typed<bf16_t>(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, (const bf16_t*)bias, (bf16_t*)y, ldy,
                                    algo, ws, ws_bytes, st);
  if (out_dtype == QTTS_F16)
    return fp8_launch_typed<f16_t>(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, (const f16_t*)bias, (f16_t*)y, ldy,
                                   algo, ws, ws_bytes, st);
  return fp8_launch_typed<float>(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, (const float*)bias, (float*)y, ldy, algo,
                                 ws, ws_bytes, st);
}
