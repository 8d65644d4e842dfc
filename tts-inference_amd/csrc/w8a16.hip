// int8 weight-only (W8A16) GEMM for gfx950: y = x @ (q * scale)^T + bias.
//
// Replaces the Triton kernel _w8_gemm_kernel (qtts/quant/kernels.py:89-135) with
// three hand-written kernels.  Weights come either row-major [N, K] (the
// reference's buffer layout) or in the strip layout of layout.h, where every
// wavefront load is one contiguous 1 KiB; the quant methods store the latter.
//
//  * skinny (M <= 16, decode rows): a workgroup owns a 16-row strip of q and a K
//    range; its waves split that range into contiguous runs.  Per 64-column chunk a
//    lane loads 16 weight bytes (one 128-bit load), converts them to bf16 in
//    registers (int8 is exact in bf16) and issues two v_mfma_f32_16x16x32_bf16 with
//    the activations as the 16-column B operand (rows >= M are zero).  A wave
//    issues all loads of its share (up to 8 chunks) before consuming any, and the
//    epilogue's scale and bias are fetched first, so a call costs one memory round
//    trip.  Waves meet in LDS; workgroups that split K further meet through the
//    workspace (splitk.h) with no second launch.
//  * tile (M > 16, prefill rows): LDS-tiled bf16 MFMA GEMM, BM x 128 x 64 tiles,
//    4 waves in 2x2, double-buffered LDS; the weight tile is dequantized to bf16 on
//    its way into LDS.
//  * generic: any dtype (fp32 activations included) and any alignment; one wave per
//    output column, lanes stride K.  Correctness path for odd shapes (row-major only).
//
// Numerics follow the reference kernel: products of the activation and the exact
// int8 weight accumulate in fp32, the fp32 sum is multiplied by f32(scale[n]),
// f32(bias[n]) is added, and the result is rounded once to the activation dtype
// (qtts/quant/kernels.py:113-135).
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "layout.h"
#include "skinny.h"
#include "splitk.h"

namespace qtts {

__device__ __forceinline__ float load_scale(const void* s, int dt, int n) {
  if (dt == QTTS_BF16) return to_f32(((const bf16_t*)s)[n]);
  if (dt == QTTS_F16) return to_f32(((const f16_t*)s)[n]);
  return ((const float*)s)[n];
}

template <typename XT>
__device__ __forceinline__ void store_out(XT* __restrict__ y, int64_t ldy, int m, int n, float acc, const void* scale,
                                          int scale_dt, const XT* __restrict__ bias) {
  float v = acc * load_scale(scale, scale_dt, n);
  if (bias) v += to_f32(bias[n]);
  y[(int64_t)m * ldy + n] = from_f32<XT>(v);
}

// ------------------------------------------------------------------------------------
// tile: M > 16
// ------------------------------------------------------------------------------------

constexpr int kTileBN = 128, kTileBK = 64, kTileLdsK = kTileBK + 8;  // padded LDS row, in elements

template <typename XT, int BM, int LAYOUT>
__global__ __launch_bounds__(256) void w8a16_tile_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ q, int N, int64_t ldq,
    const void* __restrict__ scale, int scale_dt, const XT* __restrict__ bias, XT* __restrict__ y, int64_t ldy,
    float* __restrict__ part, unsigned* __restrict__ counters, int mtiles, int ntiles, int S, int cps) {
  typedef mfma16<XT> MM;
  typedef typename MM::vec V;
  constexpr int BN = kTileBN, BK = kTileBK, LK = kTileLdsK;
  constexpr int TM = BM / 32;         // 16-row MFMA tiles per wave along M
  constexpr int TN = 4;               // 16-col MFMA tiles per wave along N
  constexpr int XL = BM * 8 / 256;    // 16-byte x chunks per thread per stage
  __shared__ __align__(16) uint16_t As[2][BM][LK];
  __shared__ __align__(16) uint16_t Bs[2][BN][LK];
  __shared__ unsigned flag;

  int tile, split;
  decode_wg(blockIdx.x, S, tile, split);
  if (tile >= mtiles * ntiles) return;
  const int mt = tile % mtiles, nt = tile / mtiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int c16 = lane & 15, g = lane >> 4;
  const int nchunks = (K + BK - 1) / BK;
  const int strips = (N + 15) / 16;
  const int k0c = split * cps;
  const int k1c = min(k0c + cps, nchunks);
  const i32x4_t zero = {0, 0, 0, 0};

  i32x4_t xr[XL], wr[2];
  auto load_stage = [&](int kc) {
#pragma unroll
    for (int l = 0; l < XL; ++l) {
      const int id = tid + 256 * l, row = id >> 3, col = (id & 7) * 8;
      const int m = m0 + row, k = kc * BK + col;
      xr[l] = (m < M && k < K) ? *(const i32x4_t*)(x + (int64_t)m * ldx + k) : zero;
    }
#pragma unroll
    for (int l = 0; l < 2; ++l) {
      const int id = tid + 256 * l;
      if constexpr (LAYOUT == kLayoutStrips) {
        // 8 strips x one chunk = 8 contiguous 1 KiB blocks; slot (id & 63) of block id / 64
        const int s = n0 / 16 + (id >> 6);
        wr[l] = s < strips ? *(const i32x4_t*)(q + ((int64_t)s * nchunks + kc) * 1024 + (id & 63) * 16) : zero;
      } else {
        const int row = id >> 2, col = (id & 3) * 16;
        const int n = n0 + row, k = kc * BK + col;
        wr[l] = (n < N && k < K) ? *(const i32x4_t*)(q + (int64_t)n * ldq + k) : zero;
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int l = 0; l < XL; ++l) {
      const int id = tid + 256 * l, row = id >> 3, col = (id & 7) * 8;
      *(i32x4_t*)&As[buf][row][col] = xr[l];
    }
#pragma unroll
    for (int l = 0; l < 2; ++l) {
      const int id = tid + 256 * l;
      int row, col;
      if constexpr (LAYOUT == kLayoutStrips) {
        row = (id >> 6) * 16 + (id & 15);
        col = ((id & 63) >> 4) * 16;
      } else {
        row = id >> 2;
        col = (id & 3) * 16;
      }
      const V lo = MM::from_i8((uint32_t)wr[l][0], (uint32_t)wr[l][1]);
      const V hi = MM::from_i8((uint32_t)wr[l][2], (uint32_t)wr[l][3]);
      *(V*)&Bs[buf][row][col] = lo;
      *(V*)&Bs[buf][row][col + 8] = hi;
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
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      V a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const V*)&As[buf][wm * (BM / 2) + i * 16 + c16][s * 32 + g * 8];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const V*)&Bs[buf][wn * 64 + j * 16 + c16][s * 32 + g * 8];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MM::mma(a[i], b[j], acc[i][j]);
    }
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

  // A = activations (rows m), B = weights (columns n): lane (c16, g) holds
  // D[4g + t][c16] of every 16x16 tile.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * 64 + j * 16 + c16;
      if (n >= N) continue;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = m0 + wm * (BM / 2) + i * 16 + 4 * g + t;
        if (m < M) store_out(y, ldy, m, n, acc[i][j][t], scale, scale_dt, bias);
      }
    }
}

// ------------------------------------------------------------------------------------
// generic: any dtype, any alignment, row-major weights
// ------------------------------------------------------------------------------------

constexpr int kGenericRows = 4;

template <typename XT>
__global__ __launch_bounds__(64) void w8a16_generic_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ q, int N, int64_t ldq,
    const void* __restrict__ scale, int scale_dt, const XT* __restrict__ bias, XT* __restrict__ y, int64_t ldy) {
  const int n = blockIdx.x, m0 = blockIdx.y * kGenericRows, lane = threadIdx.x;
  float acc[kGenericRows] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int8_t* qr = q + (int64_t)n * ldq;
  for (int k = lane; k < K; k += 64) {
    const float w = (float)qr[k];
#pragma unroll
    for (int i = 0; i < kGenericRows; ++i)
      if (m0 + i < M) acc[i] += to_f32(x[(int64_t)(m0 + i) * ldx + k]) * w;
  }
#pragma unroll
  for (int i = 0; i < kGenericRows; ++i) {
    const float s = wave_sum(acc[i]);
    if (lane == 0 && m0 + i < M) store_out(y, ldy, m0 + i, n, s, scale, scale_dt, bias);
  }
}

}  // namespace qtts

using namespace qtts;

// ---- host side ------------------------------------------------------------------------

namespace {

struct TileCfg { int bm, S, cps, mtiles, ntiles; };

TileCfg tile_cfg(int64_t m, int64_t n, int64_t k, int splits_req) {
  TileCfg c;
  c.bm = m <= 32 ? 32 : (m <= 64 ? 64 : 128);
  c.mtiles = (int)((m + c.bm - 1) / c.bm);
  c.ntiles = (int)((n + kTileBN - 1) / kTileBN);
  const int nchunks = std::max(1, (int)((k + kTileBK - 1) / kTileBK));
  int S = splits_req;
  if (S <= 0) {
    S = 1;
    const int tiles = c.mtiles * c.ntiles;
    while (tiles * S * 2 <= 512 && nchunks / (S * 2) >= 8) S *= 2;
  }
  S = std::max(1, std::min(S, nchunks));
  if ((int64_t)c.mtiles * c.ntiles > kMaxSplitTiles) S = 1;
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  return c;
}

int64_t tile_ws(const TileCfg& c) {
  if (c.S <= 1) return 0;
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  return kCounterBytes + tiles * c.S * 256 * (c.bm / 32) * 4 * 4 * 4;
}

bool grid_ok(int64_t blocks) { return blocks > 0 && blocks < (int64_t)1 << 31; }

}  // namespace

int64_t qtts_w8a16_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int stages, int shape);
int qtts_launch_w8a16_skinny_xrows(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
                                   int64_t n, const void* scale, int sdt, const void* bias, void* y, int64_t ldy,
                                   int waves, int cpw, float* part, unsigned* counters, int strips, int S, int cps,
                                   unsigned blocks, hipStream_t st);
int qtts_w8a16_xrows_built(int waves, int cpw);
int qtts_launch_w8a16_pipe(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
                           int64_t n, const void* scale, int sdt, const void* bias, void* y, int64_t ldy,
                           int splits, int stages, int shape, void* ws, int64_t ws_bytes, hipStream_t st);

int qtts_launch_w8a16_skinny_sub(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
                                 int64_t n, const void* scale, int sdt, const void* bias, void* y, int64_t ldy,
                                 int sub, int waves, int cpw, unsigned blocks, hipStream_t st);

int64_t qtts_w8a16_ws_bytes(int64_t m, int64_t n, int64_t k, int algo) {
  const int family = algo & 0xff, splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  int64_t ws = 0;
  if (family == QTTS_ALGO_SKINNY_HALF || family == QTTS_ALGO_SKINNY_QUARTER) return 0;  // no split
  const int cpw = (algo >> 24) & 0x3f;
  if (family == QTTS_ALGO_SKINNY || family == QTTS_ALGO_AUTO)
    ws = std::max(ws, skinny_ws(skinny_cfg(std::min<int64_t>(m, kSkinnyMaxM), n, k, splits, waves, cpw)));
  if (family == QTTS_ALGO_TILE || (family == QTTS_ALGO_AUTO && m > 16)) {
    ws = std::max(ws, tile_ws(tile_cfg(m, n, k, splits)));
    if (k % 64 == 0) ws = std::max(ws, qtts_w8a16_pipe_ws_bytes(m, n, k, splits, waves, (algo >> 24) & 0xff));
  }
  return ws;
}

template <typename XT, int LAYOUT>
static int launch_fast(const XT* x, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n, int64_t ldq,
                       const void* scale, int sdt, const XT* bias, XT* y, int64_t ldy, int algo, void* ws,
                       int64_t ws_bytes, hipStream_t st) {
  int family = algo & 0xff;
  const int splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  const bool wide_ok = LAYOUT == kLayoutStrips && k % 64 == 0;  // skinny beyond 16 rows
  // Row-split strips: requested by family, or the automatic choice for staged decode rows
  // where the strips alone would leave compute units idle.
  int sub = family == QTTS_ALGO_SKINNY_HALF ? 2 : (family == QTTS_ALGO_SKINNY_QUARTER ? 4 : 1);
  if (sub > 1) {
    if (LAYOUT != kLayoutStrips || splits != 0 || ((algo >> 24) & 0x40) || !skinny_sub_rows_ok(m, k, sub))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                            "w8a16 row-split strips (%d per strip) need strip weights, at most %d rows (got %lld), "
                            "K a multiple of %d (got %lld) and no split",
                            sub, sub == 2 ? kRowPartsMaxM : 16 / sub, (long long)m, 64 * sub, (long long)k);
  } else if (family == QTTS_ALGO_AUTO && LAYOUT == kLayoutStrips && splits == 0 && (algo >> 16) == 0) {
    // more than 8 rows: half strips in row parts of 8 where they pay (skinny_row_parts_sub)
    sub = m <= 8 ? skinny_auto_sub(m, n, k) : skinny_row_parts_sub(m, n, k);
  }
  if (sub > 1) {
    const int cpw = (algo >> 24) & 0x3f;
    const SkinnyCfg c = skinny_cfg_sub(n, k, sub, waves, cpw);
    const int64_t blocks = ((int64_t)c.strips * sub + 7) / 8 * 8;
    if (c.waves * c.cpw < c.cps)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 row-split strips: %d waves of %d units cover less "
                            "than the %d units of K", c.waves, c.cpw, c.cps);
    if (!grid_ok(blocks) || ldx > INT32_MAX) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16: N or ldx too large");
    const int rc = qtts_launch_w8a16_skinny_sub(x, std::is_same<XT, bf16_t>::value ? QTTS_BF16 : QTTS_F16, m, k, ldx,
                                                q, n, scale, sdt, bias, y, ldy, sub, c.waves, c.cpw,
                                                (unsigned)blocks, st);
    if (rc != 1) return rc;
    if (family != QTTS_ALGO_AUTO)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 row-split strips: %d waves of %d units are not built "
                            "for %d workgroups per strip", c.waves, c.cpw, sub);
  }
  if (family == QTTS_ALGO_AUTO)
    family = (m <= 16 || (wide_ok && m <= kSkinnyAutoMaxM && n * k <= kSkinnyAutoMaxBytes && k <= kSkinnyAutoMaxK))
                 ? QTTS_ALGO_SKINNY
                 : QTTS_ALGO_TILE;
  if (family == QTTS_ALGO_SKINNY && m > 16 && !(wide_ok && m <= kSkinnyMaxM))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                          "skinny W8A16 kernel handles M <= 16 (M <= %d on strip weights with K %% 64 == 0), got M=%lld",
                          kSkinnyMaxM, (long long)m);
  unsigned* counters = (unsigned*)ws;
  float* part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
  if (family == QTTS_ALGO_SKINNY) {
    const int cpw = (algo >> 24) & 0x3f;
    const bool direct_x = (algo >> 24) & 0x40;
    SkinnyCfg c = skinny_cfg(m, n, k, splits, waves, cpw);
    // 9-16 rows with one split on at most 128 strips: two row parts of 8 staged rows (the kernel's y0)
    const bool staged = c.mb == 1 && wide_ok && (m <= 8 || (c.S == 1 && skinny_row_parts_auto(m, n))) && !direct_x;
    // Staged rows from 2 to 8 rows: 8 waves of 12 chunks beat 16 of 6 (measured on the talker
    // down projection, K = 6144, M = 2..8; in row parts, M = 9 / 12 / 16, 16 of 6 are 0.30 / 0.26 /
    // 0.46 us a call faster).
    if (staged && m >= 2 && m <= 8 && waves == 0 && cpw == 0 && c.waves == 16 && c.S == 1 && 8 * 12 >= (k + 63) / 64)
      c = skinny_cfg(m, n, k, splits, 8, 12);
    if (!skinny_cpw_ok(c.mb, c.waves, c.cpw) && !(staged && qtts_w8a16_xrows_built(c.waves, c.cpw)))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                            "w8a16 skinny: %d chunks per wave is not built for %d waves and %d m-blocks", c.cpw,
                            c.waves, c.mb);
    const int64_t need = skinny_ws(c);
    if (need > ws_bytes || (need > 0 && !ws)) {
      if (splits > 0)
        return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 skinny with %d splits needs %lld workspace bytes, got %lld",
                              c.S, (long long)need, (long long)ws_bytes);
      // No room for a split: give each wave a longer run instead.
      const int wmax = skinny_waves_max(c.mb);
      c = skinny_cfg(m, n, k, 1, wmax, skinny_cpw_max(c.mb, wmax));
      if (c.S > 1)
        return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 skinny: K=%lld needs a split-K workspace of %lld bytes",
                              (long long)k, (long long)skinny_ws(c));
    }
    if (c.S > 65535) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 skinny: K too large (%d splits, past the grid's y limit of 65535)", c.S);
    if (c.S > 1 && c.strips > kMaxSplitTiles)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 skinny: N=%lld with K=%lld needs a split-K over more "
                            "output strips than the workspace counter block holds", (long long)n, (long long)k);
    // grid x: the strips rounded up to a multiple of 8; grid y: the K splits
    const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8;
    if (!grid_ok(blocks) || ldx > INT32_MAX) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16: N or ldx too large");
#define QTTS_SK(ST, W, CPW, FK, MBV)                                                                                \
  qtts::launch_skinny<XT, ST, W, CPW, LAYOUT, FK, MBV>(dim3((unsigned)blocks, (unsigned)c.S), dim3(W * 64), st, q, x, \
                                                       (const ST*)scale, bias, (const XT*)nullptr, (int)ldx,         \
                                                       (int)(m | (c.S << 8)), (int)k, (int)n, y, ldy, ldq, part,    \
                                                       counters, 0.0f, (const XT*)nullptr, (int64_t)0)
#define QTTS_SK_ST(W, CPW, FK, MBV)                           \
  do {                                                        \
    if (sdt == QTTS_BF16) QTTS_SK(bf16_t, W, CPW, FK, MBV);   \
    else if (sdt == QTTS_F16) QTTS_SK(f16_t, W, CPW, FK, MBV); \
    else QTTS_SK(float, W, CPW, FK, MBV);                     \
  } while (0)
#define QTTS_SK1(W, CPW)                                                 \
  do {                                                                   \
    if (wide_ok) QTTS_SK_ST(W, CPW, true, 1);                            \
    else QTTS_SK_ST(W, CPW, false, 1);                                   \
  } while (0)
    // Up to 8 rows on full-K strip weights: activation rows staged through LDS, when
    // built for this (waves, chunks) pair and not switched off by algo bit 30.
    if (staged) {
      const int rc = qtts_launch_w8a16_skinny_xrows(x, std::is_same<XT, bf16_t>::value ? QTTS_BF16 : QTTS_F16, m, k,
                                                    ldx, q, n, scale, sdt, bias, y, ldy, c.waves, c.cpw, part,
                                                    counters, c.strips, c.S, c.cps, (unsigned)blocks, st);
      if (rc != 1) return rc;
    }
    const int key = c.waves * 16 + c.cpw;
    if (c.mb == 1) {
      switch (key) {
        case 1 * 16 + 4: QTTS_SK1(1, 4); break;
        case 1 * 16 + 8: QTTS_SK1(1, 8); break;
        case 2 * 16 + 4: QTTS_SK1(2, 4); break;
        case 2 * 16 + 8: QTTS_SK1(2, 8); break;
        case 4 * 16 + 4: QTTS_SK1(4, 4); break;
        case 4 * 16 + 8: QTTS_SK1(4, 8); break;
        case 8 * 16 + 4: QTTS_SK1(8, 4); break;
        case 8 * 16 + 8: QTTS_SK1(8, 8); break;
        case 16 * 16 + 4: QTTS_SK1(16, 4); break;
        case 16 * 16 + 6: QTTS_SK1(16, 6); break;
        default:
          return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 skinny: waves per workgroup must be 1, 2, 4, 8 or 16");
      }
    } else if constexpr (LAYOUT == kLayoutStrips) {
      if (c.mb == 2) {
        switch (key) {
          case 1 * 16 + 4: QTTS_SK_ST(1, 4, true, 2); break;
          case 1 * 16 + 8: QTTS_SK_ST(1, 8, true, 2); break;
          case 2 * 16 + 4: QTTS_SK_ST(2, 4, true, 2); break;
          case 2 * 16 + 8: QTTS_SK_ST(2, 8, true, 2); break;
          case 4 * 16 + 4: QTTS_SK_ST(4, 4, true, 2); break;
          case 4 * 16 + 8: QTTS_SK_ST(4, 8, true, 2); break;
          case 8 * 16 + 4: QTTS_SK_ST(8, 4, true, 2); break;
          case 8 * 16 + 8: QTTS_SK_ST(8, 8, true, 2); break;
          case 16 * 16 + 4: QTTS_SK_ST(16, 4, true, 2); break;
          default:
            return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 skinny: unsupported waves/chunks for 2 m-blocks");
        }
      } else {
        switch (key) {
          case 1 * 16 + 4: QTTS_SK_ST(1, 4, true, 4); break;
          case 2 * 16 + 4: QTTS_SK_ST(2, 4, true, 4); break;
          case 4 * 16 + 4: QTTS_SK_ST(4, 4, true, 4); break;
          case 8 * 16 + 4: QTTS_SK_ST(8, 4, true, 4); break;
          default:
            return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 skinny: unsupported waves/chunks for 4 m-blocks");
        }
      }
    }
#undef QTTS_SK1
#undef QTTS_SK_ST
#undef QTTS_SK
    return qtts_check_launch("w8a16_skinny");
  }
  if (LAYOUT == kLayoutStrips && k % 64 == 0)
    return qtts_launch_w8a16_pipe(x, std::is_same<XT, bf16_t>::value ? QTTS_BF16 : QTTS_F16, m, k, ldx, q, n, scale,
                                  sdt, bias, y, ldy, splits, waves, (algo >> 24) & 0xff, ws, ws_bytes, st);
  TileCfg c = tile_cfg(m, n, k, splits);
  const int64_t need = tile_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 tile with %d splits needs %lld workspace bytes, got %lld", c.S,
                            (long long)need, (long long)ws_bytes);
    c = tile_cfg(m, n, k, 1);
  }
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  const int64_t blocks = (tiles + 7) / 8 * 8 * c.S;
  if (!grid_ok(blocks)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16: problem too large");
#define QTTS_TILE(BM)                                                                                          \
  qtts::launch(&w8a16_tile_kernel<XT, BM, LAYOUT>, dim3((unsigned)blocks), dim3(256), 0, st, x, (int)m, (int)k, ldx, q, (int)n, ldq, scale, \
                                                                      sdt, bias, y, ldy, part, counters, c.mtiles, \
                                                                      c.ntiles, c.S, c.cps)
  if (c.bm == 32) QTTS_TILE(32);
  else if (c.bm == 64) QTTS_TILE(64);
  else QTTS_TILE(128);
#undef QTTS_TILE
  return qtts_check_launch("w8a16_tile");
}

// layout: kLayoutRowMajor (q [n, k], row stride ldq) or kLayoutStrips (ldq ignored).
int qtts_launch_w8a16(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n,
                      int64_t ldq, int layout, const void* scale, int scale_dtype, const void* bias, void* y,
                      int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st) {
  const bool x_ok = ((uintptr_t)x % 16 == 0) && (ldx % 8 == 0) && k > 0 && (k % 16 == 0);
  const bool q_ok = layout == kLayoutStrips || (((uintptr_t)q % 16 == 0) && (ldq % 16 == 0));
  const bool fast = x_ok && q_ok && x_dtype != QTTS_F32;
  if (!fast) {
    if (layout == kLayoutStrips)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                            "strip-layout weights need bf16/fp16 activations with 16-byte aligned rows and K %% 16 == 0");
    dim3 grid((unsigned)n, (unsigned)((m + kGenericRows - 1) / kGenericRows));
    if (x_dtype == QTTS_BF16)
      qtts::launch(&w8a16_generic_kernel<bf16_t>, dim3(grid), dim3(64), 0, st, (const bf16_t*)x, (int)m, (int)k, ldx, q, (int)n, ldq, scale,
                                                        scale_dtype, (const bf16_t*)bias, (bf16_t*)y, ldy);
    else if (x_dtype == QTTS_F16)
      qtts::launch(&w8a16_generic_kernel<f16_t>, dim3(grid), dim3(64), 0, st, (const f16_t*)x, (int)m, (int)k, ldx, q, (int)n, ldq, scale,
                                                       scale_dtype, (const f16_t*)bias, (f16_t*)y, ldy);
    else
      qtts::launch(&w8a16_generic_kernel<float>, dim3(grid), dim3(64), 0, st, (const float*)x, (int)m, (int)k, ldx, q, (int)n, ldq, scale,
                                                       scale_dtype, (const float*)bias, (float*)y, ldy);
    return qtts_check_launch("w8a16_generic");
  }
  if (x_dtype == QTTS_BF16) {
    if (layout == kLayoutStrips)
      return launch_fast<bf16_t, kLayoutStrips>((const bf16_t*)x, m, k, ldx, q, n, ldq, scale, scale_dtype,
                                                (const bf16_t*)bias, (bf16_t*)y, ldy, algo, ws, ws_bytes, st);
    return launch_fast<bf16_t, kLayoutRowMajor>((const bf16_t*)x, m, k, ldx, q, n, ldq, scale, scale_dtype,
                                                (const bf16_t*)bias, (bf16_t*)y, ldy, algo, ws, ws_bytes, st);
  }
  if (layout == kLayoutStrips)
    return launch_fast<f16_t, kLayoutStrips>((const f16_t*)x, m, k, ldx, q, n, ldq, scale, scale_dtype,
                                             (const f16_t*)bias, (f16_t*)y, ldy, algo, ws, ws_bytes, st);
  return launch_fast<f16_t, kLayoutRowMajor>((const f16_t*)x, m, k, ldx, q, n, ldq, scale, scale_dtype,
                                             (const f16_t*)bias, (f16_t*)y, ldy, algo, ws, ws_bytes, st);
}
