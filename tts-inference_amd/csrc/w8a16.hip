// int8 weight-only (W8A16) GEMM for gfx950: y = x @ (q * scale)^T + bias.
//
// Replaces the Triton kernel _w8_gemm_kernel (qtts/quant/kernels.py:89-135) with
// three hand-written kernels:
//
//  * skinny (M <= 16, the decode rows): every wave owns a 16-row strip of q and a
//    share of K.  A lane loads 16 contiguous weight bytes per 64-byte chunk (one
//    128-bit load; a wave covers 16 rows x 64 B), turns them into bf16 in
//    registers (int8 is exact in bf16), and feeds two v_mfma_f32_16x16x32_bf16 with
//    the activations as the 16-column B operand (rows >= M are zero).  Waves of a
//    workgroup split K and meet in LDS; workgroups may split K further and meet
//    through a workspace, where the last-arriving workgroup of a strip sums the
//    partials in split order and runs the epilogue (no second launch).
//  * tile (M > 16, prefill rows): LDS-tiled bf16 MFMA GEMM, BM x 128 x 64 tiles,
//    4 waves in 2x2, double-buffered LDS, the weight tile dequantized to bf16 on
//    its way into LDS.
//  * generic: any dtype (fp32 activations included) and any alignment; one wave
//    per output column, lanes stride K.  Correctness path for odd shapes.
//
// Numerics match the reference kernel's order of operations: products of the
// activation and the exact int8 weight accumulate in fp32, then the fp32 sum is
// multiplied by f32(scale[n]), f32(bias[n]) is added, and the result is rounded
// to the activation dtype once (qtts/quant/kernels.py:113-135).
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace qtts {

// Workgroup id -> (strip, split) such that all splits of one strip share
// wg % 8, i.e. run on the same XCD (the dispatcher deals workgroups to the 8
// XCDs round-robin), so their partials meet in one L2.
__device__ __forceinline__ void decode_wg(int wg, int S, int& strip, int& split) {
  const int group = wg / (8 * S), within = wg - group * 8 * S;
  split = within >> 3;
  strip = group * 8 + (within & 7);
}

// Split-K meeting point.  Each workgroup stores its partial (`nv` floats per
// participating thread) into its slot, then bumps the strip's counter; the last
// arrival reads every slot back in split order.  The counter is reset by the
// last arrival, so the workspace stays zero between calls.
template <int NV>
__device__ __forceinline__ bool splitk_arrive(float (&acc)[NV], float* __restrict__ part, unsigned* __restrict__ counter,
                                              int S, int split, int tid, int nthreads, unsigned* flag_lds) {
  float* mine = part + ((int64_t)split * nthreads + tid) * NV;
#pragma unroll
  for (int v = 0; v < NV; v += 4) *(f32x4_t*)(mine + v) = f32x4_t{acc[v], acc[v + 1], acc[v + 2], acc[v + 3]};
  __threadfence();
  __syncthreads();
  if (tid == 0) *flag_lds = atomicAdd(counter, 1u);
  __syncthreads();
  if (*flag_lds != (unsigned)(S - 1)) return false;
  __threadfence();
#pragma unroll
  for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
  for (int s = 0; s < S; ++s) {
    const float* src = part + ((int64_t)s * nthreads + tid) * NV;
#pragma unroll
    for (int v = 0; v < NV; v += 4) {
      f32x4_t t = *(const f32x4_t*)(src + v);
      acc[v] += t[0];
      acc[v + 1] += t[1];
      acc[v + 2] += t[2];
      acc[v + 3] += t[3];
    }
  }
  if (tid == 0) reset_counter(counter);
  return true;
}

template <typename XT, typename ST>
__device__ __forceinline__ void store_out(XT* __restrict__ y, int64_t ldy, int m, int n, float acc,
                                          const ST* __restrict__ scale, const XT* __restrict__ bias) {
  float v = acc * to_f32(scale[n]);
  if (bias) v += to_f32(bias[n]);
  y[(int64_t)m * ldy + n] = from_f32<XT>(v);
}

// ------------------------------------------------------------------------------------
// skinny: M <= 16
// ------------------------------------------------------------------------------------

template <typename XT, typename ST, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void w8a16_skinny_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ q, int N, int64_t ldq,
    const ST* __restrict__ scale, const XT* __restrict__ bias, XT* __restrict__ y, int64_t ldy,
    float* __restrict__ part, unsigned* __restrict__ counters, int strips, int S, int cps) {
  typedef mfma16<XT> MM;
  typedef typename MM::vec V;
  __shared__ f32x4_t red[WAVES > 1 ? WAVES - 1 : 1][64];

  int strip, split;
  decode_wg(blockIdx.x, S, strip, split);
  if (strip >= strips) return;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n = strip * 16 + r;
  const bool n_ok = n < N, m_ok = r < M;
  const int nchunks = (K + 63) >> 6;
  const int c0 = split * cps;
  const int c1 = min(c0 + cps, nchunks);
  const int8_t* qp = q + (int64_t)(n_ok ? n : 0) * ldq + 16 * g;
  const XT* xp = x + (int64_t)(m_ok ? r : 0) * ldx + 16 * g;
  const i32x4_t zero = {0, 0, 0, 0};

  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = c0 + wave; c < c1; c += WAVES * U) {
    i32x4_t wv[U], xa[U], xb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + u * WAVES;
      const bool ok = cc < c1 && cc * 64 + 16 * g < K;
      wv[u] = (ok && n_ok) ? *(const i32x4_t*)(qp + (int64_t)cc * 64) : zero;
      xa[u] = (ok && m_ok) ? *(const i32x4_t*)(xp + (int64_t)cc * 64) : zero;
      xb[u] = (ok && m_ok) ? *(const i32x4_t*)(xp + (int64_t)cc * 64 + 8) : zero;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const V wlo = MM::from_i8((uint32_t)wv[u][0], (uint32_t)wv[u][1]);
      const V whi = MM::from_i8((uint32_t)wv[u][2], (uint32_t)wv[u][3]);
      acc = MM::mma(wlo, __builtin_bit_cast(V, xa[u]), acc);
      acc = MM::mma(whi, __builtin_bit_cast(V, xb[u]), acc);
    }
  }

  if (WAVES > 1) {
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < WAVES - 1; ++w) acc += red[w][lane];
  }

  if (S > 1) {
    float a[4] = {acc[0], acc[1], acc[2], acc[3]};
    // Only wave 0 is left; it is the whole "workgroup" of the meeting.
    float* pstrip = part + (int64_t)strip * S * 64 * 4;
    float* mine = pstrip + ((int64_t)split * 64 + lane) * 4;
    *(f32x4_t*)mine = acc;
    __threadfence();
    unsigned prev = 0;
    if (lane == 0) prev = atomicAdd(&counters[strip], 1u);
    prev = __shfl(prev, 0, 64);
    if (prev != (unsigned)(S - 1)) return;
    __threadfence();
    a[0] = a[1] = a[2] = a[3] = 0.0f;
    for (int s = 0; s < S; ++s) {
      const f32x4_t t = *(const f32x4_t*)(pstrip + ((int64_t)s * 64 + lane) * 4);
      a[0] += t[0];
      a[1] += t[1];
      a[2] += t[2];
      a[3] += t[3];
    }
    if (lane == 0) reset_counter(&counters[strip]);
    acc = f32x4_t{a[0], a[1], a[2], a[3]};
  }

  // D layout of the 16x16 MFMA: lane (r, g) holds rows 4g..4g+3 (weight rows n) of
  // column r (activation row m).
  if (m_ok) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nn = strip * 16 + 4 * g + i;
      if (nn < N) store_out(y, ldy, r, nn, acc[i], scale, bias);
    }
  }
}

// ------------------------------------------------------------------------------------
// tile: M > 16
// ------------------------------------------------------------------------------------

constexpr int kTileBN = 128, kTileBK = 64, kTileLdsK = kTileBK + 8;  // padded LDS row, in elements

template <typename XT, typename ST, int BM>
__global__ __launch_bounds__(256) void w8a16_tile_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ q, int N, int64_t ldq,
    const ST* __restrict__ scale, const XT* __restrict__ bias, XT* __restrict__ y, int64_t ldy,
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
      const int id = tid + 256 * l, row = id >> 2, col = (id & 3) * 16;
      const int n = n0 + row, k = kc * BK + col;
      wr[l] = (n < N && k < K) ? *(const i32x4_t*)(q + (int64_t)n * ldq + k) : zero;
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
      const int id = tid + 256 * l, row = id >> 2, col = (id & 3) * 16;
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
    float a[TM * TN * 4];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) a[(i * TN + j) * 4 + t] = acc[i][j][t];
    float* ptile = part + (int64_t)tile * S * 256 * (TM * TN * 4);
    if (!splitk_arrive<TM * TN * 4>(a, ptile, &counters[tile], S, split, tid, 256, &flag)) return;
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
        if (m < M) store_out(y, ldy, m, n, acc[i][j][t], scale, bias);
      }
    }
}

// ------------------------------------------------------------------------------------
// generic: any dtype, any alignment
// ------------------------------------------------------------------------------------

constexpr int kGenericRows = 4;

template <typename XT, typename ST>
__global__ __launch_bounds__(64) void w8a16_generic_kernel(
    const XT* __restrict__ x, int M, int K, int64_t ldx, const int8_t* __restrict__ q, int N, int64_t ldq,
    const ST* __restrict__ scale, const XT* __restrict__ bias, XT* __restrict__ y, int64_t ldy) {
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
    if (lane == 0 && m0 + i < M) store_out(y, ldy, m0 + i, n, s, scale, bias);
  }
}

}  // namespace qtts

using namespace qtts;

// ---- host side ------------------------------------------------------------------------

namespace {

struct SkinnyCfg { int waves, S, cps, strips; };
struct TileCfg { int bm, S, cps, mtiles, ntiles; };

SkinnyCfg skinny_cfg(int64_t m, int64_t n, int64_t k, int splits_req, int waves_req) {
  SkinnyCfg c;
  c.strips = (int)((n + 15) / 16);
  const int nchunks = std::max(1, (int)((k + 63) / 64));
  c.waves = waves_req > 0 ? waves_req : 4;
  int S = splits_req;
  if (S <= 0) {
    // Aim for >= 1024 workgroups (4 per CU) while keeping >= 2 chunks per wave.
    S = 1;
    while (c.strips * S * 2 <= 1024 && nchunks / (S * 2) >= 2 * c.waves) S *= 2;
  }
  S = std::max(1, std::min(S, nchunks));
  if (c.strips > kMaxSplitTiles) S = 1;
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  (void)m;
  return c;
}

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

int64_t skinny_ws(const SkinnyCfg& c) {
  if (c.S <= 1) return 0;
  return kCounterBytes + (int64_t)c.strips * c.S * 64 * 4 * 4;
}

int64_t tile_ws(const TileCfg& c) {
  if (c.S <= 1) return 0;
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  return kCounterBytes + tiles * c.S * 256 * (c.bm / 32) * 4 * 4 * 4;
}

bool grid_ok(int64_t blocks) { return blocks > 0 && blocks < (int64_t)1 << 31; }

}  // namespace

int64_t qtts_w8a16_ws_bytes(int64_t m, int64_t n, int64_t k, int algo) {
  const int family = algo & 0xff, splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  int64_t ws = 0;
  if (family == QTTS_ALGO_SKINNY || family == QTTS_ALGO_AUTO) ws = std::max(ws, skinny_ws(skinny_cfg(std::min<int64_t>(m, 16), n, k, splits, waves)));
  if (family == QTTS_ALGO_TILE || (family == QTTS_ALGO_AUTO && m > 16)) ws = std::max(ws, tile_ws(tile_cfg(m, n, k, splits)));
  return ws;
}

template <typename XT, typename ST>
static int launch_typed(const XT* x, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n, int64_t ldq,
                        const ST* scale, const XT* bias, XT* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes,
                        hipStream_t st, bool fast_ok) {
  int family = algo & 0xff;
  const int splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  if (family == QTTS_ALGO_AUTO) family = m <= 16 ? QTTS_ALGO_SKINNY : QTTS_ALGO_TILE;
  if (family == QTTS_ALGO_SKINNY && m > 16)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "skinny W8A16 kernel handles M <= 16, got M=%lld", (long long)m);
  if (std::is_same<XT, float>::value || !fast_ok) {
    dim3 grid((unsigned)n, (unsigned)((m + kGenericRows - 1) / kGenericRows));
    w8a16_generic_kernel<XT, ST><<<grid, 64, 0, st>>>(x, (int)m, (int)k, ldx, q, (int)n, ldq, scale, bias, y, ldy);
    return qtts_check_launch("w8a16_generic");
  }
  if constexpr (!std::is_same<XT, float>::value) {
  if (family == QTTS_ALGO_SKINNY) {
    SkinnyCfg c = skinny_cfg(m, n, k, splits, waves);
    const int64_t need = skinny_ws(c);
    if (need > ws_bytes || (need > 0 && !ws)) {
      if (splits > 0)
        return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 skinny with %d splits needs %lld workspace bytes, got %lld",
                              c.S, (long long)need, (long long)ws_bytes);
      c = skinny_cfg(m, n, k, 1, waves);  // no workspace: one split
    }
    unsigned* counters = (unsigned*)ws;
    float* part = c.S > 1 ? (float*)((char*)ws + kCounterBytes) : nullptr;
    const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8 * c.S;
    if (!grid_ok(blocks)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16: N too large");
#define QTTS_SKINNY(W, U)                                                                                \
  w8a16_skinny_kernel<XT, ST, W, U><<<(unsigned)blocks, W * 64, 0, st>>>(x, (int)m, (int)k, ldx, q, (int)n, ldq, \
                                                                         scale, bias, y, ldy, part, counters,  \
                                                                         c.strips, c.S, c.cps)
    switch (c.waves) {
      case 1: QTTS_SKINNY(1, 4); break;
      case 2: QTTS_SKINNY(2, 4); break;
      case 4: QTTS_SKINNY(4, 4); break;
      case 8: QTTS_SKINNY(8, 2); break;
      case 16: QTTS_SKINNY(16, 1); break;
      default:
        return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 skinny: waves per workgroup must be 1, 2, 4, 8 or 16");
    }
#undef QTTS_SKINNY
    return qtts_check_launch("w8a16_skinny");
  }
  TileCfg c = tile_cfg(m, n, k, splits);
  const int64_t need = tile_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 tile with %d splits needs %lld workspace bytes, got %lld", c.S,
                            (long long)need, (long long)ws_bytes);
    c = tile_cfg(m, n, k, 1);
  }
  const int64_t tiles = (int64_t)c.mtiles * c.ntiles;
  unsigned* counters = (unsigned*)ws;
  float* part = c.S > 1 ? (float*)((char*)ws + kCounterBytes) : nullptr;
  const int64_t blocks = (tiles + 7) / 8 * 8 * c.S;
  if (!grid_ok(blocks)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16: problem too large");
#define QTTS_TILE(BM)                                                                                       \
  w8a16_tile_kernel<XT, ST, BM><<<(unsigned)blocks, 256, 0, st>>>(x, (int)m, (int)k, ldx, q, (int)n, ldq, scale, \
                                                                  bias, y, ldy, part, counters, c.mtiles,      \
                                                                  c.ntiles, c.S, c.cps)
  if (c.bm == 32) QTTS_TILE(32);
  else if (c.bm == 64) QTTS_TILE(64);
  else QTTS_TILE(128);
#undef QTTS_TILE
  return qtts_check_launch("w8a16_tile");
  }
  return QTTS_OK;
}

int qtts_launch_w8a16(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n,
                      int64_t ldq, const void* scale, int scale_dtype, const void* bias, void* y, int64_t ldy,
                      int algo, void* ws, int64_t ws_bytes, hipStream_t st) {
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 16 == 0) && (ldx % 8 == 0) && (ldq % 16 == 0) &&
                       (k % 16 == 0) && k > 0;
#define QTTS_DISPATCH_SCALE(XT, FAST)                                                                          \
  do {                                                                                                         \
    if (scale_dtype == QTTS_F32)                                                                               \
      return launch_typed<XT, float>((const XT*)x, m, k, ldx, q, n, ldq, (const float*)scale, (const XT*)bias, \
                                     (XT*)y, ldy, algo, ws, ws_bytes, st, FAST);                               \
    if (scale_dtype == QTTS_BF16)                                                                              \
      return launch_typed<XT, bf16_t>((const XT*)x, m, k, ldx, q, n, ldq, (const bf16_t*)scale,               \
                                      (const XT*)bias, (XT*)y, ldy, algo, ws, ws_bytes, st, FAST);            \
    return launch_typed<XT, f16_t>((const XT*)x, m, k, ldx, q, n, ldq, (const f16_t*)scale, (const XT*)bias,   \
                                   (XT*)y, ldy, algo, ws, ws_bytes, st, FAST);                                 \
  } while (0)
  if (x_dtype == QTTS_BF16) QTTS_DISPATCH_SCALE(bf16_t, aligned);
  if (x_dtype == QTTS_F16) QTTS_DISPATCH_SCALE(f16_t, aligned);
  QTTS_DISPATCH_SCALE(float, false);
#undef QTTS_DISPATCH_SCALE
}
