// int8 W8A8 GEMM for gfx950: y = round((f32(sum_c qx[m,c] qw[n,c]) * sx[m]) * sw[n]
// [+ f32(bias[n])]), replacing torch._int_mm and the fp32 epilogue of Int8Method.apply
// (qtts/quant/int8.py:151-160).
//
// Both operands are int8 codes, so a lane's 16 weight bytes and 16 activation bytes
// are the operands of one v_mfma_i32_16x16x64_i8 as loaded: no conversion at all.
// The int32 accumulation is exact, so every kernel, tile shape and split count gives
// the same bits, and the only rounding is the epilogue's (int8_epilogue).
//
//  * skinny: a wave owns a 16-row strip of qw and one 16-row block of activations;
//    per 64-column chunk of K a lane loads 16 weight bytes and 16 activation bytes and
//    issues one MFMA.  Waves split K and meet in LDS; workgroups may split K further
//    and meet through the workspace (last arrival reduces).  blockIdx.y walks 16-row
//    blocks, so it serves any M (the decode path for M <= 16; on strips, up to 128 rows
//    while the row blocks times the weight stay within 24 MiB: skinny_rows_auto).
//    SUB = 2 (strip weights, M <= 8, no split): half strips, two workgroups of 8 weight
//    rows per strip, as skinny.h does for W8A16: A rows 0-7 hold chunk 2u and rows 8-15
//    chunk 2u + 1 of those rows, B columns 0-7 and 8-15 the activation rows for the same
//    two chunks, and the two diagonal 8 x 8 blocks of D are added at the end (in int32,
//    exactly: the result is the whole-strip kernel's, bit for bit).
//  * tile (the other M > 16, K % 128 == 0): pipe_w8a8.h, in tile_i8.hip / tile_i8_rows.hip.
//  * generic: any alignment and K; correctness path.
//
// Weights come row-major [N, K] or in the QTTS_STRIP_INT8 layout of layout.h (one
// 1 KiB block per strip and chunk, in MFMA lane order).  The reference's B operand
// is the transposed [K, N] copy (int8.py:138); either of these holds the same codes.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "layout.h"
#include "skinny.h"
#include "splitk.h"

namespace qtts {

template <typename OT> __device__ __forceinline__ float out_bits_f32(uint32_t b) {
  if constexpr (sizeof(OT) == 2) return to_f32(OT{(uint16_t)b});
  else return __uint_as_float(b);
}

template <typename OT, int WAVES, int U, int LAYOUT, int SUB = 1, bool NT = false>
__global__ __launch_bounds__(WAVES * 64) void int8_skinny_kernel(
    const int8_t* __restrict__ qx, const float* sx, int M, int K, int64_t ldqx,
    const int8_t* __restrict__ qw, int N, int64_t ldqw, const float* sw, const OT* bias,
    OT* __restrict__ y, int64_t ldy, int* __restrict__ part, unsigned* __restrict__ counters, int strips, int S,
    int cps) {
  static_assert(SUB == 1 || (SUB == 2 && LAYOUT == kLayoutStrips), "half strips need strip weights");
  constexpr int RP = 16 / SUB;  // weight rows per workgroup
  __shared__ i32x4_t red[WAVES > 1 ? WAVES - 1 : 1][64];
  int strip, split;
  if constexpr (SUB == 1) {
    decode_wg(blockIdx.x, S, strip, split);
  } else {  // no split: the host launches half strips with S == 1
    strip = blockIdx.x / SUB;
    split = 0;
  }
  const int part_row = SUB == 1 ? 0 : (blockIdx.x % SUB) * RP;  // this workgroup's first strip row
  if (strip >= strips) return;

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int mrow = (int)blockIdx.y * 16 + r;  // the D column lane r holds (half strips: r < 8)
  const int n = strip * 16 + r;
  const bool n_ok = n < N, m_ok = mrow < M;
  const int xrow = SUB == 1 ? mrow : r % RP;  // the activation row lane r loads (B column r)
  const bool x_ok = SUB == 1 ? m_ok : xrow < M;
  const int nchunks = (K + 63) >> 6;
  // units of SUB chunks (SUB divides nchunks, checked by the host)
  const int c0 = split * cps, c1 = min(c0 + cps, SUB == 1 ? nchunks : nchunks / SUB);
  const int cw = (c1 - c0 + WAVES - 1) / WAVES;
  const int wc0 = c0 + wave * cw, wc1 = min(wc0 + cw, c1);
  const int8_t* wp;
  int64_t wstride;
  if constexpr (LAYOUT == kLayoutStrips && SUB > 1) {
    // lane (r, g): strip row part_row + r % RP of chunk r / RP of each unit, bytes 16 g .. + 15
    wp = qw + (int64_t)strip * nchunks * 1024 + (r / RP) * 1024 + (part_row + r % RP + 16 * g) * 16;
    wstride = SUB * 1024;
  } else if constexpr (LAYOUT == kLayoutStrips) {
    wp = qw + (int64_t)strip * nchunks * 1024 + lane * 16;
    wstride = 1024;
  } else {
    wp = qw + (int64_t)(n_ok ? n : 0) * ldqw + 16 * g;
    wstride = 64;
  }
  const int8_t* xp = qx + (int64_t)(x_ok ? xrow : 0) * ldqx + (SUB == 1 ? 0 : (r / RP) * 64) + 16 * g;
  const int64_t xstride = SUB * 64;
  const i32x4_t zero = {0, 0, 0, 0};

  // A group of U chunks is issued in full before any of it is consumed.
  i32x4_t wv[U], xv[U];
  auto issue = [&](int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + u;
      const bool live = cc < wc1;
      const bool ok = live && (SUB > 1 || cc * 64 + 16 * g < K);  // half strips: K % 128 == 0
      const bool wok = LAYOUT == kLayoutStrips ? live : (ok && n_ok);
      wv[u] = wok ? load_weight<NT>(wp + (int64_t)cc * wstride) : zero;
      xv[u] = (ok && x_ok) ? *(const i32x4_t*)(xp + (int64_t)cc * xstride) : zero;
    }
  };
  i32x4_t acc = zero;
  auto consume = [&](int c) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + u < wc1) acc = mma_i8_16x16x64(wv[u], xv[u], acc);
  };
  // Epilogue operands as raw bits, loaded unconditionally (clamped in range).
  uint32_t sxv, swv[4], bi[4];
  auto issue_epilogue = [&]() {
    sxv = *(const uint32_t*)(sx + min(mrow, M - 1));
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
    for (int w = 0; w < WAVES - 1; ++w) {
      const i32x4_t o = red[w][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = (int)((unsigned)acc[i] + (unsigned)o[i]);
    }
  }

  if constexpr (SUB == 2) {
    // D rows 8 + i, columns 8 + j (the odd chunk of each unit) onto rows i, columns j: lane
    // (j, g) for g < 2 takes lane (j + 8, g + 2), i.e. lane ^ 40; int32, wrapping like the MFMA
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = (int)((unsigned)acc[i] + (unsigned)__shfl_xor(acc[i], 40, 64));
  }

  if (SUB == 1 && S > 1) {
    int a[4] = {acc[0], acc[1], acc[2], acc[3]};
    const int tile = (int)blockIdx.y * strips + strip;
    if (!splitk_meet<4>(a, part + (int64_t)tile * S * 64 * 4, &counters[tile], S, split, lane, 64, nullptr))
      return;
    acc = i32x4_t{a[0], a[1], a[2], a[3]};
  }

  if (m_ok && (SUB == 1 || r < RP)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nn = strip * 16 + part_row + 4 * g + i;
      if ((SUB == 1 || 4 * g < RP) && nn < N) {
        const float v = int8_epilogue(acc[i], __uint_as_float(sxv), __uint_as_float(swv[i]), out_bits_f32<OT>(bi[i]),
                                      bias != nullptr);
        y[(int64_t)mrow * ldy + nn] = from_f32<OT>(v);
      }
    }
  }
}

// ------------------------------------------------------------------------------------

template <typename OT>
__global__ __launch_bounds__(64) void int8_generic_kernel(
    const int8_t* __restrict__ qx, const float* __restrict__ sx, int M, int K, int64_t ldqx,
    const int8_t* __restrict__ qw, int N, int64_t ldqw, const float* __restrict__ sw, const OT* __restrict__ bias,
    OT* __restrict__ y, int64_t ldy) {
  const int n = blockIdx.x, m0 = blockIdx.y * 4, lane = threadIdx.x;
  int acc[4] = {0, 0, 0, 0};
  for (int k = lane; k < K; k += 64) {
    const int w = qw[(int64_t)n * ldqw + k];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (m0 + i < M) acc[i] = (int)((unsigned)acc[i] + (unsigned)((int)qx[(int64_t)(m0 + i) * ldqx + k] * w));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc[i] = (int)((unsigned)acc[i] + (unsigned)__shfl_xor(acc[i], o, 64));
    if (lane == 0 && m0 + i < M) {
      const float b = bias ? to_f32(bias[n]) : 0.0f;
      y[(int64_t)(m0 + i) * ldy + n] = from_f32<OT>(int8_epilogue(acc[i], sx[m0 + i], sw[n], b, bias != nullptr));
    }
  }
}

}  // namespace qtts

using namespace qtts;

int64_t qtts_int8_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int shape);
int qtts_launch_int8_pipe_strips(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                                 const int8_t* qs, int64_t n, const float* sw, const void* bias, void* y,
                                 int out_dtype, int64_t ldy, int splits, int stages, int shape, void* ws,
                                 int64_t ws_bytes, hipStream_t st);
int qtts_launch_int8_pipe_rows(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                               const int8_t* qw, int64_t n, int64_t ldqw, const float* sw, const void* bias, void* y,
                               int out_dtype, int64_t ldy, int splits, int stages, int shape, void* ws,
                               int64_t ws_bytes, hipStream_t st);

namespace {

struct I8Cfg { int family, waves, S, cps, strips, mblocks; };

constexpr int kI8CPW = 4;  // 64-byte chunks a wave keeps in flight at once

// Skinny: waves grow until each holds at most kI8CPW chunks or the grid has 2048
// waves; then workgroups split K until each wave's share fits its in-flight group.
I8Cfg int8_skinny_cfg(int64_t m, int64_t n, int64_t k, int algo) {
  I8Cfg c{};
  c.family = QTTS_ALGO_SKINNY;
  const int splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  c.strips = (int)((n + 15) / 16);
  c.mblocks = (int)((m + 15) / 16);
  const int nchunks = std::max(1, (int)((k + 63) / 64));
  int W = waves, S = splits;
  if (W <= 0) {
    W = 1;
    while (W < 16 && ((nchunks + W - 1) / W > kI8CPW || (int64_t)c.strips * c.mblocks * W < 2048)) W *= 2;
  }
  if (S <= 0) {
    S = 1;
    while ((nchunks + S * W - 1) / (S * W) > kI8CPW) S *= 2;
  }
  c.waves = W;
  S = std::max(1, std::min(S, nchunks));
  if ((int64_t)c.strips * c.mblocks > kMaxSplitTiles) S = 1;
  c.cps = (nchunks + S - 1) / S;
  c.S = (nchunks + c.cps - 1) / c.cps;
  return c;
}

int64_t int8_skinny_ws(const I8Cfg& c) {
  if (c.S <= 1) return 0;
  return kCounterBytes + (int64_t)c.strips * c.mblocks * c.S * 64 * 16;
}

bool pipe_ok(int64_t k, int64_t ldqx, const int8_t* qx, int layout, int64_t ldqw, const int8_t* qw) {
  const bool x_ok = (uintptr_t)qx % 16 == 0 && ldqx % 16 == 0 && k % 128 == 0 && k > 0;
  if (layout == kLayoutStrips) return x_ok;
  return x_ok && (uintptr_t)qw % 16 == 0 && ldqw % 16 == 0;
}

bool skinny_ok(int64_t k, int64_t ldqx, const int8_t* qx, int layout, int64_t ldqw, const int8_t* qw) {
  const bool x_ok = (uintptr_t)qx % 16 == 0 && ldqx % 16 == 0 && k % 16 == 0 && k > 0;
  if (layout == kLayoutStrips) return x_ok;
  return x_ok && (uintptr_t)qw % 16 == 0 && ldqw % 16 == 0;
}

// Up to 128 rows on strip weights the skinny kernel (one split, each 16-row block of
// activations against every strip) beats the tile kernel while the row blocks times the
// weight bytes stay within 24 MiB.  Measured (two launches with the quantization, warm
// weights, µs): talker o_proj at M = 64 9.65 -> 7.84, down_proj at M = 32 12.03 -> 9.87,
// qkv at M = 32 9.57 -> 7.77; predictor o_proj at M = 128 9.73 -> 7.92, down_proj at
// M = 64 9.84 -> 7.77; 1.01-1.36x everywhere within the bound, 0.59-0.93x past it
// (32 MiB and more).
bool skinny_rows_auto(int64_t m, int64_t n, int64_t k) {
  return m > 16 && m <= 128 && (m + 15) / 16 * n * k <= (24ll << 20);
}

int family_of(int64_t m, int64_t n, int64_t k, int layout, int algo) {
  const int f = algo & 0xff;
  if (f != QTTS_ALGO_AUTO) return f;
  return (m <= 16 || (layout == kLayoutStrips && skinny_rows_auto(m, n, k))) ? QTTS_ALGO_SKINNY : QTTS_ALGO_TILE;
}

template <typename OT>
int int8_launch_typed(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const int8_t* qw,
                      int64_t n, int64_t ldqw, int layout, const float* sw, const OT* bias, OT* y, int64_t ldy,
                      int algo, void* ws, int64_t ws_bytes, hipStream_t st) {
  constexpr int odt = std::is_same<OT, bf16_t>::value ? QTTS_BF16 : (std::is_same<OT, f16_t>::value ? QTTS_F16 : QTTS_F32);
  const int family = family_of(m, n, k, layout, algo);
  const bool fast = skinny_ok(k, ldqx, qx, layout, ldqw, qw);
  if (layout == kLayoutStrips && !fast)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT,
                          "strip-layout int8 weights need 16-byte aligned activation rows and K %% 16 == 0");
  if (family == QTTS_ALGO_TILE && pipe_ok(k, ldqx, qx, layout, ldqw, qw)) {
    const int splits = (algo >> 8) & 0xff, stages = (algo >> 16) & 0xff, shape = (algo >> 24) & 0xff;
    if (layout == kLayoutStrips)
      return qtts_launch_int8_pipe_strips(qx, sx, m, k, ldqx, qw, n, sw, bias, y, odt, ldy, splits, stages, shape, ws,
                                          ws_bytes, st);
    return qtts_launch_int8_pipe_rows(qx, sx, m, k, ldqx, qw, n, ldqw, sw, bias, y, odt, ldy, splits, stages, shape,
                                      ws, ws_bytes, st);
  }
  if (!fast) {
    dim3 grid((unsigned)n, (unsigned)((m + 3) / 4));
    qtts::launch(&int8_generic_kernel<OT>, grid, dim3(64), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw,
                 bias, y, ldy);
    return qtts_check_launch("w8a8_int8_generic");
  }
  // Half strips for decode rows where whole strips leave compute units idle (skinny.h's
  // rule: the talker's down_proj); automatic choice only.  Bit-identical to whole strips.
  if ((algo & 0xff) == QTTS_ALGO_AUTO && (algo >> 8) == 0 && layout == kLayoutStrips && m <= 8 &&
      skinny_auto_sub(m, n, k) == 2) {
    const int strips = (int)((n + 15) / 16), units = (int)(k / 128);
    int W = 1;
    while (W < 16 && ((units + W - 1) / W > kI8CPW || (int64_t)strips * 2 * W < 2048)) W *= 2;
    const int64_t blocks = ((int64_t)strips * 2 + 7) / 8 * 8;
    if ((units + W - 1) / W <= kI8CPW && blocks < ((int64_t)1 << 31)) {
#define QTTS_I8H(WV)                                                                                            \
  qtts::launch_by_policy<std::is_same<OT, bf16_t>::value>([&](auto nt) {                                        \
    qtts::launch(&int8_skinny_kernel<OT, WV, kI8CPW, kLayoutStrips, 2, decltype(nt)::value>,                    \
                 dim3((unsigned)blocks, 1), dim3(WV * 64), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw,  \
                 sw, bias, y, ldy, (int*)nullptr, (unsigned*)nullptr, strips, 1, units);                         \
  })
      switch (W) {
        case 1: QTTS_I8H(1); break;
        case 2: QTTS_I8H(2); break;
        case 4: QTTS_I8H(4); break;
        case 8: QTTS_I8H(8); break;
        default: QTTS_I8H(16); break;
      }
#undef QTTS_I8H
      return qtts_check_launch("w8a8_int8_skinny_half");
    }
  }
  // Skinny kernel: the decode path, and the fallback for tile requests the pipeline
  // cannot take (K % 128 != 0); a forced tile request keeps only its split count.
  I8Cfg c = int8_skinny_cfg(m, n, k, family == QTTS_ALGO_SKINNY ? algo : (algo & 0xff00));
  if ((algo & 0xff) == QTTS_ALGO_AUTO && (algo >> 8) == 0 && layout == kLayoutStrips && m > 8) {
    // 9-128 rows on strips: one split; 8 waves while the grid has at most 256 workgroups,
    // else 4 (the measured best of 4, 8 and 16 on every talker and predictor shape)
    const int64_t wgs = (n + 15) / 16 * ((m + 15) / 16);
    c = int8_skinny_cfg(m, n, k, QTTS_ALGO_SKINNY | (1 << 8) | ((wgs <= 256 ? 8 : 4) << 16));
  }
  const int64_t need = int8_skinny_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if ((algo >> 8) & 0xff)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a8 int8 GEMM needs %lld workspace bytes, got %lld",
                            (long long)need, (long long)ws_bytes);
    c = int8_skinny_cfg(m, n, k, QTTS_ALGO_SKINNY | (1 << 8) | (c.waves << 16));
  }
  if (c.mblocks > 65535) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a8 int8 GEMM: M too large");
  unsigned* counters = (unsigned*)ws;
  int* part = ws ? (int*)((char*)ws + kCounterBytes) : nullptr;
  const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8 * c.S;
  if (blocks >= ((int64_t)1 << 31)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a8 int8 GEMM: N too large");
  const dim3 grid((unsigned)blocks, (unsigned)c.mblocks);
#define QTTS_I8S(W)                                                                                             \
  do {                                                                                                          \
    if (layout == kLayoutStrips)                                                                                \
      /* the weight policy holds for one row block only: more row blocks re-read the weight */                \
      qtts::launch_by_policy<std::is_same<OT, bf16_t>::value>([&](auto nt) {                                    \
        if (decltype(nt)::value && c.mblocks > 1)                                                               \
          qtts::launch(&int8_skinny_kernel<OT, W, kI8CPW, kLayoutStrips>, grid, dim3(W * 64), 0, st, qx, sx,    \
                       (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, bias, y, ldy, part, counters, c.strips, c.S,  \
                       c.cps);                                                                                  \
        else                                                                                                    \
          qtts::launch(&int8_skinny_kernel<OT, W, kI8CPW, kLayoutStrips, 1, decltype(nt)::value>, grid,         \
                       dim3(W * 64), 0, st, qx, sx, (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, bias, y, ldy,    \
                       part, counters, c.strips, c.S, c.cps);                                                   \
      });                                                                                                       \
    else                                                                                                        \
      qtts::launch(&int8_skinny_kernel<OT, W, kI8CPW, kLayoutRowMajor>, grid, dim3(W * 64), 0, st, qx, sx,      \
                   (int)m, (int)k, ldqx, qw, (int)n, ldqw, sw, bias, y, ldy, part, counters, c.strips, c.S,     \
                   c.cps);                                                                                      \
  } while (0)
  switch (c.waves) {
    case 1: QTTS_I8S(1); break;
    case 2: QTTS_I8S(2); break;
    case 4: QTTS_I8S(4); break;
    case 8: QTTS_I8S(8); break;
    case 16: QTTS_I8S(16); break;
    default: return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "int8 skinny: waves must be 1, 2, 4, 8 or 16");
  }
#undef QTTS_I8S
  return qtts_check_launch("w8a8_int8_skinny");
}

}  // namespace

// Workspace of the largest automatic (or the requested) choice.
int64_t qtts_int8_gemm_ws_bytes(int64_t m, int64_t n, int64_t k, int algo) {
  const int family = family_of(m, n, k, kLayoutRowMajor, algo);  // the tile's workspace too, past 16 rows
  int64_t a = 0;
  if (family == QTTS_ALGO_SKINNY || (algo & 0xff) == QTTS_ALGO_AUTO || k % 128 != 0)
    a = int8_skinny_ws(int8_skinny_cfg(m, n, k, family == QTTS_ALGO_SKINNY ? algo : (algo & 0xff00)));
  if (family == QTTS_ALGO_TILE && k % 128 == 0)
    a = std::max(a, qtts_int8_pipe_ws_bytes(m, n, k, (algo >> 8) & 0xff, (algo >> 24) & 0xff));
  return a;
}

// layout: kLayoutRowMajor (qw [n, k], row stride ldqw) or kLayoutStrips (ldqw ignored).
int qtts_launch_int8_gemm(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const int8_t* qw,
                          int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias, void* y,
                          int out_dtype, int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (out_dtype == QTTS_BF16)
    return int8_launch_typed<bf16_t>(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, (const bf16_t*)bias, (bf16_t*)y,
                                     ldy, algo, ws, ws_bytes, st);
  if (out_dtype == QTTS_F16)
    return int8_launch_typed<f16_t>(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, (const f16_t*)bias, (f16_t*)y, ldy,
                                    algo, ws, ws_bytes, st);
  return int8_launch_typed<float>(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, (const float*)bias, (float*)y, ldy,
                                  algo, ws, ws_bytes, st);
}
