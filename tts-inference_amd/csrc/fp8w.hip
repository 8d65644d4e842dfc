// fp8 (OCP e4m3) weight-only GEMM for gfx950: y = x @ (e4m3(q) * scale)^T + bias with
// bf16 / fp16 activations, the kernel the reference's Fp8WeightOnlyMethod names as
// the right home for fp8 weights (qtts/quant/fp8.py:92-123): the W8A16 kernels
// (skinny.h for M <= 16, tile_w8a16.h above) with the weight codes converted from
// e4m3 instead of int8, two codes per v_cvt_scalef32_pk_{bf16,f16}_fp8.  Every e4m3
// value is exact in bf16 and fp16, so the arithmetic is the W8A16 kernels': fp32
// accumulation, times f32(scale[n]), plus f32(bias[n]), one rounding to the
// activation dtype (qtts/quant/kernels.py:113-135).
//
// The e4m3 codes sit in the 64-column strip layout the W8A16 kernels read
// (qtts_to_strips with QTTS_STRIP_INT8: the layout permutes bytes, whatever they
// encode).  K % 64 == 0, 16-bit activations with 16-byte aligned rows, fp32 scales.
#include "skinny.h"
#include "tile_w8a16.h"

using namespace qtts;

namespace {

template <typename XT, int W, int CPW, int MX>
void launch_sk(const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n, const float* scale,
               const void* bias, void* y, int64_t ldy, float* part, unsigned* counters, const SkinnyCfg& c,
               unsigned blocks, hipStream_t st) {
  qtts::launch_skinny<XT, float, W, CPW, kLayoutStrips, true, 1, MX, true>(
      dim3(blocks, c.S, MX > 0 ? skinny_row_parts(m) : 1), dim3(W * 64), st, (const int8_t*)qs, (const XT*)x, scale, (const XT*)bias, (const XT*)nullptr,
      (int)ldx, (int)(m | (c.S << 8)), (int)k, (int)n, (XT*)y, ldy, (int64_t)0, part, counters, 0.0f,
      (const XT*)nullptr, (int64_t)0);
}

// Returns QTTS_OK after a launch, 1 when (waves, chunks) is not built for this row mode.
template <typename XT, int MX>
int launch_wc(const SkinnyCfg& c, const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n,
              const float* scale, const void* bias, void* y, int64_t ldy, float* part, unsigned* counters,
              unsigned blocks, hipStream_t st) {
#define QTTS_F8W(W, CPW) launch_sk<XT, W, CPW, MX>(x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, c, blocks, st)
  switch (c.waves * 64 + c.cpw) {
    case 1 * 64 + 8: QTTS_F8W(1, 8); break;
    case 2 * 64 + 8: QTTS_F8W(2, 8); break;
    case 4 * 64 + 8: QTTS_F8W(4, 8); break;
    case 8 * 64 + 8: QTTS_F8W(8, 8); break;
    case 16 * 64 + 6: QTTS_F8W(16, 6); break;
    case 8 * 64 + 12:
      if constexpr (MX > 0) {
        QTTS_F8W(8, 12);
        break;
      } else {
        return 1;
      }
    default: return 1;
  }
#undef QTTS_F8W
  return QTTS_OK;
}

// Row-split strips (skinny.h, SUB = 2), the automatic choice's pairs (skinny_cfg_sub).
template <typename XT, int W, int CPW, int MX>
void launch_sub(const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n, const float* scale,
                const void* bias, void* y, int64_t ldy, unsigned blocks, hipStream_t st) {
  qtts::launch_skinny<XT, float, W, CPW, kLayoutStrips, true, 1, MX, true, kProNone, false, false, 2>(
      dim3(blocks, 1, skinny_row_parts(m)), dim3(W * 64), st, (const int8_t*)qs, (const XT*)x, scale, (const XT*)bias,
      (const XT*)nullptr, (int)ldx, (int)(m | (1 << 8)), (int)k, (int)n, (XT*)y, ldy, (int64_t)0,
      (float*)nullptr, (unsigned*)nullptr, 0.0f, (const XT*)nullptr, (int64_t)0);
}

template <typename XT, int MX>
int launch_sub_wc(const SkinnyCfg& c, const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n,
                  const float* scale, const void* bias, void* y, int64_t ldy, unsigned blocks, hipStream_t st) {
#define QTTS_F8W_SUB(W, CPW) launch_sub<XT, W, CPW, MX>(x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st)
  switch (c.waves * 64 + c.cpw) {
    case 1 * 64 + 8: QTTS_F8W_SUB(1, 8); break;
    case 2 * 64 + 8: QTTS_F8W_SUB(2, 8); break;
    case 4 * 64 + 4: QTTS_F8W_SUB(4, 4); break;
    case 4 * 64 + 8: QTTS_F8W_SUB(4, 8); break;
    case 8 * 64 + 6: QTTS_F8W_SUB(8, 6); break;
    case 16 * 64 + 3: QTTS_F8W_SUB(16, 3); break;
    default: return 1;
  }
#undef QTTS_F8W_SUB
  return QTTS_OK;
}

template <typename XT>
int launch_sub_rows(int mx, const SkinnyCfg& c, const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs,
                    int64_t n, const float* scale, const void* bias, void* y, int64_t ldy, unsigned blocks,
                    hipStream_t st) {
  switch (mx) {
    case 1: return launch_sub_wc<XT, 1>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
    case 2: return launch_sub_wc<XT, 2>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
    case 4: return launch_sub_wc<XT, 4>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
    default: return launch_sub_wc<XT, 8>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
  }
}

template <typename XT>
int launch_rows(int mx, const SkinnyCfg& c, const void* x, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs,
                int64_t n, const float* scale, const void* bias, void* y, int64_t ldy, float* part, unsigned* counters,
                unsigned blocks, hipStream_t st) {
  switch (mx) {
    case 0: return launch_wc<XT, 0>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
    case 1: return launch_wc<XT, 1>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
    case 2: return launch_wc<XT, 2>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
    case 4: return launch_wc<XT, 4>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
    default: return launch_wc<XT, 8>(c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
  }
}

int family_of(int64_t m, int algo) {
  const int f = algo & 0xff;
  return f == QTTS_ALGO_AUTO ? (m <= 16 ? QTTS_ALGO_SKINNY : QTTS_ALGO_TILE) : f;
}

// Staged rows as the W8A16 launch stages them: up to 8, or 9-16 in row parts of 8 on at most 128
// strips with one split (skinny_row_parts_auto; the split is known once the configuration is).
bool fp8w_staged(int64_t m, int64_t n, int algo, int S) {
  return (m <= 8 || (S == 1 && skinny_row_parts_auto(m, n))) && !((algo >> 24) & 0x40);
}

// The W8A16 skinny choice, including 8 waves of 12 chunks for long K from 2 to 8 rows.
SkinnyCfg fp8w_skinny_cfg(int64_t m, int64_t n, int64_t k, int algo) {
  const int splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff, cpw = (algo >> 24) & 0x3f;
  const bool staged = fp8w_staged(m, n, algo, skinny_cfg(m, n, k, splits, waves, cpw).S);
  SkinnyCfg c = skinny_cfg(m, n, k, splits, waves, cpw);
  if (staged && m >= 2 && m <= 8 && waves == 0 && cpw == 0 && c.waves == 16 && c.S == 1 && 8 * 12 >= (k + 63) / 64)
    c = skinny_cfg(m, n, k, splits, 8, 12);
  return c;
}

}  // namespace

int64_t qtts_fp8w_ws_bytes(int64_t m, int64_t n, int64_t k, int algo) {
  const int family = family_of(m, algo);
  if (family == QTTS_ALGO_SKINNY) return skinny_ws(fp8w_skinny_cfg(std::min<int64_t>(m, 16), n, k, algo));
  const int stages = pipe_stages_ok((algo >> 16) & 0xff) ? (algo >> 16) & 0xff : 0;
  return pipe_ws(pipe_cfg(m, n, k, (algo >> 8) & 0xff, stages, pipe_shape_ok((algo >> 24) & 0xff) ? (algo >> 24) & 0xff : 0));
}

// x [m, k] bf16 / fp16 (16-byte aligned rows), qs e4m3 codes in the 64-column strip
// layout, k % 64 == 0, scale [n] fp32, bias [n] of x's dtype or NULL.
int qtts_launch_fp8w(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n,
                     const float* scale, const void* bias, void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes,
                     hipStream_t st) {
  const int family = family_of(m, algo);
  const int splits = (algo >> 8) & 0xff;
  // Half strips where whole ones leave compute units idle: the W8A16 launch's automatic rule (past
  // 8 rows in row parts of 8, also in place of the tile kernel up to 64 rows).
  const int auto_sub = (algo & 0xff) == QTTS_ALGO_AUTO && (algo >> 8) == 0
                           ? (m <= 8 ? skinny_auto_sub(m, n, k) : skinny_row_parts_sub(m, n, k))
                           : 1;
  if (auto_sub == 2 && ldx <= INT32_MAX) {
    const SkinnyCfg c = skinny_cfg_sub(n, k, 2, 0, 0);
    const int64_t blocks = ((int64_t)c.strips * 2 + 7) / 8 * 8;
    if (c.waves * c.cpw >= c.cps && blocks < ((int64_t)1 << 31)) {
      const int mx = m <= 2 ? (int)m : (m <= 4 ? 4 : 8);  // the fewest staged rows built that cover m
      const int rc = x_dtype == QTTS_BF16
                         ? launch_sub_rows<bf16_t>(mx, c, x, m, k, ldx, qs, n, scale, bias, y, ldy, (unsigned)blocks, st)
                         : launch_sub_rows<f16_t>(mx, c, x, m, k, ldx, qs, n, scale, bias, y, ldy, (unsigned)blocks, st);
      if (rc != 1) return rc == QTTS_OK ? qtts_check_launch("fp8w_skinny_sub") : rc;
    }
  }
  if (family == QTTS_ALGO_TILE)
    return w8a16_pipe_launch<true>("fp8w_tile", x, x_dtype, m, k, ldx, (const int8_t*)qs, n, scale, QTTS_F32, bias, y,
                                   ldy, splits, (algo >> 16) & 0xff, (algo >> 24) & 0xff, ws, ws_bytes, st);
  if (m > 16)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8 weight-only skinny kernel handles M <= 16, got M=%lld",
                          (long long)m);
  SkinnyCfg c = fp8w_skinny_cfg(m, n, k, algo);
  const bool staged = fp8w_staged(m, n, algo, c.S);
  if (!staged && c.waves == 8 && c.cpw == 12 && ((algo >> 16) & 0xff) == 0)  // 12 chunks a wave: staged rows only
    c = skinny_cfg(m, n, k, splits, 16, 6);
  const int64_t need = skinny_ws(c);
  if (need > ws_bytes || (need > 0 && !ws)) {
    if (splits > 0)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "fp8w skinny with %d splits needs %lld workspace bytes, got %lld", c.S,
                            (long long)need, (long long)ws_bytes);
    c = skinny_cfg(m, n, k, 1, 16, 6);
    if (c.S > 1)
      return qtts_set_error(QTTS_ERR_WORKSPACE, "fp8w skinny: K=%lld needs a split-K workspace of %lld bytes",
                            (long long)k, (long long)skinny_ws(c));
  }
  if (c.S > 65535) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8w skinny: K too large (%d splits, past the grid's y limit of 65535)", c.S);
  if (c.S > 1 && c.strips > kMaxSplitTiles)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8w skinny: too many output strips for a split-K meeting");
  const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8;  // grid x; grid y: the K splits
  if (blocks <= 0 || blocks >= ((int64_t)1 << 31) || ldx > INT32_MAX)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8w: N or ldx too large");
  unsigned* counters = (unsigned*)ws;
  float* part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
  const int mx = staged ? (m <= 2 ? (int)m : (m <= 4 ? 4 : 8)) : 0;
  const int rc = x_dtype == QTTS_BF16
                     ? launch_rows<bf16_t>(mx, c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters,
                                           (unsigned)blocks, st)
                     : launch_rows<f16_t>(mx, c, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters,
                                          (unsigned)blocks, st);
  if (rc == 1)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "fp8w skinny: %d waves x %d chunks is not built%s", c.waves, c.cpw,
                          staged ? "" : " for direct activation loads");
  if (rc != QTTS_OK) return rc;
  return qtts_check_launch("fp8w_skinny");
}
