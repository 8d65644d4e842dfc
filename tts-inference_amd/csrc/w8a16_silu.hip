// GatedMLP's activation and down projection (qtts/layers/activation.py:142-147):
// y = down(silu(gate) * up) from the fused gate_up output, gfx950.
//
//  * silu_mul_vec_kernel / silu_mul_kernel: `F.silu(gate) * up` in one pass, in place
//    of torch's two elementwise kernels, with torch's rounding: silu in fp32 rounded to
//    the activation dtype, the product in fp32 rounded again (common.h: silu_mul).
//  * One decode row on full-K strip weights: the W8A16 skinny kernel computes
//    silu(gate) * up while it stages its activation row in LDS (skinny.h, SILU), so
//    the activation costs no launch and no round trip through memory.  Every
//    workgroup redoes that work; for one row it hides under the weight stream (talker
//    down: 7.0 us against 9.1 us for the two passes), from two rows on it no longer
//    pays (9.4 against 9.0 us at M = 2), and the activation kernel runs first.
#include "skinny.h"

using namespace qtts;

namespace qtts {

constexpr int kSiluThreads = 256;

// 8 elements a thread; rows 16-byte aligned, k % 8 == 0.  Grid: (vector blocks, rows).
template <typename XT>
__global__ __launch_bounds__(kSiluThreads) void silu_mul_vec_kernel(const XT* __restrict__ gu, int64_t k, int64_t ld,
                                                                    XT* __restrict__ h, int64_t ldh) {
  const int64_t r = blockIdx.y;
  const int64_t v = (int64_t)blockIdx.x * kSiluThreads + threadIdx.x;
  if (8 * v >= k) return;
  const XT* g = gu + r * ld + 8 * v;
  const i32x4_t gv = *(const i32x4_t*)g, uv = *(const i32x4_t*)(g + k);
  *(i32x4_t*)(h + r * ldh + 8 * v) = silu_mul8<XT>(gv, uv);
}

template <typename XT>
__global__ __launch_bounds__(kSiluThreads) void silu_mul_kernel(const XT* __restrict__ gu, int64_t k, int64_t ld,
                                                                XT* __restrict__ h, int64_t ldh) {
  const int64_t r = blockIdx.y;
  for (int64_t c = (int64_t)blockIdx.x * kSiluThreads + threadIdx.x; c < k; c += (int64_t)gridDim.x * kSiluThreads)
    h[r * ldh + c] = from_f32<XT>(silu_mul<XT>(to_f32(gu[r * ld + c]), to_f32(gu[r * ld + k + c])));
}

}  // namespace qtts

namespace {

template <typename XT, typename ST, int W, int CPW>
void launch_fused(const void* gu, int64_t m, int64_t k, int64_t ld, const int8_t* qs, int64_t n, const void* scale,
                  const void* bias, void* y, int64_t ldy, float* part, unsigned* counters, const SkinnyCfg& c,
                  unsigned blocks, hipStream_t st) {
  qtts::launch(&w8a16_skinny_kernel<XT, ST, W, CPW, kLayoutStrips, true, 1, 1, false, true>, dim3(blocks),
               dim3(W * 64), 0, st, (const XT*)gu, (int)m, (int)k, ld, qs, (int)n, (int64_t)0, (const ST*)scale,
               (const XT*)bias, (XT*)y, ldy, part, counters, c.strips, c.S, c.cps);
}

template <typename XT, typename ST>
int launch_wc(const SkinnyCfg& c, const void* gu, int64_t m, int64_t k, int64_t ld, const int8_t* qs, int64_t n,
              const void* scale, const void* bias, void* y, int64_t ldy, float* part, unsigned* counters,
              unsigned blocks, hipStream_t st) {
#define QTTS_SF(W, CPW) \
  launch_fused<XT, ST, W, CPW>(gu, m, k, ld, qs, n, scale, bias, y, ldy, part, counters, c, blocks, st)
  switch (c.waves * 64 + c.cpw) {
    case 1 * 64 + 8: QTTS_SF(1, 8); break;
    case 2 * 64 + 8: QTTS_SF(2, 8); break;
    case 4 * 64 + 8: QTTS_SF(4, 8); break;
    case 8 * 64 + 8: QTTS_SF(8, 8); break;
    case 16 * 64 + 6: QTTS_SF(16, 6); break;
    case 8 * 64 + 12: QTTS_SF(8, 12); break;
    default: return 1;
  }
#undef QTTS_SF
  return QTTS_OK;
}

template <typename XT>
int launch_st(int sdt, const SkinnyCfg& c, const void* gu, int64_t m, int64_t k, int64_t ld, const int8_t* qs,
              int64_t n, const void* scale, const void* bias, void* y, int64_t ldy, float* part, unsigned* counters,
              unsigned blocks, hipStream_t st) {
  if (sdt == QTTS_BF16)
    return launch_wc<XT, bf16_t>(c, gu, m, k, ld, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
  if (sdt == QTTS_F16)
    return launch_wc<XT, f16_t>(c, gu, m, k, ld, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
  return launch_wc<XT, float>(c, gu, m, k, ld, qs, n, scale, bias, y, ldy, part, counters, blocks, st);
}

int64_t al256(int64_t v) { return (v + 255) & ~(int64_t)255; }

}  // namespace

int qtts_launch_w8a16(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n,
                      int64_t ldq, int layout, const void* scale, int scale_dtype, const void* bias, void* y,
                      int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st);
int64_t qtts_w8a16_ws_bytes(int64_t m, int64_t n, int64_t k, int algo);

int qtts_launch_silu_mul(const void* gu, int x_dtype, int64_t m, int64_t k, int64_t ld, void* h, int64_t ldh,
                         hipStream_t st) {
  const bool vec = x_dtype != QTTS_F32 && k % 8 == 0 && (uintptr_t)gu % 16 == 0 && (uintptr_t)h % 16 == 0 &&
                   ld % 8 == 0 && ldh % 8 == 0 && k <= (int64_t)8 * kSiluThreads * 65535;  // one vector a thread
  const int64_t per = vec ? 8 * kSiluThreads : kSiluThreads;
  const int64_t bx = std::min<int64_t>((k + per - 1) / per, 65535);
  const dim3 grid((unsigned)bx, (unsigned)m), block(kSiluThreads);
  if (vec && x_dtype == QTTS_BF16)
    qtts::launch(&silu_mul_vec_kernel<bf16_t>, grid, block, 0, st, (const bf16_t*)gu, k, ld, (bf16_t*)h, ldh);
  else if (vec)
    qtts::launch(&silu_mul_vec_kernel<f16_t>, grid, block, 0, st, (const f16_t*)gu, k, ld, (f16_t*)h, ldh);
  else if (x_dtype == QTTS_BF16)
    qtts::launch(&silu_mul_kernel<bf16_t>, grid, block, 0, st, (const bf16_t*)gu, k, ld, (bf16_t*)h, ldh);
  else if (x_dtype == QTTS_F16)
    qtts::launch(&silu_mul_kernel<f16_t>, grid, block, 0, st, (const f16_t*)gu, k, ld, (f16_t*)h, ldh);
  else
    qtts::launch(&silu_mul_kernel<float>, grid, block, 0, st, (const float*)gu, k, ld, (float*)h, ldh);
  return qtts_check_launch("silu_mul");
}

// Workspace of qtts_w8a16_silu_mul_gemm_strips: the GEMM's own (its counter block
// always reserved), then the activation [m, k] when it is computed in a separate pass.
int64_t qtts_w8a16_silu_ws_bytes(int64_t m, int64_t n, int64_t k, int algo, int x_dtype) {
  const int64_t esz = x_dtype == QTTS_F32 ? 4 : 2;
  return al256(std::max<int64_t>(qtts_w8a16_ws_bytes(m, n, k, algo), kCounterBytes)) + al256(m * k * esz);
}

int qtts_launch_w8a16_silu(const void* gu, int x_dtype, int64_t m, int64_t k, int64_t ld, const int8_t* qs, int64_t n,
                           const void* scale, int sdt, const void* bias, void* y, int64_t ldy, int algo, void* ws,
                           int64_t ws_bytes, hipStream_t st) {
  const int family = algo & 0xff, splits = (algo >> 8) & 0xff, waves = (algo >> 16) & 0xff;
  const int cpw = (algo >> 24) & 0x3f;
  const bool direct_x = (algo >> 24) & 0x40;
  const bool fusable = m == 1 && k % 64 == 0 && x_dtype != QTTS_F32 && (uintptr_t)gu % 16 == 0 &&
                       family != QTTS_ALGO_TILE && !direct_x;
  if (fusable) {
    const SkinnyCfg c = skinny_cfg(m, n, k, splits, waves, cpw);
    const int64_t need = skinny_ws(c);
    const int64_t blocks = (int64_t)((c.strips + 7) / 8) * 8 * c.S;
    if (need <= ws_bytes && (need == 0 || ws) && !(c.S > 1 && c.strips > kMaxSplitTiles) && blocks < ((int64_t)1 << 31)) {
      unsigned* counters = (unsigned*)ws;
      float* part = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
      const int rc = x_dtype == QTTS_BF16
                         ? launch_st<bf16_t>(sdt, c, gu, m, k, ld, qs, n, scale, bias, y, ldy, part, counters,
                                             (unsigned)blocks, st)
                         : launch_st<f16_t>(sdt, c, gu, m, k, ld, qs, n, scale, bias, y, ldy, part, counters,
                                            (unsigned)blocks, st);
      if (rc == QTTS_OK) return qtts_check_launch("w8a16_silu_skinny");
      if (rc != 1) return rc;
    } else if (splits > 0) {
      return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 silu: %d splits need %lld workspace bytes, got %lld", c.S,
                            (long long)need, (long long)ws_bytes);
    }
  }
  // Two passes: the activation into the workspace tail, then the W8A16 GEMM with the
  // head of the workspace.
  const int64_t esz = x_dtype == QTTS_F32 ? 4 : 2;
  const int64_t h_bytes = al256(m * k * esz);
  if (!ws || ws_bytes < kCounterBytes + h_bytes)
    return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 silu: workspace of %lld bytes < %lld needed", (long long)ws_bytes,
                          (long long)qtts_w8a16_silu_ws_bytes(m, n, k, algo, x_dtype));
  const int64_t tail = (ws_bytes - h_bytes) & ~(int64_t)255;
  void* h = (char*)ws + tail;
  const int rc = qtts_launch_silu_mul(gu, x_dtype, m, k, ld, h, k, st);
  if (rc != QTTS_OK) return rc;
  return qtts_launch_w8a16(h, x_dtype, m, k, k, qs, n, 0, kLayoutStrips, scale, sdt, bias, y, ldy, algo, ws, tail, st);
}
