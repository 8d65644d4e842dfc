// The W8A16 skinny kernel with its activation rows staged through LDS (skinny.h,
// MX > 0): decode calls of up to 8 rows on full-K strip weights.  Kept apart from
// w8a16.hip so the two instantiation sets compile in parallel.
#include "skinny.h"

using namespace qtts;

namespace {

template <typename XT, typename ST, int W, int CPW, int MX>
void launch_xrows(const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qs, int64_t n, const void* scale,
                  const void* bias, void* y, int64_t ldy, float* part, unsigned* counters, int strips, int S, int cps,
                  unsigned blocks, hipStream_t st) {
  (void)strips;
  (void)cps;
  qtts::launch_skinny<XT, ST, W, CPW, kLayoutStrips, true, 1, MX>(
      dim3(blocks, S, skinny_row_parts(m)), dim3(W * 64), st, qs, (const XT*)x, (const ST*)scale, (const XT*)bias, (const XT*)nullptr,
      (int)ldx, (int)(m | (S << 8)), (int)k, (int)n, (XT*)y, ldy, (int64_t)0, part, counters, 0.0f, (const XT*)nullptr,
      (int64_t)0);
}

template <typename XT, typename ST, int W, int CPW>
void launch_mx(int mx, const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qs, int64_t n,
               const void* scale, const void* bias, void* y, int64_t ldy, float* part, unsigned* counters, int strips,
               int S, int cps, unsigned blocks, hipStream_t st) {
  if (mx == 1)
    launch_xrows<XT, ST, W, CPW, 1>(x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S, cps, blocks, st);
  else if (mx == 2)
    launch_xrows<XT, ST, W, CPW, 2>(x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S, cps, blocks, st);
  else if (mx == 4)
    launch_xrows<XT, ST, W, CPW, 4>(x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S, cps, blocks, st);
  else
    launch_xrows<XT, ST, W, CPW, 8>(x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S, cps, blocks, st);
}

template <typename XT, typename ST>
int launch_wc(int waves, int cpw, int mx, const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
              int64_t n, const void* scale, const void* bias, void* y, int64_t ldy, float* part, unsigned* counters,
              int strips, int S, int cps, unsigned blocks, hipStream_t st) {
#define QTTS_XR(W, CPW) \
  launch_mx<XT, ST, W, CPW>(mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S, cps, blocks, st)
  switch (waves * 64 + cpw) {  // the pairs qtts_w8a16_xrows_built lists
    case 1 * 64 + 8: QTTS_XR(1, 8); break;
    case 2 * 64 + 8: QTTS_XR(2, 8); break;
    case 4 * 64 + 8: QTTS_XR(4, 8); break;
    case 8 * 64 + 8: QTTS_XR(8, 8); break;
    case 16 * 64 + 6: QTTS_XR(16, 6); break;
    case 8 * 64 + 12: QTTS_XR(8, 12); break;
    default: return 1;
  }
#undef QTTS_XR
  return QTTS_OK;
}

}  // namespace

// Launches the staged-row skinny kernel for m <= 8 rows of 16-bit activations on full-K
// strip weights, or more rows in row parts of 8 (grid z) with one split.  Returns QTTS_OK
// after a launch, 1 when (waves, cpw) is not built with staged rows (the caller then loads the
// activations directly), or an error status.
int qtts_launch_w8a16_skinny_xrows(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
                                   int64_t n, const void* scale, int sdt, const void* bias, void* y, int64_t ldy,
                                   int waves, int cpw, float* part, unsigned* counters, int strips, int S, int cps,
                                   unsigned blocks, hipStream_t st) {
  if (m < 1 || m > kRowPartsMaxM || (m > 8 && S != 1)) return 1;
  const int mx = m <= 2 ? (int)m : (m <= 4 ? 4 : 8);
  int rc;
#define QTTS_XR_ST(XT)                                                                                                \
  do {                                                                                                                \
    if (sdt == QTTS_BF16)                                                                                             \
      rc = launch_wc<XT, bf16_t>(waves, cpw, mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S, \
                                 cps, blocks, st);                                                                    \
    else if (sdt == QTTS_F16)                                                                                         \
      rc = launch_wc<XT, f16_t>(waves, cpw, mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S,  \
                                cps, blocks, st);                                                                     \
    else                                                                                                              \
      rc = launch_wc<XT, float>(waves, cpw, mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, part, counters, strips, S,  \
                                cps, blocks, st);                                                                     \
  } while (0)
  if (x_dtype == QTTS_BF16) QTTS_XR_ST(bf16_t);
  else QTTS_XR_ST(f16_t);
#undef QTTS_XR_ST
  if (rc != QTTS_OK) return rc;
  return qtts_check_launch("w8a16_skinny");
}

// (waves, chunks per wave) pairs built with staged rows.  Staged rows hold no
// activation registers per chunk, so longer runs than the direct kernel's fit.
int qtts_w8a16_xrows_built(int waves, int cpw) {
  switch (waves * 64 + cpw) {
    case 1 * 64 + 8: case 2 * 64 + 8: case 4 * 64 + 8: case 8 * 64 + 8: case 16 * 64 + 6: case 8 * 64 + 12:
      return 1;
    default:
      return 0;
  }
}
