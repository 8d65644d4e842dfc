// The staged-row W8A16 skinny kernel over row-split strips (skinny.h, SUB > 1): SUB
// workgroups per 16-row strip, for layers whose strips alone leave compute units idle.
// Kept in its own file so its instantiations compile in parallel with the others.
#include "skinny.h"

using namespace qtts;

// (SUB, waves, units per wave) built: the automatic choices on the talker and predictor
// shapes and their neighbours for half strips; a few for quarter strips, which no
// automatic choice takes.
#define QTTS_SUB_PAIRS(X) \
  X(2, 1, 8) X(2, 2, 8) X(2, 4, 4) X(2, 4, 8) X(2, 8, 6) X(2, 16, 3) \
  X(4, 1, 8) X(4, 2, 6) X(4, 4, 6)

namespace {

template <typename XT, typename ST, int SUB, int W, int CPW, int MX>
void launch_sub(const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qs, int64_t n, const void* scale,
                const void* bias, void* y, int64_t ldy, unsigned blocks, hipStream_t st) {
  qtts::launch_skinny<XT, ST, W, CPW, kLayoutStrips, true, 1, MX, false, kProNone, false, false, SUB>(
      dim3(blocks, 1, (unsigned)((m + MX - 1) / MX)), dim3(W * 64), st, qs, (const XT*)x, (const ST*)scale, (const XT*)bias, (const XT*)nullptr,
      (int)ldx, (int)(m | (1 << 8)), (int)k, (int)n, (XT*)y, ldy, (int64_t)0, (float*)nullptr, (unsigned*)nullptr,
      0.0f, (const XT*)nullptr, (int64_t)0);
}

template <typename XT, typename ST, int SUB, int W, int CPW>
void launch_sub_mx(int mx, const void* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qs, int64_t n,
                   const void* scale, const void* bias, void* y, int64_t ldy, unsigned blocks, hipStream_t st) {
  if (mx == 1) launch_sub<XT, ST, SUB, W, CPW, 1>(x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
  else if (mx == 2) launch_sub<XT, ST, SUB, W, CPW, 2>(x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
  else if (mx == 4) launch_sub<XT, ST, SUB, W, CPW, 4>(x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
  else if constexpr (SUB == 2) launch_sub<XT, ST, SUB, W, CPW, 8>(x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);
}

template <typename XT, typename ST>
int launch_sub_wc(int sub, int waves, int cpw, int mx, const void* x, int64_t m, int64_t k, int64_t ldx,
                  const int8_t* qs, int64_t n, const void* scale, const void* bias, void* y, int64_t ldy,
                  unsigned blocks, hipStream_t st) {
#define QTTS_SUB_CASE(SUB, W, CPW)                                                                  \
  case (SUB) * 4096 + (W) * 64 + (CPW):                                                             \
    launch_sub_mx<XT, ST, SUB, W, CPW>(mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st); \
    break;
  switch (sub * 4096 + waves * 64 + cpw) {
    QTTS_SUB_PAIRS(QTTS_SUB_CASE)
    default: return 1;
  }
#undef QTTS_SUB_CASE
  return QTTS_OK;
}

}  // namespace

// Whether (sub, waves, units per wave) is built.
int qtts_w8a16_sub_built(int sub, int waves, int cpw) {
#define QTTS_SUB_CASE(SUB, W, CPW) case (SUB) * 4096 + (W) * 64 + (CPW):
  switch (sub * 4096 + waves * 64 + cpw) {
    QTTS_SUB_PAIRS(QTTS_SUB_CASE)
    return 1;
    default: return 0;
  }
#undef QTTS_SUB_CASE
}

// Launches the row-split staged kernel: m <= 16 / sub (and <= 8) rows of 16-bit activations on
// full-K strip weights, or up to 64 rows on half strips in row parts of 8 (grid z: ceil(m / MX)
// parts of MX staged rows); grid x =
// blocks (the strips times sub, rounded up to a multiple of 8).
// Returns QTTS_OK after a launch, 1 when (sub, waves, cpw) is not built, or an error status.
int qtts_launch_w8a16_skinny_sub(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
                                 int64_t n, const void* scale, int sdt, const void* bias, void* y, int64_t ldy,
                                 int sub, int waves, int cpw, unsigned blocks, hipStream_t st) {
  if (!skinny_sub_rows_ok(m, k, sub)) return 1;
  // 5-8 rows on at most 64 strips of weights the caller keeps cached (no streaming policy): two
  // row parts of 4, which fill the compute units half strips leave idle.  Measured on the code
  // predictor's frame at batch 1 (o_proj and down_proj, 64 strips): 1017.7 -> 1005.3 us; on the
  // talker's streamed 128-strip layers the second part's re-read cost 44 us a step at M = 6 and 8.
  const bool halves = sub == 2 && m >= 5 && m <= 8 && (n + 15) / 16 <= 64 && !weight_policy();
  const int mx = halves ? 4 : (m <= 2 ? (int)m : (m <= 4 ? 4 : 8));
  int rc;
#define QTTS_SUB_ST(XT)                                                                                          \
  do {                                                                                                           \
    if (sdt == QTTS_BF16)                                                                                        \
      rc = launch_sub_wc<XT, bf16_t>(sub, waves, cpw, mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st); \
    else if (sdt == QTTS_F16)                                                                                    \
      rc = launch_sub_wc<XT, f16_t>(sub, waves, cpw, mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);  \
    else                                                                                                         \
      rc = launch_sub_wc<XT, float>(sub, waves, cpw, mx, x, m, k, ldx, qs, n, scale, bias, y, ldy, blocks, st);  \
  } while (0)
  if (x_dtype == QTTS_BF16) QTTS_SUB_ST(bf16_t);
  else QTTS_SUB_ST(f16_t);
#undef QTTS_SUB_ST
  if (rc != QTTS_OK) return rc;
  return qtts_check_launch("w8a16_skinny_sub");
}
