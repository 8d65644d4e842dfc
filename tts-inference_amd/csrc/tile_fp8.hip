// fp8 (OCP e4m3) W8A8 GEMM for prefill-sized rows (M > 16) on strip-layout weights,
// gfx950: the pipelined kernel of pipe_w8a8.h with e4m3 codes.
//
// Replaces torch._scaled_mm with rowwise scales and the bias add after it
// (qtts/quant/fp8.py:79-89) for M > 16 when K % 128 == 0.  Epilogue order follows the
// reference: the fp32 accumulator times sx[m] * sw[n] is rounded to the output dtype,
// then the bias is added in the output dtype.
#include "pipe_w8a8.h"

using namespace qtts;

int64_t qtts_fp8_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int shape) {
  if (!w8a8_shape_ok(shape)) return 0;
  return w8a8_ws(w8a8_cfg(m, n, k, splits, 0, shape));
}

// qx [m, k] e4m3 (16-byte aligned rows), qs e4m3 strip layout, k % 128 == 0, m > 0.
int qtts_launch_fp8_pipe(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qs,
                         int64_t n, const float* sw, const void* bias, void* y, int out_dtype, int64_t ldy, int splits,
                         int stages, int shape, void* ws, int64_t ws_bytes, hipStream_t st) {
  const W8A8Args<PipeFp8> a{qx, sx, m, k, ldqx, qs, n, 0, sw, bias, y, ldy, nullptr, nullptr};
  return w8a8_pipe_launch<PipeFp8, kLayoutStrips, 8>("w8a8_fp8_tile", a, out_dtype, splits, stages, shape, ws,
                                                     ws_bytes, st);
}
