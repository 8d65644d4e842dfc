// int8 W8A8 GEMM for prefill-sized rows (M > 16) on row-major [N, K] int8 weights
// (16-byte aligned rows, K % 128 == 0): the pipelined kernel of pipe_w8a8.h, whose
// weight halves are then gathered 64 contiguous bytes a row like activation halves.
// Replaces torch._int_mm and the fp32 epilogue of qtts/quant/int8.py:151-160.
#include "pipe_w8a8.h"

using namespace qtts;

int qtts_launch_int8_pipe_rows(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                               const int8_t* qw, int64_t n, int64_t ldqw, const float* sw, const void* bias, void* y,
                               int out_dtype, int64_t ldy, int splits, int stages, int shape, void* ws,
                               int64_t ws_bytes, hipStream_t st) {
  const W8A8Args<PipeI8> a{qx, sx, m, k, ldqx, qw, n, ldqw, sw, bias, y, ldy, nullptr, nullptr};
  return w8a8_pipe_launch<PipeI8, kLayoutRowMajor, 4>("w8a8_int8_tile", a, out_dtype, splits, stages, shape, ws,
                                                      ws_bytes, st);
}
