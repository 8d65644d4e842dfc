// int8 W8A8 GEMM for prefill-sized rows (M > 16), gfx950: the pipelined kernel of
// pipe_w8a8.h with int8 codes on v_mfma_i32_16x16x64_i8 and the fp32 epilogue of
// Int8Method.apply (qtts/quant/int8.py:151-160), on QTTS_STRIP_INT8 weights.
// K % 128 == 0 (two 64-column strip chunks a stage).  Row-major weights: tile_i8_rows.hip.
#include "pipe_w8a8.h"

using namespace qtts;

int64_t qtts_int8_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int shape) {
  if (!w8a8_shape_ok(shape)) return 0;
  return w8a8_ws(w8a8_cfg(m, n, k, splits, 0, shape));
}

int qtts_launch_int8_pipe_strips(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                                 const int8_t* qs, int64_t n, const float* sw, const void* bias, void* y,
                                 int out_dtype, int64_t ldy, int splits, int stages, int shape, void* ws,
                                 int64_t ws_bytes, hipStream_t st) {
  const W8A8Args<PipeI8> a{qx, sx, m, k, ldqx, qs, n, 0, sw, bias, y, ldy, nullptr, nullptr};
  return w8a8_pipe_launch<PipeI8, kLayoutStrips, 4>("w8a8_int8_tile", a, out_dtype, splits, stages, shape, ws,
                                                    ws_bytes, st);
}
