// W8A16 GEMM for prefill-sized rows (M > 16) on strip-layout int8 weights, gfx950:
// the pipelined tile kernel of tile_w8a16.h.  Replaces _w8_gemm_kernel
// (qtts/quant/kernels.py:89-135) for M > 16 when K % 64 == 0.
#include "tile_w8a16.h"

using namespace qtts;

int64_t qtts_w8a16_pipe_ws_bytes(int64_t m, int64_t n, int64_t k, int splits, int stages, int shape) {
  if (!pipe_shape_ok(shape) || !pipe_stages_ok(stages)) return 0;
  return pipe_ws(pipe_cfg(m, n, k, splits, stages, shape));
}

// x [m, k] (bf16 or fp16, 16-byte aligned rows), qs strip layout, k % 64 == 0, m > 0.
int qtts_launch_w8a16_pipe(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs,
                           int64_t n, const void* scale, int sdt, const void* bias, void* y, int64_t ldy,
                           int splits, int stages, int shape, void* ws, int64_t ws_bytes, hipStream_t st) {
  return w8a16_pipe_launch<false>("w8a16_tile", x, x_dtype, m, k, ldx, qs, n, scale, sdt, bias, y, ldy, splits,
                                  stages, shape, ws, ws_bytes, st);
}
