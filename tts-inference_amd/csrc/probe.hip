// Measurement kernels for bench.py's floor mode (qtts_probe_stream, qtts_probe_empty).
// No counterpart in the reference: they bound what one kernel per linear can reach on
// this GPU.  stream_probe_kernel moves a weight-sized slice from HBM the way the decode
// GEMMs do (16 bytes a lane, every load of a wave issued before the first is used) and
// does nothing else; empty_probe_kernel measures the launch itself.
#include "common.h"

namespace qtts {

// Wave w of workgroup b reads L consecutive 1 KiB blocks starting at block
// (b * waves + w) * L, xors every 32-bit word it read and stores one word,
// sink[b * waves + w].  The whole grid covers the slice exactly (the launcher checks).
template <int L>
__global__ __launch_bounds__(1024) void stream_probe_kernel(const i32x4_t* __restrict__ src, int waves,
                                                            int* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * waves + wave;
  const i32x4_t* p = src + gw * L * 64 + lane;
  i32x4_t v[L];
#pragma unroll
  for (int u = 0; u < L; ++u) v[u] = p[u * 64];
  int acc = 0;
#pragma unroll
  for (int u = 0; u < L; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
  if (lane == 0) sink[gw] = acc;
}

__global__ void empty_probe_kernel() {}

}  // namespace qtts

extern "C" {

int qtts_probe_stream(const void* src, int64_t bytes, int waves, int loads, int32_t* sink, void* stream) {
  using namespace qtts;
  if (!src || !sink) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_stream: null pointer");
  if ((uintptr_t)src % 16) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_stream: src must be 16-byte aligned");
  if (waves < 1 || waves > 16) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_stream: waves must be 1..16");
  if (loads != 1 && loads != 2 && loads != 4 && loads != 8 && loads != 16)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_stream: loads must be 1, 2, 4, 8 or 16");
  const int64_t per_wg = (int64_t)waves * loads * 1024;
  if (bytes <= 0 || bytes % per_wg)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_stream: bytes must be a positive multiple of "
                                                     "waves * loads * 1024 = %lld", (long long)per_wg);
  const int64_t grid = bytes / per_wg;
  if (grid > 0x7fffffff) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_stream: too many workgroups");
  const hipStream_t st = (hipStream_t)stream;
  const i32x4_t* s = (const i32x4_t*)src;
  const dim3 g((unsigned)grid), b((unsigned)(64 * waves));
  switch (loads) {
    case 1: launch(stream_probe_kernel<1>, g, b, 0, st, s, waves, sink); break;
    case 2: launch(stream_probe_kernel<2>, g, b, 0, st, s, waves, sink); break;
    case 4: launch(stream_probe_kernel<4>, g, b, 0, st, s, waves, sink); break;
    case 8: launch(stream_probe_kernel<8>, g, b, 0, st, s, waves, sink); break;
    default: launch(stream_probe_kernel<16>, g, b, 0, st, s, waves, sink); break;
  }
  return qtts_check_launch("probe_stream");
}

int qtts_probe_empty(int64_t workgroups, int waves, void* stream) {
  using namespace qtts;
  if (workgroups < 1 || workgroups > 0x7fffffff || waves < 1 || waves > 16)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "probe_empty: workgroups >= 1, waves 1..16");
  launch(empty_probe_kernel, dim3((unsigned)workgroups), dim3((unsigned)(64 * waves)), 0, (hipStream_t)stream);
  return qtts_check_launch("probe_empty");
}

}  // extern "C"
