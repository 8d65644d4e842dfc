// Measurement kernels for bench.py's floor mode, built into their own library
// (libqtts_probe.so, next to this file) and never into libqtts_amd.so: they are no part of
// the quantized linear.  No counterpart in the reference: they bound what one kernel per
// linear can reach on this GPU.  stream_probe_kernel moves a weight-sized slice from HBM
// the way the decode GEMMs do (16 bytes a lane, every load of a wave issued before the
// first is used) and does nothing else; empty_probe_kernel measures the launch itself.
//
// C ABI (status 0 on success, -1 on a bad argument, -2 on a failed launch; the message of
// the last failure on this thread from qtts_probe_last_error):
//   int qtts_probe_stream(const void* src, int64_t bytes, int waves, int loads, int32_t* sink, void* stream);
//     reads `bytes` from src (16-byte aligned, contiguous) as workgroups of `waves` waves, each wave
//     `loads` consecutive 1 KiB blocks (bytes a multiple of waves * loads * 1024), and stores
//     one 32-bit xor of what each wave read to sink[wave] (sink holds bytes / (loads * 1024) words).
//   int qtts_probe_empty(int64_t workgroups, int waves, void* stream);
//   const char* qtts_probe_last_error(void);
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

typedef __attribute__((ext_vector_type(4))) int probe_i32x4_t;

namespace {

thread_local char g_probe_error[256] = "";

int probe_fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_probe_error, sizeof(g_probe_error), fmt, ap);
  va_end(ap);
  return status;
}

// Wave w of workgroup b reads L consecutive 1 KiB blocks starting at block
// (b * waves + w) * L, xors every 32-bit word it read and stores one word,
// sink[b * waves + w].  The whole grid covers the slice exactly (the launcher checks).
template <int L>
__global__ __launch_bounds__(1024) void stream_probe_kernel(const probe_i32x4_t* __restrict__ src, int waves,
                                                            int* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * waves + wave;
  const probe_i32x4_t* p = src + gw * L * 64 + lane;
  probe_i32x4_t v[L];
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

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : probe_fail(-2, "%s: launch failed: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" {

const char* qtts_probe_last_error(void) { return g_probe_error; }

int qtts_probe_stream(const void* src, int64_t bytes, int waves, int loads, int32_t* sink, void* stream) {
  if (!src || !sink) return probe_fail(-1, "probe_stream: null pointer");
  if ((uintptr_t)src % 16) return probe_fail(-1, "probe_stream: src must be 16-byte aligned");
  if (waves < 1 || waves > 16) return probe_fail(-1, "probe_stream: waves must be 1..16");
  if (loads != 1 && loads != 2 && loads != 4 && loads != 8 && loads != 16)
    return probe_fail(-1, "probe_stream: loads must be 1, 2, 4, 8 or 16");
  const int64_t per_wg = (int64_t)waves * loads * 1024;
  if (bytes <= 0 || bytes % per_wg)
    return probe_fail(-1, "probe_stream: bytes must be a positive multiple of waves * loads * 1024 = %lld",
                      (long long)per_wg);
  const int64_t grid = bytes / per_wg;
  if (grid > 0x7fffffff) return probe_fail(-1, "probe_stream: too many workgroups");
  const hipStream_t st = (hipStream_t)stream;
  const probe_i32x4_t* s = (const probe_i32x4_t*)src;
  const dim3 g((unsigned)grid), b((unsigned)(64 * waves));
  switch (loads) {
    case 1: stream_probe_kernel<1><<<g, b, 0, st>>>(s, waves, sink); break;
    case 2: stream_probe_kernel<2><<<g, b, 0, st>>>(s, waves, sink); break;
    case 4: stream_probe_kernel<4><<<g, b, 0, st>>>(s, waves, sink); break;
    case 8: stream_probe_kernel<8><<<g, b, 0, st>>>(s, waves, sink); break;
    default: stream_probe_kernel<16><<<g, b, 0, st>>>(s, waves, sink); break;
  }
  return launched("probe_stream");
}

int qtts_probe_empty(int64_t workgroups, int waves, void* stream) {
  if (workgroups < 1 || workgroups > 0x7fffffff || waves < 1 || waves > 16)
    return probe_fail(-1, "probe_empty: workgroups >= 1, waves 1..16");
  empty_probe_kernel<<<dim3((unsigned)workgroups), dim3((unsigned)(64 * waves)), 0, (hipStream_t)stream>>>();
  return launched("probe_empty");
}

}  // extern "C"
