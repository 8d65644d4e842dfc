// Row-major <-> strip layout conversion (see layout.h).  Load-time only: one thread
// per 16-byte lane slot, bounds-checked per byte at the ragged edges.
#include "common.h"
#include "layout.h"

namespace qtts {

struct SlotPos {
  int64_t row, col;  // first byte of the slot in the row-major matrix
};

__device__ __forceinline__ SlotPos slot_pos(int64_t u, int64_t nchunks, int kind) {
  const int ch = strip_chunk(kind), halves = ch / 64;
  const int lane = (int)(u & 63);
  int64_t t = u >> 6;
  const int h = (int)(t % halves);
  t /= halves;
  const int64_t c = t % nchunks, s = t / nchunks;
  return SlotPos{16 * s + (lane & 15), c * ch + (lane >> 4) * (ch / 4) + 16 * h};
}

__global__ __launch_bounds__(256) void to_strips_kernel(const uint8_t* __restrict__ src, int64_t n, int64_t k,
                                                        int64_t ld, uint8_t* __restrict__ dst, int64_t units,
                                                        int64_t nchunks, int kind) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const SlotPos p = slot_pos(u, nchunks, kind);
  uint8_t b[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) b[j] = (p.row < n && p.col + j < k) ? src[p.row * ld + p.col + j] : (uint8_t)0;
  uint4 v;
  __builtin_memcpy(&v, b, 16);
  *(uint4*)(dst + u * 16) = v;
}

__global__ __launch_bounds__(256) void from_strips_kernel(const uint8_t* __restrict__ src, int64_t n, int64_t k,
                                                          uint8_t* __restrict__ dst, int64_t ld, int64_t units,
                                                          int64_t nchunks, int kind) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const SlotPos p = slot_pos(u, nchunks, kind);
  const uint4 v = *(const uint4*)(src + u * 16);
  uint8_t b[16];
  __builtin_memcpy(b, &v, 16);
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (p.row < n && p.col + j < k) dst[p.row * ld + p.col + j] = b[j];
}

}  // namespace qtts

using namespace qtts;

int qtts_launch_to_strips(const void* src, int64_t n, int64_t k, int64_t ld, void* dst, int kind, hipStream_t st) {
  const int64_t units = strip_bytes(n, k, kind) / 16;
  if (units == 0) return QTTS_OK;
  const int64_t blocks = (units + 255) / 256;
  qtts::launch(&to_strips_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)src, n, k, ld, (uint8_t*)dst, units,
                                                     strip_nchunks(k, kind), kind);
  return qtts_check_launch("to_strips");
}

int qtts_launch_from_strips(const void* src, int64_t n, int64_t k, void* dst, int64_t ld, int kind, hipStream_t st) {
  const int64_t units = strip_bytes(n, k, kind) / 16;
  if (units == 0) return QTTS_OK;
  const int64_t blocks = (units + 255) / 256;
  qtts::launch(&from_strips_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)src, n, k, (uint8_t*)dst, ld, units,
                                                       strip_nchunks(k, kind), kind);
  return qtts_check_launch("from_strips");
}
