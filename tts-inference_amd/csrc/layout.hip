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

// w[row][col] = WT(f32(code) * f32(scale[row])) for every code of a 64-column strip
// matrix (int8 codes, or e4m3 codes with E4M3): the dequantized weight of the
// reference's eager path, q.to(dtype) * scale[:, None] (the product of a code and a
// 16-bit scale is exact in fp32, so the one rounding is torch's).  One thread per 16-byte
// lane slot, two 16-byte stores where the row is aligned and whole.  (Staging a strip's
// codes through LDS so that 16 threads store whole 1 KiB row segments measured slower:
// 23 us against 19 us for the 25 MB talker gate_up weight.)
template <typename WT, bool E4M3>
__global__ __launch_bounds__(256) void dequant_strips_kernel(const uint8_t* __restrict__ src, int64_t n, int64_t k,
                                                             const void* __restrict__ scale, int sdt,
                                                             WT* __restrict__ w, int64_t ldw, int64_t units,
                                                             int64_t nchunks) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const SlotPos p = slot_pos(u, nchunks, kStripInt8);
  if (p.row >= n || p.col >= k) return;  // padding rows and chunks
  float s;
  if (sdt == QTTS_F32) s = ((const float*)scale)[p.row];
  else if (sdt == QTTS_BF16) s = to_f32(((const bf16_t*)scale)[p.row]);
  else s = to_f32(((const f16_t*)scale)[p.row]);
  const uint4 v = *(const uint4*)(src + u * 16);
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  float f[16];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    typedef __attribute__((ext_vector_type(4))) uint32_t u4;
    const u4 c = E4M3 ? __builtin_bit_cast(u4, e4m3x8_to_bf16x8(d[2 * i], d[2 * i + 1]))
                      : __builtin_bit_cast(u4, i8x8_to_bf16x8(d[2 * i], d[2 * i + 1]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[8 * i + 2 * j] = __uint_as_float(c[j] << 16);  // the codes, exact in bf16
      f[8 * i + 2 * j + 1] = __uint_as_float(c[j] & 0xffff0000u);
    }
  }
  WT* dst = w + p.row * ldw + p.col;
  if constexpr (sizeof(WT) == 2) {
    if (p.col + 16 <= k && ((uintptr_t)dst & 15) == 0) {
      uint32_t o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = pack2_f32<WT>(f[2 * j] * s, f[2 * j + 1] * s);
      *(uint4*)dst = make_uint4(o[0], o[1], o[2], o[3]);
      *(uint4*)(dst + 8) = make_uint4(o[4], o[5], o[6], o[7]);
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (p.col + j < k) dst[j] = from_f32<WT>(f[j] * s);
}

}  // namespace qtts

using namespace qtts;

int qtts_launch_dequant_strips(const void* qs, int codes, int64_t n, int64_t k, const void* scale, int sdt, void* w,
                               int w_dtype, int64_t ldw, hipStream_t st) {
  const int64_t units = strip_bytes(n, k, kStripInt8) / 16;
  if (units == 0) return QTTS_OK;
  const int64_t blocks = (units + 255) / 256;
  if (blocks >= ((int64_t)1 << 31)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "dequant_strips: too large");
  const int64_t nch = strip_nchunks(k, kStripInt8);
#define QTTS_DQ(WT, E)                                                                                          \
  qtts::launch(&dequant_strips_kernel<WT, E>, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)qs, n, k, \
               scale, sdt, (WT*)w, ldw, units, nch)
  const bool e4 = codes == QTTS_CODE_E4M3;
  if (w_dtype == QTTS_BF16) { if (e4) QTTS_DQ(bf16_t, true); else QTTS_DQ(bf16_t, false); }
  else if (w_dtype == QTTS_F16) { if (e4) QTTS_DQ(f16_t, true); else QTTS_DQ(f16_t, false); }
  else { if (e4) QTTS_DQ(float, true); else QTTS_DQ(float, false); }
#undef QTTS_DQ
  return qtts_check_launch("dequant_strips");
}

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
