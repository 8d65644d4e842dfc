// The strip weight layout: the [N, K] byte matrix re-tiled so that every wavefront
// load of the GEMM kernels is one contiguous, aligned 1 KiB.
//
//   strip s   = rows [16 s, 16 s + 16)          strips  = ceil(N / 16)
//   chunk c   = columns [CH c, CH c + CH)       nchunks = ceil(K / CH)
//   block(s, c) = 16 * CH bytes at ((s * nchunks) + c) * 16 * CH
//   inside a block, half h in [0, CH / 64) and lane l in [0, 64) own the 16 bytes at
//   h * 1024 + l * 16, which hold row 16 s + (l % 16), columns
//   CH c + (l / 16) * (CH / 4) + 16 h ... + 15.
//
// CH = 64 for int8 weights (one 16x16x32 bf16 MFMA pair per 16-byte lane slot) and
// CH = 128 for e4m3 weights (one 16x16x128 fp8 MFMA per two slots).  Rows past N and
// columns past K are zero.  Lane l's bytes are exactly the MFMA A-operand fragment of
// lane l (row l % 16, K group l / 16), so a wave turns one 1 KiB load into MFMA
// operands with no shuffling.
#pragma once

#include <stdint.h>

namespace qtts {

enum : int { kLayoutRowMajor = 0, kLayoutStrips = 1 };
enum : int { kStripInt8 = 0, kStripFp8 = 1 };

__host__ __device__ constexpr int strip_chunk(int kind) { return kind == kStripFp8 ? 128 : 64; }

__host__ __device__ constexpr int64_t strip_count(int64_t n) { return (n + 15) / 16; }

__host__ __device__ constexpr int64_t strip_nchunks(int64_t k, int kind) {
  return (k + strip_chunk(kind) - 1) / strip_chunk(kind);
}

__host__ __device__ constexpr int64_t strip_bytes(int64_t n, int64_t k, int kind) {
  return strip_count(n) * strip_nchunks(k, kind) * 16 * strip_chunk(kind);
}

}  // namespace qtts
