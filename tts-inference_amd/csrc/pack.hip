// Weight packers and per-token activation quantization.
//
// Load-time packers (int8, e4m3) and the run-time fp8 and int8 activation quantizers.  One
// workgroup of 256 threads owns one row: a coalesced pass finds the row's absmax,
// a second pass divides, rounds and stores.  All arithmetic is IEEE fp32 (hipcc's
// default correctly-rounded division; no fast-math), so results are bit-exact with
// the reference's torch expressions (see the oracle tests).
#include "common.h"

namespace qtts {

constexpr int kPackThreads = 256;

template <typename T>
__device__ __forceinline__ float row_absmax(const T* __restrict__ row, int64_t k, float* red) {
  float m = 0.0f;
  for (int64_t c = threadIdx.x; c < k; c += kPackThreads) m = fmaxf(m, fabsf(to_f32(row[c])));
  m = wave_max(m);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return m;
}

// quantize_weight_per_channel, qtts/quant/int8.py:45-56 (+ stored scale cast, :105).
template <typename SrcT, typename StoreT>
__global__ __launch_bounds__(kPackThreads) void pack_int8_kernel(
    const SrcT* __restrict__ src, int64_t k, int64_t ld, int8_t* __restrict__ q,
    StoreT* __restrict__ scale_out, float* __restrict__ scale_f32, int div_mode) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const SrcT* row = src + r * ld;
  float amax = row_absmax(row, k, red);
  amax = fmaxf(amax, 1e-12f);  // clamp_min(1e-12)
  const float scale = scalar_div(amax, 127.0f, div_mode);
  int8_t* qrow = q + r * k;
  for (int64_t c = threadIdx.x; c < k; c += kPackThreads) {
    float v = __builtin_rintf(to_f32(row[c]) / scale);  // round half to even
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    qrow[c] = (int8_t)(int)v;
  }
  if (threadIdx.x == 0) {
    scale_out[r] = from_f32<StoreT>(scale);
    if (scale_f32) scale_f32[r] = scale;
  }
}

// quantize_weight_fp8, qtts/quant/fp8.py:45-49.
template <typename SrcT>
__global__ __launch_bounds__(kPackThreads) void pack_fp8_kernel(
    const SrcT* __restrict__ src, int64_t k, int64_t ld, uint8_t* __restrict__ q,
    float* __restrict__ scale_out, int div_mode) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const SrcT* row = src + r * ld;
  float amax = fmaxf(row_absmax(row, k, red), 1e-12f);
  const float scale = scalar_div(amax, 448.0f, div_mode);
  uint8_t* qrow = q + r * k;
  for (int64_t c = threadIdx.x; c < k; c += kPackThreads) qrow[c] = (uint8_t)e4m3_encode(to_f32(row[c]) / scale);
  if (threadIdx.x == 0) scale_out[r] = scale;
}

// Activation half of Fp8Method.apply, qtts/quant/fp8.py:77-78.  The absmax and the
// 1e-6 clamp happen in the activation dtype (exact for max/abs; the clamp value is
// 1e-6 rounded to that dtype), then the scale is formed in fp32.
template <typename XT>
__global__ __launch_bounds__(kPackThreads) void quant_act_fp8_kernel(
    const XT* __restrict__ x, int64_t k, int64_t ld, uint8_t* __restrict__ qx,
    float* __restrict__ sx, int div_mode) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const XT* row = x + r * ld;
  const float floor_v = round_through<XT>(1e-6f);
  const float amax = fmaxf(row_absmax(row, k, red), floor_v);
  const float s = scalar_div(amax, 448.0f, div_mode);
  uint8_t* qrow = qx + r * k;
  for (int64_t c = threadIdx.x; c < k; c += kPackThreads) qrow[c] = (uint8_t)e4m3_encode(to_f32(row[c]) / s);
  if (threadIdx.x == 0) sx[r] = s;
}

// Vectorized quant_act_fp8_kernel for 16-bit activations with 16-byte aligned rows and
// k % 8 == 0: every thread loads up to V 8-element vectors of its row at once (one
// memory round trip), the row maximum goes through one LDS exchange, and the codes
// come from a correctly rounded quotient (the row's reciprocal plus one FMA
// correction) and v_cvt_pk_fp8_f32 -- the same codes as the scalar kernel.
template <typename XT, int V>
__global__ __launch_bounds__(kPackThreads) void quant_act_fp8_vec_kernel(
    const XT* __restrict__ x, int64_t k, int64_t ld, uint8_t* __restrict__ qx,
    float* __restrict__ sx, int div_mode) {
  __shared__ float red[kPackThreads / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int nv = (int)(k >> 3);
  const XT* row = x + r * ld;
  i32x4_t v[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int idx = tid + kPackThreads * j;
    v[j] = *(const i32x4_t*)(row + 8 * (int64_t)min(idx, nv - 1));  // clamped: in the row
  }
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (tid + kPackThreads * j < nv) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t pr = (uint32_t)v[j][e];
        mx = fmaxf(mx, fmaxf(fabsf(to_f32(XT{(uint16_t)pr})), fabsf(to_f32(XT{(uint16_t)(pr >> 16)}))));
      }
    }
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kPackThreads / 64; ++w) mx = fmaxf(mx, red[w]);
  const float s = scalar_div(fmaxf(mx, round_through<XT>(1e-6f)), 448.0f, div_mode);
  const float rs = 1.0f / s;
  uint8_t* qrow = qx + r * k;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int idx = tid + kPackThreads * j;
    if (idx < nv) {
      uint32_t w[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t p0 = (uint32_t)v[j][2 * h], p1 = (uint32_t)v[j][2 * h + 1];
        const uint32_t c01 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
            div_by(to_f32(XT{(uint16_t)p0}), s, rs), div_by(to_f32(XT{(uint16_t)(p0 >> 16)}), s, rs), 0, false);
        const uint32_t c23 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
            div_by(to_f32(XT{(uint16_t)p1}), s, rs), div_by(to_f32(XT{(uint16_t)(p1 >> 16)}), s, rs), 0, false);
        w[h] = (c01 & 0xffffu) | (c23 << 16);
      }
      *(uint2*)(qrow + 8 * (int64_t)idx) = make_uint2(w[0], w[1]);
    }
  }
  if (tid == 0) sx[r] = s;
}

// ---- int8 activations: Int8Method.apply, qtts/quant/int8.py:147-149 ----------------
// Everything happens in the activation dtype XT: the absmax, the 1e-6 clamp, the
// division by 127 (div_mode) and the quotient x / scale, each rounded to XT as torch
// rounds an XT tensor op; .round() is half-to-even on that XT value.  The scale is
// stored widened to fp32 (exact).  A NaN quotient (0 / 0, which the fp16 scale of a
// row with absmax below ~3.8e-6 produces, since that scale rounds to zero) stores
// code 0, what the reference's float -> int8 cast gives it.

template <typename XT>
__global__ __launch_bounds__(kPackThreads) void quant_act_int8_kernel(
    const XT* __restrict__ x, int64_t k, int64_t ld, int8_t* __restrict__ qx, float* __restrict__ sx,
    int div_mode) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const XT* row = x + r * ld;
  const float s = int8_act_scale<XT>(row_absmax(row, k, red), div_mode);
  int8_t* qrow = qx + r * k;
  for (int64_t c = threadIdx.x; c < k; c += kPackThreads) qrow[c] = (int8_t)int8_act_code<XT>(to_f32(row[c]), s);
  if (threadIdx.x == 0) sx[r] = s;
}

// Vectorized form for 16-bit activations with 16-byte aligned rows and k % 8 == 0:
// each thread holds up to V 8-element vectors of the row in registers across both
// passes, so the row is read once.
template <typename XT, int V>
__global__ __launch_bounds__(kPackThreads) void quant_act_int8_vec_kernel(
    const XT* __restrict__ x, int64_t k, int64_t ld, int8_t* __restrict__ qx, float* __restrict__ sx,
    int div_mode) {
  __shared__ float red[kPackThreads / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int nv = (int)(k >> 3);
  const XT* row = x + r * ld;
  i32x4_t v[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int idx = tid + kPackThreads * j;
    v[j] = *(const i32x4_t*)(row + 8 * (int64_t)min(idx, nv - 1));  // clamped: in the row
  }
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (tid + kPackThreads * j < nv) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t pr = (uint32_t)v[j][e];
        mx = fmaxf(mx, fmaxf(fabsf(to_f32(XT{(uint16_t)pr})), fabsf(to_f32(XT{(uint16_t)(pr >> 16)}))));
      }
    }
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kPackThreads / 64; ++w) mx = fmaxf(mx, red[w]);
  const float s = int8_act_scale<XT>(mx, div_mode);
  int8_t* qrow = qx + r * k;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int idx = tid + kPackThreads * j;
    if (idx < nv) {
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t pr = (uint32_t)v[j][e];
        const uint32_t c0 = (uint32_t)int8_act_code<XT>(to_f32(XT{(uint16_t)pr}), s) & 0xffu;
        const uint32_t c1 = (uint32_t)int8_act_code<XT>(to_f32(XT{(uint16_t)(pr >> 16)}), s) & 0xffu;
        w[e >> 1] |= (c0 | (c1 << 8)) << (16 * (e & 1));
      }
      *(uint2*)(qrow + 8 * (int64_t)idx) = make_uint2(w[0], w[1]);
    }
  }
  if (tid == 0) sx[r] = s;
}

}  // namespace qtts

using namespace qtts;

int qtts_launch_pack_int8(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld, int8_t* q,
                          void* scale_out, int scale_dtype, float* scale_f32, int div_mode, hipStream_t st) {
  dim3 grid((unsigned)n), block(kPackThreads);
#define QTTS_PACK_I8(ST, DT)                                                                         \
  do {                                                                                               \
    if (scale_dtype == QTTS_F32)                                                                     \
      qtts::launch(&pack_int8_kernel<ST, float>, dim3(grid), dim3(block), 0, st, (const ST*)src, k, ld, q, (float*)scale_out, \
                                                          scale_f32, div_mode);                      \
    else if (scale_dtype == QTTS_BF16)                                                               \
      qtts::launch(&pack_int8_kernel<ST, bf16_t>, dim3(grid), dim3(block), 0, st, (const ST*)src, k, ld, q, (bf16_t*)scale_out, \
                                                           scale_f32, div_mode);                     \
    else                                                                                             \
      qtts::launch(&pack_int8_kernel<ST, f16_t>, dim3(grid), dim3(block), 0, st, (const ST*)src, k, ld, q, (f16_t*)scale_out, \
                                                          scale_f32, div_mode);                      \
  } while (0)
  if (src_dtype == QTTS_F32) QTTS_PACK_I8(float, 0);
  else if (src_dtype == QTTS_BF16) QTTS_PACK_I8(bf16_t, 1);
  else QTTS_PACK_I8(f16_t, 2);
#undef QTTS_PACK_I8
  return qtts_check_launch("pack_int8_rowwise");
}

int qtts_launch_pack_fp8(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld, uint8_t* q,
                         float* scale, int div_mode, hipStream_t st) {
  dim3 grid((unsigned)n), block(kPackThreads);
  if (src_dtype == QTTS_F32) qtts::launch(&pack_fp8_kernel<float>, dim3(grid), dim3(block), 0, st, (const float*)src, k, ld, q, scale, div_mode);
  else if (src_dtype == QTTS_BF16) qtts::launch(&pack_fp8_kernel<bf16_t>, dim3(grid), dim3(block), 0, st, (const bf16_t*)src, k, ld, q, scale, div_mode);
  else qtts::launch(&pack_fp8_kernel<f16_t>, dim3(grid), dim3(block), 0, st, (const f16_t*)src, k, ld, q, scale, div_mode);
  return qtts_check_launch("pack_fp8_e4m3_rowwise");
}

int qtts_launch_quant_act_fp8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ld, uint8_t* qx,
                              float* sx, int div_mode, hipStream_t st) {
  dim3 grid((unsigned)m), block(kPackThreads);
  const int64_t nv = k / 8;
  if (x_dtype != QTTS_F32 && k % 8 == 0 && k > 0 && (uintptr_t)x % 16 == 0 && ld % 8 == 0 && (uintptr_t)qx % 8 == 0 &&
      nv <= 4 * kPackThreads) {
#define QTTS_QA_VEC(XT)                                                                                          \
  do {                                                                                                           \
    if (nv <= kPackThreads)                                                                                      \
      qtts::launch(&quant_act_fp8_vec_kernel<XT, 1>, grid, block, 0, st, (const XT*)x, k, ld, qx, sx, div_mode); \
    else if (nv <= 2 * kPackThreads)                                                                             \
      qtts::launch(&quant_act_fp8_vec_kernel<XT, 2>, grid, block, 0, st, (const XT*)x, k, ld, qx, sx, div_mode); \
    else                                                                                                         \
      qtts::launch(&quant_act_fp8_vec_kernel<XT, 4>, grid, block, 0, st, (const XT*)x, k, ld, qx, sx, div_mode); \
  } while (0)
    if (x_dtype == QTTS_BF16) QTTS_QA_VEC(bf16_t);
    else QTTS_QA_VEC(f16_t);
#undef QTTS_QA_VEC
    return qtts_check_launch("quant_act_fp8_rows");
  }
  if (x_dtype == QTTS_F32) qtts::launch(&quant_act_fp8_kernel<float>, dim3(grid), dim3(block), 0, st, (const float*)x, k, ld, qx, sx, div_mode);
  else if (x_dtype == QTTS_BF16) qtts::launch(&quant_act_fp8_kernel<bf16_t>, dim3(grid), dim3(block), 0, st, (const bf16_t*)x, k, ld, qx, sx, div_mode);
  else qtts::launch(&quant_act_fp8_kernel<f16_t>, dim3(grid), dim3(block), 0, st, (const f16_t*)x, k, ld, qx, sx, div_mode);
  return qtts_check_launch("quant_act_fp8_rows");
}

int qtts_launch_quant_act_int8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ld, int8_t* qx,
                               float* sx, int div_mode, hipStream_t st) {
  dim3 grid((unsigned)m), block(kPackThreads);
  const int64_t nv = k / 8;
  if (x_dtype != QTTS_F32 && k % 8 == 0 && k > 0 && (uintptr_t)x % 16 == 0 && ld % 8 == 0 && (uintptr_t)qx % 8 == 0 &&
      nv <= 4 * kPackThreads) {
#define QTTS_QA8_VEC(XT)                                                                                          \
  do {                                                                                                            \
    if (nv <= kPackThreads)                                                                                       \
      qtts::launch(&quant_act_int8_vec_kernel<XT, 1>, grid, block, 0, st, (const XT*)x, k, ld, qx, sx, div_mode); \
    else if (nv <= 2 * kPackThreads)                                                                              \
      qtts::launch(&quant_act_int8_vec_kernel<XT, 2>, grid, block, 0, st, (const XT*)x, k, ld, qx, sx, div_mode); \
    else                                                                                                          \
      qtts::launch(&quant_act_int8_vec_kernel<XT, 4>, grid, block, 0, st, (const XT*)x, k, ld, qx, sx, div_mode); \
  } while (0)
    if (x_dtype == QTTS_BF16) QTTS_QA8_VEC(bf16_t);
    else QTTS_QA8_VEC(f16_t);
#undef QTTS_QA8_VEC
    return qtts_check_launch("quant_act_int8_rows");
  }
  if (x_dtype == QTTS_F32)
    qtts::launch(&quant_act_int8_kernel<float>, grid, block, 0, st, (const float*)x, k, ld, qx, sx, div_mode);
  else if (x_dtype == QTTS_BF16)
    qtts::launch(&quant_act_int8_kernel<bf16_t>, grid, block, 0, st, (const bf16_t*)x, k, ld, qx, sx, div_mode);
  else
    qtts::launch(&quant_act_int8_kernel<f16_t>, grid, block, 0, st, (const f16_t*)x, k, ld, qx, sx, div_mode);
  return qtts_check_launch("quant_act_int8_rows");
}
