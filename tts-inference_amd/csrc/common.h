// Shared device helpers for the gfx950 quantized-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qtts_amd.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(8))) int i32x8_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;

namespace qtts {

// Workspace layout shared by every op: a fixed block of split-K counters first
// (one 32-bit counter per output tile, reset to zero by the workgroup that
// consumes it), then op-specific scratch.  The counter block does not depend on
// the shape, so one call's scratch can never overlap another call's counters.
constexpr int64_t kCounterBytes = 65536;
constexpr int64_t kMaxSplitTiles = kCounterBytes / 4;

__host__ __device__ constexpr int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// A weight block of 16 bytes, loaded as the caller's weight policy asks: NT for weights
// that a step reads once and that cannot stay cached between steps (`global_load_dwordx4
// ... nt`, so the stream neither evicts the activation rows and scales nor the Infinity
// Cache lines of weights that are reused); plain loads for weights small enough to stay
// resident (QTTS_ALGO_STREAM in include/qtts_amd.h picks NT per call).  The decode kernels
// take NT as a template parameter: a run-time branch around the loads joins before their
// first use, where the compiler's wait counting loses the per-load order and waits for every
// weight block before the first MFMA (measured 8% slower on the talker stack).
template <bool NT> __device__ __forceinline__ i32x4_t load_weight(const void* p) {
  if constexpr (NT) return __builtin_nontemporal_load((const i32x4_t*)p);
  else return *(const i32x4_t*)p;
}

// Reset a split-K counter: an agent-scope atomic store (written through to the
// coherence point), so the next kernel's atomics see zero from any XCD.
__device__ __forceinline__ void reset_counter(unsigned* c) {
  __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- scalar element access by dtype code ------------------------------------------

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return __uint_as_float((uint32_t)v.bits << 16); }
__device__ __forceinline__ float to_f32(f16_t v) {
  _Float16 h;
  __builtin_memcpy(&h, &v.bits, 2);
  return (float)h;
}

// fp32 -> 16-bit float, round to nearest even, by the hardware conversions
// (v_cvt_pk_bf16_f32 on gfx950, v_cvt_f16_f32): branch-free, NaN becomes a quiet NaN.
// The fp16 conversion is written as the instruction itself: left to the compiler, a
// conversion of a product or an fma result is folded into v_fma_mixlo_f16, which rounds
// the exact result once (and turns -0 * s into +0), where fp32 arithmetic followed by
// the conversion -- torch's order -- rounds twice.
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
  return bf16_t{__builtin_bit_cast(uint16_t, (__bf16)v)};
}
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float v) {
  uint32_t h;
  asm("v_cvt_f16_f32 %0, %1" : "=v"(h) : "v"(v));
  return f16_t{(uint16_t)h};
}

// Two values rounded to T and packed low-first into 32 bits (one conversion for bf16).
template <typename T> __device__ __forceinline__ uint32_t pack2_f32(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2_f32<bf16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack2_f32<f16_t>(float a, float b) {
  return (uint32_t)from_f32<f16_t>(a).bits | ((uint32_t)from_f32<f16_t>(b).bits << 16);
}

// Round to T and widen back (identity for fp32).
template <typename T> __device__ __forceinline__ float round_through(float v) { return to_f32(from_f32<T>(v)); }

// acc + lo^2 + hi^2 of a packed pair of 16-bit floats in one v_dot2c_f32_{bf16,f16} (the
// products are exact in fp32).
template <typename XT> __device__ __forceinline__ float sq2_acc(uint32_t p, float acc) {
  typedef __attribute__((ext_vector_type(2))) _Float16 h2_t;
  if constexpr (std::is_same<XT, bf16_t>::value)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, p), __builtin_bit_cast(bf16x2_t, p), acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, p), __builtin_bit_cast(h2_t, p), acc, false);
}

// ---- int8 -> 16-bit float vectors for the MFMA operands ---------------------------
// Every int8 value is exact in bf16 and fp16.  Each byte goes through one
// v_cvt_f32_i32 with an SDWA sign-extended byte select (written out: the compiler
// shifts bytes 1 and 3 first, an extra instruction each), then pairs are rounded
// into bf16 by one v_cvt_pk_bf16_f32 (exact: the floats are small integers).

template <int B> __device__ __forceinline__ float sbyte_to_f32(uint32_t w) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
  return r;
}

__device__ __forceinline__ uint32_t sbytes_to_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

__device__ __forceinline__ bf16x8_t i8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  typedef __attribute__((ext_vector_type(4))) uint32_t u4;
  const u4 v = {sbytes_to_bf16x2(sbyte_to_f32<0>(lo), sbyte_to_f32<1>(lo)),
                sbytes_to_bf16x2(sbyte_to_f32<2>(lo), sbyte_to_f32<3>(lo)),
                sbytes_to_bf16x2(sbyte_to_f32<0>(hi), sbyte_to_f32<1>(hi)),
                sbytes_to_bf16x2(sbyte_to_f32<2>(hi), sbyte_to_f32<3>(hi))};
  return __builtin_bit_cast(bf16x8_t, v);
}

// Exact, by the exponent trick: code c becomes the fp16 bit pattern 0x6400 | (c + 128), i.e.
// 1024 + 128 + c (the ulp at 1024 is 1), then one v_pk_add_f16 of -1152 per two codes leaves
// c (+0 for c = 0, as the integer conversion gives).  Five instructions per four codes.
__device__ __forceinline__ f16x8_t i8x8_to_f16x8(uint32_t lo, uint32_t hi) {
  typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
  const uint32_t tl = lo ^ 0x80808080u, th = hi ^ 0x80808080u;  // c + 128 in each byte
  const f16x2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  // v_perm_b32: bytes 0-3 from the second operand, 4-7 from the first (0x64 each)
  auto pair = [&](uint32_t t, uint32_t sel) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, t, sel)) + off);
  };
  typedef __attribute__((ext_vector_type(4))) uint32_t u4;
  const u4 v = {pair(tl, 0x04010400u), pair(tl, 0x04030402u), pair(th, 0x04010400u), pair(th, 0x04030402u)};
  return __builtin_bit_cast(f16x8_t, v);
}

// ---- OCP e4m3 -> 16-bit float vectors (fp8 weight-only GEMM) ---------------------
// Every e4m3 value (3 mantissa bits, exponents 2^-9 .. 2^8) is exact in bf16 and
// fp16.  v_cvt_scalef32_pk_{bf16,f16}_fp8 converts two codes per instruction; the
// unit scale leaves the values unchanged.

__device__ __forceinline__ bf16x8_t e4m3x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  typedef __attribute__((ext_vector_type(4))) uint32_t u4;
  const u4 v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true))};
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f16x8_t e4m3x8_to_f16x8(uint32_t lo, uint32_t hi) {
  typedef __attribute__((ext_vector_type(4))) uint32_t u4;
  const u4 v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true))};
  return __builtin_bit_cast(f16x8_t, v);
}

// 16-bit activation element types mapped to their MFMA operand vector.
template <typename XT> struct mfma16;
template <> struct mfma16<bf16_t> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ vec from_i8(uint32_t lo, uint32_t hi) { return i8x8_to_bf16x8(lo, hi); }
  static __device__ __forceinline__ vec from_e4m3(uint32_t lo, uint32_t hi) { return e4m3x8_to_bf16x8(lo, hi); }
  static __device__ __forceinline__ f32x4_t mma(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct mfma16<f16_t> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ vec from_i8(uint32_t lo, uint32_t hi) { return i8x8_to_f16x8(lo, hi); }
  static __device__ __forceinline__ vec from_e4m3(uint32_t lo, uint32_t hi) { return e4m3x8_to_f16x8(lo, hi); }
  static __device__ __forceinline__ f32x4_t mma(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Weight codes (8 per call: two packed dwords) to the MFMA operand: int8, or OCP
// e4m3 for the fp8 weight-only kernels (F8W).
template <bool F8W, typename XT> __device__ __forceinline__ typename mfma16<XT>::vec wcvt(uint32_t lo, uint32_t hi) {
  if constexpr (F8W) return mfma16<XT>::from_e4m3(lo, hi);
  else return mfma16<XT>::from_i8(lo, hi);
}

// fp8 x fp8 (OCP e4m3 on gfx950) 16x16x128 MFMA, unit block scales (E8M0 127 = 2^0).
__device__ __forceinline__ f32x4_t mma_fp8_16x16x128(i32x8_t a, i32x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// int8 x int8 -> int32 16x16x64 MFMA.  Integer accumulation is exact (and wraps
// modulo 2^32 past |sum| >= 2^31, which needs K > 133,000 at +-127 codes), so any
// K order and any split give the same result.
__device__ __forceinline__ i32x4_t mma_i8_16x16x64(i32x4_t a, i32x4_t b, i32x4_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// The fp32 epilogue of Int8Method.apply (qtts/quant/int8.py:157-160): the int32
// accumulator converted to fp32, times the token scale, times the channel scale,
// plus the bias, each step rounded on its own (the reference runs them as separate
// elementwise kernels, so nothing may fuse into an FMA here).
__device__ __forceinline__ float int8_epilogue(int acc, float sx, float sw, float bias, bool has_bias) {
#pragma clang fp contract(off)
  float v = (float)acc * sx;
  v = v * sw;
  return has_bias ? v + bias : v;
}

// GatedMLP's activation, qtts/layers/activation.py:147, `F.silu(gate) * up` on tensors
// of dtype T: silu in fp32 with torch's formula x / (1 + exp(-x)), rounded to T; the
// product in fp32, rounded to T.
template <typename T> __device__ __forceinline__ float silu_mul(float g, float u) {
  const float s = round_through<T>(g / (1.0f + expf(-g)));
  return round_through<T>(s * u);
}

// Eight 16-bit values of type T packed in an i32x4: silu_mul element by element.
template <typename T> __device__ __forceinline__ i32x4_t silu_mul8(i32x4_t g, i32x4_t u) {
  i32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t gp = (uint32_t)g[i], up = (uint32_t)u[i];
    const float lo = silu_mul<T>(to_f32(T{(uint16_t)gp}), to_f32(T{(uint16_t)up}));
    const float hi = silu_mul<T>(to_f32(T{(uint16_t)(gp >> 16)}), to_f32(T{(uint16_t)(up >> 16)}));
    r[i] = (int)pack2_f32<T>(lo, hi);
  }
  return r;
}

// ---- OCP e4m3fn encode (round to nearest even, non-saturating like torch's cast) ---

__device__ __forceinline__ uint32_t e4m3_encode(float f) {
  uint32_t u = __float_as_uint(f), s = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return s | 0x7fu;
  if (a < 0x3c800000u) {  // below 2^-6: subnormal grid of 2^-9
    float v = __uint_as_float(a) * 512.0f;
    return s | (uint32_t)__builtin_rintf(v);
  }
  int32_t e = (int32_t)(a >> 23) - 120;
  uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  uint32_t r = mant >> 20, rem = mant & 0xfffffu;
  r += (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ? 1u : 0u;
  if (r == 16u) { r = 8u; e++; }
  uint32_t code = ((uint32_t)e << 3) | (r & 7u);
  return s | ((e > 15 || code >= 0x7fu) ? 0x7fu : code);
}

// x / s, correctly rounded, from rs = RN(1/s): q0 = RN(x rs) is within an ulp of the
// quotient, the residual x - q0 s is exact in one FMA, and one FMA step with rs
// rounds the corrected quotient (Markstein's theorem).  An exact q0 (zero residual)
// is returned as is, which keeps the sign of a zero quotient.
__device__ __forceinline__ float div_by(float x, float s, float rs) {
  const float q0 = x * rs;
  const float r = __builtin_fmaf(-q0, s, x);
  return r == 0.0f ? q0 : __builtin_fmaf(r, rs, q0);
}

// `num / c` with the reference's scalar-division semantics (qtts_div_mode).
__device__ __forceinline__ float scalar_div(float num, float c, int div_mode) {
  return div_mode == QTTS_DIV_DEVICE ? num * (1.0f / c) : num / c;
}

// Per-token int8 activation quantization (qtts/quant/int8.py:146-149), every step in
// the activation dtype XT as the reference computes it on an XT tensor:
// s = XT(max(amax, XT(1e-6)) / 127), code = clamp(rint(XT(x / s)), -127, 127), and a
// NaN quotient (0 / 0 when an fp16 scale underflows to zero) gives code 0.
template <typename XT> __device__ __forceinline__ float int8_act_scale(float amax, int div_mode) {
  return round_through<XT>(scalar_div(fmaxf(amax, round_through<XT>(1e-6f)), 127.0f, div_mode));
}

template <typename XT> __device__ __forceinline__ int int8_act_code(float x, float s) {
  const float v = __builtin_rintf(round_through<XT>(x / s));
  return v != v ? 0 : (int)fminf(fmaxf(v, -127.0f), 127.0f);
}

// ---- wave64 reductions ----------------------------------------------------------------

template <int CTRL> __device__ __forceinline__ float dpp_max(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                        false)));
}

// Max over each aligned group of G lanes (16, 32 or 64), in every lane of the group:
// within rows of 16 by DPP (swap neighbours, swap pairs, mirror half rows, mirror rows),
// across rows by lane swizzles.
template <int G> __device__ __forceinline__ float group_max(float v) {
  v = dpp_max<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_max<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_max<0x141>(v);  // row_half_mirror
  v = dpp_max<0x140>(v);  // row_mirror
  if constexpr (G >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}


__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// v + v of the lane DPP control CTRL names (a VALU operation, no LDS round trip).
template <int CTRL> __device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, uniform result, without the LDS permutes __shfl_xor compiles to:
// within each row of 16 lanes by DPP (swap neighbours, swap pairs, mirror each half row,
// mirror the row), then the four row sums read out lane by lane, ((r0 + r1) + (r2 + r3)).
__device__ __forceinline__ float wave_sum_rows(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

}  // namespace qtts

// ---- host-side error plumbing (abi.hip) -------------------------------------------------

int qtts_set_error(int status, const char* fmt, ...);
int qtts_check_launch(const char* what);

// ---- kernel launches and the kernel timer (abi.hip) -------------------------------------
// Every kernel of the library is launched through qtts::launch.  While the kernel
// timer is armed (qtts_kernel_timer_begin), each launch outside stream capture
// takes a start/stop event pair that hipExtLaunchKernel binds to the kernel's own
// dispatch, so the elapsed time is the kernel's duration, without launch gaps or
// the cost of separate event records.

#include <hip/hip_ext.h>

bool qtts_timer_slot(hipStream_t st, hipEvent_t* start, hipEvent_t* stop);

namespace qtts {

template <typename... Params, typename... Args>
inline void launch(void (*kernel)(Params...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
                   Args... args) {
  static_assert(sizeof...(Params) == sizeof...(Args), "kernel argument count");
  hipEvent_t a = nullptr, b = nullptr;
  qtts_timer_slot(st, &a, &b);
  hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, a, b, 0u, static_cast<Params>(args)...);
}

}  // namespace qtts

// ---- the weight policy of the call in progress (abi.hip) ----------------------------------
// A public entry point whose `algo` carries QTTS_ALGO_STREAM holds a WeightPolicy for the
// call; the decode launchers on the same thread read it with weight_policy() and launch the
// kernels' NT instantiation where one is built.  Launches happen on the calling thread, inside
// the entry point, so a thread-local value is exactly the call's.

namespace qtts {

extern thread_local int g_weight_policy;

inline bool weight_policy() { return g_weight_policy != 0; }

class WeightPolicy {
 public:
  // Takes QTTS_ALGO_STREAM out of `algo` (the kernels' choice never sees it) and sets the
  // policy until the scope ends.
  explicit WeightPolicy(int& algo) : saved_(g_weight_policy) {
    g_weight_policy = (algo & QTTS_ALGO_STREAM) ? 1 : 0;
    algo &= ~QTTS_ALGO_STREAM;
  }
  ~WeightPolicy() { g_weight_policy = saved_; }
  WeightPolicy(const WeightPolicy&) = delete;
  WeightPolicy& operator=(const WeightPolicy&) = delete;

 private:
  int saved_;
};

// f(std::true_type{}) when the NT instantiation is built (NT_BUILT) and the caller's weight
// policy streams, else f(std::false_type{}); f launches its kernel's NT or plain instantiation
// (a generic lambda: the NT one is instantiated only where NT_BUILT).
template <bool NT_BUILT, typename F> inline void launch_by_policy(F&& f) {
  if constexpr (NT_BUILT) {
    if (weight_policy()) {
      f(std::true_type{});
      return;
    }
  }
  f(std::false_type{});
}

}  // namespace qtts
