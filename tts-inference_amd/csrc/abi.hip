// C ABI entry points (include/qtts_amd.h): argument checks, device gating, error
// strings and dispatch to the kernel launchers in pack.hip, w8a16.hip, fp8.hip and
// w8a8_int8.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"
#include "layout.h"
#include "qtts_amd.h"

// Launchers implemented next to their kernels.
int qtts_launch_pack_int8(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld, int8_t* q,
                          void* scale_out, int scale_dtype, float* scale_f32, int div_mode, hipStream_t st);
int qtts_launch_pack_fp8(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld, uint8_t* q, float* scale,
                         int div_mode, hipStream_t st);
int qtts_launch_quant_act_fp8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ld, uint8_t* qx, float* sx,
                              int div_mode, hipStream_t st);
int qtts_launch_w8a16(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n,
                      int64_t ldq, int layout, const void* scale, int scale_dtype, const void* bias, void* y,
                      int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st);
int64_t qtts_w8a16_ws_bytes(int64_t m, int64_t n, int64_t k, int algo);
int qtts_launch_fp8_gemm(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qw,
                         int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias, void* y,
                         int out_dtype, int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st);
int qtts_launch_to_strips(const void* src, int64_t n, int64_t k, int64_t ld, void* dst, int kind, hipStream_t st);
int qtts_launch_from_strips(const void* src, int64_t n, int64_t k, void* dst, int64_t ld, int kind, hipStream_t st);
int qtts_launch_dequant_strips(const void* qs, int codes, int64_t n, int64_t k, const void* scale, int sdt, void* w,
                               int w_dtype, int64_t ldw, hipStream_t st);
int64_t qtts_fp8_gemm_ws_bytes(int64_t m, int64_t n, int64_t k, int algo);
int qtts_fp8_fused_ok(int64_t m, int64_t n, int64_t k, int waves);
int qtts_launch_quant_act_int8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ld, int8_t* qx, float* sx,
                               int div_mode, hipStream_t st);
int qtts_launch_int8_gemm(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const int8_t* qw,
                          int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias, void* y,
                          int out_dtype, int64_t ldy, int algo, void* ws, int64_t ws_bytes, hipStream_t st);
int64_t qtts_int8_gemm_ws_bytes(int64_t m, int64_t n, int64_t k, int algo);
int64_t qtts_fp8w_ws_bytes(int64_t m, int64_t n, int64_t k, int algo);
int qtts_launch_fp8w(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n,
                     const float* scale, const void* bias, void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes,
                     hipStream_t st);
int qtts_launch_silu_mul(const void* gu, int x_dtype, int64_t m, int64_t k, int64_t ld, void* h, int64_t ldh,
                         hipStream_t st);
int64_t qtts_w8a16_silu_ws_bytes(int64_t m, int64_t n, int64_t k, int algo, int x_dtype);
int qtts_launch_w8a16_silu(const void* gu, int x_dtype, int64_t m, int64_t k, int64_t ld, const int8_t* qs, int64_t n,
                           const void* scale, int sdt, const void* bias, void* y, int64_t ldy, int algo, void* ws,
                           int64_t ws_bytes, hipStream_t st);
int qtts_launch_rms_norm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* w, float eps,
                         void* y, int64_t ldy, hipStream_t st);
int qtts_launch_w8a16_gate_up_silu(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int pro,
                                   const void* nw, float eps, const int8_t* qs, int64_t n, const void* scale, int sdt,
                                   const void* bias, void* act, int64_t ldact, int algo, void* ws, int64_t ws_bytes,
                                   hipStream_t st);
int64_t qtts_w8a16_fused_ws_bytes(int64_t m, int64_t n, int64_t k, int algo, int x_dtype);
int qtts_launch_w8a16_fused(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int pro, const void* nw,
                            float eps, const int8_t* qs, int64_t n, const void* scale, int sdt, const void* bias,
                            const void* res, int64_t ldr, void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes,
                            hipStream_t st);
int qtts_launch_fp8_linear_fused(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qws,
                                 int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode,
                                 int waves, hipStream_t st);
int qtts_int8_fused_ok(int64_t m, int64_t n, int64_t k, int waves);
int qtts_launch_int8_linear_fused(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qws,
                                  int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode,
                                  int waves, hipStream_t st);

static thread_local char g_last_error[512] = "";

// The weight policy of the entry point running on this thread (common.h: WeightPolicy).
thread_local int qtts::g_weight_policy = 0;

int qtts_set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int qtts_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return qtts_set_error(QTTS_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return QTTS_OK;
}

// ---- kernel timer -----------------------------------------------------------------------
// Armed by qtts_kernel_timer_begin with a fixed pool of event pairs; qtts::launch takes
// the next pair for each launch that is not being captured into a graph.

namespace {
std::mutex g_timer_mu;
std::atomic<bool> g_timer_armed{false};
std::vector<hipEvent_t> g_timer_events;  // start0, stop0, start1, stop1, ...
size_t g_timer_used = 0;
int64_t g_timer_untimed = 0;

void timer_release() {
  for (hipEvent_t e : g_timer_events) (void)hipEventDestroy(e);
  g_timer_events.clear();
  g_timer_used = 0;
}
}  // namespace

bool qtts_timer_slot(hipStream_t st, hipEvent_t* start, hipEvent_t* stop) {
  if (!g_timer_armed.load(std::memory_order_acquire)) return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (cs != hipStreamCaptureStatusNone) return false;
  std::lock_guard<std::mutex> lock(g_timer_mu);
  if (!g_timer_armed.load(std::memory_order_relaxed)) return false;
  if (g_timer_used + 2 > g_timer_events.size()) {
    g_timer_untimed++;
    return false;
  }
  *start = g_timer_events[g_timer_used];
  *stop = g_timer_events[g_timer_used + 1];
  g_timer_used += 2;
  return true;
}

// ---- device gating: gfx950 only ---------------------------------------------------------

namespace {

constexpr int kMaxDevices = 64;
std::atomic<int> g_dev_state[kMaxDevices];  // 0 unknown, 1 supported, 2 unsupported

bool dtype_ok(int d) { return d == QTTS_F32 || d == QTTS_BF16 || d == QTTS_F16; }
int64_t dtype_size(int d) { return d == QTTS_F32 ? 4 : 2; }
bool div_ok(int d) { return d == QTTS_DIV_DEVICE || d == QTTS_DIV_IEEE; }
bool algo_ok(int a) {
  const int f = a & 0xff;
  return f == QTTS_ALGO_AUTO || f == QTTS_ALGO_SKINNY || f == QTTS_ALGO_TILE;
}
// The families of the W8A16 strip GEMM: the others plus the row-split skinny kernels.
bool algo_ok_rows(int a) {
  const int f = a & 0xff;
  return algo_ok(a) || f == QTTS_ALGO_SKINNY_HALF || f == QTTS_ALGO_SKINNY_QUARTER;
}
int64_t al256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// Whether the byte spans of two [rows, cols] matrices (row strides lda, ldb, elements
// of esz bytes) intersect.
bool ranges_overlap(const void* a, int64_t rows_a, int64_t lda, const void* b, int64_t rows_b, int64_t ldb,
                    int64_t cols, int64_t esz) {
  const uintptr_t a0 = (uintptr_t)a, a1 = a0 + (uintptr_t)(((rows_a - 1) * lda + cols) * esz);
  const uintptr_t b0 = (uintptr_t)b, b1 = b0 + (uintptr_t)(((rows_b - 1) * ldb + cols) * esz);
  return a0 < b1 && b0 < a1;
}

// Floor division for a positive divisor.
int64_t floor_div(int64_t a, int64_t d) { return a >= 0 ? a / d : -((-a + d - 1) / d); }

// Whether an [rows_a, cols_a] matrix at a (row stride lda, elements of esz_a bytes) and an
// [rows_b, cols_b] matrix at b (row stride ldb, elements of esz_b bytes) share a byte.  Row by
// row: two column blocks of one buffer whose rows interleave (x = buf[:, :k], y = buf[:, k:])
// share none.  Row i of a covers [a + i * La, a + i * La + Ca) (La = lda * esz_a, Ca = cols_a *
// esz_a), likewise for b; for each row i of a, the rows j of b that meet it satisfy
// j * Lb in (a + i * La - b - Cb, a + i * La - b + Ca).  The loop runs over a's rows once the
// whole spans are known to intersect; more than 2^22 rows are taken to overlap.
bool spans_overlap(const void* a, int64_t rows_a, int64_t lda, int64_t cols_a, int64_t esz_a, const void* b,
                   int64_t rows_b, int64_t ldb, int64_t cols_b, int64_t esz_b) {
  if (rows_a <= 0 || cols_a <= 0 || rows_b <= 0 || cols_b <= 0) return false;
  const int64_t La = lda * esz_a, Ca = cols_a * esz_a, Lb = ldb * esz_b, Cb = cols_b * esz_b;
  const uintptr_t a0 = (uintptr_t)a, a1 = a0 + (uintptr_t)((rows_a - 1) * La + Ca);
  const uintptr_t b0 = (uintptr_t)b, b1 = b0 + (uintptr_t)((rows_b - 1) * Lb + Cb);
  if (!(a0 < b1 && b0 < a1)) return false;
  if (rows_a > (1 << 22) || La <= 0 || Lb <= 0) return true;
  const int64_t d = (int64_t)(a0 - b0);  // a - b, bytes (the spans intersect, so this is small)
  for (int64_t i = 0; i < rows_a; ++i) {
    const int64_t lo = d + i * La - Cb, hi = d + i * La + Ca;  // open interval for j * Lb
    const int64_t j0 = std::max<int64_t>(floor_div(lo, Lb) + 1, 0);
    if (j0 < rows_b && j0 * Lb < hi) return true;
  }
  return false;
}

// Workspace of the one-call linears: the GEMM's own part (its split-K counter block
// always reserved, so the quantized activations never land on counters that later
// calls expect at zero), then the activation codes and their scales.
int64_t linear_ws(int64_t gemm_ws, int64_t m, int64_t k) {
  return al256(std::max<int64_t>(gemm_ws, qtts::kCounterBytes)) + al256(m * k) + al256(m * 4);
}

int current_device_check() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return qtts_set_error(QTTS_ERR_UNSUPPORTED, "no HIP device: %s", hipGetErrorString(e));
  if (qtts_device_supported(dev) != 1)
    return qtts_set_error(QTTS_ERR_UNSUPPORTED, "device %d is not a gfx950 (MI355X-class) GPU", dev);
  return QTTS_OK;
}

#define QTTS_REQUIRE(cond, ...) \
  do {                          \
    if (!(cond)) return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define QTTS_TRY(expr)               \
  do {                               \
    int _s = (expr);                 \
    if (_s != QTTS_OK) return _s;    \
  } while (0)

}  // namespace

extern "C" {

int qtts_abi_version(void) { return QTTS_ABI_VERSION; }

const char* qtts_last_error(void) { return g_last_error; }

int qtts_device_supported(int device) {
  if (device < 0 || device >= kMaxDevices) return 0;
  int s = g_dev_state[device].load(std::memory_order_acquire);
  if (s == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    s = (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : 2;
    g_dev_state[device].store(s, std::memory_order_release);
  }
  return s == 1 ? 1 : 0;
}

int64_t qtts_workspace_bytes(int op, int64_t m, int64_t n, int64_t k, int algo) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  const bool rows_ok = op == QTTS_OP_W8A16 || op == QTTS_OP_W8A16_FUSED || op == QTTS_OP_W8A16_SILU;
  // sizes past 2^31 are rejected as every entry point rejects them (and m * k stays in range)
  if (m < 0 || n < 0 || k < 0 || m >= (1ll << 31) || n >= (1ll << 31) || k >= (1ll << 31) ||
      !(rows_ok ? algo_ok_rows(algo) : algo_ok(algo)))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "bad workspace query");
  if (m == 0 || n == 0) return 0;
  switch (op) {
    case QTTS_OP_W8A16: return qtts_w8a16_ws_bytes(m, n, k, algo);
    case QTTS_OP_W8A8_FP8: return qtts_fp8_gemm_ws_bytes(m, n, k, algo);
    case QTTS_OP_FP8_LINEAR: return linear_ws(qtts_fp8_gemm_ws_bytes(m, n, k, algo), m, k);
    case QTTS_OP_W8A8_INT8: return qtts_int8_gemm_ws_bytes(m, n, k, algo);
    case QTTS_OP_INT8_LINEAR: return linear_ws(qtts_int8_gemm_ws_bytes(m, n, k, algo), m, k);
    case QTTS_OP_FP8W: return qtts_fp8w_ws_bytes(m, n, k, algo);
    case QTTS_OP_W8A16_SILU: return qtts_w8a16_silu_ws_bytes(m, n, k, algo, QTTS_BF16);
    case QTTS_OP_W8A16_FUSED: return qtts_w8a16_fused_ws_bytes(m, n, k, algo, QTTS_BF16);
    default: return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "unknown op %d", op);
  }
}

int qtts_pack_int8_rowwise(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld_src, int8_t* q_out,
                           void* scale_out, int scale_dtype, float* scale_f32_out, int div_mode, void* stream) {
  QTTS_REQUIRE(n >= 0 && k >= 0, "pack_int8_rowwise: negative size (n=%lld, k=%lld)", (long long)n, (long long)k);
  QTTS_REQUIRE(dtype_ok(src_dtype) && dtype_ok(scale_dtype), "pack_int8_rowwise: bad dtype code");
  QTTS_REQUIRE(div_ok(div_mode), "pack_int8_rowwise: bad div_mode %d", div_mode);
  QTTS_REQUIRE(ld_src >= k, "pack_int8_rowwise: ld_src %lld < k %lld", (long long)ld_src, (long long)k);
  QTTS_REQUIRE(n < (1ll << 31), "pack_int8_rowwise: n too large");
  if (n == 0) return QTTS_OK;
  QTTS_REQUIRE(scale_out && (k == 0 || (src && q_out)), "pack_int8_rowwise: null pointer");
  QTTS_TRY(current_device_check());
  return qtts_launch_pack_int8(src, src_dtype, n, k, ld_src, q_out, scale_out, scale_dtype, scale_f32_out, div_mode,
                               (hipStream_t)stream);
}

int qtts_pack_fp8_e4m3_rowwise(const void* src, int src_dtype, int64_t n, int64_t k, int64_t ld_src,
                               uint8_t* q_out, float* scale_out, int div_mode, void* stream) {
  QTTS_REQUIRE(n >= 0 && k >= 0, "pack_fp8_e4m3_rowwise: negative size");
  QTTS_REQUIRE(dtype_ok(src_dtype), "pack_fp8_e4m3_rowwise: bad dtype code");
  QTTS_REQUIRE(div_ok(div_mode), "pack_fp8_e4m3_rowwise: bad div_mode %d", div_mode);
  QTTS_REQUIRE(ld_src >= k, "pack_fp8_e4m3_rowwise: ld_src < k");
  QTTS_REQUIRE(n < (1ll << 31), "pack_fp8_e4m3_rowwise: n too large");
  if (n == 0) return QTTS_OK;
  QTTS_REQUIRE(scale_out && (k == 0 || (src && q_out)), "pack_fp8_e4m3_rowwise: null pointer");
  QTTS_TRY(current_device_check());
  return qtts_launch_pack_fp8(src, src_dtype, n, k, ld_src, q_out, scale_out, div_mode, (hipStream_t)stream);
}

int qtts_w8a16_gemm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* q, int64_t n,
                    int64_t ldq, const void* scale, int scale_dtype, const void* bias, void* y, int64_t ldy, int algo,
                    void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a16_gemm: negative size (m=%lld, n=%lld, k=%lld)", (long long)m,
               (long long)n, (long long)k);
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "w8a16_gemm: size too large");
  QTTS_REQUIRE(dtype_ok(x_dtype) && dtype_ok(scale_dtype), "w8a16_gemm: bad dtype code");
  QTTS_REQUIRE(algo_ok(algo), "w8a16_gemm: bad algo %d", algo);
  QTTS_REQUIRE(ldx >= k && ldq >= k && ldy >= n, "w8a16_gemm: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a16_gemm: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(scale && y && (k == 0 || (x && q)), "w8a16_gemm: null pointer");
  // Every workgroup reads all x rows of its K range while others write y.
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, k, dtype_size(x_dtype), y, m, ldy, n, dtype_size(x_dtype)),
               "w8a16_gemm: y overlaps x");
  QTTS_TRY(current_device_check());
  return qtts_launch_w8a16(x, x_dtype, m, k, ldx, q, n, ldq, qtts::kLayoutRowMajor, scale, scale_dtype, bias, y, ldy,
                           algo, ws, ws_bytes, (hipStream_t)stream);
}

int qtts_w8a16_gemm_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qs, int64_t n,
                           const void* scale, int scale_dtype, const void* bias, void* y, int64_t ldy, int algo,
                           void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a16_gemm_strips: negative size (m=%lld, n=%lld, k=%lld)", (long long)m,
               (long long)n, (long long)k);
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "w8a16_gemm_strips: size too large");
  QTTS_REQUIRE(dtype_ok(x_dtype) && dtype_ok(scale_dtype), "w8a16_gemm_strips: bad dtype code");
  QTTS_REQUIRE(algo_ok_rows(algo), "w8a16_gemm_strips: bad algo %d", algo);
  QTTS_REQUIRE(ldx >= k && ldy >= n, "w8a16_gemm_strips: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a16_gemm_strips: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(scale && y && x && qs, "w8a16_gemm_strips: null pointer");
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, k, dtype_size(x_dtype), y, m, ldy, n, dtype_size(x_dtype)),
               "w8a16_gemm_strips: y overlaps x");
  QTTS_TRY(current_device_check());
  return qtts_launch_w8a16(x, x_dtype, m, k, ldx, qs, n, 0, qtts::kLayoutStrips, scale, scale_dtype, bias, y, ldy,
                           algo, ws, ws_bytes, (hipStream_t)stream);
}

int qtts_quant_act_fp8_rows(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, uint8_t* qx, float* sx,
                            int div_mode, void* stream) {
  QTTS_REQUIRE(m >= 0 && k >= 0, "quant_act_fp8_rows: negative size");
  QTTS_REQUIRE(m < (1ll << 31), "quant_act_fp8_rows: m too large");
  QTTS_REQUIRE(dtype_ok(x_dtype), "quant_act_fp8_rows: bad dtype code");
  QTTS_REQUIRE(div_ok(div_mode), "quant_act_fp8_rows: bad div_mode %d", div_mode);
  QTTS_REQUIRE(ldx >= k, "quant_act_fp8_rows: ldx < k");
  if (m == 0) return QTTS_OK;
  QTTS_REQUIRE(sx && (k == 0 || (x && qx)), "quant_act_fp8_rows: null pointer");
  QTTS_TRY(current_device_check());
  return qtts_launch_quant_act_fp8(x, x_dtype, m, k, ldx, qx, sx, div_mode, (hipStream_t)stream);
}

int qtts_w8a8_fp8_gemm(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const uint8_t* qw,
                       int64_t n, int64_t ldqw, const float* sw, const void* bias, void* y, int out_dtype,
                       int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a8_fp8_gemm: negative size");
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "w8a8_fp8_gemm: size too large");
  QTTS_REQUIRE(dtype_ok(out_dtype), "w8a8_fp8_gemm: bad dtype code");
  QTTS_REQUIRE(algo_ok(algo), "w8a8_fp8_gemm: bad algo %d", algo);
  QTTS_REQUIRE(ldqx >= k && ldqw >= k && ldy >= n, "w8a8_fp8_gemm: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a8_fp8_gemm: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(sx && sw && y && (k == 0 || (qx && qw)), "w8a8_fp8_gemm: null pointer");
  QTTS_REQUIRE(!spans_overlap(qx, m, ldqx, k, 1, y, m, ldy, n, dtype_size(out_dtype)), "w8a8_fp8_gemm: y overlaps qx");
  QTTS_TRY(current_device_check());
  return qtts_launch_fp8_gemm(qx, sx, m, k, ldqx, qw, n, ldqw, qtts::kLayoutRowMajor, sw, bias, y, out_dtype, ldy,
                              algo, ws, ws_bytes, (hipStream_t)stream);
}

int qtts_w8a8_fp8_gemm_strips(const uint8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                              const uint8_t* qws, int64_t n, const float* sw, const void* bias, void* y, int out_dtype,
                              int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a8_fp8_gemm_strips: negative size");
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "w8a8_fp8_gemm_strips: size too large");
  QTTS_REQUIRE(dtype_ok(out_dtype), "w8a8_fp8_gemm_strips: bad dtype code");
  QTTS_REQUIRE(algo_ok(algo), "w8a8_fp8_gemm_strips: bad algo %d", algo);
  QTTS_REQUIRE(ldqx >= k && ldy >= n, "w8a8_fp8_gemm_strips: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a8_fp8_gemm_strips: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(qx && sx && qws && sw && y, "w8a8_fp8_gemm_strips: null pointer");
  QTTS_REQUIRE(!spans_overlap(qx, m, ldqx, k, 1, y, m, ldy, n, dtype_size(out_dtype)),
               "w8a8_fp8_gemm_strips: y overlaps qx");
  QTTS_TRY(current_device_check());
  return qtts_launch_fp8_gemm(qx, sx, m, k, ldqx, qws, n, 0, qtts::kLayoutStrips, sw, bias, y, out_dtype, ldy, algo,
                              ws, ws_bytes, (hipStream_t)stream);
}

static int fp8_linear_impl(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qw,
                           int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias, void* y,
                           int64_t ldy, int div_mode, int algo, void* ws, int64_t ws_bytes, void* stream) {
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "fp8_linear: negative size");
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "fp8_linear: size too large");
  QTTS_REQUIRE(dtype_ok(x_dtype), "fp8_linear: bad dtype code");
  QTTS_REQUIRE(div_ok(div_mode), "fp8_linear: bad div_mode %d", div_mode);
  QTTS_REQUIRE(algo_ok(algo), "fp8_linear: bad algo %d", algo);
  QTTS_REQUIRE(ldx >= k && (layout == qtts::kLayoutStrips || ldqw >= k) && ldy >= n,
               "fp8_linear: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "fp8_linear: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(sw && y && (k == 0 || (x && qw)), "fp8_linear: null pointer");
  // The decode kernel has every workgroup read all of x while others write y.
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, k, dtype_size(x_dtype), y, m, ldy, n, dtype_size(x_dtype)),
               "fp8_linear: y overlaps x");
  // Decode rows on strip weights: quantization fused into the GEMM, one kernel, no
  // workspace.  A wave count alone (family SKINNY or AUTO, no split count or chunk
  // count) sets the fused kernel's waves; an explicit split count keeps the two-kernel path.
  const int fused_waves = (algo >> 16) & 0xff;
  if (layout == qtts::kLayoutStrips && (algo & 0xff) != QTTS_ALGO_TILE && ((algo >> 8) & 0xff) == 0 &&
      (algo >> 24) == 0 && x_dtype != QTTS_F32 && (uintptr_t)x % 16 == 0 && ldx % 8 == 0 &&
      qtts_fp8_fused_ok(m, n, k, fused_waves)) {
    QTTS_TRY(current_device_check());
    return qtts_launch_fp8_linear_fused(x, x_dtype, m, k, ldx, qw, n, sw, bias, y, ldy, div_mode, fused_waves,
                                        (hipStream_t)stream);
  }
  // Layout: the GEMM's own workspace (split-K counters first) from the start, the
  // quantized activations and their scales at the end.
  const int64_t qx_bytes = al256(m * k), sx_bytes = al256(m * 4);
  const int64_t need = linear_ws(qtts_fp8_gemm_ws_bytes(m, n, k, algo), m, k);
  QTTS_REQUIRE(ws != nullptr, "fp8_linear: a workspace of %lld bytes is required", (long long)need);
  if (ws_bytes < qtts::kCounterBytes + qx_bytes + sx_bytes)
    return qtts_set_error(QTTS_ERR_WORKSPACE, "fp8_linear: workspace of %lld bytes < %lld needed", (long long)ws_bytes,
                          (long long)need);
  const int64_t tail = (ws_bytes - qx_bytes - sx_bytes) & ~(int64_t)255;
  QTTS_TRY(current_device_check());
  uint8_t* qx = (uint8_t*)ws + tail;
  float* sx = (float*)((char*)ws + tail + qx_bytes);
  QTTS_TRY(qtts_launch_quant_act_fp8(x, x_dtype, m, k, ldx, qx, sx, div_mode, (hipStream_t)stream));
  return qtts_launch_fp8_gemm(qx, sx, m, k, k, qw, n, ldqw, layout, sw, bias, y, x_dtype, ldy, algo,
                              tail > 0 ? ws : nullptr, tail, (hipStream_t)stream);
}

int qtts_fp8_linear(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qw, int64_t n,
                    int64_t ldqw, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode, int algo,
                    void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  return fp8_linear_impl(x, x_dtype, m, k, ldx, qw, n, ldqw, qtts::kLayoutRowMajor, sw, bias, y, ldy, div_mode, algo, ws,
                         ws_bytes, stream);
}

int qtts_fp8_linear_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qws,
                           int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode, int algo,
                           void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  return fp8_linear_impl(x, x_dtype, m, k, ldx, qws, n, 0, qtts::kLayoutStrips, sw, bias, y, ldy, div_mode, algo, ws,
                         ws_bytes, stream);
}

}  // extern "C"

// ---- the fp8 linear on a library-owned workspace (qtts_fp8_linear_strips_static) ---------
// `scratch` is that workspace: one array per GPU, kept until the process ends.  In host code
// its name is a host-side stand-in, never a device address; the device address of each
// GPU's copy comes from hipGetSymbolAddress, with that GPU current, and only that address
// is handed to kernels.
static __device__ __align__(256) unsigned char scratch[QTTS_STATIC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void zero_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The current GPU's scratch address, resolved once per GPU.  On that first call the split-K
// counter block at its start is cleared with a kernel on `st` (the loader zero-fills the
// array too; every later call leaves the counters at zero again).
int scratch_of_current_device(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return qtts_set_error(QTTS_ERR_UNSUPPORTED, "no HIP device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return qtts_set_error(QTTS_ERR_UNSUPPORTED, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return qtts_set_error(QTTS_ERR_HIP, "static scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                            hipGetErrorString(e));
    const int words = (int)(qtts::kCounterBytes / 4);
    qtts::launch(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, st, (uint32_t*)p, words);
    QTTS_TRY(qtts_check_launch("static scratch clear"));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return QTTS_OK;
}
}  // namespace

extern "C" {

int qtts_fp8_linear_strips_static(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qws,
                                  int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode,
                                  int algo, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "fp8_linear_strips_static: negative size");
  QTTS_REQUIRE(m < (1ll << 31) && k < (1ll << 31), "fp8_linear_strips_static: size too large");
  // The activation codes, their scales and the counter block must fit; a split-K choice that
  // does not fit in what is left runs without the split.
  const int64_t least = qtts::kCounterBytes + al256(m * k) + al256(m * 4);
  if (least > QTTS_STATIC_SCRATCH_BYTES)
    return qtts_set_error(QTTS_ERR_WORKSPACE,
                          "fp8_linear_strips_static: m * k = %lld activation bytes need %lld workspace bytes, "
                          "more than the %lld of the static scratch",
                          (long long)(m * k), (long long)least, (long long)QTTS_STATIC_SCRATCH_BYTES);
  if (m == 0 || n == 0) return fp8_linear_impl(x, x_dtype, m, k, ldx, qws, n, 0, qtts::kLayoutStrips, sw, bias, y,
                                               ldy, div_mode, algo, nullptr, 0, stream);
  QTTS_TRY(current_device_check());
  void* ws = nullptr;
  QTTS_TRY(scratch_of_current_device((hipStream_t)stream, &ws));
  return fp8_linear_impl(x, x_dtype, m, k, ldx, qws, n, 0, qtts::kLayoutStrips, sw, bias, y, ldy, div_mode, algo, ws,
                         QTTS_STATIC_SCRATCH_BYTES, stream);
}

int qtts_quant_act_int8_rows(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qx, float* sx,
                             int div_mode, void* stream) {
  QTTS_REQUIRE(m >= 0 && k >= 0, "quant_act_int8_rows: negative size");
  QTTS_REQUIRE(m < (1ll << 31), "quant_act_int8_rows: m too large");
  QTTS_REQUIRE(dtype_ok(x_dtype), "quant_act_int8_rows: bad dtype code");
  QTTS_REQUIRE(div_ok(div_mode), "quant_act_int8_rows: bad div_mode %d", div_mode);
  QTTS_REQUIRE(ldx >= k, "quant_act_int8_rows: ldx < k");
  if (m == 0) return QTTS_OK;
  QTTS_REQUIRE(sx && (k == 0 || (x && qx)), "quant_act_int8_rows: null pointer");
  QTTS_TRY(current_device_check());
  return qtts_launch_quant_act_int8(x, x_dtype, m, k, ldx, qx, sx, div_mode, (hipStream_t)stream);
}

static int int8_gemm_impl(const char* what, const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                          const int8_t* qw, int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias,
                          void* y, int out_dtype, int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "%s: negative size", what);
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "%s: size too large", what);
  QTTS_REQUIRE(dtype_ok(out_dtype), "%s: bad dtype code", what);
  QTTS_REQUIRE(algo_ok(algo), "%s: bad algo %d", what, algo);
  QTTS_REQUIRE(ldqx >= k && (layout == qtts::kLayoutStrips || ldqw >= k) && ldy >= n,
               "%s: leading dimension smaller than the row", what);
  QTTS_REQUIRE(ws_bytes >= 0, "%s: negative workspace size", what);
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(sx && sw && y && (k == 0 || (qx && qw)), "%s: null pointer", what);
  QTTS_REQUIRE(!spans_overlap(qx, m, ldqx, k, 1, y, m, ldy, n, dtype_size(out_dtype)), "%s: y overlaps qx", what);
  QTTS_TRY(current_device_check());
  return qtts_launch_int8_gemm(qx, sx, m, k, ldqx, qw, n, ldqw, layout, sw, bias, y, out_dtype, ldy, algo, ws, ws_bytes,
                               (hipStream_t)stream);
}

int qtts_w8a8_int8_gemm(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx, const int8_t* qw,
                        int64_t n, int64_t ldqw, const float* sw, const void* bias, void* y, int out_dtype,
                        int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  return int8_gemm_impl("w8a8_int8_gemm", qx, sx, m, k, ldqx, qw, n, ldqw, qtts::kLayoutRowMajor, sw, bias, y,
                        out_dtype, ldy, algo, ws, ws_bytes, stream);
}

int qtts_w8a8_int8_gemm_strips(const int8_t* qx, const float* sx, int64_t m, int64_t k, int64_t ldqx,
                               const int8_t* qws, int64_t n, const float* sw, const void* bias, void* y, int out_dtype,
                               int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  return int8_gemm_impl("w8a8_int8_gemm_strips", qx, sx, m, k, ldqx, qws, n, 0, qtts::kLayoutStrips, sw, bias, y,
                        out_dtype, ldy, algo, ws, ws_bytes, stream);
}

static int int8_linear_impl(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qw,
                            int64_t n, int64_t ldqw, int layout, const float* sw, const void* bias, void* y,
                            int64_t ldy, int div_mode, int algo, void* ws, int64_t ws_bytes, void* stream) {
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "int8_linear: negative size");
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "int8_linear: size too large");
  QTTS_REQUIRE(dtype_ok(x_dtype), "int8_linear: bad dtype code");
  QTTS_REQUIRE(div_ok(div_mode), "int8_linear: bad div_mode %d", div_mode);
  QTTS_REQUIRE(algo_ok(algo), "int8_linear: bad algo %d", algo);
  QTTS_REQUIRE(ldx >= k && (layout == qtts::kLayoutStrips || ldqw >= k) && ldy >= n,
               "int8_linear: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "int8_linear: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(sw && y && (k == 0 || (x && qw)), "int8_linear: null pointer");
  // The decode kernel has every workgroup read all of x while others write y.
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, k, dtype_size(x_dtype), y, m, ldy, n, dtype_size(x_dtype)),
               "int8_linear: y overlaps x");
  // Decode rows on strip weights: quantization fused into the GEMM, one kernel, no
  // workspace.  A wave count alone (family SKINNY or AUTO, no split count or chunk
  // count) sets the fused kernel's waves; an explicit split count keeps the two-kernel path.
  const int fused_waves = (algo >> 16) & 0xff;
  if (layout == qtts::kLayoutStrips && (algo & 0xff) != QTTS_ALGO_TILE && ((algo >> 8) & 0xff) == 0 &&
      (algo >> 24) == 0 && x_dtype != QTTS_F32 && (uintptr_t)x % 16 == 0 && ldx % 8 == 0 &&
      qtts_int8_fused_ok(m, n, k, fused_waves)) {
    QTTS_TRY(current_device_check());
    return qtts_launch_int8_linear_fused(x, x_dtype, m, k, ldx, qw, n, sw, bias, y, ldy, div_mode, fused_waves,
                                         (hipStream_t)stream);
  }
  // Layout: the GEMM's own workspace (split-K counters first) from the start, the
  // quantized activations (rows of k bytes, 16-byte aligned when k % 16 == 0) and
  // their scales at the end.
  const int64_t qx_bytes = al256(m * k), sx_bytes = al256(m * 4);
  const int64_t need = linear_ws(qtts_int8_gemm_ws_bytes(m, n, k, algo), m, k);
  QTTS_REQUIRE(ws != nullptr, "int8_linear: a workspace of %lld bytes is required", (long long)need);
  if (ws_bytes < qtts::kCounterBytes + qx_bytes + sx_bytes)
    return qtts_set_error(QTTS_ERR_WORKSPACE, "int8_linear: workspace of %lld bytes < %lld needed", (long long)ws_bytes,
                          (long long)need);
  const int64_t tail = (ws_bytes - qx_bytes - sx_bytes) & ~(int64_t)255;
  QTTS_TRY(current_device_check());
  int8_t* qx = (int8_t*)ws + tail;
  float* sx = (float*)((char*)ws + tail + qx_bytes);
  QTTS_TRY(qtts_launch_quant_act_int8(x, x_dtype, m, k, ldx, qx, sx, div_mode, (hipStream_t)stream));
  return qtts_launch_int8_gemm(qx, sx, m, k, k, qw, n, ldqw, layout, sw, bias, y, x_dtype, ldy, algo,
                               tail > 0 ? ws : nullptr, tail, (hipStream_t)stream);
}

int qtts_int8_linear(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qw, int64_t n,
                     int64_t ldqw, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode, int algo,
                     void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  return int8_linear_impl(x, x_dtype, m, k, ldx, qw, n, ldqw, qtts::kLayoutRowMajor, sw, bias, y, ldy, div_mode, algo,
                          ws, ws_bytes, stream);
}

int qtts_int8_linear_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const int8_t* qws,
                            int64_t n, const float* sw, const void* bias, void* y, int64_t ldy, int div_mode, int algo,
                            void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  return int8_linear_impl(x, x_dtype, m, k, ldx, qws, n, 0, qtts::kLayoutStrips, sw, bias, y, ldy, div_mode, algo, ws,
                          ws_bytes, stream);
}

int qtts_silu_mul(const void* gate_up, int x_dtype, int64_t m, int64_t k, int64_t ld_gate_up, void* h, int64_t ldh,
                  void* stream) {
  QTTS_REQUIRE(m >= 0 && k >= 0, "silu_mul: negative size");
  QTTS_REQUIRE(m < 65536 && k < (1ll << 31), "silu_mul: size too large");
  QTTS_REQUIRE(dtype_ok(x_dtype), "silu_mul: bad dtype code");
  QTTS_REQUIRE(ld_gate_up >= 2 * k && ldh >= k, "silu_mul: leading dimension smaller than the row");
  if (m == 0 || k == 0) return QTTS_OK;
  QTTS_REQUIRE(gate_up && h, "silu_mul: null pointer");
  QTTS_TRY(current_device_check());
  return qtts_launch_silu_mul(gate_up, x_dtype, m, k, ld_gate_up, h, ldh, (hipStream_t)stream);
}

int qtts_w8a16_silu_mul_gemm_strips(const void* gate_up, int x_dtype, int64_t m, int64_t k, int64_t ld_gate_up,
                                    const int8_t* qs, int64_t n, const void* scale, int scale_dtype, const void* bias,
                                    void* y, int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a16_silu_mul_gemm_strips: negative size");
  QTTS_REQUIRE(m < 65536 && n < (1ll << 31) && k < (1ll << 30), "w8a16_silu_mul_gemm_strips: size too large");
  QTTS_REQUIRE(x_dtype == QTTS_BF16 || x_dtype == QTTS_F16, "w8a16_silu_mul_gemm_strips: activations must be bf16 or fp16");
  QTTS_REQUIRE(dtype_ok(scale_dtype), "w8a16_silu_mul_gemm_strips: bad scale dtype code");
  QTTS_REQUIRE(algo_ok_rows(algo), "w8a16_silu_mul_gemm_strips: bad algo %d", algo);
  QTTS_REQUIRE(k % 16 == 0, "w8a16_silu_mul_gemm_strips: K %% 16 != 0 (K=%lld)", (long long)k);
  QTTS_REQUIRE(ld_gate_up >= 2 * k && ldy >= n, "w8a16_silu_mul_gemm_strips: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a16_silu_mul_gemm_strips: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(gate_up && qs && scale && y, "w8a16_silu_mul_gemm_strips: null pointer");
  QTTS_REQUIRE(!spans_overlap(gate_up, m, ld_gate_up, 2 * k, 2, y, m, ldy, n, 2),
               "w8a16_silu_mul_gemm_strips: y overlaps gate_up");
  QTTS_TRY(current_device_check());
  return qtts_launch_w8a16_silu(gate_up, x_dtype, m, k, ld_gate_up, qs, n, scale, scale_dtype, bias, y, ldy, algo, ws,
                                ws_bytes, (hipStream_t)stream);
}

int qtts_rms_norm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* weight, float eps, void* y,
                  int64_t ldy, void* stream) {
  QTTS_REQUIRE(m >= 0 && k >= 0, "rms_norm: negative size");
  QTTS_REQUIRE(m < (1ll << 31) && k < (1ll << 31), "rms_norm: size too large");
  QTTS_REQUIRE(dtype_ok(x_dtype), "rms_norm: bad dtype code");
  QTTS_REQUIRE(ldx >= k && ldy >= k, "rms_norm: leading dimension smaller than the row");
  if (m == 0 || k == 0) return QTTS_OK;
  QTTS_REQUIRE(x && weight && y, "rms_norm: null pointer");
  QTTS_TRY(current_device_check());
  return qtts_launch_rms_norm(x, x_dtype, m, k, ldx, weight, eps, y, ldy, (hipStream_t)stream);
}

int qtts_w8a16_fused_gemm_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int prologue,
                                 const void* norm_weight, float eps, const int8_t* qs, int64_t n, const void* scale,
                                 int scale_dtype, const void* bias, const void* residual, int64_t ldr, void* y,
                                 int64_t ldy, int algo, void* ws, int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a16_fused_gemm_strips: negative size");
  QTTS_REQUIRE(m < 65536 && n < (1ll << 31) && k < (1ll << 30), "w8a16_fused_gemm_strips: size too large");
  QTTS_REQUIRE(x_dtype == QTTS_BF16 || x_dtype == QTTS_F16, "w8a16_fused_gemm_strips: activations must be bf16 or fp16");
  QTTS_REQUIRE(dtype_ok(scale_dtype), "w8a16_fused_gemm_strips: bad scale dtype code");
  QTTS_REQUIRE(algo_ok_rows(algo), "w8a16_fused_gemm_strips: bad algo %d", algo);
  QTTS_REQUIRE(prologue == QTTS_PRO_NONE || prologue == QTTS_PRO_SILU_MUL || prologue == QTTS_PRO_RMS_NORM,
               "w8a16_fused_gemm_strips: bad prologue %d", prologue);
  QTTS_REQUIRE(k % 64 == 0, "w8a16_fused_gemm_strips: K %% 64 != 0 (K=%lld)", (long long)k);
  QTTS_REQUIRE(ldx >= (prologue == QTTS_PRO_SILU_MUL ? 2 * k : k) && ldy >= n && (!residual || ldr >= n),
               "w8a16_fused_gemm_strips: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a16_fused_gemm_strips: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(x && qs && scale && y && (prologue != QTTS_PRO_RMS_NORM || norm_weight),
               "w8a16_fused_gemm_strips: null pointer");
  QTTS_REQUIRE(prologue != QTTS_PRO_NONE || ((uintptr_t)x % 16 == 0 && (m == 1 || ldx % 8 == 0)),
               "w8a16_fused_gemm_strips: activation rows must be 16-byte aligned");
  QTTS_REQUIRE(!residual || residual == y || !ranges_overlap(residual, m, ldr, y, m, ldy, n, 2),
               "w8a16_fused_gemm_strips: residual overlaps y without being y");
  QTTS_REQUIRE(!residual || residual != y || ldr == ldy, "w8a16_fused_gemm_strips: residual is y with another stride");
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, prologue == QTTS_PRO_SILU_MUL ? 2 * k : k, 2, y, m, ldy, n, 2),
               "w8a16_fused_gemm_strips: y overlaps x");
  QTTS_TRY(current_device_check());
  return qtts_launch_w8a16_fused(x, x_dtype, m, k, ldx, prologue, norm_weight, eps, qs, n, scale, scale_dtype, bias,
                                 residual, ldr, y, ldy, algo, ws, ws_bytes, (hipStream_t)stream);
}

int qtts_w8a16_gate_up_silu_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int prologue,
                                   const void* norm_weight, float eps, const int8_t* qs, int64_t n, const void* scale,
                                   int scale_dtype, const void* bias, void* act, int64_t ldact, int algo, void* ws,
                                   int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "w8a16_gate_up_silu_strips: negative size");
  QTTS_REQUIRE(m < 65536 && n < (1ll << 31) && k < (1ll << 30), "w8a16_gate_up_silu_strips: size too large");
  QTTS_REQUIRE(x_dtype == QTTS_BF16 || x_dtype == QTTS_F16,
               "w8a16_gate_up_silu_strips: activations must be bf16 or fp16");
  QTTS_REQUIRE(dtype_ok(scale_dtype), "w8a16_gate_up_silu_strips: bad scale dtype code");
  QTTS_REQUIRE(algo_ok_rows(algo), "w8a16_gate_up_silu_strips: bad algo %d", algo);
  QTTS_REQUIRE(prologue == QTTS_PRO_NONE || prologue == QTTS_PRO_RMS_NORM,
               "w8a16_gate_up_silu_strips: prologue must be none or RMSNorm, got %d", prologue);
  QTTS_REQUIRE(k % 64 == 0, "w8a16_gate_up_silu_strips: K %% 64 != 0 (K=%lld)", (long long)k);
  QTTS_REQUIRE(n % 2 == 0, "w8a16_gate_up_silu_strips: gate_up width %lld is odd", (long long)n);
  QTTS_REQUIRE(ldx >= k && ldact >= n / 2, "w8a16_gate_up_silu_strips: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "w8a16_gate_up_silu_strips: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(x && qs && scale && act && (prologue != QTTS_PRO_RMS_NORM || norm_weight),
               "w8a16_gate_up_silu_strips: null pointer");
  QTTS_REQUIRE((uintptr_t)x % 16 == 0 && (m == 1 || ldx % 8 == 0),
               "w8a16_gate_up_silu_strips: activation rows must be 16-byte aligned");
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, k, 2, act, m, ldact, n / 2, 2), "w8a16_gate_up_silu_strips: act overlaps x");
  QTTS_TRY(current_device_check());
  return qtts_launch_w8a16_gate_up_silu(x, x_dtype, m, k, ldx, prologue, norm_weight, eps, qs, n, scale, scale_dtype,
                                        bias, act, ldact, algo, ws, ws_bytes, (hipStream_t)stream);
}

int qtts_fp8w_gemm_strips(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* qs, int64_t n,
                          const float* scale, const void* bias, void* y, int64_t ldy, int algo, void* ws,
                          int64_t ws_bytes, void* stream) {
  const qtts::WeightPolicy policy(algo);  // takes QTTS_ALGO_STREAM out of algo
  QTTS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "fp8w_gemm_strips: negative size (m=%lld, n=%lld, k=%lld)", (long long)m,
               (long long)n, (long long)k);
  QTTS_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), "fp8w_gemm_strips: size too large");
  QTTS_REQUIRE(x_dtype == QTTS_BF16 || x_dtype == QTTS_F16, "fp8w_gemm_strips: activations must be bf16 or fp16");
  QTTS_REQUIRE(algo_ok(algo), "fp8w_gemm_strips: bad algo %d", algo);
  QTTS_REQUIRE(k % 64 == 0, "fp8w_gemm_strips: K %% 64 != 0 (K=%lld)", (long long)k);
  QTTS_REQUIRE(ldx >= k && ldy >= n, "fp8w_gemm_strips: leading dimension smaller than the row");
  QTTS_REQUIRE(ws_bytes >= 0, "fp8w_gemm_strips: negative workspace size");
  if (m == 0 || n == 0) return QTTS_OK;
  QTTS_REQUIRE(x && qs && scale && y, "fp8w_gemm_strips: null pointer");
  QTTS_REQUIRE((uintptr_t)x % 16 == 0 && (m == 1 || ldx % 8 == 0), "fp8w_gemm_strips: activation rows must be 16-byte aligned");
  QTTS_REQUIRE(!spans_overlap(x, m, ldx, k, 2, y, m, ldy, n, 2), "fp8w_gemm_strips: y overlaps x");
  QTTS_TRY(current_device_check());
  return qtts_launch_fp8w(x, x_dtype, m, k, ldx, qs, n, scale, bias, y, ldy, algo, ws, ws_bytes, (hipStream_t)stream);
}

int64_t qtts_strip_bytes(int64_t n, int64_t k, int kind) {
  if (n < 0 || k < 0 || n >= (1ll << 31) || k >= (1ll << 31) || (kind != QTTS_STRIP_INT8 && kind != QTTS_STRIP_FP8))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "strip_bytes: bad arguments");
  return qtts::strip_bytes(n, k, kind);
}

int qtts_to_strips(const void* src, int64_t n, int64_t k, int64_t ld_src, int kind, void* dst, void* stream) {
  QTTS_REQUIRE(n >= 0 && k >= 0 && n < (1ll << 31) && k < (1ll << 31) && ld_src >= k, "to_strips: bad sizes");
  QTTS_REQUIRE(kind == QTTS_STRIP_INT8 || kind == QTTS_STRIP_FP8, "to_strips: bad kind %d", kind);
  if (n == 0 || k == 0) return QTTS_OK;
  QTTS_REQUIRE(src && dst, "to_strips: null pointer");
  QTTS_REQUIRE((uintptr_t)dst % 16 == 0, "to_strips: destination must be 16-byte aligned");
  QTTS_TRY(current_device_check());
  return qtts_launch_to_strips(src, n, k, ld_src, dst, kind, (hipStream_t)stream);
}

int qtts_from_strips(const void* src, int64_t n, int64_t k, int kind, void* dst, int64_t ld_dst, void* stream) {
  QTTS_REQUIRE(n >= 0 && k >= 0 && n < (1ll << 31) && k < (1ll << 31) && ld_dst >= k, "from_strips: bad sizes");
  QTTS_REQUIRE(kind == QTTS_STRIP_INT8 || kind == QTTS_STRIP_FP8, "from_strips: bad kind %d", kind);
  if (n == 0 || k == 0) return QTTS_OK;
  QTTS_REQUIRE(src && dst, "from_strips: null pointer");
  QTTS_REQUIRE((uintptr_t)src % 16 == 0, "from_strips: source must be 16-byte aligned");
  QTTS_TRY(current_device_check());
  return qtts_launch_from_strips(src, n, k, dst, ld_dst, kind, (hipStream_t)stream);
}

int qtts_dequant_strips(const void* qs, int codes, int64_t n, int64_t k, const void* scale, int scale_dtype, void* w,
                        int w_dtype, int64_t ldw, void* stream) {
  QTTS_REQUIRE(n >= 0 && k >= 0 && n < (1ll << 31) && k < (1ll << 31) && ldw >= k, "dequant_strips: bad sizes");
  QTTS_REQUIRE(n < (1ll << 31) && k < (1ll << 31), "dequant_strips: size too large");
  QTTS_REQUIRE(codes == QTTS_CODE_INT8 || codes == QTTS_CODE_E4M3, "dequant_strips: bad code kind %d", codes);
  QTTS_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(w_dtype), "dequant_strips: bad dtype code");
  if (n == 0 || k == 0) return QTTS_OK;
  QTTS_REQUIRE(qs && scale && w, "dequant_strips: null pointer");
  QTTS_REQUIRE((uintptr_t)qs % 16 == 0, "dequant_strips: strip buffer must be 16-byte aligned");
  QTTS_TRY(current_device_check());
  return qtts_launch_dequant_strips(qs, codes, n, k, scale, scale_dtype, w, w_dtype, ldw, (hipStream_t)stream);
}

int qtts_kernel_timer_begin(int max_launches) {
  QTTS_REQUIRE(max_launches > 0 && max_launches <= (1 << 20), "kernel timer: max_launches must be in [1, 2^20]");
  std::lock_guard<std::mutex> lock(g_timer_mu);
  if (g_timer_armed.load(std::memory_order_relaxed))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "kernel timer: already armed");
  timer_release();
  g_timer_events.reserve(2 * (size_t)max_launches);
  for (int i = 0; i < 2 * max_launches; ++i) {
    hipEvent_t e = nullptr;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      timer_release();
      return qtts_set_error(QTTS_ERR_HIP, "kernel timer: hipEventCreate failed: %s", hipGetErrorString(err));
    }
    g_timer_events.push_back(e);
  }
  g_timer_untimed = 0;
  g_timer_armed.store(true, std::memory_order_release);
  return QTTS_OK;
}

int qtts_kernel_timer_end(double* total_ms, int64_t* launches, int64_t* untimed) {
  QTTS_REQUIRE(total_ms && launches && untimed, "kernel timer: null pointer");
  std::lock_guard<std::mutex> lock(g_timer_mu);
  if (!g_timer_armed.load(std::memory_order_relaxed))
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "kernel timer: not armed");
  g_timer_armed.store(false, std::memory_order_release);
  double sum = 0.0;
  int status = QTTS_OK;
  for (size_t i = 0; i + 1 < g_timer_used; i += 2) {
    float ms = 0.0f;
    hipError_t err = hipEventSynchronize(g_timer_events[i + 1]);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, g_timer_events[i], g_timer_events[i + 1]);
    if (err != hipSuccess) {
      status = qtts_set_error(QTTS_ERR_HIP, "kernel timer: %s", hipGetErrorString(err));
      break;
    }
    sum += ms;
  }
  *total_ms = sum;
  *launches = (int64_t)(g_timer_used / 2);
  *untimed = g_timer_untimed;
  timer_release();
  return status;
}

}  // extern "C"
