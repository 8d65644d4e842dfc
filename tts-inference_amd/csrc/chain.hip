// A chain of dependent W8A16 decode linears in one persistent launch (gfx950).
//
// The decoder layer of the talker (qtts/models/talker.py:246-271) runs, between two
// attention calls, four linears that each read what the previous one wrote:
//
//   h1  = h + o_proj(attn)                              link 0: residual epilogue
//   act = silu(gate) * up,
//         gate | up = gate_up_proj(post_attention_layernorm(h1))
//                                                       link 1: RMSNorm prologue,
//                                                               SiLU * mul epilogue
//   h2  = h1 + down_proj(act)                           link 2: residual epilogue
//   qkv = qkv_proj(input_layernorm(h2))  (next layer)   link 3: RMSNorm prologue
//
// One kernel per linear pays a launch boundary each time: the grid drains (its
// slowest workgroups are the tail), then the next one ramps up from an idle memory
// pipe.  Here one grid works through all links.  Work items are handed out in link
// order from a ticket counter; a workgroup issues an item's weight loads first and
// only then waits for the link it depends on, so the next linear's weights stream
// in while the previous one finishes.
//
// Work item: 8 waves.  Each output strip (16 weight rows) gets `wps` waves that split
// its K range into runs of `cw` <= 12 chunks (64 columns, 1 KiB of strip bytes a
// chunk); an item holds 8 / wps strips.  With the SiLU epilogue an item pairs gate
// strip s with up strip s + N/32, so one workgroup holds both halves of its output
// columns and writes silu(gate) * up directly: the gate_up output itself is never
// stored, and the down projection reads the activation as is.
//
// Workgroup w runs items w, w + G, w + 2G, ... of the grid of G workgroups, in order,
// and an item waits only for items of earlier links, which hold smaller indices.  The
// host sizes the grid so that every workgroup is resident at once (occupancy), so the
// unfinished item with the smallest index is always running and never waits: every
// item finishes.  Each wait is still bounded (kChainSpin polls): past it the kernel
// raises the control block's timeout flag and carries on, so no launch can hang.
//
// Coherence across the 8 XCDs (each has its own L2): every value one workgroup
// writes for another (activations, residual stream) is stored with agent-scope
// stores (sc1, written through), and the writer waits for their completion
// (vmcnt(0)) before its workgroup sets the item's flag; readers poll the flags and
// then load with agent-scope loads (sc1), which do not hit stale L2 lines.  No
// buffer_wbl2 / buffer_inv: only these accesses need coherence.  Weights, scales,
// biases and norm weights are constant for the launch and use plain loads.
//
// Synchronisation uses per-item flags only, no atomics (see the control block below).
#include <algorithm>

#include "skinny.h"

using namespace qtts;

namespace qtts {

constexpr int kChainWaves = 8;         // waves per workgroup (and per work item)
constexpr int kChainMaxChunks = 12;    // chunks in flight per wave
constexpr int kChainMaxK = 8192;       // staged K per row (two 8-element vectors a thread)
constexpr int kChainSpin = 1 << 18;    // polls before a wait gives up (~0.3 s)
constexpr int kLdsChainMax = 160 * 1024;
enum : int { kEpiStore = 0, kEpiResidual = 1, kEpiSiluMul = 2 };
// The chain's control block (32-bit words), owned by one chain: word 0 is the timeout
// flag, word kCtlFlags + t the completion flag of work item t.  No word is ever the
// target of an atomic (atomics on one address serialize at the memory side, tens of
// nanoseconds each).  Every launch has an epoch E: item t's flag is set to E once the
// item's outputs are visible, and consumers wait for flags equal to E.  Each launch of
// one chain runs the same items on the same grid, with workgroup w running items w,
// w + G, ...; item w's flag is written by workgroup w alone, so at the start of a launch
// it still holds the previous launch's epoch, and E = flag[w] + 1 is the same in every
// workgroup.  Nothing is ever reset; a zero-filled block starts at epoch 1.
constexpr int kCtlTimeout = 0;
constexpr int kCtlFlags = 64;
constexpr int kPollUnroll = 8;  // flag loads a lane issues at once
// One flag per 256-byte line: every waiting workgroup reads all flags of the link it
// waits for, and packed flags would put that whole stream of reads on one memory channel.
constexpr int kFlagStride = 64;  // words
static_assert(kCtlTimeout * 4 == QTTS_CHAIN_TIMEOUT_BYTE && kCtlFlags * 4 == QTTS_CHAIN_FLAGS_BYTE,
              "control block layout");

struct ChainLink {
  const void* x;
  const int8_t* qs;
  const void* scale;
  const void* bias;
  const void* nw;
  const void* res;
  void* y;
  int64_t ldx, ldr, ldy;
  float eps;
  int n, k, pro, epi, after;
  int wps, cw, items, item0, nbytes_x, nbytes_r;
  int waited;  // some later link waits for this one
};

struct ChainArgs {
  ChainLink L[QTTS_CHAIN_MAX_LINKS];
  unsigned* ctl;
  int count, m, total;
};

// LDS: cross-wave partial sums, norm partials, a word of flags, then the staged rows.
constexpr int kRedBytes = kChainWaves * 64 * 16;
constexpr int kNssOff = kRedBytes;
constexpr int kFlagsOff = kNssOff + kChainWaves * 8 * 4;
constexpr int kXsOff = kFlagsOff + 16;

typedef __attribute__((ext_vector_type(2))) int i32x2_t;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t chain_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
// 16 / 8 bytes at byte offset `off`, agent-scope coherent (sc1); out of range reads 0.
__device__ __forceinline__ i32x4_t load16_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}
__device__ __forceinline__ i32x2_t load8_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16);
}

template <typename T> __device__ __forceinline__ float elem(uint32_t pair, int hi) {
  return to_f32(T{(uint16_t)(hi ? pair >> 16 : pair)});
}

// One work item of link L: item j (ticket minus the link's first ticket).  C >= L.cw
// is the number of weight loads each wave keeps in flight.  KNOWN: the link L waits
// for (if any) is already known complete, so the activation rows are requested
// first and the whole item is one memory round trip; otherwise the weights go out
// first, wave 0 polls the link's done counter (its first poll issued before the
// weights, so a satisfied dependency costs no wait for them) and the rows follow.
//
// Every load before the first wait is unconditional (clamped addresses for waves
// without work): the compiler's wait counting is not path-sensitive, and a load
// under a branch would make the first wait cover every load in flight.
template <typename XT, typename ST, int MX, int C, bool KNOWN>
__device__ __forceinline__ void chain_item(const ChainArgs& a, const ChainLink& L, int j, char* smem,
                                           unsigned epoch, bool waited) {
  typedef mfma16<XT> MM;
  typedef typename MM::vec V;
  f32x4_t* red = (f32x4_t*)smem;
  float* nss = (float*)(smem + kNssOff);
  unsigned* known = (unsigned*)(smem + kFlagsOff + 4);
  uint16_t* xs = (uint16_t*)(smem + kXsOff);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int M = a.m, K = L.k, P = K + 8;  // P: LDS row pitch in elements (+16 bytes: no bank aliasing)
  const int wps = L.wps, sidx = wave / wps, kslot = wave - sidx * wps;
  const int nstrips = L.n >> 4, nchunks = K >> 6;
  const bool silu = L.epi == kEpiSiluMul, norm = L.pro == QTTS_PRO_RMS_NORM;
  int strip;
  if (silu) {
    const int half = nstrips >> 1, pair = j * (kChainWaves / wps / 2) + (sidx >> 1);
    strip = pair < half ? pair + (sidx & 1) * half : nstrips;
  } else {
    strip = j * (kChainWaves / wps) + sidx;
  }
  const bool sv = strip < nstrips;
  const int c0 = kslot * L.cw, c1 = min(c0 + L.cw, nchunks);
  const bool has = sv && c0 < c1;
  // The wave that runs the epilogue of its strip (of the pair, with SiLU).
  const bool lead = sv && kslot == 0 && !(silu && (sidx & 1));
  const i32x4_t zero = {0, 0, 0, 0};
  const int sl = sv ? strip : 0;  // clamped: loads of waves without work stay in bounds
  const int nn0 = sl * 16 + 4 * g;

  // Activation rows, coherent: row m's vector v (8 elements) goes to thread v mod 512;
  // the residual of the lead waves' output columns.
  i32x4_t xv[MX][2], nwv[2];
  i32x2_t rv = {0, 0};
  auto issue_x = [&]() {
    const __amdgpu_buffer_rsrc_t xr = chain_rsrc(L.x, L.nbytes_x);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = min(8 * (tid + 512 * i), K - 8);
#pragma unroll
      for (int m = 0; m < MX; ++m)
        xv[m][i] = load16_coherent(xr, (int)(2 * ((int64_t)min(m, M - 1) * L.ldx + e)));
      if (norm) nwv[i] = *(const i32x4_t*)((const XT*)L.nw + e);
    }
    if (L.epi == kEpiResidual) {
      const __amdgpu_buffer_rsrc_t rr = chain_rsrc(L.res, L.nbytes_r);
      rv = load8_coherent(rr, (int)(2 * ((int64_t)min(r, M - 1) * L.ldr + nn0)));
    }
  };

  // 1. The first poll (wave 0), the rows if the dependency is known, the weights and
  // the epilogue constants: every load of the item goes out before anything waits.
  // Wave 0 watches the flags of the awaited link's items, lane l the items l + 64 j.
  const int dep = L.after >= 0 ? L.after : 0;
  const int d0 = a.L[dep].item0, dn = a.L[dep].items;
  // Flags past the link's last item read as zero from the bounded buffer resource
  // (no memory request) and count as ready.
  const __amdgpu_buffer_rsrc_t fr = chain_rsrc(a.ctl + kCtlFlags + d0 * kFlagStride, dn * kFlagStride * 4);
  bool ready = true;
  auto flag_at = [&](int i) {
    return (unsigned)__builtin_amdgcn_raw_buffer_load_b32(fr, i * kFlagStride * 4, 0, 16);
  };
  auto poll = [&](int base) {  // items base .. base + 64 kPollUnroll - 1 of the link
    unsigned f[kPollUnroll];
#pragma unroll
    for (int j = 0; j < kPollUnroll; ++j) f[j] = flag_at(base + lane + 64 * j);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kPollUnroll; ++j) ok = ok && (f[j] == epoch || base + lane + 64 * j >= dn);
    return ok;
  };
  unsigned f0[kPollUnroll];
  if (!KNOWN && wave == 0) {
#pragma unroll
    for (int j = 0; j < kPollUnroll; ++j) f0[j] = flag_at(lane + 64 * j);
  }
  if (KNOWN) issue_x();
  i32x4_t w[C];
  {
    const int8_t* wp = L.qs + (int64_t)sl * nchunks * 1024 + lane * 16;
    const int cl = has ? c1 - 1 : 0;
#pragma unroll
    for (int u = 0; u < C; ++u) w[u] = *(const i32x4_t*)(wp + (int64_t)min(c0 + u, cl) * 1024);
  }
  // scale and bias of rows 4g..4g+3, and of the paired up rows with SiLU (the scale
  // stands in for a missing bias; its bits are then never used).
  uint32_t sc[4], bi[4], su[4], bu[4];
  {
    const void* bsrc = L.bias ? L.bias : L.scale;
    // Only gate strips' lead waves use the up rows; other waves' indices stay below n.
    const int nu = silu ? min(nn0 + (L.n >> 1), L.n - 4) : nn0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = load_bits((const ST*)L.scale + nn0 + i);
      bi[i] = load_bits((const XT*)bsrc + nn0 + i);
      su[i] = load_bits((const ST*)L.scale + nu + i);
      bu[i] = load_bits((const XT*)bsrc + nu + i);
    }
  }

  // 2. Wait for the link whose outputs this one reads (the weights stay in flight),
  // then request the rows.
  if (!KNOWN) {
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < kPollUnroll; ++j) ready = ready && (f0[j] == epoch || lane + 64 * j >= dn);
      int it = 0, nap = 1;
      for (int base = 0; base < dn;) {
        if (!__builtin_amdgcn_ballot_w64(!ready)) {
          base += 64 * kPollUnroll;
          ready = base >= dn || poll(base);
          continue;
        }
        if (++it == kChainSpin) {
          if (lane == 0) store_coherent(a.ctl + kCtlTimeout, 1u);
          break;
        }
        for (int z = 0; z < nap; ++z) __builtin_amdgcn_s_sleep(2);  // backing off up to ~0.4 us
        nap = min(2 * nap, 8);
        ready = poll(base);
      }
      if (lane == 0) *known |= 1u << L.after;
    }
    barrier_only();
    issue_x();
  }

  // 3. RMSNorm: per-row sums of squares, in thread then wave then workgroup order.
  float inv[MX];
  if (norm) {
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      float ss = 0.0f;
      if (m < M) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (8 * (tid + 512 * i) < K) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float lo = elem<XT>((uint32_t)xv[m][i][q], 0), hi = elem<XT>((uint32_t)xv[m][i][q], 1);
              ss = __builtin_fmaf(lo, lo, ss);
              ss = __builtin_fmaf(hi, hi, ss);
            }
          }
        }
      }
      ss = wave_sum_rows(ss);
      if (lane == 0) nss[wave * 8 + m] = ss;
    }
    wait_lgkmcnt0();
    barrier_only();
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      float ss = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < kChainWaves; ++w2) ss += nss[w2 * 8 + m];
      inv[m] = 1.0f / __builtin_sqrtf(ss / (float)K + L.eps);
    }
  }

  // 4. Stage the rows in LDS (normalized and rounded to XT with the norm prologue).
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int e = 8 * (tid + 512 * i);
    if (e < K) {
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        if (m < M) {
          i32x4_t v = xv[m][i];
          if (norm) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t p = (uint32_t)v[q], wq = (uint32_t)nwv[i][q];
              const float h0 = (elem<XT>(p, 0) * inv[m]) * elem<XT>(wq, 0);
              const float h1 = (elem<XT>(p, 1) * inv[m]) * elem<XT>(wq, 1);
              v[q] = (int)pack2_f32<XT>(h0, h1);
            }
          }
          *(i32x4_t*)(xs + m * P + e) = v;
        }
      }
    }
  }
  wait_lgkmcnt0();
  barrier_only();

  // 5. MFMAs: the weight strip is the A operand, the staged rows the B operand (lanes
  // of rows >= M read row 0; their D columns are never stored).  Unconditional: zeroed
  // weights past the wave's range.
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  {
    const uint16_t* xb = xs + (r < M ? r : 0) * P + 16 * g;
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const bool live = has && c0 + u < c1;
      const int cu = max(min(c0 + u, c1 - 1), 0);
      const i32x4_t wv = live ? w[u] : zero;
      const i32x4_t x0 = *(const i32x4_t*)(xb + 64 * cu), x1 = *(const i32x4_t*)(xb + 64 * cu + 8);
      acc = MM::mma(wcvt<false, XT>((uint32_t)wv[0], (uint32_t)wv[1]), __builtin_bit_cast(V, x0), acc);
      acc = MM::mma(wcvt<false, XT>((uint32_t)wv[2], (uint32_t)wv[3]), __builtin_bit_cast(V, x1), acc);
    }
  }

  // 6. Cross-wave sums: every non-lead wave of a valid strip parks its partial.
  if (sv && !lead) red[wave * 64 + lane] = acc;
  wait_lgkmcnt0();
  barrier_only();
  if (!lead) {
    // Loads whose values a path never used (rows past M) have long completed; waiting
    // here tells the compiler so, or it waits for them before reusing their registers
    // in the next item, behind that item's own first loads.
    wait_vmem();
    return;
  }
  for (int w2 = 1; w2 < wps; ++w2) acc += red[(wave + w2) * 64 + lane];
  f32x4_t up = {0.0f, 0.0f, 0.0f, 0.0f};
  if (silu)
    for (int w2 = 0; w2 < wps; ++w2) up += red[(wave + wps + w2) * 64 + lane];

  // 7. Epilogue: lane (r, g) holds weight rows 4g..4g+3 of the strip for activation
  // row r; four consecutive outputs, one 8-byte coherent store.
  if (r < M) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t = acc[i] * bits_to_f32<ST>(sc[i]);
      if (L.bias) t += bits_to_f32<XT>(bi[i]);
      if (L.epi == kEpiResidual) {
        t = elem<XT>((uint32_t)rv[i >> 1], i & 1) + round_through<XT>(t);
      } else if (silu) {
        float u = up[i] * bits_to_f32<ST>(su[i]);
        if (L.bias) u += bits_to_f32<XT>(bu[i]);
        t = silu_mul<XT>(round_through<XT>(t), round_through<XT>(u));
      }
      v[i] = t;
    }
    const uint64_t packed = (uint64_t)pack2_f32<XT>(v[0], v[1]) | ((uint64_t)pack2_f32<XT>(v[2], v[3]) << 32);
    store_coherent((uint64_t*)((XT*)L.y + (int64_t)r * L.ldy + nn0), packed);
  }
  // A later link reads these outputs: they are complete before the item's flag is set.
  if (waited) wait_vmem();
}

template <typename XT, typename ST, int MX, int C>
__device__ __forceinline__ void chain_item_any(const ChainArgs& a, const ChainLink& L, int j, char* smem,
                                               bool known, unsigned epoch, bool waited) {
  if (known) chain_item<XT, ST, MX, C, true>(a, L, j, smem, epoch, waited);
  else chain_item<XT, ST, MX, C, false>(a, L, j, smem, epoch, waited);
}

template <typename XT, typename ST, int MX>
__global__ __launch_bounds__(kChainWaves * 64) void w8a16_chain_kernel(ChainArgs a) {
  extern __shared__ __align__(16) char smem[];
  unsigned* kmask = (unsigned*)(smem + kFlagsOff + 4);  // bit i: link i seen complete here
  const int tid = threadIdx.x, lane = tid & 63, G = gridDim.x, wg = blockIdx.x;
  const bool wave0 = tid < 64;
  // The launch's epoch, needed by wave 0 only (it polls and writes every flag); its load
  // overlaps the first item's loads.
  unsigned epoch = 0;
  if (wave0) epoch = load_coherent(a.ctl + kCtlFlags + wg * kFlagStride) + 1u;
  if (tid == 0) *kmask = 0u;
  wait_lgkmcnt0();
  barrier_only();
  // Static assignment: workgroup wg runs items wg, wg + G, ... in order.  Every
  // workgroup of the grid is resident at once (the host sizes the grid by occupancy),
  // so an item's wait for earlier items always ends.
  int li = 0;
  for (int t = wg; t < a.total; t += G) {
    while (li + 1 < a.count && t >= a.L[li + 1].item0) ++li;
    li = __builtin_amdgcn_readfirstlane(li);
    const ChainLink& L = a.L[li];
    // The dependency is known complete once this workgroup has seen it so (the mask
    // is written by wave 0 before a barrier of an earlier item).
    const bool known = L.after < 0 || ((__builtin_amdgcn_readfirstlane((int)*kmask) >> L.after) & 1);
    const bool waited = L.waited;
    if (L.cw <= 4) chain_item_any<XT, ST, MX, 4>(a, L, t - L.item0, smem, known, epoch, waited);
    else if (L.cw <= 8) chain_item_any<XT, ST, MX, 8>(a, L, t - L.item0, smem, known, epoch, waited);
    else chain_item_any<XT, ST, MX, kChainMaxChunks>(a, L, t - L.item0, smem, known, epoch, waited);
    wait_lgkmcnt0();
    barrier_only();  // a waited-for item's stores are complete (each storing wave waited)
    if (tid == 0) store_coherent(a.ctl + kCtlFlags + t * kFlagStride, epoch);
  }
  (void)lane;
}

}  // namespace qtts

namespace {

template <typename XT, typename ST, int MX>
int launch_chain(const ChainArgs& a, int kmax, int grid_req, hipStream_t st) {
  auto* ker = &w8a16_chain_kernel<XT, ST, MX>;
  const int smem = kXsOff + MX * (kmax + 8) * 2;
  static int configured[64] = {0};  // per device: max dynamic LDS raised once
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return qtts_set_error(QTTS_ERR_HIP, "w8a16 chain: no current device");
  if (!configured[dev]) {
    if (hipFuncSetAttribute((const void*)ker, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsChainMax) != hipSuccess)
      return qtts_set_error(QTTS_ERR_HIP, "w8a16 chain: cannot raise the LDS limit");
    if (hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return qtts_set_error(QTTS_ERR_HIP, "w8a16 chain: cannot read the CU count");
    configured[dev] = 1;
  }
  // Every workgroup must be resident at once: the grid never exceeds what fits.
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, (const void*)ker, kChainWaves * 64, smem) != hipSuccess ||
      nb < 1)
    return qtts_set_error(QTTS_ERR_HIP, "w8a16 chain: occupancy query failed");
  const int capacity = cus[dev] * nb;
  int grid = grid_req > 0 ? std::min(grid_req, capacity) : capacity;
  grid = std::max(1, std::min(grid, a.total));
  qtts::launch(ker, dim3(grid), dim3(kChainWaves * 64), (uint32_t)smem, st, a);
  return qtts_check_launch("w8a16_chain");
}

template <typename XT, typename ST>
int launch_chain_mx(const ChainArgs& a, int kmax, int grid, hipStream_t st) {
  if (a.m <= 1) return launch_chain<XT, ST, 1>(a, kmax, grid, st);
  if (a.m <= 2) return launch_chain<XT, ST, 2>(a, kmax, grid, st);
  if (a.m <= 4) return launch_chain<XT, ST, 4>(a, kmax, grid, st);
  return launch_chain<XT, ST, 8>(a, kmax, grid, st);
}

bool al(const void* p, int bytes) { return (uintptr_t)p % bytes == 0; }

}  // namespace

namespace {

// Validates the links and fills the kernel's view of them.  Returns QTTS_OK or an error.
int prepare_chain(const qtts_chain_link* links, int count, int64_t m, ChainArgs& a, int& kmax) {
  if (!links || count < 1 || count > QTTS_CHAIN_MAX_LINKS)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain: %d links (1..%d)", count, QTTS_CHAIN_MAX_LINKS);
  if (m < 0 || m > QTTS_CHAIN_MAX_ROWS)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain: m = %lld rows (0..%d)", (long long)m,
                          QTTS_CHAIN_MAX_ROWS);
  a = ChainArgs{};
  a.count = count;
  a.m = (int)m;
  kmax = 64;
  int item0 = 0;
  for (int i = 0; i < count; ++i) {
    const qtts_chain_link& s = links[i];
    ChainLink& d = a.L[i];
    const int64_t n = s.n, k = s.k;
    if (n < 16 || n % 16 || k < 64 || k % 64 || k > kChainMaxK || n > (1 << 24))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: n %% 16 == 0 and k %% 64 == 0, "
                            "k <= %d (got n=%lld, k=%lld)", i, kChainMaxK, (long long)n, (long long)k);
    if (m > 0 && (!s.x || !s.qs || !s.scale || !s.y))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: null x, weight, scale or y", i);
    if (s.after < -1 || s.after >= i)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: `after` must name an earlier link", i);
    if (s.prologue != QTTS_PRO_NONE && s.prologue != QTTS_PRO_RMS_NORM)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: prologue must be none or RMSNorm", i);
    if (s.prologue == QTTS_PRO_RMS_NORM && (!s.norm_weight || !al(s.norm_weight, 16)))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: RMSNorm needs a 16-byte aligned weight", i);
    if (s.epilogue != QTTS_EPI_STORE && s.epilogue != QTTS_EPI_RESIDUAL && s.epilogue != QTTS_EPI_SILU_MUL)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: unknown epilogue %d", i, s.epilogue);
    if (s.epilogue == QTTS_EPI_RESIDUAL && (!s.residual || !al(s.residual, 8) || (m > 1 && s.ldr % 4)))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: residual rows must be 8-byte aligned", i);
    if (!al(s.x, 16) || (m > 1 && s.ldx % 8) || !al(s.y, 8) || (m > 1 && s.ldy % 4))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: x rows must be 16-byte aligned and "
                            "y rows 8-byte aligned", i);
    const int64_t out_cols = s.epilogue == QTTS_EPI_SILU_MUL ? n / 2 : n;
    if ((m > 1 && (s.ldx < k || s.ldy < out_cols)) || (s.epilogue == QTTS_EPI_RESIDUAL && m > 1 && s.ldr < n))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: a row stride is below the row", i);
    const int64_t xb = ((m > 0 ? m - 1 : 0) * s.ldx + k) * 2, rb = ((m > 0 ? m - 1 : 0) * s.ldr + n) * 2;
    if (xb >= ((int64_t)1 << 31) || (s.epilogue == QTTS_EPI_RESIDUAL && rb >= ((int64_t)1 << 31)))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: activation rows above 2 GiB", i);
    const int nchunks = (int)(k / 64);
    int wps = 1;
    while (wps < kChainWaves && (nchunks + wps - 1) / wps > kChainMaxChunks) wps *= 2;
    const int spi = kChainWaves / wps, nstrips = (int)(n / 16);
    if (s.epilogue == QTTS_EPI_SILU_MUL && (spi < 2 || nstrips % 2))
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain link %d: the SiLU epilogue needs n %% 32 == 0 "
                            "and k <= %d", i, 4 * kChainMaxChunks * 64);
    d.x = s.x;
    d.qs = s.qs;
    d.scale = s.scale;
    d.bias = s.bias;
    d.nw = s.norm_weight;
    d.res = s.residual;
    d.y = s.y;
    d.ldx = m > 1 ? s.ldx : k;
    d.ldr = m > 1 ? s.ldr : n;
    d.ldy = m > 1 ? s.ldy : out_cols;
    d.eps = s.eps;
    d.n = (int)n;
    d.k = (int)k;
    d.pro = s.prologue;
    d.epi = s.epilogue;
    d.after = s.after;
    d.wps = wps;
    d.cw = (nchunks + wps - 1) / wps;
    d.items = s.epilogue == QTTS_EPI_SILU_MUL ? (nstrips / 2 + spi / 2 - 1) / (spi / 2) : (nstrips + spi - 1) / spi;
    d.item0 = item0;
    d.nbytes_x = (int)xb;
    d.nbytes_r = s.epilogue == QTTS_EPI_RESIDUAL ? (int)rb : 0;
    d.waited = 0;
    if (s.after >= 0) a.L[s.after].waited = 1;
    item0 += d.items;
    kmax = std::max<int>(kmax, (int)k);
    if (item0 > QTTS_CHAIN_MAX_ITEMS)
      return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain: more than %d work items",
                            QTTS_CHAIN_MAX_ITEMS);
  }
  a.total = item0;
  return QTTS_OK;
}

}  // namespace

extern "C" int64_t qtts_w8a16_chain_ctl_bytes(const qtts_chain_link* links, int count, int64_t m) {
  ChainArgs a;
  int kmax = 0;
  const int rc = prepare_chain(links, count, m, a, kmax);
  if (rc != QTTS_OK) return rc;
  return ((int64_t)kCtlFlags + (int64_t)a.total * kFlagStride) * 4;
}

extern "C" int qtts_w8a16_chain_strips(const qtts_chain_link* links, int count, int x_dtype, int scale_dtype,
                                       int64_t m, int algo, void* ctl, int64_t ctl_bytes, void* stream) {
  // bf16 only, the talker's dtype: the fp16 build of this kernel spills (the int8 ->
  // fp16 conversion is per element), and fp16 callers keep the per-linear launches.
  if (x_dtype != QTTS_BF16)
    return qtts_set_error(QTTS_ERR_UNSUPPORTED, "w8a16 chain: activations must be bf16");
  if (scale_dtype != x_dtype && scale_dtype != QTTS_F32)
    return qtts_set_error(QTTS_ERR_INVALID_ARGUMENT, "w8a16 chain: scales must be fp32 or of the activation dtype");
  ChainArgs a;
  int kmax = 0;
  int rc = prepare_chain(links, count, m, a, kmax);
  if (rc != QTTS_OK) return rc;
  const int64_t need = ((int64_t)kCtlFlags + (int64_t)a.total * kFlagStride) * 4;
  if (!ctl || ctl_bytes < need || !al(ctl, 256))
    return qtts_set_error(QTTS_ERR_WORKSPACE, "w8a16 chain: needs a 256-byte aligned control block of %lld bytes, "
                          "got %lld", (long long)need, (long long)ctl_bytes);
  a.ctl = (unsigned*)ctl;
  if (m == 0) return QTTS_OK;
  const int grid = (algo >> 8) & 0xffff;  // bits 8-23: workgroups (0: as many as fit at once)
  hipStream_t st = (hipStream_t)stream;
  return scale_dtype == QTTS_F32 ? launch_chain_mx<bf16_t, float>(a, kmax, grid, st)
                                 : launch_chain_mx<bf16_t, bf16_t>(a, kmax, grid, st);
}
