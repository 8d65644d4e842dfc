// Launch plumbing of the W8A16 skinny kernel's fused variants (skinny.h: PRO, RES):
// one row set of template instantiations per (prologue, residual, staged rows), each
// built in one translation unit (w8a16_fused.hip, w8a16_fused_res.hip).
#pragma once

#include "skinny.h"

namespace qtts {

struct FusedArgs {
  const void* x;
  int64_t m, k, ldx;
  const int8_t* qs;
  int64_t n;
  const void* scale;
  const void* bias;
  const void* aux;  // the norm weight (kProRmsNorm)
  float eps;
  const void* res;  // residual rows (RES)
  int64_t ldr;
  void* y;
  int64_t ldy;
  float* part;
  unsigned* counters;
  SkinnyCfg c;
  int sub;  // workgroups per strip (row-split strips when > 1)
  unsigned blocks;
  hipStream_t st;
};

template <typename XT, typename ST, int W, int CPW, int MX, int PRO, bool RES, bool PAIR = false, int SUB = 1>
void launch_fused_one(const FusedArgs& a) {
  launch_skinny<XT, ST, W, CPW, kLayoutStrips, true, 1, MX, false, PRO, RES, PAIR, SUB>(
      dim3(a.blocks, a.c.S, skinny_row_parts(a.m)), dim3(W * 64), a.st, a.qs, (const XT*)a.x, (const ST*)a.scale, (const XT*)a.bias,
      (const XT*)a.aux, (int)a.ldx, (int)(a.m | (a.c.S << 8)), (int)a.k, (int)a.n, (XT*)a.y, a.ldy, (int64_t)0, a.part,
      a.counters, a.eps, (const XT*)a.res, a.ldr);
}

// The row-split pairs built for the fused kernels: the automatic choices of the half-strip
// layers (skinny_auto_sub, skinny_cfg_sub), for the residual epilogue and the SiLU prologue.
inline bool fused_sub_built(int sub, int waves, int cpw) {
  return sub == 2 && ((waves == 4 && (cpw == 4 || cpw == 8)) || (waves == 8 && cpw == 6));
}

// The (waves, chunks) pairs built with staged rows (qtts_w8a16_xrows_built), and the
// half-strip ones of fused_sub_built (at most 8 rows; not with the RMSNorm prologue).
template <typename XT, typename ST, int MX, int PRO, bool RES>
int launch_fused_wc(const FusedArgs& a) {
  if (a.sub > 1) {
    if constexpr (PRO != kProRmsNorm && MX <= 8) {
      if (a.sub == 2) {
        switch (a.c.waves * 64 + a.c.cpw) {
          case 4 * 64 + 4: launch_fused_one<XT, ST, 4, 4, MX, PRO, RES, false, 2>(a); return 0;
          case 4 * 64 + 8: launch_fused_one<XT, ST, 4, 8, MX, PRO, RES, false, 2>(a); return 0;
          case 8 * 64 + 6: launch_fused_one<XT, ST, 8, 6, MX, PRO, RES, false, 2>(a); return 0;
          default: break;
        }
      }
    }
    return 1;
  }
  switch (a.c.waves * 64 + a.c.cpw) {
    case 1 * 64 + 8: launch_fused_one<XT, ST, 1, 8, MX, PRO, RES>(a); break;
    case 2 * 64 + 8: launch_fused_one<XT, ST, 2, 8, MX, PRO, RES>(a); break;
    case 4 * 64 + 8: launch_fused_one<XT, ST, 4, 8, MX, PRO, RES>(a); break;
    case 8 * 64 + 8: launch_fused_one<XT, ST, 8, 8, MX, PRO, RES>(a); break;
    case 16 * 64 + 6: launch_fused_one<XT, ST, 16, 6, MX, PRO, RES>(a); break;
    case 8 * 64 + 12: launch_fused_one<XT, ST, 8, 12, MX, PRO, RES>(a); break;
    default: return 1;
  }
  return 0;
}

// The SiLU-pair variants (PAIR).  Two-strip (a gate strip and its up strip a workgroup, each
// wave carrying both strips' chunks): 2, 4, 8 and 16 waves of 4 chunks and 1, 2, 4 and 8 waves
// of 8 chunks.  Half strips (sub = 2: 8 gate rows and their up rows a workgroup): 1, 2, 4 and 8
// waves of 8 chunks, the plain GEMM's automatic choices up to K = 4096.
template <typename XT, typename ST, int MX, int PRO>
int launch_pair_wc(const FusedArgs& a) {
  if (a.sub == 2) {  // half strips (skinny.h: PAIR with SUB = 2), the plain GEMM's configurations
    switch (a.c.waves * 64 + a.c.cpw) {
      case 1 * 64 + 8: launch_fused_one<XT, ST, 1, 8, MX, PRO, false, true, 2>(a); break;
      case 2 * 64 + 8: launch_fused_one<XT, ST, 2, 8, MX, PRO, false, true, 2>(a); break;
      case 4 * 64 + 8: launch_fused_one<XT, ST, 4, 8, MX, PRO, false, true, 2>(a); break;
      case 8 * 64 + 8: launch_fused_one<XT, ST, 8, 8, MX, PRO, false, true, 2>(a); break;
      default: return 1;
    }
    return 0;
  }
  switch (a.c.waves * 64 + a.c.cpw) {
    case 2 * 64 + 4: launch_fused_one<XT, ST, 2, 4, MX, PRO, false, true>(a); break;
    case 4 * 64 + 4: launch_fused_one<XT, ST, 4, 4, MX, PRO, false, true>(a); break;
    case 8 * 64 + 4: launch_fused_one<XT, ST, 8, 4, MX, PRO, false, true>(a); break;
    case 16 * 64 + 4: launch_fused_one<XT, ST, 16, 4, MX, PRO, false, true>(a); break;
    case 1 * 64 + 8: launch_fused_one<XT, ST, 1, 8, MX, PRO, false, true>(a); break;
    case 2 * 64 + 8: launch_fused_one<XT, ST, 2, 8, MX, PRO, false, true>(a); break;
    case 4 * 64 + 8: launch_fused_one<XT, ST, 4, 8, MX, PRO, false, true>(a); break;
    case 8 * 64 + 8: launch_fused_one<XT, ST, 8, 8, MX, PRO, false, true>(a); break;
    default: return 1;
  }
  return 0;
}
inline bool pair_half_built(int waves, int cpw) {
  return cpw == 8 && (waves == 1 || waves == 2 || waves == 4 || waves == 8);
}
inline bool pair_built(int waves, int cpw) {
  return (cpw == 4 && (waves == 2 || waves == 4 || waves == 8 || waves == 16)) ||
         (cpw == 8 && (waves == 1 || waves == 2 || waves == 4 || waves == 8));
}

// Returns 0 after a launch, 1 when the combination is not built.  Scales are either
// of the activation dtype (Int8WeightOnlyMethod) or fp32.
template <int PRO, bool RES, int MX, bool PAIR = false>
int launch_fused(int x_dtype, bool f32_scale, const FusedArgs& a) {
  if constexpr (PAIR) {
    if (x_dtype == QTTS_BF16)
      return f32_scale ? launch_pair_wc<bf16_t, float, MX, PRO>(a) : launch_pair_wc<bf16_t, bf16_t, MX, PRO>(a);
    return f32_scale ? launch_pair_wc<f16_t, float, MX, PRO>(a) : launch_pair_wc<f16_t, f16_t, MX, PRO>(a);
  } else {
    if (x_dtype == QTTS_BF16)
      return f32_scale ? launch_fused_wc<bf16_t, float, MX, PRO, RES>(a)
                       : launch_fused_wc<bf16_t, bf16_t, MX, PRO, RES>(a);
    return f32_scale ? launch_fused_wc<f16_t, float, MX, PRO, RES>(a) : launch_fused_wc<f16_t, f16_t, MX, PRO, RES>(a);
  }
}

// Residual-only variants (w8a16_fused_res.hip) for 1, 2, 4 and 8 staged rows.
extern template int launch_fused<kProNone, true, 1>(int, bool, const FusedArgs&);
extern template int launch_fused<kProNone, true, 2>(int, bool, const FusedArgs&);
extern template int launch_fused<kProNone, true, 4>(int, bool, const FusedArgs&);
extern template int launch_fused<kProNone, true, 8>(int, bool, const FusedArgs&);
// RMSNorm prologue for 2, 4 and 8 staged rows (w8a16_fused_norm.hip).
extern template int launch_fused<kProRmsNorm, false, 2>(int, bool, const FusedArgs&);
extern template int launch_fused<kProRmsNorm, false, 4>(int, bool, const FusedArgs&);
extern template int launch_fused<kProRmsNorm, false, 8>(int, bool, const FusedArgs&);
// SiLU-pair gate_up, with or without the RMSNorm prologue (w8a16_fused_pair.hip,
// w8a16_fused_pair_norm.hip).
extern template int launch_fused<kProNone, false, 1, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProNone, false, 2, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProNone, false, 4, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProNone, false, 8, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProRmsNorm, false, 1, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProRmsNorm, false, 2, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProRmsNorm, false, 4, true>(int, bool, const FusedArgs&);
extern template int launch_fused<kProRmsNorm, false, 8, true>(int, bool, const FusedArgs&);

}  // namespace qtts
