// Binary32 exponential and (max, sum of exp) pairs shared by the sampler and
// the LM head's statistics epilogue.  Every operation is fixed so that the
// CPU restatement reproduces the bits: compile with contraction off.
#pragma once

#include "sg_common.h"

namespace sg {

#define SG_LOG2E 0x1.715476p+0f
#define SG_LN2_HI 0x1.62e4p-1f
#define SG_LN2_LO 0x1.7f7d1cp-20f
#define SG_C6 0x1.6c16c2p-10f
#define SG_C5 0x1.111112p-7f
#define SG_C4 0x1.555556p-5f
#define SG_C3 0x1.555556p-3f

// E(x): 0 below -87 (and for NaN), Cody-Waite reduction with a split ln2,
// degree-6 Taylor polynomial in Horner form, exact scale by 2^n.
__device__ __forceinline__ float sg_exp(float x) {
  const bool live = x >= -87.0f;
  const float xc = fminf(fmaxf(x, -87.0f), 88.0f);
  const float n = __builtin_rintf(xc * SG_LOG2E);
  float r = __builtin_fmaf(-n, SG_LN2_HI, xc);
  r = __builtin_fmaf(-n, SG_LN2_LO, r);
  float p = SG_C6;
  p = __builtin_fmaf(p, r, SG_C5);
  p = __builtin_fmaf(p, r, SG_C4);
  p = __builtin_fmaf(p, r, SG_C3);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  // p * 2^n, exact scale (n in [-126, 127]); ldexp rounds a subnormal result
  // exactly as the multiplication by the normal power of two would.
  float y = __builtin_ldexpf(p, static_cast<int>(n));
  y = (x > 88.0f) ? __builtin_inff() : y;
  return live ? y : 0.0f;
}

// E(x) for x <= 0 (every argument of the form value - max): the same
// operations as sg_exp without the upper clamp and overflow select, which
// cannot apply there, and without the lower clamp: it leaves every live x
// (x >= -87) unchanged, and the final select returns 0 for the others
// whatever the polynomial gave them.  The results are identical.
__device__ __forceinline__ float sg_exp_nonpos(float x) {
  const bool live = x >= -87.0f;
  const float xc = x;
  const float n = __builtin_rintf(xc * SG_LOG2E);
  float r = __builtin_fmaf(-n, SG_LN2_HI, xc);
  r = __builtin_fmaf(-n, SG_LN2_LO, r);
  float p = SG_C6;
  p = __builtin_fmaf(p, r, SG_C5);
  p = __builtin_fmaf(p, r, SG_C4);
  p = __builtin_fmaf(p, r, SG_C3);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float y = __builtin_ldexpf(p, static_cast<int>(n));
  return live ? y : 0.0f;
}

struct MZ {
  float m;
  float z;
};

__device__ __forceinline__ MZ merge_mz(MZ a, MZ b) {
  MZ out;
  out.m = fmaxf(a.m, b.m);
  const float left = a.z * sg_exp(a.m - out.m);
  const float right = b.z * sg_exp(b.m - out.m);
  out.z = (out.m == -__builtin_inff()) ? 0.0f : left + right;
  return out;
}

}  // namespace sg
