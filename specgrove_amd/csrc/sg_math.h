// Binary32 exponential and (max, sum of exp) pairs shared by the sampler and
// the LM head's statistics epilogue.  Every operation is fixed so that the
// CPU restatement reproduces the bits: compile with contraction off.
#pragma once

#include "sg_common.h"

namespace sg {

#define SG_LOG2E 0x1.715476p+0f
#define SG_LN2_HI 0x1.62e4p-1f
#define SG_LN2_LO 0x1.7f7d1cp-20f
// e^r on |r| <= ln2/2 as 1 + r + C2 r^2 + ... + C5 r^5: a relative-error
// fit (iteratively reweighted least squares over Chebyshev nodes, float64,
// then rounded to binary32); its own error is 1.06e-7, below the 1.6e-7 of
// the degree-6 Taylor polynomial on the same interval.
#define SG_C5 0x1.10625ap-7f
#define SG_C4 0x1.5729eep-5f
#define SG_C3 0x1.5557aep-3f
#define SG_C2 0x1.fffdfcp-2f
// Lower clamp of the argument: -inf, NaN and everything below land here, where
// n = -173 and the scale underflows to exactly 0.
#define SG_EXP_LO (-120.0f)
#define SG_EXP_HI 88.0f

// E(x): Cody-Waite reduction x = n ln2 + r with a split ln2 (both steps by
// fma), the degree-5 polynomial above in Horner form, and p * 2^n by ldexp,
// which rounds a subnormal result once (as p * 2^(n+64) * 2^-64 would).  The
// argument is clamped to [-120, 88] first: E is exactly 0 below about
// -103.3 (n <= -151), a subnormal between there and -87.3, and +inf above 88.
// Over every binary32 x in [-87, 0] its relative error against exp is at
// most 1.8e-7.
__device__ __forceinline__ float sg_exp(float x) {
  const float xc = fminf(fmaxf(x, SG_EXP_LO), SG_EXP_HI);
  const float n = __builtin_rintf(xc * SG_LOG2E);
  float r = __builtin_fmaf(-n, SG_LN2_HI, xc);
  r = __builtin_fmaf(-n, SG_LN2_LO, r);
  float p = SG_C5;
  p = __builtin_fmaf(p, r, SG_C4);
  p = __builtin_fmaf(p, r, SG_C3);
  p = __builtin_fmaf(p, r, SG_C2);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float y = __builtin_ldexpf(p, static_cast<int>(n));
  return (x > SG_EXP_HI) ? __builtin_inff() : y;
}

// E(x) for x <= 0 (every argument of the form value - max): sg_exp without
// the upper clamp and the overflow select, which cannot apply there.  The
// results are identical.
__device__ __forceinline__ float sg_exp_nonpos(float x) {
  const float xc = fmaxf(x, SG_EXP_LO);
  const float n = __builtin_rintf(xc * SG_LOG2E);
  float r = __builtin_fmaf(-n, SG_LN2_HI, xc);
  r = __builtin_fmaf(-n, SG_LN2_LO, r);
  float p = SG_C5;
  p = __builtin_fmaf(p, r, SG_C4);
  p = __builtin_fmaf(p, r, SG_C3);
  p = __builtin_fmaf(p, r, SG_C2);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, static_cast<int>(n));
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
