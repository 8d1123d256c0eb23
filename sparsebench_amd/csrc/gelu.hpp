// The GELU of the SDD epilogues (the reference applies F.gelu's exact erf
// form in fp32 before rounding to bf16: csrc/sdd.cu:41, 104-110).
#pragma once

#include "common.hpp"

namespace sb {

// Exact-erf GELU, 0.5 v (1 + erf(v / sqrt 2)), in fp32.
//
// erfc(u) for u >= 0 by Abramowitz & Stegun 7.1.26 (Hastings' rational
// approximation, |error| <= 1.5e-7): erfc(u) = t P(t) exp(-u^2),
// t = 1 / (1 + p u), u = |v| / sqrt 2. With h = 0.5 |v| erfc(u),
//   GELU(v) = v - h for v >= 0 and -h for v < 0, that is max(v, 0) - h,
// so no select on the sign, and for v < 0 no cancellation. In terms of
// a = |v| sqrt(log2(e) / 2), exp(-u^2) = 2^(-a^2), t = 1 / (1 + a p / sqrt(log2 e))
// and h = a t P(t) 2^(-a^2) / sqrt(2 log2 e): the constants fold into the
// coefficients below (A&S's p, a1..a5 scaled), leaving 12 VALU operations
// plus one reciprocal and one exp2 per value. The epilogue is bound by
// this VALU work (one workgroup per CU, nothing overlaps it).
// Special values: GELU(+-0) = +0 (zero rows stay zero), GELU(+inf) = +inf,
// NaN stays NaN; GELU(-inf) = 0 where erf's formula gives NaN.
__device__ __forceinline__ float gelu_erf_fast(float v) {
  const float a = fabsf(v) * 0.8493218002880191f;  // sqrt(log2(e) / 2)
  const float t = __builtin_amdgcn_rcpf(fmaf(0.2727374808792225f, a, 1.0f));  // p / sqrt(log2 e)
  // a1..a5 / sqrt(2 log2 e)
  float q = fmaf(0.6248546950284685f, t, -0.8554778804142388f);
  q = fmaf(q, t, 0.8367933923973075f);
  q = fmaf(q, t, -0.1674846541696695f);
  q = fmaf(q, t, 0.1500194578271646f);
  const float g = q * t * __builtin_amdgcn_exp2f(-(a * a));
  // max(v, +0) on the bits (one integer max: fmaxf also quiets NaN inputs
  // first, a second instruction); a is clamped so that g = 0 with a = inf
  // gives 0, not NaN.
  const float pos = __int_as_float(max(__float_as_int(v), 0));
  return fmaf(-g, fminf(a, 3.40282347e38f), pos);
}

// The same with the device library's erff (reference accuracy, slower).
__device__ __forceinline__ float gelu_erf_libm(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f)); }

}  // namespace sb
