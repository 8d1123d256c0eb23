// The GELU of the SDD epilogues (the reference applies F.gelu's exact erf
// form in fp32 before rounding to bf16: csrc/sdd.cu:41, 104-110).
#pragma once

#include "common.hpp"

namespace sb {

// Exact-erf GELU, 0.5 v (1 + erf(v / sqrt 2)), in fp32.
//
// erfc(u) for u >= 0 by Abramowitz & Stegun 7.1.26 (Hastings' rational
// approximation, |error| <= 1.5e-7): erfc(u) = t P(t) exp(-u^2),
// t = 1 / (1 + p u). Branch-free, about fifteen instructions, and for
// v < 0 it forms 1 - erf(u) = erfc(u) directly, with no cancellation.
__device__ __forceinline__ float gelu_erf_fast(float v) {
  const float u = fabsf(v) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, u, 1.0f));
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  const float erfc_u = poly * t * __builtin_amdgcn_exp2f(-u * u * 1.44269504088896341f);
  return v >= 0.0f ? v * (1.0f - 0.5f * erfc_u) : 0.5f * v * erfc_u;
}

// The same with the device library's erff (reference accuracy, slower).
__device__ __forceinline__ float gelu_erf_libm(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f)); }

}  // namespace sb
