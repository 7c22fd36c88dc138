// Exact (erf) GELU and its derivative in fp32 for the gfx950 kernels.
//
// erf uses Abramowitz & Stegun, Handbook of Mathematical Functions, eq. 7.1.26
// (|error| <= 1.5e-7), far below the bf16 rounding the results get:
//   erf(x) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-x^2),
//   t = 1 / (1 + p x),  x >= 0.
#pragma once

#include "common.h"

namespace mednext {

// 1 - erf(|x|) without the final subtraction: returns p * t and exp(-x^2) parts.
__device__ inline void erfc_parts(float ax, float& poly, float& ex) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, ax, 1.0f));
  float p = fmaf(1.061405429f, t, -1.453152027f);
  p = fmaf(p, t, 1.421413741f);
  p = fmaf(p, t, -0.284496736f);
  p = fmaf(p, t, 0.254829592f);
  poly = p * t;
  ex = __expf(-ax * ax);
}

__device__ inline float erf_as(float x) {
  float poly, ex;
  erfc_parts(fabsf(x), poly, ex);
  return copysignf(1.0f - poly * ex, x);
}

__device__ inline float gelu_f(float h) { return 0.5f * h * (1.0f + erf_as(h * 0.7071067811865476f)); }

// d/dh of h * Phi(h) = Phi(h) + h * phi(h); phi(h) = exp(-h^2 / 2) / sqrt(2 pi)
// shares its exponential with the erf approximation.
__device__ inline float gelu_grad_f(float h) {
  float poly, ex;
  erfc_parts(fabsf(h) * 0.7071067811865476f, poly, ex);
  const float cdf = 0.5f + 0.5f * copysignf(1.0f - poly * ex, h);
  return fmaf(h * 0.3989422804014327f, ex, cdf);
}

// GELU(h) and GELU'(h) from one exponential.
__device__ inline void gelu_pair(float h, float& g, float& dg) {
  float poly, ex;
  erfc_parts(fabsf(h) * 0.7071067811865476f, poly, ex);
  const float cdf = 0.5f + 0.5f * copysignf(1.0f - poly * ex, h);
  g = h * cdf;
  dg = fmaf(h * 0.3989422804014327f, ex, cdf);
}

// The value a bf16 tensor holding GELU(h) would store.
__device__ inline float gelu_bf16(float h) { return bf16_to_f32(f32_to_bf16(gelu_f(h))); }

}  // namespace mednext
