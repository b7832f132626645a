// Closed-form Gaussian moment helpers shared by several kernel files.
#pragma once
#include "tagi_common.h"

namespace tagi {

#define INV_SQRT_2PI 0.3989422804014327f
#define INV_SQRT_2 0.7071067811865476f

// ------------------------------------------------------------------------------ ReLU
// relu.py:43-86: exact rectified-Gaussian moments; Phi by erf, replaced by the
// asymptotic pdf/(-alpha) when alpha < -5; variance floored at 0.
// Variance of max(0, z) given its mean mu = sigma (phi + alpha Phi):
//   -mu^2 + 2 mu mz - mz sigma phi + (S - mz^2) Phi          (the reference's form)
//   = S [Phi + alpha^2 Phi Q + alpha phi (Q - Phi) - phi^2],   Q = 1 - Phi
// The identity holds for any Phi value (it only uses mu = sigma phi + mz Phi), so it also
// covers the asymptotic branch; the second form has no O(alpha^2) cancellation in fp32.
__device__ __forceinline__ float rect_var(float S, float alpha, float pdf, float cdf, float Q) {
  return S * (cdf + alpha * alpha * cdf * Q + alpha * pdf * (Q - cdf) - pdf * pdf);
}

__device__ __forceinline__ void relu_moments(float mz, float Sz, float& ma, float& Sa, float& J) {
  const float Ss = fmaxf(Sz, 1e-30f);
  const float sig = sqrtf(Ss);
  const float alpha = mz / sig;
  const float pdf = expf(-0.5f * alpha * alpha) * INV_SQRT_2PI;
  // Phi(alpha) = 0.5 (1 + erf(alpha/sqrt2)) evaluated as 0.5 erfc(-alpha/sqrt2): equal in
  // exact arithmetic, without the fp32 cancellation of the erf form for alpha < 0.
  const bool asym = alpha < -5.0f;
  // one erfc gives the smaller tail; the other side is its complement (no cancellation)
  const float tail = 0.5f * erfcf(fabsf(alpha) * INV_SQRT_2);
  const float cdf_e = alpha >= 0.0f ? 1.0f - tail : tail;
  const float cdf = asym ? pdf / (-alpha) : cdf_e;
  const float Q = asym ? 1.0f - cdf : (alpha >= 0.0f ? tail : 1.0f - tail);
  ma = sig * pdf + mz * cdf;
  Sa = fmaxf(rect_var(Ss, alpha, pdf, cdf, Q), 0.0f);
  J = cdf;
}

}  // namespace tagi
