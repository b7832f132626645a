// Closed-form Gaussian moment helpers shared by several kernel files.
#pragma once
#include "tagi_common.h"

namespace tagi {

#define INV_SQRT_2PI 0.3989422804014327f
#define INV_SQRT_2 0.7071067811865476f

// ------------------------------------------------------------------------ fast fp32 math
// The moment helpers below turn off the compiler's implicit contraction of a * b + c into
// fused multiply-adds (#pragma clang fp contract(off)) and write every fused multiply-add
// they use as fmaf: whether an implicit contraction happens depends on the code around
// the inlined helper, and kernels that share the row math (the fused attention forward
// and the two-call Remax, the conv epilogue's ReLU statistics and the ReLU/BatchNorm
// pass) must round the same way to give the same bits.
// The hardware transcendental instructions (v_rcp_f32, v_rsq_f32, v_exp_f32)
// are accurate to about 1 ulp on normal operands. The library forms add range reduction,
// denormal scaling and correct rounding that the moment formulas below do not need: their
// results are checked at a relative tolerance of 1e-4, and every use here is a few ulp.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_rsqrt(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ float fast_div(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }

// exp(x) = 2^(x log2 e). The product x log2 e is carried as p + e (e from an fma and the
// low part of log2 e), so its rounding (up to |x| 2^-24 absolute) does not reach the
// result: 2^(p + e) = 2^p (1 + e ln 2) to second order in e. Relative error about 2 ulp
// for results above 2^-126; smaller results (x < -87.3) flush to 0.
__device__ __forceinline__ float fast_exp(float x) {
#pragma clang fp contract(off)
  const float L2E = 1.44269502162933349609375f;   // log2(e) rounded to fp32
  const float L2E_LO = 1.925963033500011e-8f;     // log2(e) - L2E
  const float p = x * L2E;
  const float e = fmaf(x, L2E_LO, fmaf(x, L2E, -p));
  return __builtin_amdgcn_exp2f(p) * fmaf(e, 0.6931471805599453f, 1.0f);
}

// Upper tail of the standard normal, Q(a) = 0.5 erfc(a / sqrt 2), for a >= 0, by the
// Chebyshev-fitted erfc of Press et al., Numerical Recipes in C, 2nd ed., sec. 6.2
// ("erfcc": fractional error below 1.2e-7 in exact arithmetic; about 2e-6 evaluated in
// fp32 for a < 5, 1e-5 for a < 13; 0 beyond a = 13, where Q < 1e-38).
__device__ __forceinline__ float normal_tail(float a) {
  const float z = a * INV_SQRT_2;
  const float t = fast_rcp(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  p = fmaf(p, t, -1.26551223f);
  return 0.5f * t * fast_exp(fmaf(-z, z, p));
}

// Phi(alpha) and 1 - Phi(alpha) from one tail evaluation: the smaller of the two is the
// tail itself and the other its complement, so neither side cancels.
__device__ __forceinline__ void normal_cdf_pair(float alpha, float& cdf, float& ccdf) {
  const float tail = normal_tail(fabsf(alpha));
  cdf = alpha >= 0.0f ? 1.0f - tail : tail;
  ccdf = alpha >= 0.0f ? tail : 1.0f - tail;
}

// ----------------------------------------------------------------------- Capped update
// One parameter's capped update (parameters.py:58-96): each of the mean and variance
// deltas is clipped to sqrt(max(S, 1e-10)) / cap in magnitude, keeping its sign, and a
// variance that would end at or below 0 becomes 1e-5. Used by the update kernels and by
// the parameter-delta GEMM epilogue that applies the update in place; contraction is off
// so that both round alike.
__device__ __forceinline__ float signf_(float x) { return x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f); }

__device__ __forceinline__ void capped(float& m, float& S, float dm, float dS, float cap) {
#pragma clang fp contract(off)
  const float bar = sqrtf(fmaxf(S, 1e-10f)) / cap;
  m = m + signf_(dm) * fminf(fabsf(dm), bar);
  const float Sr = S + signf_(dS) * fminf(fabsf(dS), bar);
  S = (Sr <= 0.f) ? 1e-5f : Sr;
}

// ------------------------------------------------------------------------------ ReLU
// relu.py:43-86: exact rectified-Gaussian moments; Phi by erf, replaced by the
// asymptotic pdf/(-alpha) when alpha < -5; variance floored at 0.
// Variance of max(0, z) given its mean mu = sigma (phi + alpha Phi):
//   -mu^2 + 2 mu mz - mz sigma phi + (S - mz^2) Phi          (the reference's form)
//   = S [Phi + alpha^2 Phi Q + alpha phi (Q - Phi) - phi^2],   Q = 1 - Phi
// The identity holds for any Phi value (it only uses mu = sigma phi + mz Phi), so it also
// covers the asymptotic branch; the second form has no O(alpha^2) cancellation in fp32.
__device__ __forceinline__ float rect_var(float S, float alpha, float pdf, float cdf, float Q) {
#pragma clang fp contract(off)
  return S * (cdf + alpha * alpha * cdf * Q + alpha * pdf * (Q - cdf) - pdf * pdf);
}

// 1 - x R(x) and (1 + x^2) R(x) - x for x >= 2, where R = Q / phi is the Mills ratio.
// They are about 1/x^2 and 2/x^3, differences of terms near 1 and x: formed from R they
// would carry R's relative rounding multiplied by about x^2 and x^4 / 2 (1e-4 of the
// variance near x = 4). They are evaluated from their own fits instead, g1 = x^2 u1 and
// g2 = x^3 u2 / 2 (both tend to 1 as x grows) as polynomials in t = 1 / (1 + x / (2 sqrt 2)),
// the variable of the erfc fit, t in (0, 0.586] for x >= 2: least squares on Chebyshev
// nodes of values computed at 90 digits (gen_mills_fit.py next to this file), relative
// error 6e-8 / 9e-8 in exact arithmetic and below 2e-7 / 4e-7 in fp32 Horner evaluation.
// No cancellation at any x: t = 0 (x = inf) gives u1 = u2 = 0.
__device__ __forceinline__ void mills_differences(float a, float t, float& u1, float& u2) {
#pragma clang fp contract(off)
  float g1 = 4.963217913e-02f;
  g1 = fmaf(g1, t, -3.676841643e+00f);
  g1 = fmaf(g1, t, 7.277117302e+00f);
  g1 = fmaf(g1, t, -2.912598560e+00f);
  g1 = fmaf(g1, t, 3.630294165e-01f);
  g1 = fmaf(g1, t, -1.046916153e+00f);
  g1 = fmaf(g1, t, -7.352366037e-01f);
  g1 = fmaf(g1, t, -3.756972988e-01f);
  g1 = fmaf(g1, t, 1.265216389e-05f);
  g1 = fmaf(g1, t, 9.999999624e-01f);
  float g2 = 1.280788407e+01f;
  g2 = fmaf(g2, t, -2.014247635e+01f);
  g2 = fmaf(g2, t, -3.991492743e+00f);
  g2 = fmaf(g2, t, 1.672760442e+01f);
  g2 = fmaf(g2, t, -3.405939506e+00f);
  g2 = fmaf(g2, t, 1.312790107e+00f);
  g2 = fmaf(g2, t, -1.765867478e+00f);
  g2 = fmaf(g2, t, -1.482223791e+00f);
  g2 = fmaf(g2, t, -7.507189017e-01f);
  g2 = fmaf(g2, t, 1.112854611e-05f);
  g2 = fmaf(g2, t, 9.999999719e-01f);
  const float r = fast_rcp(a);
  const float r2 = r * r;
  u1 = g1 * r2;
  u2 = 2.0f * g2 * r2 * r;
}

// Moments of max(z, 0) for z ~ N(mz, S), sd = sqrt(S), alpha = mz / sd, without the
// fp32 cancellation of their two terms for alpha < 0 (layers/remax.py:60-75 in exact
// arithmetic). Out: mean, variance and Phi(alpha) (the density pdf is returned too).
// With a = |alpha|, the Chebyshev fit of normal_tail writes Q(a) = 0.5 t exp(-a^2/2 + P(t));
// its part without the Gaussian factor is the Mills ratio R(a) = Q(a) / phi(a) =
// sqrt(pi/2) t exp(P(t)), so the tail is phi(a) R(a), one exp(-a^2/2) shared by the density
// and the tail. For alpha = -x < 0, with Phi = phi R:
//   mean     = mz Phi + sd phi                         = sd phi (1 - x R)
//   variance = S [Phi + alpha^2 Phi Q + alpha phi (Q - Phi) - phi^2]
//            = S phi [((1 + x^2) R - x) - phi (1 - x R)^2]
// 1 - x R (about 1/x^2) and (1 + x^2) R - x (about 2/x^3) cancel by about x^2 and x^4 / 2.
// Below x = 2 (at most 8-fold) they are formed from R with exact products (fma), so the
// cancellation meets only R's own rounding (a few 1e-7) and not the independent roundings
// of two exponentials; from x = 2 on they come from fits of their own
// (mills_differences), without cancellation. Either way the variance near alpha = -4,
// which sits just above the Remax's 1e-6 floor there and sets its Jacobian, keeps the
// relative accuracy of its terms (the density and the tail formed independently gave
// 1e-4 of it). For alpha >= 0 the terms do not cancel and the forms are the reference's
// (mean) and rect_var's (variance).
__device__ __forceinline__ void rect_moments(float mz, float S, float sd, float alpha, float& mean, float& var,
                                             float& cdf, float& pdf) {
#pragma clang fp contract(off)
  const float a = fabsf(alpha);
  const float z = a * INV_SQRT_2;
  const float t = fast_rcp(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  p = fmaf(p, t, -1.26551223f);
  const float SQRT_PI_2 = 1.2533141373155003f;  // sqrt(pi / 2)
  // p lies in [-1.266, 0] for t in (0, 1], so the rounding of p log2(e) moves exp(p) by at
  // most 1e-7 relative: the plain 2^(p log2 e) serves, without fast_exp's split product
  const float mills = SQRT_PI_2 * t * __builtin_amdgcn_exp2f(p * 1.44269502162933349609375f);
  pdf = INV_SQRT_2PI * fast_exp(-0.5f * a * a);
  const float tail = pdf * mills;
  if (alpha >= 0.0f) {
    cdf = 1.0f - tail;
    mean = fmaf(mz, cdf, sd * pdf);
    var = rect_var(S, alpha, pdf, cdf, tail);
  } else {
    float u1, u2;
    if (a >= 2.0f) {
      mills_differences(a, t, u1, u2);
    } else {
      u1 = fmaf(-a, mills, 1.0f);                 // 1 - x R
      u2 = fmaf(fmaf(a, a, 1.0f), mills, -a);      // (1 + x^2) R - x
    }
    cdf = tail;
    mean = sd * pdf * u1;
    var = S * pdf * fmaf(-pdf * u1, u1, u2);
  }
}

__device__ __forceinline__ void relu_moments(float mz, float Sz, float& ma, float& Sa, float& J) {
#pragma clang fp contract(off)
  const float Ss = fmaxf(Sz, 1e-30f);
  const float rs = fast_rsqrt(Ss);
  const float sig = Ss * rs;
  const float alpha = mz * rs;
  const float pdf = fast_exp(-0.5f * alpha * alpha) * INV_SQRT_2PI;
  // Phi(alpha) = 0.5 (1 + erf(alpha/sqrt2)) is taken from the normal tail: equal in exact
  // arithmetic, without the fp32 cancellation of the erf form for alpha < 0.
  const bool asym = alpha < -5.0f;
  float cdf_e, Q_e;
  normal_cdf_pair(alpha, cdf_e, Q_e);
  const float cdf = asym ? fast_div(pdf, -alpha) : cdf_e;
  const float Q = asym ? 1.0f - cdf : Q_e;
  ma = fmaf(mz, cdf, sig * pdf);
  Sa = fmaxf(rect_var(Ss, alpha, pdf, cdf, Q), 0.0f);
  J = cdf;
}

// Sum over a 64-lane wavefront; every lane gets the same total. Pairs of lanes are added
// in registers, without the LDS crossbar that __shfl_xor goes through: DPP quad
// permutations (lane ^ 1, lane ^ 2), the 8-lane and 16-lane mirrors (lane i with 7 - i,
// then with 15 - i, within each 16-lane row), then v_permlane16_swap (rows 0 <-> 1,
// 2 <-> 3) and v_permlane32_swap (lanes 0-31 <-> 32-63). Each step adds two partial sums
// that cover disjoint lane sets, and fp32 addition commutes, so all lanes hold the
// bit-identical total.
__device__ __forceinline__ float wave_sum(float v) {
  int x;
  x = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  v += __int_as_float(x);
  x = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  v += __int_as_float(x);
  x = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __int_as_float(x);
  x = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false);  // row_mirror
  v += __int_as_float(x);
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Remax of one row of K <= 64*EPT classes held by a wavefront (remax.py:33-114): lane
// holds classes lane + 64e. In: the row's moments (any values past K). Out: mu_a, S_a and
// the Jacobian J = cov(a, z) / S_z, valid for the lane's classes below K.
template <int EPT>
__device__ __forceinline__ void remax_row(const float (&mz)[EPT], const float (&Sz)[EPT], int lane, int K,
                                          float (&ma)[EPT], float (&Sa)[EPT], float (&Jo)[EPT]) {
#pragma clang fp contract(off)
  const float EPS = 1e-6f;
  float var_z[EPT], mu_m[EPT], var_m[EPT], jcb[EPT];
  float s_mu = 0.f, s_var = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const bool ok = lane + 64 * e < K;
    const float m = mz[e];
    const float v = Sz[e];
    const float rs = fast_rsqrt(v);
    const float sd = v * rs;
    const float al = m * rs;
    float mraw, vrect, cdf, pdf;
    rect_moments(m, v, sd, al, mraw, vrect, cdf, pdf);
    const float mm = fmaxf(mraw, EPS);
    // The reference's variance -mm^2 + 2 mm m - m sd pdf + (v - m^2) cdf (remax.py:68-73)
    // with mm its floored mean equals vrect + (mraw - mm)(mraw + mm - 2 m) exactly, vrect
    // being the variance of max(z, 0) at its own mean mraw (see rect_moments): the second
    // term is 0 while the floor is inactive and is formed from two differences otherwise.
    const float vraw = (mraw >= EPS) ? vrect : fmaf(mraw - EPS, (mraw + EPS) - 2.0f * m, vrect);
    const float vm = fmaxf(vraw, EPS);
    var_z[e] = v;
    mu_m[e] = mm;
    var_m[e] = vm;
    jcb[e] = cdf;
    if (ok) {
      s_mu += mm;
      s_var += vm;
    }
  }
  const float mu_mt = fmaxf(wave_sum(s_mu), EPS);
  const float var_mt = fmaxf(wave_sum(s_var), EPS);
  const float inv_mt = fast_rcp(mu_mt);
  // The reference's log-normal stage (remax.py:82-105) in closed form. With
  //   x = S_m / mu_m^2,  y = S_mt / mu_mt^2,  w = S_m / (mu_m mu_mt)
  // its logarithms are var_log_m = log(1+x), var_log_mt = log(1+y), cov_log_m_mt = log(1+w),
  // and its exponentials collapse to
  //   mu_a_raw = exp(mu_log_a + var_log_a / 2)      = (mu_m / mu_mt) (1+y) / (1+w)
  //   exp(var_log_a) - 1 = (1+x)(1+y)/(1+w)^2 - 1    = (x - w + y - w + xy - w^2) / (1+w)^2
  //   exp(cov_log_a_log_m) - 1 = (1+x)/(1+w) - 1     = (x - w) / (1+w)
  // Both differences are >= 0 in exact arithmetic (mu_m <= mu_mt and S_m <= S_mt give
  // w <= x and w^2 <= xy, so (1+w)^2 <= (1+x)(1+y)); the reference's clamp of var_log_a at 0
  // and the one here act on rounding only. No logarithm or exponential is left, and the
  // small differences are formed from their terms (absolute error a few ulp of x, y, w)
  // instead of from logarithms of 1 + x (an fp32 emulation against float64 puts this form
  // at or below the log form's error on every row distribution tried).
  const float y = var_mt * inv_mt * inv_mt;
  const float c_mt = inv_mt * (1.0f + y);
  float x_m[EPT], w_m[EPT], rw_m[EPT], mu_a_raw[EPT];
  float s_a = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const float rm = fast_rcp(mu_m[e]);
    const float vr = var_m[e] * rm;
    const float x = vr * rm;
    const float w = vr * inv_mt;
    const float rw = fast_rcp(1.0f + w);
    const float mar = fmaxf(mu_m[e] * c_mt * rw, EPS);
    x_m[e] = x;
    w_m[e] = w;
    rw_m[e] = rw;
    mu_a_raw[e] = mar;
    if (lane + 64 * e < K) s_a += mar;
  }
  const float inv_sum_a = fast_rcp(fmaxf(wave_sum(s_a), EPS));
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const float mua = mu_a_raw[e] * inv_sum_a;
    const float x = x_m[e], w = w_m[e], rw = rw_m[e];
    const float xw = x - w;
    const float num = (xw + (y - w)) + fmaf(x, y, -(w * w));
    const float vara = fmaxf(num, 0.0f) * rw * rw * mua * mua;
    const float cov_am = fmaxf(xw, 0.0f) * rw * mua * mu_m[e];
    const float cs = __builtin_amdgcn_sqrtf(vara * var_z[e]);
    const float cov_az = fminf(cs, cov_am * fast_rcp(fmaxf(jcb[e], EPS)));
    ma[e] = mua;
    Sa[e] = vara;
    Jo[e] = cov_az * fast_rcp(var_z[e]);
  }
}

}  // namespace tagi
