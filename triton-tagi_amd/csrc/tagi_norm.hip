// BatchNorm2D, RMSNorm, Embedding and positional-encoding kernels.
//
// Per-channel / per-column reductions are two-stage and deterministic: blocks write
// partial sums to a caller-provided workspace in a fixed layout, and a small finalize
// kernel adds them in a fixed order (no float atomics anywhere).
#include "tagi_common.h"
#include "tagi_moments.h"

namespace tagi {


// BatchNorm2D on channels-last data: a (rows = N*H*W) x C matrix, channel = column.
// Blocks own contiguous row ranges; in the float4 path each thread keeps one group of 4
// channels for the whole block (C divides 1024), so per-channel constants and partial
// sums stay in registers and every load is a coalesced float4.
static inline bool bn_vec(int64_t C) { return C % 4 == 0 && C <= 1024 && 1024 % C == 0; }

// Reduction grid: blocks own contiguous ranges of about 32 or more rows (at most 1024
// ranges, so a channel has at most 1024 partials) and, in the float4 path, a chunk of the
// channels: chunks halve (down to 16 channels) until the grid has 512 blocks, which keeps
// small layers spread over the CUs while the partials stay a few percent of the traffic.
// Partials are stored quantity-major then channel then row range,
// ws[(q * C + c) * nbr + b], so the finalize pass reads each channel's contiguously.
static inline int red_rows(int64_t rows) {
  int64_t b = cdiv(rows, 32);
  if (b > 1024) b = 1024;
  return (int)(b < 1 ? 1 : b);
}
static inline int red_chunks(int nbr, int64_t C, bool vec) {
  int ncc = 1;
  if (!vec) return ncc;
  for (int64_t W = C; (int64_t)nbr * ncc < 512 && W >= 32; W >>= 1) ncc <<= 1;
  return ncc;
}

// Per-block partial sums over the block's rows (finalized by the kernels below).
//   MODE 0  statistics of (mu, S):                   sums mu, S, mu^2
//   MODE 1  statistics of ReLU(mu, S), writes y0 = J: sums mu_a, S_a, mu_a^2
//   MODE 2  backward, x0 = dmu, x1 = dS, x2 = mhat:   y0 = dmu g/sqrt(var+eps),
//           y1 = dS g^2/(var+eps); sums dmu mhat, dS mhat^2, dmu, dS
//   MODE 3  MODE 2 followed by the Jacobian of the ReLU in front of the BN (x3 = J):
//           y0 = (dmu g/sqrt(var+eps)) J, y1 = (dS g^2/(var+eps)) J^2; same sums
//   MODE 4  MODE 3, plus the sums of y0 and y1 (the bias sums of the convolution in
//           front of the ReLU, whose output deltas y0, y1 are)
template <int MODE>
struct BnRed {
  static constexpr int NQ = MODE == 4 ? 6 : (MODE >= 2 ? 4 : 3);
  __device__ __forceinline__ static void elem(float a, float b, float h, float j, float km, float kS, float* acc,
                                              float& o0, float& o1) {
    if constexpr (MODE == 0) {
      acc[0] += a;
      acc[1] += b;
      acc[2] += a * a;
    } else if constexpr (MODE == 1) {
      float ma, Sa, J;
      relu_moments(a, b, ma, Sa, J);
      acc[0] += ma;
      acc[1] += Sa;
      acc[2] += ma * ma;
      o0 = J;
    } else {
      acc[0] += a * h;
      acc[1] += b * h * h;
      acc[2] += a;
      acc[3] += b;
      o0 = a * km;
      o1 = b * kS;
      if constexpr (MODE >= 3) {
        o0 = o0 * j;
        o1 = o1 * j * j;
      }
      if constexpr (MODE == 4) {
        acc[4] += o0;
        acc[5] += o1;
      }
    }
  }
};

template <int MODE, bool VEC>
__global__ void __launch_bounds__(256) bn_reduce_kernel(const float* __restrict__ x0, const float* __restrict__ x1,
                                                        const float* __restrict__ x2, const float* __restrict__ x3,
                                                        float* __restrict__ ws, int64_t rows, int C, int nblk,
                                                        const float* __restrict__ var, const float* __restrict__ mg,
                                                        float* __restrict__ y0, float* __restrict__ y1, float eps) {
  using R = BnRed<MODE>;
  constexpr int NQ = R::NQ;
  // per-thread partials, quantity-major with the thread index fastest (one bank per lane
  // on the stores); the combine reads them with the channel's 4 lanes of a float4 group
  // spread over the rows
  constexpr int RP = 256 + 4;
  __shared__ float red[4 * NQ * RP];
  const int64_t r0 = rows * blockIdx.x / nblk, r1 = rows * (blockIdx.x + 1) / nblk;
  const int t = threadIdx.x;
  if constexpr (VEC) {
    const int W = C / (int)gridDim.y, c0 = (int)blockIdx.y * W;  // this block's channel chunk
    const int cq = W >> 2, rpi = 256 / cq;
    const int c4 = t % cq, rr = t / cq;
    float acc[4][NQ];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < NQ; ++q) acc[j][q] = 0.f;
    float km[4] = {0, 0, 0, 0}, kS[4] = {0, 0, 0, 0};
    if constexpr (MODE >= 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = c0 + 4 * c4 + j;
        const float rv = var[c] + eps;
        km[j] = mg[c] * (1.0f / sqrtf(rv));
        kS[j] = mg[c] * mg[c] * (1.0f / rv);
      }
    }
#pragma unroll 2
    for (int64_t row = r0 + rr; row < r1; row += rpi) {
      const int64_t off = row * C + c0 + 4 * c4;
      const float4 a = *reinterpret_cast<const float4*>(x0 + off);
      const float4 b = *reinterpret_cast<const float4*>(x1 + off);
      float4 h = make_float4(0.f, 0.f, 0.f, 0.f), jj = h;
      if constexpr (MODE >= 2) h = *reinterpret_cast<const float4*>(x2 + off);
      if constexpr (MODE >= 3) jj = *reinterpret_cast<const float4*>(x3 + off);
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
      const float hv[4] = {h.x, h.y, h.z, h.w}, jv[4] = {jj.x, jj.y, jj.z, jj.w};
      float o0[4], o1[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) R::elem(av[j], bv[j], hv[j], jv[j], km[j], kS[j], acc[j], o0[j], o1[j]);
      if constexpr (MODE >= 1) *reinterpret_cast<float4*>(y0 + off) = make_float4(o0[0], o0[1], o0[2], o0[3]);
      if constexpr (MODE >= 2) *reinterpret_cast<float4*>(y1 + off) = make_float4(o1[0], o1[1], o1[2], o1[3]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < NQ; ++q) red[(q * 4 + j) * RP + t] = acc[j][q];
    __syncthreads();
    // thread u combines channel 4 * g4 + j of the chunk, u = j * cq + g4 (lanes of one j
    // read consecutive words)
    for (int u = t; u < W; u += 256) {
      const int j = u / cq, g4 = u - j * cq;
      const int cl = 4 * g4 + j;
      for (int q = 0; q < NQ; ++q) {
        float sum = 0.f;
        for (int r = 0; r < rpi; ++r) sum += red[(q * 4 + j) * RP + r * cq + g4];
        ws[((int64_t)q * C + c0 + cl) * nblk + blockIdx.x] = sum;
      }
    }
  } else {
    for (int c = t; c < C; c += 256) {
      float acc[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) acc[q] = 0.f;
      float kmc = 0.f, kSc = 0.f;
      if constexpr (MODE >= 2) {
        const float rv = var[c] + eps;
        kmc = mg[c] * (1.0f / sqrtf(rv));
        kSc = mg[c] * mg[c] * (1.0f / rv);
      }
      for (int64_t row = r0; row < r1; ++row) {
        const int64_t off = row * C + c;
        const float h = MODE >= 2 ? x2[off] : 0.f;
        const float j = MODE >= 3 ? x3[off] : 0.f;
        float o0 = 0.f, o1 = 0.f;
        R::elem(x0[off], x1[off], h, j, kmc, kSc, acc, o0, o1);
        if constexpr (MODE >= 1) y0[off] = o0;
        if constexpr (MODE >= 2) y1[off] = o1;
      }
      for (int q = 0; q < NQ; ++q) ws[((int64_t)q * C + c) * nblk + blockIdx.x] = acc[q];
    }
  }
}

// One 256-thread block per channel: thread t adds partials t, t + 256, ... (contiguous
// across the block), then a fixed butterfly within each wave and a fixed-order sum over
// the four waves, so the result does not depend on timing.
__device__ __forceinline__ float wave_reduce(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int NQ>
__device__ __forceinline__ void channel_sums(const float* __restrict__ ws, int C, int c, int nblk, float* out) {
  __shared__ float part[4][NQ];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  float acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = 0.f;
  // at most 1024 partials: up to 4 iterations, all loads issued together
#pragma unroll 4
  for (int b = t; b < nblk; b += 256) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[q] += ws[((int64_t)q * C + c) * nblk + b];
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = wave_reduce(acc[q]);
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) part[w][q] = acc[q];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NQ; ++q) out[q] = (part[0][q] + part[1][q]) + (part[2][q] + part[3][q]);
}

__global__ void __launch_bounds__(256) bn_stats_finalize_kernel(const float* __restrict__ ws, float* __restrict__ bmean,
                                         float* __restrict__ bvar, float* __restrict__ rmean,
                                         float* __restrict__ rvar, float* __restrict__ mg, int C, int nblk,
                                         double n, float momentum, float eps, int first_call, int preserve_var) {
  const int c = blockIdx.x;
  float sums[3];
  channel_sums<3>(ws, C, c, nblk, sums);
  const float a = sums[0], b = sums[1], q = sums[2];
  if (threadIdx.x != 0) return;
  const float inv = (float)(1.0 / n);
  const float mean = a * inv;
  const float bessel = (float)(n / (n - 1.0));
  const float var = (b * inv + q * inv - mean * mean) * bessel;
  bmean[c] = mean;
  bvar[c] = var;
  if (rmean && rvar) {
    if (first_call) {
      rmean[c] = mean;
      rvar[c] = var;
      if (preserve_var && mg) mg[c] = sqrtf(var + eps);
    } else {
      rmean[c] = (1.0f - momentum) * rmean[c] + momentum * mean;
      rvar[c] = (1.0f - momentum) * rvar[c] + momentum * var;
    }
  }
}

// --------------------------------------------------------------------- BN apply
// Normalise + Gaussian affine (batchnorm2d.py:59-126), optionally on the ReLU moments of
// the input (RELU: the rectified moments are recomputed from mu, S instead of being
// read back) and optionally adding a second Gaussian stream to the output (ADD: the
// residual shortcut of the block the BN closes).
template <bool RELU>
__device__ __forceinline__ void bn_in(float m, float s, float& x, float& v) {
  if constexpr (RELU) {
    float J;
    relu_moments(m, s, x, v, J);
  } else {
    x = m;
    v = s;
  }
}

template <bool RELU, bool ADD>
__global__ void __launch_bounds__(256) bn_apply_vec_kernel(
    const float* __restrict__ mz, const float* __restrict__ Sz, const float* __restrict__ mean,
    const float* __restrict__ var, const float* __restrict__ mg, const float* __restrict__ Sg,
    const float* __restrict__ mb, const float* __restrict__ Sb, const float* __restrict__ am,
    const float* __restrict__ aS, float* __restrict__ ma, float* __restrict__ Sa, float* __restrict__ mhat,
    float* __restrict__ Shat, int64_t rows, int C, int64_t rows_per_block, float eps) {
  const int cq = C >> 2, rpi = 256 / cq;
  const int t = threadIdx.x, c4 = t % cq, rr = t / cq;
  float k_mean[4], k_irv[4], k_is[4], k_g[4], k_sg[4], k_b[4], k_sb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = 4 * c4 + j;
    k_mean[j] = mean[c];
    const float rv = var[c] + eps;
    k_irv[j] = 1.0f / rv;
    k_is[j] = 1.0f / sqrtf(rv);
    k_g[j] = mg[c];
    k_sg[j] = Sg[c];
    k_b[j] = mb[c];
    k_sb[j] = Sb[c];
  }
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
#pragma unroll 2
  for (int64_t row = r0 + rr; row < r1; row += rpi) {
    const int64_t off = row * C + 4 * c4;
    const float4 m4 = *reinterpret_cast<const float4*>(mz + off);
    const float4 s4 = *reinterpret_cast<const float4*>(Sz + off);
    float4 a4 = make_float4(0.f, 0.f, 0.f, 0.f), b4 = a4;
    if constexpr (ADD) {
      a4 = *reinterpret_cast<const float4*>(am + off);
      b4 = *reinterpret_cast<const float4*>(aS + off);
    }
    const float mv[4] = {m4.x, m4.y, m4.z, m4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
    const float av[4] = {a4.x, a4.y, a4.z, a4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
    float mh[4], sh[4], om[4], os[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x, v;
      bn_in<RELU>(mv[j], sv[j], x, v);
      mh[j] = (x - k_mean[j]) * k_is[j];
      sh[j] = v * k_irv[j];
      om[j] = k_g[j] * mh[j] + k_b[j];
      os[j] = k_g[j] * k_g[j] * sh[j] + k_sg[j] * mh[j] * mh[j] + k_sg[j] * sh[j] + k_sb[j];
      if constexpr (ADD) {
        om[j] = om[j] + av[j];
        os[j] = os[j] + bv[j];
      }
    }
    *reinterpret_cast<float4*>(ma + off) = make_float4(om[0], om[1], om[2], om[3]);
    *reinterpret_cast<float4*>(Sa + off) = make_float4(os[0], os[1], os[2], os[3]);
    *reinterpret_cast<float4*>(mhat + off) = make_float4(mh[0], mh[1], mh[2], mh[3]);
    if (Shat) *reinterpret_cast<float4*>(Shat + off) = make_float4(sh[0], sh[1], sh[2], sh[3]);
  }
}

template <bool RELU, bool ADD>
__global__ void bn_apply_scalar_kernel(const float* __restrict__ mz, const float* __restrict__ Sz,
                                       const float* __restrict__ mean, const float* __restrict__ var,
                                       const float* __restrict__ mg, const float* __restrict__ Sg,
                                       const float* __restrict__ mb, const float* __restrict__ Sb,
                                       const float* __restrict__ am, const float* __restrict__ aS,
                                       float* __restrict__ ma, float* __restrict__ Sa, float* __restrict__ mhat,
                                       float* __restrict__ Shat, int64_t total, int C, float eps) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int c = (int)(i % C);
    const float rv = var[c] + eps;
    const float inv_std = 1.0f / sqrtf(rv);
    const float g = mg[c], sg = Sg[c];
    float x, v;
    bn_in<RELU>(mz[i], Sz[i], x, v);
    const float mh = (x - mean[c]) * inv_std;
    const float sh = v * (1.0f / rv);
    float om = g * mh + mb[c];
    float os = g * g * sh + sg * mh * mh + sg * sh + Sb[c];
    if constexpr (ADD) {
      om = om + am[i];
      os = os + aS[i];
    }
    ma[i] = om;
    Sa[i] = os;
    mhat[i] = mh;
    if (Shat) Shat[i] = sh;
  }
}

__global__ void __launch_bounds__(256) bn_bwd_finalize_kernel(const float* __restrict__ ws, const float* __restrict__ Sg,
                                       const float* __restrict__ Sb, float* __restrict__ dmg, float* __restrict__ dSg,
                                       float* __restrict__ dmb, float* __restrict__ dSb, int C, int nblk) {
  const int c = blockIdx.x;
  float sums[4];
  channel_sums<4>(ws, C, c, nblk, sums);
  const float s0 = sums[0], s1 = sums[1], s2 = sums[2], s3 = sums[3];
  if (threadIdx.x != 0) return;
  const float g = Sg[c], b = Sb[c];
  dmg[c] = g * s0;
  dSg[c] = g * g * s1;
  dmb[c] = b * s2;
  dSb[c] = b * b * s3;
}

// The BatchNorm2D parameter-delta pass of several layers in one launch: block b finalizes
// channel b - start[t] of layer t (the same fixed-order sums as bn_bwd_finalize_kernel).
constexpr int kBnMulti = 32;
struct BnFinalizeMulti {
  const float* ws[kBnMulti];
  const float* Sg[kBnMulti];
  const float* Sb[kBnMulti];
  float* dmg[kBnMulti];
  float* dSg[kBnMulti];
  float* dmb[kBnMulti];
  float* dSb[kBnMulti];
  const float* cSb[kBnMulti];  // bias variances of the conv in front (six-sum layers), else null
  float* cdmb[kBnMulti];
  float* cdSb[kBnMulti];
  int C[kBnMulti];
  int nblk[kBnMulti];
  int start[kBnMulti + 1];
  int count;
};

__global__ void __launch_bounds__(256) bn_bwd_finalize_multi_kernel(BnFinalizeMulti a) {
  const int b = blockIdx.x;
  int t = 0;
  while (t + 1 < a.count && a.start[t + 1] <= b) ++t;
  const int c = b - a.start[t];
  float sums[6];
  const bool conv_bias = a.cdmb[t] != nullptr;
  if (conv_bias)
    channel_sums<6>(a.ws[t], a.C[t], c, a.nblk[t], sums);
  else
    channel_sums<4>(a.ws[t], a.C[t], c, a.nblk[t], sums);
  if (threadIdx.x != 0) return;
  const float g = a.Sg[t][c], bb = a.Sb[t][c];
  a.dmg[t][c] = g * sums[0];
  a.dSg[t][c] = g * g * sums[1];
  a.dmb[t][c] = bb * sums[2];
  a.dSb[t][c] = bb * bb * sums[3];
  if (conv_bias) {
    const float cb = a.cSb[t][c];
    a.cdmb[t][c] = cb * sums[4];
    a.cdSb[t][c] = cb * cb * sums[5];
  }
}

// --------------------------------------------------------------------- RMSNorm
// One wavefront per row (rms_norm.py:99-110).
template <int EPT>
__global__ void __launch_bounds__(256) rmsnorm_fwd_kernel(const float* __restrict__ ma, const float* __restrict__ Sa,
                                                          const float* __restrict__ mw, const float* __restrict__ Sw,
                                                          float* __restrict__ mz, float* __restrict__ Sz,
                                                          float* __restrict__ inv_rms, int64_t rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* pm = ma + row * D;
  const float* ps = Sa + row * D;
  float m[EPT], s[EPT];
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = lane + 64 * e;
    m[e] = c < D ? pm[c] : 0.f;
    s[e] = c < D ? ps[c] : 0.f;
    acc += m[e] * m[e] + s[e];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  const float rms = acc / (float)D;
  const float inv = 1.0f / sqrtf(rms + eps);
  if (lane == 0) inv_rms[row] = inv;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = lane + 64 * e;
    if (c >= D) continue;
    const float w = mw[c], sw = Sw[c];
    mz[row * D + c] = inv * m[e] * w;
    Sz[row * D + c] = (inv * inv) * (s[e] * (w * w + sw) + sw * m[e] * m[e]);
  }
}

// Backward (rms_norm.py:115-134): per-row scaling of the deltas plus two per-column sums
// (the weight deltas). Blocks own contiguous row ranges, rows * b / nblk ..; partial sums
// go to ws[(q * D + c) * nblk + b] and are added by the finalize kernel in a fixed order.
// Float4 path (D % 4 == 0 and D divides 1024): each thread keeps one group of 4 columns
// for the block's whole row range, as the BatchNorm reductions do.
__global__ void __launch_bounds__(256) rmsnorm_bwd_partial_vec_kernel(
    const float* __restrict__ dmz, const float* __restrict__ dSz, const float* __restrict__ ma,
    const float* __restrict__ inv_rms, const float* __restrict__ mw, float* __restrict__ dma,
    float* __restrict__ dSa, float* __restrict__ ws, int64_t rows, int D, int nblk) {
  __shared__ float red[256 * 4 * 2];
  const int64_t r0 = rows * blockIdx.x / nblk, r1 = rows * (blockIdx.x + 1) / nblk;
  const int W = D / (int)gridDim.y, c0 = (int)blockIdx.y * W;  // this block's column chunk
  const int cq = W >> 2, rpi = 256 / cq;
  const int t = threadIdx.x, c4 = t % cq, rr = t / cq;
  const float4 w4 = *reinterpret_cast<const float4*>(mw + c0 + 4 * c4);
  const float w[4] = {w4.x, w4.y, w4.z, w4.w};
  float am[4] = {0.f, 0.f, 0.f, 0.f}, as[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int64_t row = r0 + rr; row < r1; row += rpi) {
    const float inv = inv_rms[row];
    const int64_t off = row * D + c0 + 4 * c4;
    const float4 d4 = *reinterpret_cast<const float4*>(dmz + off);
    const float4 s4 = *reinterpret_cast<const float4*>(dSz + off);
    const float4 m4 = *reinterpret_cast<const float4*>(ma + off);
    const float dm[4] = {d4.x, d4.y, d4.z, d4.w}, ds[4] = {s4.x, s4.y, s4.z, s4.w}, m[4] = {m4.x, m4.y, m4.z, m4.w};
    float o0[4], o1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float k = inv * w[j];
      o0[j] = k * dm[j];
      o1[j] = k * k * ds[j];
      am[j] += inv * m[j] * dm[j];
      as[j] += inv * inv * m[j] * m[j] * ds[j];
    }
    *reinterpret_cast<float4*>(dma + off) = make_float4(o0[0], o0[1], o0[2], o0[3]);
    *reinterpret_cast<float4*>(dSa + off) = make_float4(o1[0], o1[1], o1[2], o1[3]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    red[(t * 4 + j) * 2] = am[j];
    red[(t * 4 + j) * 2 + 1] = as[j];
  }
  __syncthreads();
  for (int cl = t; cl < W; cl += 256) {
    const int g4 = cl >> 2, j = cl & 3;
    for (int q = 0; q < 2; ++q) {
      float sum = 0.f;
      for (int r = 0; r < rpi; ++r) sum += red[((r * cq + g4) * 4 + j) * 2 + q];
      ws[((int64_t)q * D + c0 + cl) * nblk + blockIdx.x] = sum;
    }
  }
}

// Scalar path: threads stride over the columns and walk the block's rows.
__global__ void __launch_bounds__(256) rmsnorm_bwd_partial_kernel(
    const float* __restrict__ dmz, const float* __restrict__ dSz, const float* __restrict__ ma,
    const float* __restrict__ inv_rms, const float* __restrict__ mw, float* __restrict__ dma,
    float* __restrict__ dSa, float* __restrict__ ws, int64_t rows, int D, int nblk) {
  const int64_t r0 = rows * blockIdx.x / nblk, r1 = rows * (blockIdx.x + 1) / nblk;
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    const float w = mw[c];
    float s_mu = 0.f, s_var = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
      const float inv = inv_rms[r];
      const int64_t i = r * D + c;
      const float dm = dmz[i], ds = dSz[i], m = ma[i];
      const float k = inv * w;
      dma[i] = k * dm;
      dSa[i] = k * k * ds;
      s_mu += inv * m * dm;
      s_var += inv * inv * m * m * ds;
    }
    ws[(int64_t)c * nblk + blockIdx.x] = s_mu;
    ws[((int64_t)D + c) * nblk + blockIdx.x] = s_var;
  }
}

// One 256-thread block per column (same fixed-order sum as the BatchNorm finalize).
__global__ void __launch_bounds__(256) rmsnorm_bwd_finalize_kernel(const float* __restrict__ ws,
                                                                   const float* __restrict__ Sw,
                                                                   float* __restrict__ dmw, float* __restrict__ dSw,
                                                                   int D, int nblk) {
  const int c = blockIdx.x;
  float sums[2];
  channel_sums<2>(ws, D, c, nblk, sums);
  if (threadIdx.x != 0) return;
  const float sw = Sw[c];
  dmw[c] = sums[0] * sw;
  dSw[c] = sums[1] * sw * sw;
}

// --------------------------------------------------------------------- LayerNorm
// Per-row statistics over the features (layernorm.py:101-135):
//   mu = mean(m),  var = (sum (m - mu)^2 + sum S) / (D - 1),  inv = 1/sqrt(var + eps)
//   mz = inv (m - mu) g + b,   Sz = inv^2 (S (g^2 + Sg) + Sg (m - mu)^2) + Sb
// The mean is formed first and the squared deviations are summed from it, as written.
// One wavefront per row with the row in registers for D <= 1024; one block per row,
// re-reading the row, above that.
template <int EPT>
__global__ void __launch_bounds__(256) layernorm_fwd_kernel(
    const float* __restrict__ ma, const float* __restrict__ Sa, const float* __restrict__ mw,
    const float* __restrict__ Sw, const float* __restrict__ mb, const float* __restrict__ Sb, float* __restrict__ mz,
    float* __restrict__ Sz, float* __restrict__ mu_ra, float* __restrict__ var_ra, int64_t rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* pm = ma + row * D;
  const float* ps = Sa + row * D;
  float m[EPT], s[EPT];
  float sm = 0.f, ss = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = lane + 64 * e;
    m[e] = c < D ? pm[c] : 0.f;
    s[e] = c < D ? ps[c] : 0.f;
    sm += m[e];
    ss += s[e];
  }
  const float mu = wave_reduce(sm) / (float)D;
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const float d = m[e] - mu;
    if (lane + 64 * e < D) sq += d * d;
  }
  const float var = (wave_reduce(sq) + wave_reduce(ss)) / (float)(D - 1);
  const float inv = 1.0f / sqrtf(var + eps);
  if (lane == 0) {
    mu_ra[row] = mu;
    var_ra[row] = var;
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = lane + 64 * e;
    if (c >= D) continue;
    const float g = mw[c], sg = Sw[c], d = m[e] - mu;
    mz[row * D + c] = inv * d * g + mb[c];
    Sz[row * D + c] = (inv * inv) * (s[e] * (g * g + sg) + sg * d * d) + Sb[c];
  }
}

__device__ __forceinline__ float block_sum256(float v, float* sh) {
  v = wave_reduce(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(256) layernorm_fwd_row_kernel(
    const float* __restrict__ ma, const float* __restrict__ Sa, const float* __restrict__ mw,
    const float* __restrict__ Sw, const float* __restrict__ mb, const float* __restrict__ Sb, float* __restrict__ mz,
    float* __restrict__ Sz, float* __restrict__ mu_ra, float* __restrict__ var_ra, int D, float eps) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const float* pm = ma + row * D;
  const float* ps = Sa + row * D;
  float sm = 0.f, ss = 0.f;
  for (int c = threadIdx.x; c < D; c += 256) {
    sm += pm[c];
    ss += ps[c];
  }
  const float mu = block_sum256(sm, sh) / (float)D;
  float sq = 0.f;
  for (int c = threadIdx.x; c < D; c += 256) {
    const float d = pm[c] - mu;
    sq += d * d;
  }
  const float var = (block_sum256(sq, sh) + block_sum256(ss, sh)) / (float)(D - 1);
  const float inv = 1.0f / sqrtf(var + eps);
  if (threadIdx.x == 0) {
    mu_ra[row] = mu;
    var_ra[row] = var;
  }
  for (int c = threadIdx.x; c < D; c += 256) {
    const float g = mw[c], sg = Sw[c], d = pm[c] - mu;
    mz[row * D + c] = inv * d * g + mb[c];
    Sz[row * D + c] = (inv * inv) * (ps[c] * (g * g + sg) + sg * d * d) + Sb[c];
  }
}

// Backward (layernorm.py:140-175), diagonal Jacobian J = inv g per element:
//   delta_m = J delta_mz, delta_S = J^2 delta_Sz, and four per-column sums with
//   h = inv (m - mu): sum h delta_mz, sum h^2 delta_Sz, sum delta_mz, sum delta_Sz,
// scaled by Sg, Sg^2, Sb, Sb^2 in the finalize kernel. Partials as for RMSNorm.
__global__ void __launch_bounds__(256) layernorm_bwd_partial_vec_kernel(
    const float* __restrict__ dmz, const float* __restrict__ dSz, const float* __restrict__ ma,
    const float* __restrict__ mu_ra, const float* __restrict__ var_ra, const float* __restrict__ mw,
    float* __restrict__ dma, float* __restrict__ dSa, float* __restrict__ ws, int64_t rows, int D, int nblk,
    float eps) {
  __shared__ float red[256 * 4 * 4];
  const int64_t r0 = rows * blockIdx.x / nblk, r1 = rows * (blockIdx.x + 1) / nblk;
  const int W = D / (int)gridDim.y, c0 = (int)blockIdx.y * W;  // this block's column chunk
  const int cq = W >> 2, rpi = 256 / cq;
  const int t = threadIdx.x, c4 = t % cq, rr = t / cq;
  const float4 w4 = *reinterpret_cast<const float4*>(mw + c0 + 4 * c4);
  const float w[4] = {w4.x, w4.y, w4.z, w4.w};
  float acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[j][q] = 0.f;
#pragma unroll 2
  for (int64_t row = r0 + rr; row < r1; row += rpi) {
    const float mu = mu_ra[row];
    const float inv = 1.0f / sqrtf(var_ra[row] + eps);
    const int64_t off = row * D + c0 + 4 * c4;
    const float4 d4 = *reinterpret_cast<const float4*>(dmz + off);
    const float4 s4 = *reinterpret_cast<const float4*>(dSz + off);
    const float4 m4 = *reinterpret_cast<const float4*>(ma + off);
    const float dm[4] = {d4.x, d4.y, d4.z, d4.w}, ds[4] = {s4.x, s4.y, s4.z, s4.w}, m[4] = {m4.x, m4.y, m4.z, m4.w};
    float o0[4], o1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float k = inv * w[j];
      const float h = inv * (m[j] - mu);
      o0[j] = k * dm[j];
      o1[j] = k * k * ds[j];
      acc[j][0] += h * dm[j];
      acc[j][1] += h * h * ds[j];
      acc[j][2] += dm[j];
      acc[j][3] += ds[j];
    }
    *reinterpret_cast<float4*>(dma + off) = make_float4(o0[0], o0[1], o0[2], o0[3]);
    *reinterpret_cast<float4*>(dSa + off) = make_float4(o1[0], o1[1], o1[2], o1[3]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(t * 4 + j) * 4 + q] = acc[j][q];
  __syncthreads();
  for (int cl = t; cl < W; cl += 256) {
    const int g4 = cl >> 2, j = cl & 3;
    for (int q = 0; q < 4; ++q) {
      float sum = 0.f;
      for (int r = 0; r < rpi; ++r) sum += red[((r * cq + g4) * 4 + j) * 4 + q];
      ws[((int64_t)q * D + c0 + cl) * nblk + blockIdx.x] = sum;
    }
  }
}

__global__ void __launch_bounds__(256) layernorm_bwd_partial_kernel(
    const float* __restrict__ dmz, const float* __restrict__ dSz, const float* __restrict__ ma,
    const float* __restrict__ mu_ra, const float* __restrict__ var_ra, const float* __restrict__ mw,
    float* __restrict__ dma, float* __restrict__ dSa, float* __restrict__ ws, int64_t rows, int D, int nblk,
    float eps) {
  const int64_t r0 = rows * blockIdx.x / nblk, r1 = rows * (blockIdx.x + 1) / nblk;
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    const float w = mw[c];
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t r = r0; r < r1; ++r) {
      const float inv = 1.0f / sqrtf(var_ra[r] + eps);
      const int64_t i = r * D + c;
      const float dm = dmz[i], ds = dSz[i], h = inv * (ma[i] - mu_ra[r]);
      const float k = inv * w;
      dma[i] = k * dm;
      dSa[i] = k * k * ds;
      acc[0] += h * dm;
      acc[1] += h * h * ds;
      acc[2] += dm;
      acc[3] += ds;
    }
    for (int q = 0; q < 4; ++q) ws[((int64_t)q * D + c) * nblk + blockIdx.x] = acc[q];
  }
}

__global__ void __launch_bounds__(256) layernorm_bwd_finalize_kernel(const float* __restrict__ ws,
                                                                     const float* __restrict__ Sw,
                                                                     const float* __restrict__ Sb,
                                                                     float* __restrict__ dmw, float* __restrict__ dSw,
                                                                     float* __restrict__ dmb, float* __restrict__ dSb,
                                                                     int D, int nblk) {
  const int c = blockIdx.x;
  float sums[4];
  channel_sums<4>(ws, D, c, nblk, sums);
  if (threadIdx.x != 0) return;
  const float sw = Sw[c], sb = Sb[c];
  dmw[c] = sw * sums[0];
  dSw[c] = sw * sw * sums[1];
  dmb[c] = sb * sums[2];
  dSb[c] = sb * sb * sums[3];
}

// ------------------------------------------------------------------- Embedding
__device__ __forceinline__ int64_t token_id(float t) { return (int64_t)t; }  // truncation, as .long()

__global__ void embedding_fwd_kernel(const float* __restrict__ tokens, const float* __restrict__ mw,
                                     const float* __restrict__ Sw, float* __restrict__ mz, float* __restrict__ Sz,
                                     int64_t n_tokens, int64_t V, int D, int64_t padding_idx) {
  const int64_t total = n_tokens * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / D;
    const int d = (int)(i - t * D);
    const int64_t cat = token_id(tokens[t]);
    const bool ok = cat >= 0 && cat < V && cat != padding_idx;
    mz[i] = ok ? mw[cat * D + d] : 0.f;
    Sz[i] = ok ? Sw[cat * D + d] : 0.f;
  }
}

// Float4 gather (D % 4 == 0 and D / 4 dividing 256): D/4 threads per token, 256 / (D/4)
// tokens per block.
__global__ void __launch_bounds__(256) embedding_fwd_vec_kernel(const float* __restrict__ tokens,
                                                                const float* __restrict__ mw,
                                                                const float* __restrict__ Sw, float* __restrict__ mz,
                                                                float* __restrict__ Sz, int64_t n_tokens, int64_t V,
                                                                int D, int64_t padding_idx) {
  const int D4 = D >> 2, tpb = 256 / D4;
  const int64_t t = (int64_t)blockIdx.x * tpb + threadIdx.x / D4;
  const int d = (threadIdx.x % D4) * 4;
  if (t >= n_tokens) return;
  const int64_t cat = token_id(tokens[t]);
  const bool ok = cat >= 0 && cat < V && cat != padding_idx;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 m = ok ? *reinterpret_cast<const float4*>(mw + cat * D + d) : z;
  const float4 v = ok ? *reinterpret_cast<const float4*>(Sw + cat * D + d) : z;
  *reinterpret_cast<float4*>(mz + t * D + d) = m;
  *reinterpret_cast<float4*>(Sz + t * D + d) = v;
}

// -------------------------------------------------------------------------- PE
__global__ void pe_add_kernel(const float* __restrict__ ma, const float* __restrict__ pe, float* __restrict__ out,
                              int64_t total, int64_t SE) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = ma[i] + pe[i % SE];
}


}  // namespace tagi

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

extern "C" int64_t tagi_bn_stats_ws_bytes(int64_t N, int64_t C, int64_t HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  return (int64_t)red_rows(N * HW) * C * 3 * (int64_t)sizeof(float);
}

static inline bool al16p(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int tagi::bn_stats_finalize(const char* what, const float* ws, int nblk, int64_t rows, int64_t C, float* batch_mean,
                            float* batch_var, float* running_mean, float* running_var, float* mg, float momentum,
                            float eps, int first_call, int preserve_var, hipStream_t s) {
  hipLaunchKernelGGL(bn_stats_finalize_kernel, dim3((unsigned)C), dim3(256), 0, s, ws, batch_mean, batch_var,
                     running_mean, running_var, mg, (int)C, nblk, (double)rows, momentum, eps, first_call,
                     preserve_var);
  return check_launch(what);
}

// Statistics pass (MODE 0 or 1) + finalize: batch mean/var and running-stat bookkeeping.
static int bn_stats_impl(const char* what, bool relu, const float* mz, const float* Sz, float* J, float* batch_mean,
                         float* batch_var, float* running_mean, float* running_var, float* mg, int64_t N, int64_t C,
                         int64_t HW, float momentum, float eps, int first_call, int preserve_var, float* ws,
                         int64_t ws_bytes, tagi_stream_t stream) {
  TAGI_REQUIRE(mz && Sz && batch_mean && batch_var && ws && (!relu || J), "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && HW > 0 && N * HW > 1, "%s: bad sizes", what);
  TAGI_REQUIRE(N * C * HW < (1ll << 40), "%s: too large", what);
  TAGI_REQUIRE(ws_bytes >= tagi_bn_stats_ws_bytes(N, C, HW), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BN_STATS, s, 0.0, (relu ? 12.0 : 8.0) * N * C * HW);
  const int64_t rows = N * HW;
  const int nblk = red_rows(rows);
  const bool vec = bn_vec(C) && al16p(mz) && al16p(Sz) && (!relu || al16p(J));
  const dim3 grid(nblk, red_chunks(nblk, C, vec)), blk(256);
  if (relu) {
    if (vec)
      hipLaunchKernelGGL((bn_reduce_kernel<1, true>), grid, blk, 0, s, mz, Sz, nullptr, nullptr, ws, rows, (int)C,
                         nblk, nullptr, nullptr, J, nullptr, 0.f);
    else
      hipLaunchKernelGGL((bn_reduce_kernel<1, false>), grid, blk, 0, s, mz, Sz, nullptr, nullptr, ws, rows, (int)C,
                         nblk, nullptr, nullptr, J, nullptr, 0.f);
  } else {
    if (vec)
      hipLaunchKernelGGL((bn_reduce_kernel<0, true>), grid, blk, 0, s, mz, Sz, nullptr, nullptr, ws, rows, (int)C,
                         nblk, nullptr, nullptr, nullptr, nullptr, 0.f);
    else
      hipLaunchKernelGGL((bn_reduce_kernel<0, false>), grid, blk, 0, s, mz, Sz, nullptr, nullptr, ws, rows, (int)C,
                         nblk, nullptr, nullptr, nullptr, nullptr, 0.f);
  }
  int rc = check_launch(what);
  if (rc) return rc;
  return bn_stats_finalize(what, ws, nblk, rows, C, batch_mean, batch_var, running_mean, running_var, mg, momentum,
                           eps, first_call, preserve_var, s);
}

extern "C" int tagi_bn_stats(const float* mz, const float* Sz, float* batch_mean, float* batch_var,
                             float* running_mean, float* running_var, float* mg, int64_t N, int64_t C, int64_t HW,
                             float momentum, float eps, int first_call, int preserve_var, float* ws, int64_t ws_bytes,
                             tagi_stream_t stream) {
  return bn_stats_impl("tagi_bn_stats", false, mz, Sz, nullptr, batch_mean, batch_var, running_mean, running_var, mg,
                       N, C, HW, momentum, eps, first_call, preserve_var, ws, ws_bytes, stream);
}

extern "C" int tagi_relu_bn_stats(const float* mz, const float* Sz, float* J, float* batch_mean, float* batch_var,
                                  float* running_mean, float* running_var, float* mg, int64_t N, int64_t C, int64_t HW,
                                  float momentum, float eps, int first_call, int preserve_var, float* ws,
                                  int64_t ws_bytes, tagi_stream_t stream) {
  return bn_stats_impl("tagi_relu_bn_stats", true, mz, Sz, J, batch_mean, batch_var, running_mean, running_var, mg,
                       N, C, HW, momentum, eps, first_call, preserve_var, ws, ws_bytes, stream);
}

static int bn_apply_impl(const char* what, bool relu, const float* mz, const float* Sz, const float* mean,
                         const float* var, const float* mg, const float* Sg, const float* mb, const float* Sb,
                         const float* am, const float* aS, float* ma, float* Sa, float* mhat, float* Shat, int64_t N,
                         int64_t C, int64_t HW, float eps, tagi_stream_t stream) {
  TAGI_REQUIRE(mz && Sz && mean && var && mg && Sg && mb && Sb && ma && Sa && mhat, "%s: null pointer", what);
  TAGI_REQUIRE((am == nullptr) == (aS == nullptr), "%s: add_m and add_S must both be given or both be NULL", what);
  TAGI_REQUIRE(N > 0 && C > 0 && HW > 0, "%s: bad sizes", what);
  hipStream_t s = as_stream(stream);
  const int64_t total = N * C * HW;
  const bool add = am != nullptr;
  ProfScope ps(FAM_BN_FWD, s, 0.0, 4.0 * total * ((Shat ? 6 : 5) + (add ? 2 : 0)));
  const bool vec = bn_vec(C) && al16p(mz) && al16p(Sz) && al16p(ma) && al16p(Sa) && al16p(mhat) &&
                   (Shat == nullptr || al16p(Shat)) && (!add || (al16p(am) && al16p(aS)));
  if (vec) {
    const int64_t rows = N * HW;
    const int rpi = (int)(256 / (C / 4));
    // up to four float4 rows per thread, fewer when that leaves under ~1024 blocks
    int64_t per = cdiv(rows, (int64_t)rpi * 1024);
    per = per < 1 ? 1 : (per > 4 ? 4 : per);
    const int64_t rpb = (int64_t)rpi * per;
    const int64_t blocks = cdiv(rows, rpb);
    const dim3 grid((unsigned)blocks), blk(256);
#define TAGI_BN_APPLY(R, A)                                                                                         \
  hipLaunchKernelGGL((bn_apply_vec_kernel<R, A>), grid, blk, 0, s, mz, Sz, mean, var, mg, Sg, mb, Sb, am, aS, ma, \
                     Sa, mhat, Shat, rows, (int)C, rpb, eps)
    if (relu && add) TAGI_BN_APPLY(true, true);
    else if (relu) TAGI_BN_APPLY(true, false);
    else if (add) TAGI_BN_APPLY(false, true);
    else TAGI_BN_APPLY(false, false);
#undef TAGI_BN_APPLY
  } else {
    const dim3 grid(ew_blocks(total, 256)), blk(256);
#define TAGI_BN_APPLY(R, A)                                                                                           \
  hipLaunchKernelGGL((bn_apply_scalar_kernel<R, A>), grid, blk, 0, s, mz, Sz, mean, var, mg, Sg, mb, Sb, am, aS, ma, \
                     Sa, mhat, Shat, total, (int)C, eps)
    if (relu && add) TAGI_BN_APPLY(true, true);
    else if (relu) TAGI_BN_APPLY(true, false);
    else if (add) TAGI_BN_APPLY(false, true);
    else TAGI_BN_APPLY(false, false);
#undef TAGI_BN_APPLY
  }
  return check_launch(what);
}

extern "C" int tagi_bn_fwd(const float* mz, const float* Sz, const float* mean, const float* var, const float* mg,
                           const float* Sg, const float* mb, const float* Sb, float* ma, float* Sa, float* mhat,
                           float* Shat, int64_t N, int64_t C, int64_t HW, float eps, tagi_stream_t stream) {
  return bn_apply_impl("tagi_bn_fwd", false, mz, Sz, mean, var, mg, Sg, mb, Sb, nullptr, nullptr, ma, Sa, mhat, Shat,
                       N, C, HW, eps, stream);
}

extern "C" int tagi_relu_bn_fwd(const float* mz, const float* Sz, const float* mean, const float* var,
                                const float* mg, const float* Sg, const float* mb, const float* Sb, const float* add_m,
                                const float* add_S, float* ma, float* Sa, float* mhat, int64_t N, int64_t C,
                                int64_t HW, float eps, tagi_stream_t stream) {
  return bn_apply_impl("tagi_relu_bn_fwd", true, mz, Sz, mean, var, mg, Sg, mb, Sb, add_m, add_S, ma, Sa, mhat,
                       nullptr, N, C, HW, eps, stream);
}

extern "C" int64_t tagi_bn_bwd_ws_bytes(int64_t N, int64_t C, int64_t HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  return (int64_t)red_rows(N * HW) * C * 4 * (int64_t)sizeof(float);
}

extern "C" int64_t tagi_bn_relu_bwd_bias_ws_bytes(int64_t N, int64_t C, int64_t HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  return (int64_t)red_rows(N * HW) * C * 6 * (int64_t)sizeof(float);
}

static int bn_bwd_impl(const char* what, const float* dma, const float* dSa, const float* mhat, const float* J,
                       const float* var, const float* mg, const float* Sg, const float* Sb, float* dmz, float* dSz,
                       float* dmg, float* dSg, float* dmb, float* dSb, int64_t N, int64_t C, int64_t HW, float eps,
                       float* ws, int64_t ws_bytes, tagi_stream_t stream, bool jac, bool finalize = true,
                       bool bias_sums = false) {
  TAGI_REQUIRE(dma && dSa && mhat && var && mg && dmz && dSz && ws && (!jac || J) &&
                   (!finalize || (Sg && Sb && dmg && dSg && dmb && dSb)),
               "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && HW > 0, "%s: bad sizes", what);
  TAGI_REQUIRE(ws_bytes >= (bias_sums ? tagi_bn_relu_bwd_bias_ws_bytes(N, C, HW) : tagi_bn_bwd_ws_bytes(N, C, HW)),
               "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BN_BWD, s, 0.0, (jac ? 24.0 : 20.0) * N * C * HW);
  const int64_t rows = N * HW;
  const int nblk = red_rows(rows);
  const bool vec = bn_vec(C) && al16p(dma) && al16p(dSa) && al16p(mhat) && al16p(dmz) && al16p(dSz) &&
                   (!jac || al16p(J));
  const dim3 grid(nblk, red_chunks(nblk, C, vec)), blk(256);
  if (bias_sums) {
    if (vec)
      hipLaunchKernelGGL((bn_reduce_kernel<4, true>), grid, blk, 0, s, dma, dSa, mhat, J, ws, rows, (int)C, nblk, var,
                         mg, dmz, dSz, eps);
    else
      hipLaunchKernelGGL((bn_reduce_kernel<4, false>), grid, blk, 0, s, dma, dSa, mhat, J, ws, rows, (int)C, nblk,
                         var, mg, dmz, dSz, eps);
  } else if (jac) {
    if (vec)
      hipLaunchKernelGGL((bn_reduce_kernel<3, true>), grid, blk, 0, s, dma, dSa, mhat, J, ws, rows, (int)C, nblk, var,
                         mg, dmz, dSz, eps);
    else
      hipLaunchKernelGGL((bn_reduce_kernel<3, false>), grid, blk, 0, s, dma, dSa, mhat, J, ws, rows, (int)C, nblk,
                         var, mg, dmz, dSz, eps);
  } else {
    if (vec)
      hipLaunchKernelGGL((bn_reduce_kernel<2, true>), grid, blk, 0, s, dma, dSa, mhat, nullptr, ws, rows, (int)C,
                         nblk, var, mg, dmz, dSz, eps);
    else
      hipLaunchKernelGGL((bn_reduce_kernel<2, false>), grid, blk, 0, s, dma, dSa, mhat, nullptr, ws, rows, (int)C,
                         nblk, var, mg, dmz, dSz, eps);
  }
  int rc = check_launch(what);
  if (rc || !finalize) return rc;
  hipLaunchKernelGGL(bn_bwd_finalize_kernel, dim3((unsigned)C), dim3(256), 0, s, (const float*)ws, Sg, Sb,
                     dmg, dSg, dmb, dSb, (int)C, nblk);
  return check_launch(what);
}

extern "C" int tagi_bn_bwd(const float* dma, const float* dSa, const float* mhat, const float* var, const float* mg,
                           const float* Sg, const float* Sb, float* dmz, float* dSz, float* dmg, float* dSg,
                           float* dmb, float* dSb, int64_t N, int64_t C, int64_t HW, float eps, float* ws,
                           int64_t ws_bytes, tagi_stream_t stream) {
  return bn_bwd_impl("tagi_bn_bwd", dma, dSa, mhat, nullptr, var, mg, Sg, Sb, dmz, dSz, dmg, dSg, dmb, dSb, N, C, HW,
                     eps, ws, ws_bytes, stream, false);
}

extern "C" int tagi_bn_relu_bwd(const float* dma, const float* dSa, const float* mhat, const float* J,
                                const float* var, const float* mg, const float* Sg, const float* Sb, float* dmz,
                                float* dSz, float* dmg, float* dSg, float* dmb, float* dSb, int64_t N, int64_t C,
                                int64_t HW, float eps, float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  return bn_bwd_impl("tagi_bn_relu_bwd", dma, dSa, mhat, J, var, mg, Sg, Sb, dmz, dSz, dmg, dSg, dmb, dSb, N, C, HW,
                     eps, ws, ws_bytes, stream, true);
}

extern "C" int tagi_bn_relu_bwd_partials(const float* dma, const float* dSa, const float* mhat, const float* J,
                                         const float* var, const float* mg, float* dmz, float* dSz, int64_t N,
                                         int64_t C, int64_t HW, float eps, float* ws, int64_t ws_bytes,
                                         tagi_stream_t stream) {
  return bn_bwd_impl("tagi_bn_relu_bwd_partials", dma, dSa, mhat, J, var, mg, nullptr, nullptr, dmz, dSz, nullptr,
                     nullptr, nullptr, nullptr, N, C, HW, eps, ws, ws_bytes, stream, true, false);
}

extern "C" int tagi_bn_relu_bwd_partials_bias(const float* dma, const float* dSa, const float* mhat, const float* J,
                                              const float* var, const float* mg, float* dmz, float* dSz, int64_t N,
                                              int64_t C, int64_t HW, float eps, float* ws, int64_t ws_bytes,
                                              tagi_stream_t stream) {
  return bn_bwd_impl("tagi_bn_relu_bwd_partials_bias", dma, dSa, mhat, J, var, mg, nullptr, nullptr, dmz, dSz, nullptr,
                     nullptr, nullptr, nullptr, N, C, HW, eps, ws, ws_bytes, stream, true, false, true);
}

extern "C" int tagi_bn_bwd_finalize_multi(const tagi_bn_bwd_pending* items, int64_t count, tagi_stream_t stream) {
  const char* what = "tagi_bn_bwd_finalize_multi";
  TAGI_REQUIRE(count >= 0 && (count == 0 || items), "%s: bad table", what);
  hipStream_t s = as_stream(stream);
  int64_t bytes = 0;
  for (int64_t i = 0; i < count; ++i) {
    const tagi_bn_bwd_pending& p = items[i];
    TAGI_REQUIRE(p.ws && p.Sg && p.Sb && p.dmg && p.dSg && p.dmb && p.dSb, "%s: null pointer at %lld", what,
                 (long long)i);
    TAGI_REQUIRE(p.N > 0 && p.C > 0 && p.HW > 0 && p.C < (1 << 24), "%s: bad sizes at %lld", what, (long long)i);
    TAGI_REQUIRE((p.cdmb == nullptr) == (p.cdSb == nullptr) && (p.cdmb == nullptr || p.cSb != nullptr),
                 "%s: conv bias outputs at %lld must be all given or all NULL", what, (long long)i);
    const bool cb = p.cdmb != nullptr;
    TAGI_REQUIRE(p.nblk >= 0 && p.nblk < (1ll << 31), "%s: bad nblk at %lld", what, (long long)i);
    bytes += (p.nblk > 0 ? p.nblk : (int64_t)red_rows(p.N * p.HW)) * p.C * (cb ? 24 : 16) + (cb ? 36 : 24) * p.C;
  }
  ProfScope ps(FAM_BN_BWD, s, 0.0, (double)bytes);
  for (int64_t t0 = 0; t0 < count; t0 += kBnMulti) {
    BnFinalizeMulti a{};
    int c = 0, blocks = 0;
    for (int64_t t = t0; t < count && c < kBnMulti; ++t, ++c) {
      const tagi_bn_bwd_pending& p = items[t];
      a.ws[c] = p.ws;
      a.Sg[c] = p.Sg;
      a.Sb[c] = p.Sb;
      a.dmg[c] = p.dmg;
      a.dSg[c] = p.dSg;
      a.dmb[c] = p.dmb;
      a.dSb[c] = p.dSb;
      a.cSb[c] = p.cSb;
      a.cdmb[c] = p.cdmb;
      a.cdSb[c] = p.cdSb;
      a.C[c] = (int)p.C;
      a.nblk[c] = p.nblk > 0 ? (int)p.nblk : red_rows(p.N * p.HW);
      a.start[c] = blocks;
      blocks += (int)p.C;
    }
    a.start[c] = blocks;
    a.count = c;
    hipLaunchKernelGGL(bn_bwd_finalize_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    int rc = check_launch(what);
    if (rc) return rc;
  }
  return TAGI_OK;
}

extern "C" int tagi_rmsnorm_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw, float* mz,
                                float* Sz, float* inv_rms, int64_t rows, int64_t D, float eps, tagi_stream_t stream) {
  const char* what = "tagi_rmsnorm_fwd";
  TAGI_REQUIRE(ma && Sa && mw && Sw && mz && Sz && inv_rms, "%s: null pointer", what);
  TAGI_REQUIRE(rows >= 0 && D > 0, "%s: bad sizes", what);
  if (rows == 0) return TAGI_OK;
  if (D > 1024) return fail(TAGI_ERR_UNSUPPORTED, "%s: rows longer than 1024 features", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_RMSNORM, s, 0.0, 16.0 * rows * D + 4.0 * rows);
  const unsigned blocks = (unsigned)cdiv(rows, 4);
  if (D <= 64)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<1>, dim3(blocks), dim3(256), 0, s, ma, Sa, mw, Sw, mz, Sz, inv_rms, rows,
                       (int)D, eps);
  else if (D <= 256)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<4>, dim3(blocks), dim3(256), 0, s, ma, Sa, mw, Sw, mz, Sz, inv_rms, rows,
                       (int)D, eps);
  else
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<16>, dim3(blocks), dim3(256), 0, s, ma, Sa, mw, Sw, mz, Sz, inv_rms, rows,
                       (int)D, eps);
  return check_launch(what);
}

extern "C" int64_t tagi_rmsnorm_bwd_ws_bytes(int64_t rows, int64_t D) {
  if (rows <= 0 || D <= 0) return 0;
  return (int64_t)red_rows(rows) * 2 * D * (int64_t)sizeof(float);
}

extern "C" int tagi_rmsnorm_bwd(const float* dmz, const float* dSz, const float* ma, const float* inv_rms,
                                const float* mw, const float* Sw, float* dma, float* dSa, float* dmw, float* dSw,
                                int64_t rows, int64_t D, float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_rmsnorm_bwd";
  TAGI_REQUIRE(dmz && dSz && ma && inv_rms && mw && Sw && dma && dSa && dmw && dSw && ws, "%s: null pointer", what);
  TAGI_REQUIRE(rows > 0 && D > 0, "%s: bad sizes", what);
  TAGI_REQUIRE(ws_bytes >= tagi_rmsnorm_bwd_ws_bytes(rows, D), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_RMSNORM, s, 0.0, 20.0 * rows * D);
  const int nblk = red_rows(rows);
  const bool vec = bn_vec(D) && al16p(dmz) && al16p(dSz) && al16p(ma) && al16p(mw) && al16p(dma) && al16p(dSa);
  if (vec)
    hipLaunchKernelGGL(rmsnorm_bwd_partial_vec_kernel, dim3((unsigned)nblk, red_chunks(nblk, D, true)), dim3(256), 0,
                       s, dmz, dSz, ma, inv_rms,
                       mw, dma, dSa, ws, rows, (int)D, nblk);
  else
    hipLaunchKernelGGL(rmsnorm_bwd_partial_kernel, dim3((unsigned)nblk), dim3(256), 0, s, dmz, dSz, ma, inv_rms, mw,
                       dma, dSa, ws, rows, (int)D, nblk);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(rmsnorm_bwd_finalize_kernel, dim3((unsigned)D), dim3(256), 0, s, (const float*)ws, Sw, dmw, dSw,
                     (int)D, nblk);
  return check_launch(what);
}

extern "C" int tagi_layernorm_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw, const float* mb,
                                  const float* Sb, float* mz, float* Sz, float* mu_ra, float* var_ra, int64_t rows,
                                  int64_t D, float eps, tagi_stream_t stream) {
  const char* what = "tagi_layernorm_fwd";
  TAGI_REQUIRE(rows >= 0 && D > 0 && D < (1ll << 31), "%s: bad sizes", what);
  if (rows == 0) return TAGI_OK;
  TAGI_REQUIRE(ma && Sa && mw && Sw && mb && Sb && mz && Sz && mu_ra && var_ra, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_LAYERNORM, s, 0.0, 16.0 * rows * D + 8.0 * rows);
  const unsigned blocks = (unsigned)cdiv(rows, 4);
  if (D <= 64)
    hipLaunchKernelGGL(layernorm_fwd_kernel<1>, dim3(blocks), dim3(256), 0, s, ma, Sa, mw, Sw, mb, Sb, mz, Sz, mu_ra,
                       var_ra, rows, (int)D, eps);
  else if (D <= 256)
    hipLaunchKernelGGL(layernorm_fwd_kernel<4>, dim3(blocks), dim3(256), 0, s, ma, Sa, mw, Sw, mb, Sb, mz, Sz, mu_ra,
                       var_ra, rows, (int)D, eps);
  else if (D <= 1024)
    hipLaunchKernelGGL(layernorm_fwd_kernel<16>, dim3(blocks), dim3(256), 0, s, ma, Sa, mw, Sw, mb, Sb, mz, Sz,
                       mu_ra, var_ra, rows, (int)D, eps);
  else {
    TAGI_REQUIRE(rows < (1ll << 31), "%s: more than 2^31 rows", what);
    hipLaunchKernelGGL(layernorm_fwd_row_kernel, dim3((unsigned)rows), dim3(256), 0, s, ma, Sa, mw, Sw, mb, Sb, mz, Sz,
                       mu_ra, var_ra, (int)D, eps);
  }
  return check_launch(what);
}

extern "C" int64_t tagi_layernorm_bwd_ws_bytes(int64_t rows, int64_t D) {
  if (rows <= 0 || D <= 0) return 0;
  return (int64_t)red_rows(rows) * 4 * D * (int64_t)sizeof(float);
}

extern "C" int tagi_layernorm_bwd(const float* dmz, const float* dSz, const float* ma, const float* mu_ra,
                                  const float* var_ra, const float* mw, const float* Sw, const float* Sb, float* dma,
                                  float* dSa, float* dmw, float* dSw, float* dmb, float* dSb, int64_t rows, int64_t D,
                                  float eps, float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_layernorm_bwd";
  TAGI_REQUIRE(dmz && dSz && ma && mu_ra && var_ra && mw && Sw && Sb && dma && dSa && dmw && dSw && dmb && dSb && ws,
               "%s: null pointer", what);
  TAGI_REQUIRE(rows > 0 && D > 0 && D < (1ll << 31), "%s: bad sizes", what);
  TAGI_REQUIRE(ws_bytes >= tagi_layernorm_bwd_ws_bytes(rows, D), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_LAYERNORM, s, 0.0, 20.0 * rows * D + 8.0 * rows);
  const int nblk = red_rows(rows);
  const bool vec = bn_vec(D) && al16p(dmz) && al16p(dSz) && al16p(ma) && al16p(mw) && al16p(dma) && al16p(dSa);
  if (vec)
    hipLaunchKernelGGL(layernorm_bwd_partial_vec_kernel, dim3((unsigned)nblk, red_chunks(nblk, D, true)), dim3(256),
                       0, s, dmz, dSz, ma, mu_ra, var_ra, mw, dma, dSa, ws, rows, (int)D, nblk, eps);
  else
    hipLaunchKernelGGL(layernorm_bwd_partial_kernel, dim3((unsigned)nblk), dim3(256), 0, s, dmz, dSz, ma, mu_ra,
                       var_ra, mw, dma, dSa, ws, rows, (int)D, nblk, eps);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(layernorm_bwd_finalize_kernel, dim3((unsigned)D), dim3(256), 0, s, (const float*)ws, Sw, Sb, dmw,
                     dSw, dmb, dSb, (int)D, nblk);
  return check_launch(what);
}

extern "C" int tagi_embedding_fwd(const float* tokens, const float* mw, const float* Sw, float* mz, float* Sz,
                                  int64_t n_tokens, int64_t V, int64_t D, int64_t padding_idx, tagi_stream_t stream) {
  const char* what = "tagi_embedding_fwd";
  TAGI_REQUIRE(tokens && mw && Sw && mz && Sz, "%s: null pointer", what);
  TAGI_REQUIRE(n_tokens >= 0 && V > 0 && D > 0, "%s: bad sizes", what);
  if (n_tokens == 0) return TAGI_OK;
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_EMBEDDING, s, 0.0, 4.0 * n_tokens + 16.0 * n_tokens * D);
  const bool vec = D % 4 == 0 && D <= 1024 && 256 % (D / 4) == 0 && al16p(mw) && al16p(Sw) && al16p(mz) && al16p(Sz);
  if (vec)
    hipLaunchKernelGGL(embedding_fwd_vec_kernel, dim3((unsigned)cdiv(n_tokens, 256 / (D / 4))), dim3(256), 0, s, tokens,
                       mw, Sw, mz, Sz, n_tokens, V, (int)D, padding_idx);
  else
    hipLaunchKernelGGL(embedding_fwd_kernel, dim3(ew_blocks(n_tokens * D, 256)), dim3(256), 0, s, tokens, mw, Sw, mz,
                       Sz, n_tokens, V, (int)D, padding_idx);
  return check_launch(what);
}

extern "C" int tagi_pe_add(const float* ma, const float* pe, float* out, int64_t B, int64_t S, int64_t E,
                           tagi_stream_t stream) {
  const char* what = "tagi_pe_add";
  TAGI_REQUIRE(ma && pe && out, "%s: null pointer", what);
  TAGI_REQUIRE(B >= 0 && S > 0 && E > 0, "%s: bad sizes", what);
  if (B == 0) return TAGI_OK;
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_PE, s, 0.0, 8.0 * B * S * E + 4.0 * S * E);
  hipLaunchKernelGGL(pe_add_kernel, dim3(ew_blocks(B * S * E, 256)), dim3(256), 0, s, ma, pe, out, B * S * E, S * E);
  return check_launch(what);
}
