// MaxPool2D with the hard-argmax moment rule (maxpool2d.py:62-126): the output takes the
// mean and variance of the window position with the largest mean; the backward pass
// routes each output delta to that position.
//
// Tensors are (N, C, H, W) in either NCHW or channels-last storage (one flag for all of
// them). One thread per output element in the forward pass; the backward pass gathers
// instead of scattering: one thread per input element adds, in ascending (h_out, w_out)
// order, the deltas of the windows that picked it. That order is scatter_add's, every
// input is written once (no memset) and the result does not depend on timing.
#include "tagi_common.h"

namespace tagi {

struct PoolGeom {
  int64_t N;
  int C, H, W, Ho, Wo, k, s, p;
  bool cl;  // channels-last storage
};

__device__ __forceinline__ int64_t in_off(const PoolGeom& g, int64_t n, int c, int h, int w) {
  return g.cl ? ((n * g.H + h) * g.W + w) * g.C + c : ((n * g.C + c) * g.H + h) * (int64_t)g.W + w;
}
__device__ __forceinline__ int64_t out_off(const PoolGeom& g, int64_t n, int c, int h, int w) {
  return g.cl ? ((n * g.Ho + h) * g.Wo + w) * g.C + c : ((n * g.C + c) * g.Ho + h) * (int64_t)g.Wo + w;
}
// (n, c, h, w) of flat storage position e of a tensor with spatial size (h_n, w_n).
// IT is uint32_t when every flat index fits (32-bit division is a short sequence;
// 64-bit division is a long software routine), int64_t otherwise.
template <typename IT>
__device__ __forceinline__ void decode(const PoolGeom& g, IT e, int h_n, int w_n, int64_t& n, int& c, int& h,
                                       int& w) {
  if (g.cl) {
    c = (int)(e % (IT)g.C);
    e /= (IT)g.C;
    w = (int)(e % (IT)w_n);
    e /= (IT)w_n;
    h = (int)(e % (IT)h_n);
    n = (int64_t)(e / (IT)h_n);
  } else {
    w = (int)(e % (IT)w_n);
    e /= (IT)w_n;
    h = (int)(e % (IT)h_n);
    e /= (IT)h_n;
    c = (int)(e % (IT)g.C);
    n = (int64_t)(e / (IT)g.C);
  }
}

// The first in-window position starts as the pick with value -inf; a later position
// replaces it when its mean is larger or NaN (torch's max_pool2d selection rule).
template <typename IT>
__global__ void __launch_bounds__(256) maxpool_fwd_kernel(PoolGeom g, const float* __restrict__ ma,
                                                          const float* __restrict__ Sa, float* __restrict__ mz,
                                                          float* __restrict__ Sz, int32_t* __restrict__ pool_idx) {
  const int64_t total = g.N * g.C * (int64_t)g.Ho * g.Wo;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    int64_t n;
    int c, ho, wo;
    decode<IT>(g, (IT)e, g.Ho, g.Wo, n, c, ho, wo);
    const int h0 = ho * g.s - g.p, w0 = wo * g.s - g.p;
    const int ha = max(h0, 0), hb = min(h0 + g.k, g.H), wa = max(w0, 0), wb = min(w0 + g.k, g.W);
    float best = -__builtin_inff();
    int bh = ha, bw = wa;
    for (int h = ha; h < hb; ++h)
      for (int w = wa; w < wb; ++w) {
        const float v = ma[in_off(g, n, c, h, w)];
        if (v > best || v != v) {
          best = v;
          bh = h;
          bw = w;
        }
      }
    const int64_t src = in_off(g, n, c, bh, bw);
    mz[e] = ma[src];
    Sz[e] = Sa[src];
    pool_idx[e] = bh * g.W + bw;
  }
}

template <typename IT>
__global__ void __launch_bounds__(256) maxpool_bwd_kernel(PoolGeom g, const float* __restrict__ dmz,
                                                          const float* __restrict__ dSz,
                                                          const int32_t* __restrict__ pool_idx,
                                                          float* __restrict__ dma, float* __restrict__ dSa) {
  const int64_t total = g.N * g.C * (int64_t)g.H * g.W;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    int64_t n;
    int c, h, w;
    decode<IT>(g, (IT)e, g.H, g.W, n, c, h, w);
    // windows ho with ho*s - p <= h <= ho*s - p + k - 1
    const int hp = h + g.p, wp = w + g.p;
    const int ho_a = hp - g.k + 1 <= 0 ? 0 : (hp - g.k + 1 + g.s - 1) / g.s;
    const int ho_b = min(hp / g.s, g.Ho - 1);
    const int wo_a = wp - g.k + 1 <= 0 ? 0 : (wp - g.k + 1 + g.s - 1) / g.s;
    const int wo_b = min(wp / g.s, g.Wo - 1);
    const int32_t me = h * g.W + w;
    float am = 0.f, aS = 0.f;
    for (int ho = ho_a; ho <= ho_b; ++ho)
      for (int wo = wo_a; wo <= wo_b; ++wo) {
        const int64_t o = out_off(g, n, c, ho, wo);
        if (pool_idx[o] == me) {
          am += dmz[o];
          aS += dSz[o];
        }
      }
    dma[e] = am;
    dSa[e] = aS;
  }
}

}  // namespace tagi

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

static int pool_geom(const char* what, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k, int64_t stride,
                     int64_t pad, int channels_last, PoolGeom* g) {
  TAGI_REQUIRE(N >= 0 && C > 0 && H > 0 && W > 0, "%s: bad sizes", what);
  TAGI_REQUIRE(k > 0 && stride > 0 && pad >= 0 && 2 * pad <= k, "%s: need k > 0, stride > 0, 0 <= pad <= k/2",
               what);
  TAGI_REQUIRE(C < (1ll << 31) && H * W < (1ll << 31), "%s: plane or channel count above 2^31", what);
  const int64_t Ho = (H + 2 * pad - k) / stride + 1, Wo = (W + 2 * pad - k) / stride + 1;
  TAGI_REQUIRE(H + 2 * pad >= k && W + 2 * pad >= k, "%s: window larger than the padded input", what);
  *g = PoolGeom{N, (int)C, (int)H, (int)W, (int)Ho, (int)Wo, (int)k, (int)stride, (int)pad, channels_last != 0};
  return TAGI_OK;
}

extern "C" int tagi_maxpool2d_fwd(const float* ma, const float* Sa, float* mz, float* Sz, int32_t* pool_idx,
                                  int64_t N, int64_t C, int64_t H, int64_t W, int64_t k, int64_t stride, int64_t pad,
                                  int channels_last, tagi_stream_t stream) {
  const char* what = "tagi_maxpool2d_fwd";
  PoolGeom g;
  int rc = pool_geom(what, N, C, H, W, k, stride, pad, channels_last, &g);
  if (rc) return rc;
  if (N == 0) return TAGI_OK;
  TAGI_REQUIRE(ma && Sa && mz && Sz && pool_idx, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  const int64_t out = N * C * (int64_t)g.Ho * g.Wo;
  ProfScope ps(FAM_MAXPOOL, s, 0.0, 4.0 * N * C * H * W + 12.0 * out);
  if (out < (1ll << 32))
    hipLaunchKernelGGL(maxpool_fwd_kernel<uint32_t>, dim3(ew_blocks(out, 256)), dim3(256), 0, s, g, ma, Sa, mz, Sz,
                       pool_idx);
  else
    hipLaunchKernelGGL(maxpool_fwd_kernel<int64_t>, dim3(ew_blocks(out, 256)), dim3(256), 0, s, g, ma, Sa, mz, Sz,
                       pool_idx);
  return check_launch(what);
}

extern "C" int tagi_maxpool2d_bwd(const float* dmz, const float* dSz, const int32_t* pool_idx, float* dma,
                                  float* dSa, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k, int64_t stride,
                                  int64_t pad, int channels_last, tagi_stream_t stream) {
  const char* what = "tagi_maxpool2d_bwd";
  PoolGeom g;
  int rc = pool_geom(what, N, C, H, W, k, stride, pad, channels_last, &g);
  if (rc) return rc;
  if (N == 0) return TAGI_OK;
  TAGI_REQUIRE(dmz && dSz && pool_idx && dma && dSa, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  const int64_t total = N * C * H * W;
  ProfScope ps(FAM_MAXPOOL, s, 0.0, 12.0 * N * C * (int64_t)g.Ho * g.Wo + 8.0 * total);
  if (total < (1ll << 32))
    hipLaunchKernelGGL(maxpool_bwd_kernel<uint32_t>, dim3(ew_blocks(total, 256)), dim3(256), 0, s, g, dmz, dSz,
                       pool_idx, dma, dSa);
  else
    hipLaunchKernelGGL(maxpool_bwd_kernel<int64_t>, dim3(ew_blocks(total, 256)), dim3(256), 0, s, g, dmz, dSz,
                       pool_idx, dma, dSa);
  return check_launch(what);
}
