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

// Channels-last with C % 4 == 0 and 16-byte aligned tensors: one thread per four
// consecutive channels of one output (forward) or input (backward) pixel, float4 loads
// and stores along the channels; the same selection and summation order per channel.
template <typename IT>
__global__ void __launch_bounds__(256) maxpool_fwd_cl4_kernel(PoolGeom g, const float* __restrict__ ma,
                                                              const float* __restrict__ Sa, float* __restrict__ mz,
                                                              float* __restrict__ Sz, int32_t* __restrict__ pool_idx) {
  const int C4 = g.C >> 2;
  const int64_t total = g.N * g.Ho * (int64_t)g.Wo * C4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    IT q = (IT)e;
    const int c = (int)(q % (IT)C4) * 4;
    q /= (IT)C4;
    const int wo = (int)(q % (IT)g.Wo);
    q /= (IT)g.Wo;
    const int ho = (int)(q % (IT)g.Ho);
    const int64_t n = (int64_t)(q / (IT)g.Ho);
    const int h0 = ho * g.s - g.p, w0 = wo * g.s - g.p;
    const int ha = max(h0, 0), hb = min(h0 + g.k, g.H), wa = max(w0, 0), wb = min(w0 + g.k, g.W);
    float best[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    int pick[4] = {ha * g.W + wa, ha * g.W + wa, ha * g.W + wa, ha * g.W + wa};
    const int64_t img = n * g.H * (int64_t)g.W;
    for (int h = ha; h < hb; ++h)
      for (int w = wa; w < wb; ++w) {
        const float4 v4 = *reinterpret_cast<const float4*>(ma + (img + (int64_t)h * g.W + w) * g.C + c);
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (v[j] > best[j] || v[j] != v[j]) {
            best[j] = v[j];
            pick[j] = h * g.W + w;
          }
      }
    float sv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sv[j] = Sa[(img + pick[j]) * g.C + c + j];
    const int64_t o = e * 4;  // output (n, ho, wo, c) in channels-last order
    *reinterpret_cast<float4*>(mz + o) = make_float4(best[0], best[1], best[2], best[3]);
    *reinterpret_cast<float4*>(Sz + o) = make_float4(sv[0], sv[1], sv[2], sv[3]);
    *reinterpret_cast<int4*>(pool_idx + o) = make_int4(pick[0], pick[1], pick[2], pick[3]);
  }
}

template <typename IT>
__global__ void __launch_bounds__(256) maxpool_bwd_cl4_kernel(PoolGeom g, const float* __restrict__ dmz,
                                                              const float* __restrict__ dSz,
                                                              const int32_t* __restrict__ pool_idx,
                                                              float* __restrict__ dma, float* __restrict__ dSa) {
  const int C4 = g.C >> 2;
  const int64_t total = g.N * g.H * (int64_t)g.W * C4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    IT q = (IT)e;
    const int c = (int)(q % (IT)C4) * 4;
    q /= (IT)C4;
    const int w = (int)(q % (IT)g.W);
    q /= (IT)g.W;
    const int h = (int)(q % (IT)g.H);
    const int64_t n = (int64_t)(q / (IT)g.H);
    const int hp = h + g.p, wp = w + g.p;
    const int ho_a = hp - g.k + 1 <= 0 ? 0 : (hp - g.k + 1 + g.s - 1) / g.s;
    const int ho_b = min(hp / g.s, g.Ho - 1);
    const int wo_a = wp - g.k + 1 <= 0 ? 0 : (wp - g.k + 1 + g.s - 1) / g.s;
    const int wo_b = min(wp / g.s, g.Wo - 1);
    const int32_t me = h * g.W + w;
    float am[4] = {0.f, 0.f, 0.f, 0.f}, aS[4] = {0.f, 0.f, 0.f, 0.f};
    if (g.k <= 2 * g.s) {
      // at most 2 x 2 windows cover a position: the indices and deltas of all of them are
      // loaded at once, then the matching ones are added in the (ho, wo) order of the loop
      // below
      int4 p4[2][2];
      float4 m4[2][2], s4[2][2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          p4[i][j] = make_int4(-1, -1, -1, -1);
          m4[i][j] = s4[i][j] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (ho_a + i <= ho_b && wo_a + j <= wo_b) {
            const int64_t o = ((n * g.Ho + ho_a + i) * g.Wo + wo_a + j) * g.C + c;
            p4[i][j] = *reinterpret_cast<const int4*>(pool_idx + o);
            m4[i][j] = *reinterpret_cast<const float4*>(dmz + o);
            s4[i][j] = *reinterpret_cast<const float4*>(dSz + o);
          }
        }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int p[4] = {p4[i][j].x, p4[i][j].y, p4[i][j].z, p4[i][j].w};
          const float m[4] = {m4[i][j].x, m4[i][j].y, m4[i][j].z, m4[i][j].w};
          const float sv[4] = {s4[i][j].x, s4[i][j].y, s4[i][j].z, s4[i][j].w};
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (p[q] == me) {
              am[q] += m[q];
              aS[q] += sv[q];
            }
        }
      *reinterpret_cast<float4*>(dma + e * 4) = make_float4(am[0], am[1], am[2], am[3]);
      *reinterpret_cast<float4*>(dSa + e * 4) = make_float4(aS[0], aS[1], aS[2], aS[3]);
      continue;
    }
    for (int ho = ho_a; ho <= ho_b; ++ho)
      for (int wo = wo_a; wo <= wo_b; ++wo) {
        const int64_t o = ((n * g.Ho + ho) * g.Wo + wo) * g.C + c;
        const int4 p4 = *reinterpret_cast<const int4*>(pool_idx + o);
        const int p[4] = {p4.x, p4.y, p4.z, p4.w};
        if (p[0] != me && p[1] != me && p[2] != me && p[3] != me) continue;
        const float4 m4 = *reinterpret_cast<const float4*>(dmz + o);
        const float4 s4 = *reinterpret_cast<const float4*>(dSz + o);
        const float m[4] = {m4.x, m4.y, m4.z, m4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (p[j] == me) {
            am[j] += m[j];
            aS[j] += sv[j];
          }
      }
    *reinterpret_cast<float4*>(dma + e * 4) = make_float4(am[0], am[1], am[2], am[3]);
    *reinterpret_cast<float4*>(dSa + e * 4) = make_float4(aS[0], aS[1], aS[2], aS[3]);
  }
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// one float4 group per thread up to 2^28 groups, so the gathers of many positions are in
// flight at once
static inline unsigned bwd_blocks(int64_t items) { return (unsigned)std::min<int64_t>(cdiv(items, 256), 1ll << 20); }

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
  if (g.cl && C % 4 == 0 && al16(ma) && al16(Sa) && al16(mz) && al16(Sz) && al16(pool_idx)) {
    const int64_t items = out / 4;
    if (items < (1ll << 32))
      hipLaunchKernelGGL(maxpool_fwd_cl4_kernel<uint32_t>, dim3(ew_blocks(items, 256)), dim3(256), 0, s, g, ma, Sa,
                         mz, Sz, pool_idx);
    else
      hipLaunchKernelGGL(maxpool_fwd_cl4_kernel<int64_t>, dim3(ew_blocks(items, 256)), dim3(256), 0, s, g, ma, Sa,
                         mz, Sz, pool_idx);
  } else if (out < (1ll << 32))
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
  if (g.cl && C % 4 == 0 && al16(dmz) && al16(dSz) && al16(pool_idx) && al16(dma) && al16(dSa)) {
    const int64_t items = total / 4;
    if (items < (1ll << 32))
      hipLaunchKernelGGL(maxpool_bwd_cl4_kernel<uint32_t>, dim3(bwd_blocks(items)), dim3(256), 0, s, g, dmz, dSz,
                         pool_idx, dma, dSa);
    else
      hipLaunchKernelGGL(maxpool_bwd_cl4_kernel<int64_t>, dim3(bwd_blocks(items)), dim3(256), 0, s, g, dmz, dSz,
                         pool_idx, dma, dSa);
  } else if (total < (1ll << 32))
    hipLaunchKernelGGL(maxpool_bwd_kernel<uint32_t>, dim3(ew_blocks(total, 256)), dim3(256), 0, s, g, dmz, dSz,
                       pool_idx, dma, dSa);
  else
    hipLaunchKernelGGL(maxpool_bwd_kernel<int64_t>, dim3(ew_blocks(total, 256)), dim3(256), 0, s, g, dmz, dSz,
                       pool_idx, dma, dSa);
  return check_launch(what);
}
