// Bandwidth-bound TAGI kernels: rectified-Gaussian moments, Remax, output innovation,
// capped parameter update, moment add, average pooling and the Jacobian backward.
//
// Elementwise kernels are grid-stride loops over float4 when every pointer is 16-byte
// aligned (the torch caching allocator's normal case), scalar otherwise. One lane owns
// four consecutive elements, so a wavefront moves 1 KiB per access.
#include "tagi_common.h"
#include "tagi_moments.h"

namespace tagi {

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename F>
__device__ __forceinline__ void for_each_vec(int64_t n, F f) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) f(i);
}

template <bool VEC>
__global__ void relu_kernel(const float* __restrict__ mz, const float* __restrict__ Sz, float* __restrict__ ma,
                            float* __restrict__ Sa, float* __restrict__ J, int64_t n) {
  if constexpr (VEC) {
    const int64_t n4 = n >> 2;
    for_each_vec(n4, [&](int64_t i) {
      const float4 m = reinterpret_cast<const float4*>(mz)[i];
      const float4 s = reinterpret_cast<const float4*>(Sz)[i];
      float4 a, b, j;
      relu_moments(m.x, s.x, a.x, b.x, j.x);
      relu_moments(m.y, s.y, a.y, b.y, j.y);
      relu_moments(m.z, s.z, a.z, b.z, j.z);
      relu_moments(m.w, s.w, a.w, b.w, j.w);
      reinterpret_cast<float4*>(ma)[i] = a;
      reinterpret_cast<float4*>(Sa)[i] = b;
      reinterpret_cast<float4*>(J)[i] = j;
    });
    // tail
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
      const int64_t i = (n4 << 2) + threadIdx.x;
      relu_moments(mz[i], Sz[i], ma[i], Sa[i], J[i]);
    }
  } else {
    for_each_vec(n, [&](int64_t i) { relu_moments(mz[i], Sz[i], ma[i], Sa[i], J[i]); });
  }
}

// -------------------------------------------------------------- Jacobian backward
template <bool VEC>
__global__ void jacobian_kernel(const float* __restrict__ dm, const float* __restrict__ dS,
                                const float* __restrict__ J, float* __restrict__ om, float* __restrict__ oS,
                                int64_t n) {
  if constexpr (VEC) {
    const int64_t n4 = n >> 2;
    for_each_vec(n4, [&](int64_t i) {
      const float4 a = reinterpret_cast<const float4*>(dm)[i];
      const float4 b = reinterpret_cast<const float4*>(dS)[i];
      const float4 j = reinterpret_cast<const float4*>(J)[i];
      reinterpret_cast<float4*>(om)[i] = make_float4(a.x * j.x, a.y * j.y, a.z * j.z, a.w * j.w);
      reinterpret_cast<float4*>(oS)[i] =
          make_float4(b.x * j.x * j.x, b.y * j.y * j.y, b.z * j.z * j.z, b.w * j.w * j.w);
    });
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
      const int64_t i = (n4 << 2) + threadIdx.x;
      om[i] = dm[i] * J[i];
      oS[i] = dS[i] * J[i] * J[i];
    }
  } else {
    for_each_vec(n, [&](int64_t i) {
      om[i] = dm[i] * J[i];
      oS[i] = dS[i] * J[i] * J[i];
    });
  }
}

// ------------------------------------------------------------------------ Innovation
template <bool VEC>
__global__ void innovation_kernel(const float* __restrict__ y, const float* __restrict__ mu,
                                  const float* __restrict__ var, float sv2, float* __restrict__ dm,
                                  float* __restrict__ dS, int64_t n) {
  for_each_vec(n, [&](int64_t i) {
    const float Sy = var[i] + sv2;
    dm[i] = (y[i] - mu[i]) / Sy;
    dS[i] = -1.0f / Sy;
  });
}

// -------------------------------------------------------------------- Capped update
// capped() (tagi_moments.h) is shared with the parameter-delta GEMM epilogue, which can
// apply the same update while it forms the deltas.
template <bool VEC>
__global__ void update_kernel(float* __restrict__ m, float* __restrict__ S, const float* __restrict__ dm,
                              const float* __restrict__ dS, float cap, int64_t n) {
  if constexpr (VEC) {
    const int64_t n4 = n >> 2;
    for_each_vec(n4, [&](int64_t i) {
      float4 a = reinterpret_cast<float4*>(m)[i];
      float4 b = reinterpret_cast<float4*>(S)[i];
      const float4 c = reinterpret_cast<const float4*>(dm)[i];
      const float4 d = reinterpret_cast<const float4*>(dS)[i];
      capped(a.x, b.x, c.x, d.x, cap);
      capped(a.y, b.y, c.y, d.y, cap);
      capped(a.z, b.z, c.z, d.z, cap);
      capped(a.w, b.w, c.w, d.w, cap);
      reinterpret_cast<float4*>(m)[i] = a;
      reinterpret_cast<float4*>(S)[i] = b;
    });
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
      const int64_t i = (n4 << 2) + threadIdx.x;
      capped(m[i], S[i], dm[i], dS[i], cap);
    }
  } else {
    for_each_vec(n, [&](int64_t i) { capped(m[i], S[i], dm[i], dS[i], cap); });
  }
}

constexpr int kMultiMax = 48;
constexpr int kMultiChunk = 4096;  // elements per block (a multiple of 4)
struct MultiUpdateArgs {
  float* m[kMultiMax];
  float* S[kMultiMax];
  const float* dm[kMultiMax];
  const float* dS[kMultiMax];
  int64_t n[kMultiMax];
  int64_t block_start[kMultiMax + 1];
  unsigned long long vec_mask;  // bit t: tensor t's four arrays are 16-byte aligned
  int count;
  float cap;
};

// One launch for many parameter tensors: blocks are dealt to tensors by a prefix table.
__global__ void update_multi_kernel(MultiUpdateArgs a) {
  const int64_t b = blockIdx.x;
  int t = 0;
  while (t + 1 < a.count && a.block_start[t + 1] <= b) ++t;
  const int64_t base = (b - a.block_start[t]) * kMultiChunk;
  const int64_t n = a.n[t];
  float* m = a.m[t];
  float* S = a.S[t];
  const float* dm = a.dm[t];
  const float* dS = a.dS[t];
  const int64_t end = base + kMultiChunk < n ? base + kMultiChunk : n;
  if ((a.vec_mask >> t) & 1ull) {
    // float4 groups of the chunk, then the tensor's last n % 4 elements one by one
    const int64_t e4 = base + ((end - base) & ~(int64_t)3);
    for (int64_t i = base + 4 * (int64_t)threadIdx.x; i < e4; i += 4 * (int64_t)blockDim.x) {
      float4 x = *reinterpret_cast<float4*>(m + i);
      float4 y = *reinterpret_cast<float4*>(S + i);
      const float4 c = *reinterpret_cast<const float4*>(dm + i);
      const float4 d = *reinterpret_cast<const float4*>(dS + i);
      capped(x.x, y.x, c.x, d.x, a.cap);
      capped(x.y, y.y, c.y, d.y, a.cap);
      capped(x.z, y.z, c.z, d.z, a.cap);
      capped(x.w, y.w, c.w, d.w, a.cap);
      *reinterpret_cast<float4*>(m + i) = x;
      *reinterpret_cast<float4*>(S + i) = y;
    }
    for (int64_t i = e4 + threadIdx.x; i < end; i += blockDim.x) {
      float mm = m[i], ss = S[i];
      capped(mm, ss, dm[i], dS[i], a.cap);
      m[i] = mm;
      S[i] = ss;
    }
    return;
  }
  for (int64_t i = base + threadIdx.x; i < end; i += blockDim.x) {
    float mm = m[i], ss = S[i];
    capped(mm, ss, dm[i], dS[i], a.cap);
    m[i] = mm;
    S[i] = ss;
  }
}

// ------------------------------------------------------------------------ Add
template <bool VEC>
__global__ void add_kernel(const float* __restrict__ ms, const float* __restrict__ vs, float* __restrict__ ma,
                           float* __restrict__ va, int64_t n) {
  if constexpr (VEC) {
    const int64_t n4 = n >> 2;
    for_each_vec(n4, [&](int64_t i) {
      float4 a = reinterpret_cast<float4*>(ma)[i];
      float4 b = reinterpret_cast<float4*>(va)[i];
      const float4 c = reinterpret_cast<const float4*>(ms)[i];
      const float4 d = reinterpret_cast<const float4*>(vs)[i];
      a.x += c.x; a.y += c.y; a.z += c.z; a.w += c.w;
      b.x += d.x; b.y += d.y; b.z += d.z; b.w += d.w;
      reinterpret_cast<float4*>(ma)[i] = a;
      reinterpret_cast<float4*>(va)[i] = b;
    });
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
      const int64_t i = (n4 << 2) + threadIdx.x;
      ma[i] += ms[i];
      va[i] += vs[i];
    }
  } else {
    for_each_vec(n, [&](int64_t i) {
      ma[i] += ms[i];
      va[i] += vs[i];
    });
  }
}

// -------------------------------------------------------------------- AvgPool2D
// Channels-last: one lane per (output pixel, group of V channels); consecutive lanes walk
// channels, so every window read is a coalesced row of C floats. V = 4 moves float4 when
// C % 4 == 0 and the pointers are 16-byte aligned; IT = uint32_t when every flat index of
// the input fits in 31 bits (the index decode is then 32-bit division). Each component
// sums its window in the same (row, column) order for every V, so the results do not
// depend on the vector width.
template <int V>
struct vec_of;
template <>
struct vec_of<1> {
  using T = float;
  static __device__ __forceinline__ T zero() { return 0.f; }
  static __device__ __forceinline__ void add(T& a, T b) { a += b; }
  static __device__ __forceinline__ T scale(T a, float s) { return a * s; }
  static __device__ __forceinline__ T mul(T a, T b) { return a * b; }
  static __device__ __forceinline__ void relu(T m, T s, T& a, T& b, T& j) { relu_moments(m, s, a, b, j); }
  static __device__ __forceinline__ float lane(T a, int) { return a; }
  static __device__ __forceinline__ void set_lane(T& a, int, float x) { a = x; }
};
template <>
struct vec_of<4> {
  using T = float4;
  static __device__ __forceinline__ T zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
  static __device__ __forceinline__ void add(T& a, T b) {
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
  }
  static __device__ __forceinline__ T scale(T a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
  static __device__ __forceinline__ T mul(T a, T b) { return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w); }
  static __device__ __forceinline__ void relu(T m, T s, T& a, T& b, T& j) {
    relu_moments(m.x, s.x, a.x, b.x, j.x);
    relu_moments(m.y, s.y, a.y, b.y, j.y);
    relu_moments(m.z, s.z, a.z, b.z, j.z);
    relu_moments(m.w, s.w, a.w, b.w, j.w);
  }
  static __device__ __forceinline__ float lane(T a, int v) { return v == 0 ? a.x : (v == 1 ? a.y : (v == 2 ? a.z : a.w)); }
  static __device__ __forceinline__ void set_lane(T& a, int v, float x) {
    if (v == 0) a.x = x;
    else if (v == 1) a.y = x;
    else if (v == 2) a.z = x;
    else a.w = x;
  }
};

template <typename IT, int V>
__global__ void __launch_bounds__(256) avgpool_fwd_kernel(const float* __restrict__ ma, const float* __restrict__ Sa,
                                                          float* __restrict__ mo, float* __restrict__ So, IT N, IT H,
                                                          IT W, IT C, IT k, float inv_k2, float var_scale) {
  using VO = vec_of<V>;
  using T = typename VO::T;
  const T* m = reinterpret_cast<const T*>(ma);
  const T* S = reinterpret_cast<const T*>(Sa);
  const IT Ho = H / k, Wo = W / k, Cv = C / V;
  const IT total = N * Ho * Wo * Cv;
  const IT stride = (IT)gridDim.x * blockDim.x;
  for (IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const IT c = i % Cv, pix = i / Cv;
    const IT ow = pix % Wo, t = pix / Wo;
    const IT oh = t % Ho, n = t / Ho;
    const IT base = ((n * H + oh * k) * W + ow * k) * Cv + c;
    T sm = VO::zero(), ss = VO::zero();
    for (IT a = 0; a < k; ++a)
      for (IT b = 0; b < k; ++b) {
        const IT off = base + (a * W + b) * Cv;
        VO::add(sm, m[off]);
        VO::add(ss, S[off]);
      }
    reinterpret_cast<T*>(mo)[i] = VO::scale(sm, inv_k2);
    reinterpret_cast<T*>(So)[i] = VO::scale(ss, var_scale);
  }
}

// Input positions past the last whole window (H % k rows, W % k columns) receive zeros.
template <typename IT, int V>
__global__ void __launch_bounds__(256) avgpool_bwd_kernel(const float* __restrict__ dm, const float* __restrict__ dS,
                                                          float* __restrict__ om, float* __restrict__ oS, IT N, IT H,
                                                          IT W, IT C, IT k, float inv_k2, float var_scale) {
  using VO = vec_of<V>;
  using T = typename VO::T;
  const IT Ho = H / k, Wo = W / k, Cv = C / V;
  const IT total = N * H * W * Cv;
  const IT stride = (IT)gridDim.x * blockDim.x;
  for (IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const IT c = i % Cv, pix = i / Cv;
    const IT w = pix % W, t = pix / W;
    const IT h = t % H, n = t / H;
    const IT oh = h / k, ow = w / k;
    T a = VO::zero(), b = VO::zero();
    if (oh < Ho && ow < Wo) {
      const IT j = ((n * Ho + oh) * Wo + ow) * Cv + c;
      a = VO::scale(reinterpret_cast<const T*>(dm)[j], inv_k2);
      b = VO::scale(reinterpret_cast<const T*>(dS)[j], var_scale);
    }
    reinterpret_cast<T*>(om)[i] = a;
    reinterpret_cast<T*>(oS)[i] = b;
  }
}

// ReLU followed by AvgPool2D in one pass (relu.py:94-122, then avgpool2d.py:38-90): each
// thread takes V channels of one pooled pixel, forms the rectified moments and J of its
// k x k inputs (J stored for the backward pass) and sums them in avgpool_fwd_kernel's
// order, so the outputs are the two launches' bit for bit; the ReLU output is never
// written. H and W are multiples of k (every input lies in one window).
template <typename IT, int V, bool NCHW>
__global__ void __launch_bounds__(256) relu_avgpool_fwd_kernel(const float* __restrict__ mz,
                                                               const float* __restrict__ Sz, float* __restrict__ J,
                                                               float* __restrict__ mo, float* __restrict__ So, IT N,
                                                               IT H, IT W, IT C, IT k, float inv_k2,
                                                               float var_scale) {
  using VO = vec_of<V>;
  using T = typename VO::T;
  const T* m = reinterpret_cast<const T*>(mz);
  const T* S = reinterpret_cast<const T*>(Sz);
  T* Jv = reinterpret_cast<T*>(J);
  const IT Ho = H / k, Wo = W / k, Cv = C / V;
  const IT total = N * Ho * Wo * Cv;
  const IT stride = (IT)gridDim.x * blockDim.x;
  for (IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const IT c = i % Cv, pix = i / Cv;
    const IT ow = pix % Wo, t = pix / Wo;
    const IT oh = t % Ho, n = t / Ho;
    const IT base = ((n * H + oh * k) * W + ow * k) * Cv + c;
    T sm = VO::zero(), ss = VO::zero();
    for (IT a = 0; a < k; ++a)
      for (IT b = 0; b < k; ++b) {
        const IT off = base + (a * W + b) * Cv;
        T am, as, jj;
        VO::relu(m[off], S[off], am, as, jj);
        Jv[off] = jj;
        VO::add(sm, am);
        VO::add(ss, as);
      }
    if constexpr (NCHW) {
      // pooled moments laid out (N, C, Ho, Wo) row-major, as a following Flatten reads them
      const T pm = VO::scale(sm, inv_k2), ps = VO::scale(ss, var_scale);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const IT o = ((n * C + c * V + v) * Ho + oh) * Wo + ow;
        mo[o] = VO::lane(pm, v);
        So[o] = VO::lane(ps, v);
      }
    } else {
      reinterpret_cast<T*>(mo)[i] = VO::scale(sm, inv_k2);
      reinterpret_cast<T*>(So)[i] = VO::scale(ss, var_scale);
    }
  }
}

// AvgPool2D backward followed by the ReLU Jacobian (avgpool2d.py:92-130, relu.py:152-169):
// each input element gets its window's deltas scaled as avgpool_bwd_kernel scales them,
// times J and J^2 as jacobian_kernel multiplies (the same bits as the two launches; the
// unpooled deltas are never written). H and W are multiples of k.
template <typename IT, int V, bool NCHW>
__global__ void __launch_bounds__(256) avgpool_relu_bwd_kernel(const float* __restrict__ dm,
                                                               const float* __restrict__ dS,
                                                               const float* __restrict__ J, float* __restrict__ om,
                                                               float* __restrict__ oS, IT N, IT H, IT W, IT C, IT k,
                                                               float inv_k2, float var_scale) {
  using VO = vec_of<V>;
  using T = typename VO::T;
  const IT Ho = H / k, Wo = W / k, Cv = C / V;
  const IT total = N * H * W * Cv;
  const IT stride = (IT)gridDim.x * blockDim.x;
  for (IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const IT c = i % Cv, pix = i / Cv;
    const IT w = pix % W, t = pix / W;
    const IT h = t % H, n = t / H;
    T a, b;
    if constexpr (NCHW) {
      // pooled deltas laid out (N, C, Ho, Wo) row-major, as a following Flatten passes them
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const IT j = ((n * C + c * V + v) * Ho + h / k) * Wo + w / k;
        VO::set_lane(a, v, dm[j]);
        VO::set_lane(b, v, dS[j]);
      }
    } else {
      const IT j = ((n * Ho + h / k) * Wo + w / k) * Cv + c;
      a = reinterpret_cast<const T*>(dm)[j];
      b = reinterpret_cast<const T*>(dS)[j];
    }
    a = VO::scale(a, inv_k2);
    b = VO::scale(b, var_scale);
    const T jj = reinterpret_cast<const T*>(J)[i];
    reinterpret_cast<T*>(om)[i] = VO::mul(a, jj);
    reinterpret_cast<T*>(oS)[i] = VO::mul(VO::mul(b, jj), jj);
  }
}

// ------------------------------------------------------------------------ Remax
// remax.py:33-114. One wavefront per row (the row math is remax_row in tagi_moments.h).
template <int EPT>
__global__ void __launch_bounds__(256) remax_kernel(const float* __restrict__ mz, const float* __restrict__ Sz,
                                                    float* __restrict__ ma, float* __restrict__ Sa,
                                                    float* __restrict__ Jo, int64_t rows, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* pm = mz + row * K;
  const float* ps = Sz + row * K;
  float m[EPT], v[EPT], mua[EPT], vara[EPT], jo[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = lane + 64 * e;
    const bool ok = c < K;
    m[e] = ok ? pm[c] : 0.f;
    v[e] = ok ? ps[c] : 1.f;
  }
  remax_row<EPT>(m, v, lane, K, mua, vara, jo);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = lane + 64 * e;
    if (c >= K) continue;
    ma[row * K + c] = mua[e];
    Sa[row * K + c] = vara[e];
    Jo[row * K + c] = jo[e];
  }
}

}  // namespace tagi

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

extern "C" int tagi_relu_fwd(const float* mz, const float* Sz, float* ma, float* Sa, float* J, int64_t n,
                             tagi_stream_t stream) {
  TAGI_REQUIRE(n >= 0, "tagi_relu_fwd: n < 0");
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(mz && Sz && ma && Sa && J, "tagi_relu_fwd: null pointer");
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_RELU, s, 0.0, 20.0 * n);
  const bool vec = aligned16(mz) && aligned16(Sz) && aligned16(ma) && aligned16(Sa) && aligned16(J);
  if (vec)
    hipLaunchKernelGGL(relu_kernel<true>, dim3(ew_blocks(n / 4 + 1, 256)), dim3(256), 0, s, mz, Sz, ma, Sa, J, n);
  else
    hipLaunchKernelGGL(relu_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, mz, Sz, ma, Sa, J, n);
  return check_launch("tagi_relu_fwd");
}

extern "C" int tagi_jacobian_bwd(const float* dm, const float* dS, const float* J, float* dm_out, float* dS_out,
                                 int64_t n, tagi_stream_t stream) {
  TAGI_REQUIRE(n >= 0, "tagi_jacobian_bwd: n < 0");
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(dm && dS && J && dm_out && dS_out, "tagi_jacobian_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_JACOBIAN, s, 0.0, 20.0 * n);
  const bool vec = aligned16(dm) && aligned16(dS) && aligned16(J) && aligned16(dm_out) && aligned16(dS_out);
  if (vec)
    hipLaunchKernelGGL(jacobian_kernel<true>, dim3(ew_blocks(n / 4 + 1, 256)), dim3(256), 0, s, dm, dS, J, dm_out,
                       dS_out, n);
  else
    hipLaunchKernelGGL(jacobian_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, dm, dS, J, dm_out, dS_out,
                       n);
  return check_launch("tagi_jacobian_bwd");
}

extern "C" int tagi_innovation(const float* y, const float* mu, const float* var, float sigma_v2, float* dm,
                               float* dS, int64_t n, tagi_stream_t stream) {
  TAGI_REQUIRE(n >= 0, "tagi_innovation: n < 0");
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(y && mu && var && dm && dS, "tagi_innovation: null pointer");
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_INNOVATION, s, 0.0, 20.0 * n);
  hipLaunchKernelGGL(innovation_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, y, mu, var, sigma_v2, dm,
                     dS, n);
  return check_launch("tagi_innovation");
}

extern "C" int tagi_capped_update(float* m, float* S, const float* dm, const float* dS, float cap_factor, int64_t n,
                                  tagi_stream_t stream) {
  TAGI_REQUIRE(n >= 0, "tagi_capped_update: n < 0");
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(m && S && dm && dS, "tagi_capped_update: null pointer");
  TAGI_REQUIRE(cap_factor > 0.f, "tagi_capped_update: cap_factor must be positive");
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_UPDATE, s, 0.0, 24.0 * n);
  const bool vec = aligned16(m) && aligned16(S) && aligned16(dm) && aligned16(dS);
  if (vec)
    hipLaunchKernelGGL(update_kernel<true>, dim3(ew_blocks(n / 4 + 1, 256)), dim3(256), 0, s, m, S, dm, dS,
                       cap_factor, n);
  else
    hipLaunchKernelGGL(update_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, m, S, dm, dS, cap_factor, n);
  return check_launch("tagi_capped_update");
}

extern "C" int tagi_capped_update_multi(float* const* m, float* const* S, const float* const* dm,
                                        const float* const* dS, const int64_t* n, int64_t count, float cap_factor,
                                        tagi_stream_t stream) {
  TAGI_REQUIRE(count >= 0, "tagi_capped_update_multi: count < 0");
  TAGI_REQUIRE(count == 0 || (m && S && dm && dS && n), "tagi_capped_update_multi: null table");
  TAGI_REQUIRE(cap_factor > 0.f, "tagi_capped_update_multi: cap_factor must be positive");
  hipStream_t s = as_stream(stream);
  int64_t total = 0;
  for (int64_t t = 0; t < count; ++t) {
    TAGI_REQUIRE(n[t] >= 0, "tagi_capped_update_multi: negative size at %lld", (long long)t);
    TAGI_REQUIRE(n[t] == 0 || (m[t] && S[t] && dm[t] && dS[t]), "tagi_capped_update_multi: null pointer at %lld",
                 (long long)t);
    total += n[t];
  }
  ProfScope ps(FAM_UPDATE, s, 0.0, 24.0 * total);
  // one cursor over the table: each launch takes the next (up to) kMultiMax non-empty
  // groups, so every group is updated exactly once whatever the empty groups between them
  int64_t t = 0;
  while (t < count) {
    MultiUpdateArgs a{};
    a.cap = cap_factor;
    int c = 0;
    int64_t blocks = 0;
    for (; t < count && c < kMultiMax; ++t) {
      if (n[t] == 0) continue;
      a.m[c] = m[t];
      a.S[c] = S[t];
      a.dm[c] = dm[t];
      a.dS[c] = dS[t];
      a.n[c] = n[t];
      if (aligned16(m[t]) && aligned16(S[t]) && aligned16(dm[t]) && aligned16(dS[t])) a.vec_mask |= 1ull << c;
      a.block_start[c] = blocks;
      blocks += cdiv(n[t], kMultiChunk);
      ++c;
    }
    a.block_start[c] = blocks;
    a.count = c;
    if (c == 0) continue;
    hipLaunchKernelGGL(update_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    int rc = check_launch("tagi_capped_update_multi");
    if (rc) return rc;
  }
  return TAGI_OK;
}

extern "C" int tagi_add_inplace(const float* mu_s, const float* var_s, float* mu_a, float* var_a, int64_t n,
                                tagi_stream_t stream) {
  TAGI_REQUIRE(n >= 0, "tagi_add_inplace: n < 0");
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(mu_s && var_s && mu_a && var_a, "tagi_add_inplace: null pointer");
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_ADD, s, 0.0, 24.0 * n);
  const bool vec = aligned16(mu_s) && aligned16(var_s) && aligned16(mu_a) && aligned16(var_a);
  if (vec)
    hipLaunchKernelGGL(add_kernel<true>, dim3(ew_blocks(n / 4 + 1, 256)), dim3(256), 0, s, mu_s, var_s, mu_a, var_a,
                       n);
  else
    hipLaunchKernelGGL(add_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, mu_s, var_s, mu_a, var_a, n);
  return check_launch("tagi_add_inplace");
}

template <bool FWD, typename IT, int V>
static void launch_avgpool_as(const float* a, const float* b, float* c, float* d, IT N, IT C, IT H, IT W, IT k,
                              float var_scale, unsigned blocks, hipStream_t s) {
  const float inv_k2 = 1.0f / (float)(k * k);
  if constexpr (FWD)
    hipLaunchKernelGGL((avgpool_fwd_kernel<IT, V>), dim3(blocks), dim3(256), 0, s, a, b, c, d, N, H, W, C, k, inv_k2,
                       var_scale);
  else
    hipLaunchKernelGGL((avgpool_bwd_kernel<IT, V>), dim3(blocks), dim3(256), 0, s, a, b, c, d, N, H, W, C, k, inv_k2,
                       var_scale);
}

template <bool FWD>
static void launch_avgpool(const float* a, const float* b, float* c, float* d, int64_t N, int64_t C, int64_t H,
                           int64_t W, int64_t k, float var_scale, int64_t items, hipStream_t s) {
  const bool v4 = C % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(c) && aligned16(d);
  const bool small = N * C * H * W < (1ll << 31);
  const unsigned blocks = ew_blocks(v4 ? items / 4 : items, 256);
  if (small && v4)
    launch_avgpool_as<FWD, uint32_t, 4>(a, b, c, d, (uint32_t)N, (uint32_t)C, (uint32_t)H, (uint32_t)W, (uint32_t)k,
                                        var_scale, blocks, s);
  else if (small)
    launch_avgpool_as<FWD, uint32_t, 1>(a, b, c, d, (uint32_t)N, (uint32_t)C, (uint32_t)H, (uint32_t)W, (uint32_t)k,
                                        var_scale, blocks, s);
  else if (v4)
    launch_avgpool_as<FWD, int64_t, 4>(a, b, c, d, N, C, H, W, k, var_scale, blocks, s);
  else
    launch_avgpool_as<FWD, int64_t, 1>(a, b, c, d, N, C, H, W, k, var_scale, blocks, s);
}

extern "C" int tagi_avgpool2d_fwd(const float* ma, const float* Sa, float* ma_out, float* Sa_out, int64_t N,
                                  int64_t C, int64_t H, int64_t W, int64_t k, float var_scale, tagi_stream_t stream) {
  TAGI_REQUIRE(ma && Sa && ma_out && Sa_out, "tagi_avgpool2d_fwd: null pointer");
  TAGI_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && k > 0 && H >= k && W >= k, "tagi_avgpool2d_fwd: bad sizes");
  hipStream_t s = as_stream(stream);
  const int64_t out = N * C * (H / k) * (W / k);
  ProfScope ps(FAM_AVGPOOL, s, 0.0, 8.0 * (N * C * H * W + out));
  launch_avgpool<true>(ma, Sa, ma_out, Sa_out, N, C, H, W, k, var_scale, out, s);
  return check_launch("tagi_avgpool2d_fwd");
}

extern "C" int tagi_avgpool2d_bwd(const float* dm, const float* dS, float* dm_out, float* dS_out, int64_t N,
                                  int64_t C, int64_t H, int64_t W, int64_t k, float var_scale, tagi_stream_t stream) {
  TAGI_REQUIRE(dm && dS && dm_out && dS_out, "tagi_avgpool2d_bwd: null pointer");
  TAGI_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && k > 0 && H >= k && W >= k, "tagi_avgpool2d_bwd: bad sizes");
  hipStream_t s = as_stream(stream);
  const int64_t total = N * C * H * W;
  ProfScope ps(FAM_AVGPOOL, s, 0.0, 8.0 * (total + N * C * (H / k) * (W / k)));
  launch_avgpool<false>(dm, dS, dm_out, dS_out, N, C, H, W, k, var_scale, total, s);
  return check_launch("tagi_avgpool2d_bwd");
}

template <bool FWD, typename IT, int V, bool NCHW>
static void launch_pool_relu_lay(const float* a, const float* b, float* J, float* c, float* d, IT N, IT C, IT H,
                                 IT W, IT k, float var_scale, unsigned blocks, hipStream_t s) {
  const float inv_k2 = 1.0f / (float)(k * k);
  if constexpr (FWD)
    hipLaunchKernelGGL((relu_avgpool_fwd_kernel<IT, V, NCHW>), dim3(blocks), dim3(256), 0, s, a, b, J, c, d, N, H, W,
                       C, k, inv_k2, var_scale);
  else
    hipLaunchKernelGGL((avgpool_relu_bwd_kernel<IT, V, NCHW>), dim3(blocks), dim3(256), 0, s, a, b, J, c, d, N, H, W,
                       C, k, inv_k2, var_scale);
}

template <bool FWD, typename IT, int V>
static void launch_pool_relu_as(const float* a, const float* b, float* J, float* c, float* d, IT N, IT C, IT H, IT W,
                                IT k, float var_scale, bool nchw, unsigned blocks, hipStream_t s) {
  if (nchw)
    launch_pool_relu_lay<FWD, IT, V, true>(a, b, J, c, d, N, C, H, W, k, var_scale, blocks, s);
  else
    launch_pool_relu_lay<FWD, IT, V, false>(a, b, J, c, d, N, C, H, W, k, var_scale, blocks, s);
}

// FWD: a, b the conv output moments, J written, c, d the pooled moments; backward: a, b the
// pooled deltas, J read, c, d the deltas at the ReLU input. items: threads' work units.
template <bool FWD>
static void launch_pool_relu(const float* a, const float* b, const float* J, float* c, float* d, int64_t N, int64_t C,
                             int64_t H, int64_t W, int64_t k, float var_scale, bool nchw, int64_t items,
                             hipStream_t s) {
  // the pooled side (c, d forward; a, b backward) is read or written lane by lane when NCHW
  const bool v4 = C % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(J) && aligned16(c) && aligned16(d);
  const bool small = N * C * H * W < (1ll << 31);
  const unsigned blocks = ew_blocks(v4 ? items / 4 : items, 256);
  float* Jm = const_cast<float*>(J);
  if (small && v4)
    launch_pool_relu_as<FWD, uint32_t, 4>(a, b, Jm, c, d, (uint32_t)N, (uint32_t)C, (uint32_t)H, (uint32_t)W,
                                          (uint32_t)k, var_scale, nchw, blocks, s);
  else if (small)
    launch_pool_relu_as<FWD, uint32_t, 1>(a, b, Jm, c, d, (uint32_t)N, (uint32_t)C, (uint32_t)H, (uint32_t)W,
                                          (uint32_t)k, var_scale, nchw, blocks, s);
  else if (v4)
    launch_pool_relu_as<FWD, int64_t, 4>(a, b, Jm, c, d, N, C, H, W, k, var_scale, nchw, blocks, s);
  else
    launch_pool_relu_as<FWD, int64_t, 1>(a, b, Jm, c, d, N, C, H, W, k, var_scale, nchw, blocks, s);
}

extern "C" int tagi_relu_avgpool2d_fwd(const float* mz, const float* Sz, float* J, float* ma_out, float* Sa_out,
                                       int64_t N, int64_t C, int64_t H, int64_t W, int64_t k, float var_scale,
                                       int pooled_nchw, tagi_stream_t stream) {
  const char* what = "tagi_relu_avgpool2d_fwd";
  TAGI_REQUIRE(mz && Sz && J && ma_out && Sa_out, "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && k > 0 && H >= k && W >= k, "%s: bad sizes", what);
  if (H % k || W % k)
    return fail(TAGI_ERR_UNSUPPORTED, "%s: H and W must be multiples of the window (use tagi_relu_fwd and "
                "tagi_avgpool2d_fwd)", what);
  hipStream_t s = as_stream(stream);
  const int64_t out = N * C * (H / k) * (W / k);
  ProfScope ps(FAM_AVGPOOL, s, 0.0, 12.0 * N * C * H * W + 8.0 * out);
  launch_pool_relu<true>(mz, Sz, J, ma_out, Sa_out, N, C, H, W, k, var_scale, pooled_nchw != 0, out, s);
  return check_launch(what);
}

extern "C" int tagi_avgpool2d_relu_bwd(const float* dm, const float* dS, const float* J, float* dm_out,
                                       float* dS_out, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k,
                                       float var_scale, int pooled_nchw, tagi_stream_t stream) {
  const char* what = "tagi_avgpool2d_relu_bwd";
  TAGI_REQUIRE(dm && dS && J && dm_out && dS_out, "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && k > 0 && H >= k && W >= k, "%s: bad sizes", what);
  if (H % k || W % k)
    return fail(TAGI_ERR_UNSUPPORTED, "%s: H and W must be multiples of the window (use tagi_avgpool2d_bwd and "
                "tagi_jacobian_bwd)", what);
  hipStream_t s = as_stream(stream);
  const int64_t total = N * C * H * W;
  ProfScope ps(FAM_AVGPOOL, s, 0.0, 12.0 * total + 8.0 * N * C * (H / k) * (W / k));
  launch_pool_relu<false>(dm, dS, J, dm_out, dS_out, N, C, H, W, k, var_scale, pooled_nchw != 0, total, s);
  return check_launch(what);
}

extern "C" int tagi_remax_fwd(const float* mz, const float* Sz, float* ma, float* Sa, float* J, int64_t rows,
                              int64_t K, tagi_stream_t stream) {
  TAGI_REQUIRE(mz && Sz && ma && Sa && J, "tagi_remax_fwd: null pointer");
  TAGI_REQUIRE(rows >= 0 && K > 0, "tagi_remax_fwd: bad sizes");
  if (rows == 0) return TAGI_OK;
  if (K > 1024) return fail(TAGI_ERR_UNSUPPORTED, "tagi_remax_fwd: rows longer than 1024 classes (K=%lld)", (long long)K);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_REMAX, s, 0.0, 20.0 * rows * K);
  const unsigned blocks = (unsigned)cdiv(rows, 4);
  if (K <= 64)
    hipLaunchKernelGGL(remax_kernel<1>, dim3(blocks), dim3(256), 0, s, mz, Sz, ma, Sa, J, rows, (int)K);
  else if (K <= 256)
    hipLaunchKernelGGL(remax_kernel<4>, dim3(blocks), dim3(256), 0, s, mz, Sz, ma, Sa, J, rows, (int)K);
  else
    hipLaunchKernelGGL(remax_kernel<16>, dim3(blocks), dim3(256), 0, s, mz, Sz, ma, Sa, J, rows, (int)K);
  return check_launch("tagi_remax_fwd");
}
