// BatchNorm2D, RMSNorm, Embedding and positional-encoding kernels.
//
// Per-channel / per-column reductions are two-stage and deterministic: blocks write
// partial sums to a caller-provided workspace in a fixed layout, and a small finalize
// kernel adds them in a fixed order (no float atomics anywhere).
#include "tagi_common.h"

namespace tagi {

__device__ __forceinline__ float block_sum(float v, float* red) {
  // 256-thread block: wave reduction, then across the 4 waves through LDS.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  const int nw = blockDim.x >> 6;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// Split of the N images of one channel over `splits` blocks.
static inline int bn_splits(int64_t N, int64_t C, int64_t HW) {
  int64_t per_channel = N * HW;
  int64_t want = cdiv(2048, C);  // aim for >= 2048 blocks in total
  int64_t by_size = cdiv(per_channel, 8192);
  int64_t sp = want < by_size ? want : by_size;
  if (sp > N) sp = N;
  if (sp < 1) sp = 1;
  return (int)sp;
}

// ----------------------------------------------------------------- BN statistics
// grid (C, splits); block sums mu, S, mu^2 over its slice of images of channel c.
__global__ void __launch_bounds__(256) bn_stats_partial_kernel(const float* __restrict__ mz,
                                                               const float* __restrict__ Sz, float* __restrict__ ws,
                                                               int N, int C, int HW, int splits) {
  __shared__ float red[4];
  const int c = blockIdx.x, sp = blockIdx.y;
  const int n0 = (int)((int64_t)N * sp / splits), n1 = (int)((int64_t)N * (sp + 1) / splits);
  float a = 0.f, b = 0.f, q = 0.f;
  for (int n = n0; n < n1; ++n) {
    const float* pm = mz + ((int64_t)n * C + c) * HW;
    const float* ps = Sz + ((int64_t)n * C + c) * HW;
    if ((HW & 3) == 0 && (((uintptr_t)pm | (uintptr_t)ps) & 15) == 0) {
      for (int i = threadIdx.x; i < (HW >> 2); i += blockDim.x) {
        const float4 m = reinterpret_cast<const float4*>(pm)[i];
        const float4 s = reinterpret_cast<const float4*>(ps)[i];
        a += (m.x + m.y) + (m.z + m.w);
        b += (s.x + s.y) + (s.z + s.w);
        q += (m.x * m.x + m.y * m.y) + (m.z * m.z + m.w * m.w);
      }
    } else {
      for (int i = threadIdx.x; i < HW; i += blockDim.x) {
        const float m = pm[i];
        a += m;
        b += ps[i];
        q += m * m;
      }
    }
  }
  a = block_sum(a, red);
  b = block_sum(b, red);
  q = block_sum(q, red);
  if (threadIdx.x == 0) {
    float* o = ws + ((int64_t)c * splits + sp) * 3;
    o[0] = a;
    o[1] = b;
    o[2] = q;
  }
}

__global__ void bn_stats_finalize_kernel(const float* __restrict__ ws, float* __restrict__ bmean,
                                         float* __restrict__ bvar, float* __restrict__ rmean,
                                         float* __restrict__ rvar, float* __restrict__ mg, int C, int splits,
                                         double n, float momentum, float eps, int first_call, int preserve_var) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float a = 0.f, b = 0.f, q = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float* p = ws + ((int64_t)c * splits + s) * 3;
    a += p[0];
    b += p[1];
    q += p[2];
  }
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
__global__ void bn_fwd_kernel(const float* __restrict__ mz, const float* __restrict__ Sz,
                              const float* __restrict__ mean, const float* __restrict__ var,
                              const float* __restrict__ mg, const float* __restrict__ Sg,
                              const float* __restrict__ mb, const float* __restrict__ Sb, float* __restrict__ ma,
                              float* __restrict__ Sa, float* __restrict__ mhat, float* __restrict__ Shat, int64_t total,
                              int C, int HW, float eps, bool vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (vec) {
    const int64_t t4 = total >> 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < t4; i += stride) {
      const int c = (int)(((i << 2) / HW) % C);
      const float rv = var[c] + eps;
      const float inv_std = 1.0f / sqrtf(rv);
      const float mu = mean[c], g = mg[c], sg = Sg[c], b = mb[c], sb = Sb[c];
      const float4 m = reinterpret_cast<const float4*>(mz)[i];
      const float4 s = reinterpret_cast<const float4*>(Sz)[i];
      float4 mh, sh, om, os;
#define BNF(X)                                           \
  mh.X = (m.X - mu) * inv_std;                           \
  sh.X = s.X / rv;                                       \
  om.X = g * mh.X + b;                                   \
  os.X = g * g * sh.X + sg * mh.X * mh.X + sg * sh.X + sb;
      BNF(x) BNF(y) BNF(z) BNF(w)
#undef BNF
      reinterpret_cast<float4*>(ma)[i] = om;
      reinterpret_cast<float4*>(Sa)[i] = os;
      reinterpret_cast<float4*>(mhat)[i] = mh;
      if (Shat) reinterpret_cast<float4*>(Shat)[i] = sh;
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int c = (int)((i / HW) % C);
      const float rv = var[c] + eps;
      const float inv_std = 1.0f / sqrtf(rv);
      const float g = mg[c], sg = Sg[c];
      const float mh = (mz[i] - mean[c]) * inv_std;
      const float sh = Sz[i] / rv;
      ma[i] = g * mh + mb[c];
      Sa[i] = g * g * sh + sg * mh * mh + sg * sh + Sb[c];
      mhat[i] = mh;
      if (Shat) Shat[i] = sh;
    }
  }
}

// ------------------------------------------------------------------- BN backward
// grid (C, splits): propagated deltas for the block's slice + 4 partial channel sums.
__global__ void __launch_bounds__(256) bn_bwd_partial_kernel(
    const float* __restrict__ dma, const float* __restrict__ dSa, const float* __restrict__ mhat,
    const float* __restrict__ var, const float* __restrict__ mg, float* __restrict__ dmz, float* __restrict__ dSz,
    float* __restrict__ ws, int N, int C, int HW, int splits, float eps) {
  __shared__ float red[4];
  const int c = blockIdx.x, sp = blockIdx.y;
  const int n0 = (int)((int64_t)N * sp / splits), n1 = (int)((int64_t)N * (sp + 1) / splits);
  const float rv = var[c] + eps;
  const float g = mg[c];
  const float km = g * (1.0f / sqrtf(rv));
  const float kS = g * g * (1.0f / rv);
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  for (int n = n0; n < n1; ++n) {
    const int64_t base = ((int64_t)n * C + c) * HW;
    for (int i = threadIdx.x; i < HW; i += blockDim.x) {
      const float dm = dma[base + i], ds = dSa[base + i], mh = mhat[base + i];
      s0 += dm * mh;
      s1 += ds * mh * mh;
      s2 += dm;
      s3 += ds;
      dmz[base + i] = dm * km;
      dSz[base + i] = ds * kS;
    }
  }
  s0 = block_sum(s0, red);
  s1 = block_sum(s1, red);
  s2 = block_sum(s2, red);
  s3 = block_sum(s3, red);
  if (threadIdx.x == 0) {
    float* o = ws + ((int64_t)c * splits + sp) * 4;
    o[0] = s0;
    o[1] = s1;
    o[2] = s2;
    o[3] = s3;
  }
}

__global__ void bn_bwd_finalize_kernel(const float* __restrict__ ws, const float* __restrict__ Sg,
                                       const float* __restrict__ Sb, float* __restrict__ dmg, float* __restrict__ dSg,
                                       float* __restrict__ dmb, float* __restrict__ dSb, int C, int splits) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float* p = ws + ((int64_t)c * splits + s) * 4;
    s0 += p[0];
    s1 += p[1];
    s2 += p[2];
    s3 += p[3];
  }
  const float g = Sg[c], b = Sb[c];
  dmg[c] = g * s0;
  dSg[c] = g * g * s1;
  dmb[c] = b * s2;
  dSb[c] = b * b * s3;
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

// Backward: each block owns a slab of rows; threads stride over the D columns, so the
// per-column partial sums need no cross-thread reduction.
__global__ void rmsnorm_bwd_partial_kernel(const float* __restrict__ dmz, const float* __restrict__ dSz,
                                           const float* __restrict__ ma, const float* __restrict__ inv_rms,
                                           const float* __restrict__ mw, float* __restrict__ dma,
                                           float* __restrict__ dSa, float* __restrict__ ws, int64_t rows, int D,
                                           int rows_per_block) {
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = min(rows, r0 + rows_per_block);
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    const float w = mw[c];
    float s_mu = 0.f, s_var = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
      const float inv = inv_rms[r];
      const int64_t i = r * D + c;
      const float dm = dmz[i], ds = dSz[i], m = ma[i];
      const float t = inv * w;
      dma[i] = t * dm;
      dSa[i] = t * t * ds;
      s_mu += inv * m * dm;
      s_var += inv * inv * m * m * ds;
    }
    ws[((int64_t)blockIdx.x * 2) * D + c] = s_mu;
    ws[((int64_t)blockIdx.x * 2 + 1) * D + c] = s_var;
  }
}

__global__ void rmsnorm_bwd_finalize_kernel(const float* __restrict__ ws, const float* __restrict__ Sw,
                                            float* __restrict__ dmw, float* __restrict__ dSw, int D, int nblk) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= D) return;
  float a = 0.f, b = 0.f;
  for (int k = 0; k < nblk; ++k) {
    a += ws[((int64_t)k * 2) * D + c];
    b += ws[((int64_t)k * 2 + 1) * D + c];
  }
  const float sw = Sw[c];
  dmw[c] = a * sw;
  dSw[c] = b * sw * sw;
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

// grid (slabs of columns, chunks of tokens); block threads own one column each and walk
// the chunk's tokens in order, accumulating into an LDS table [V][slab].
__global__ void embedding_bwd_partial_kernel(const float* __restrict__ tokens, const float* __restrict__ dmz,
                                             const float* __restrict__ dSz, const float* __restrict__ Sw,
                                             float* __restrict__ ws, int64_t n_tokens, int V, int D,
                                             int64_t padding_idx, int slab, int chunk) {
  extern __shared__ float tab[];  // [2][V][slab]
  const int d = blockIdx.x * slab + threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.y * chunk;
  const int64_t t1 = min(n_tokens, t0 + chunk);
  for (int i = threadIdx.x; i < 2 * V * slab; i += blockDim.x) tab[i] = 0.f;
  __syncthreads();
  if (threadIdx.x < slab && d < D) {
    for (int64_t t = t0; t < t1; ++t) {
      const int64_t cat = token_id(tokens[t]);
      if (cat < 0 || cat >= V || cat == padding_idx) continue;
      const float sw = Sw[cat * D + d];
      tab[cat * slab + threadIdx.x] += dmz[t * D + d] * sw;
      tab[(V + cat) * slab + threadIdx.x] += dSz[t * D + d] * sw * sw;
    }
  }
  __syncthreads();
  if (threadIdx.x < slab && d < D) {
    for (int v = 0; v < V; ++v) {
      ws[(((int64_t)blockIdx.y * 2) * V + v) * D + d] = tab[v * slab + threadIdx.x];
      ws[(((int64_t)blockIdx.y * 2 + 1) * V + v) * D + d] = tab[(V + v) * slab + threadIdx.x];
    }
  }
}

__global__ void embedding_bwd_finalize_kernel(const float* __restrict__ ws, float* __restrict__ dmw,
                                              float* __restrict__ dSw, int V, int D, int nchunks) {
  const int64_t total = (int64_t)V * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float a = 0.f, b = 0.f;
    for (int k = 0; k < nchunks; ++k) {
      a += ws[((int64_t)k * 2) * total + i];
      b += ws[((int64_t)k * 2 + 1) * total + i];
    }
    dmw[i] = a;
    dSw[i] = b;
  }
}

// -------------------------------------------------------------------------- PE
__global__ void pe_add_kernel(const float* __restrict__ ma, const float* __restrict__ pe, float* __restrict__ out,
                              int64_t total, int64_t SE) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = ma[i] + pe[i % SE];
}

static inline void emb_plan(int64_t n_tokens, int64_t V, int64_t D, int* slab, int* chunk, int* nchunks) {
  int s = (int)(65536 / (8 * V));
  s = (s / 32) * 32;
  if (s > 256) s = 256;
  if (s > D) s = (int)(((D + 31) / 32) * 32);
  *slab = s;
  *chunk = 256;
  *nchunks = (int)cdiv(n_tokens, 256);
}

}  // namespace tagi

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

extern "C" int64_t tagi_bn_stats_ws_bytes(int64_t N, int64_t C, int64_t HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  return (int64_t)C * bn_splits(N, C, HW) * 3 * (int64_t)sizeof(float);
}

extern "C" int tagi_bn_stats(const float* mz, const float* Sz, float* batch_mean, float* batch_var,
                             float* running_mean, float* running_var, float* mg, int64_t N, int64_t C, int64_t HW,
                             float momentum, float eps, int first_call, int preserve_var, float* ws, int64_t ws_bytes,
                             tagi_stream_t stream) {
  const char* what = "tagi_bn_stats";
  TAGI_REQUIRE(mz && Sz && batch_mean && batch_var && ws, "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && HW > 0 && N * HW > 1, "%s: bad sizes", what);
  TAGI_REQUIRE(N * C * HW < (1ll << 40) && C < 65536, "%s: too large", what);
  TAGI_REQUIRE(ws_bytes >= tagi_bn_stats_ws_bytes(N, C, HW), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BN_STATS, s, 0.0, 8.0 * N * C * HW);
  const int sp = bn_splits(N, C, HW);
  hipLaunchKernelGGL(bn_stats_partial_kernel, dim3((unsigned)C, (unsigned)sp), dim3(256), 0, s, mz, Sz, ws, (int)N,
                     (int)C, (int)HW, sp);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(bn_stats_finalize_kernel, dim3((unsigned)cdiv(C, 256)), dim3(256), 0, s, (const float*)ws,
                     batch_mean, batch_var, running_mean, running_var, mg, (int)C, sp, (double)(N * HW), momentum, eps,
                     first_call, preserve_var);
  return check_launch(what);
}

extern "C" int tagi_bn_fwd(const float* mz, const float* Sz, const float* mean, const float* var, const float* mg,
                           const float* Sg, const float* mb, const float* Sb, float* ma, float* Sa, float* mhat,
                           float* Shat, int64_t N, int64_t C, int64_t HW, float eps, tagi_stream_t stream) {
  const char* what = "tagi_bn_fwd";
  TAGI_REQUIRE(mz && Sz && mean && var && mg && Sg && mb && Sb && ma && Sa && mhat, "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && HW > 0, "%s: bad sizes", what);
  hipStream_t s = as_stream(stream);
  const int64_t total = N * C * HW;
  ProfScope ps(FAM_BN_FWD, s, 0.0, 4.0 * total * (Shat ? 6 : 5));
  const bool vec = (HW % 4 == 0) && ((((uintptr_t)mz | (uintptr_t)Sz | (uintptr_t)ma | (uintptr_t)Sa |
                                       (uintptr_t)mhat | (uintptr_t)(Shat ? Shat : ma)) & 15) == 0);
  hipLaunchKernelGGL(bn_fwd_kernel, dim3(ew_blocks(vec ? total / 4 : total, 256)), dim3(256), 0, s, mz, Sz, mean, var,
                     mg, Sg, mb, Sb, ma, Sa, mhat, Shat, total, (int)C, (int)HW, eps, vec);
  return check_launch(what);
}

extern "C" int64_t tagi_bn_bwd_ws_bytes(int64_t N, int64_t C, int64_t HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  return (int64_t)C * bn_splits(N, C, HW) * 4 * (int64_t)sizeof(float);
}

extern "C" int tagi_bn_bwd(const float* dma, const float* dSa, const float* mhat, const float* var, const float* mg,
                           const float* Sg, const float* Sb, float* dmz, float* dSz, float* dmg, float* dSg,
                           float* dmb, float* dSb, int64_t N, int64_t C, int64_t HW, float eps, float* ws,
                           int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_bn_bwd";
  TAGI_REQUIRE(dma && dSa && mhat && var && mg && Sg && Sb && dmz && dSz && dmg && dSg && dmb && dSb && ws,
               "%s: null pointer", what);
  TAGI_REQUIRE(N > 0 && C > 0 && HW > 0 && C < 65536, "%s: bad sizes", what);
  TAGI_REQUIRE(ws_bytes >= tagi_bn_bwd_ws_bytes(N, C, HW), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BN_BWD, s, 0.0, 20.0 * N * C * HW);
  const int sp = bn_splits(N, C, HW);
  hipLaunchKernelGGL(bn_bwd_partial_kernel, dim3((unsigned)C, (unsigned)sp), dim3(256), 0, s, dma, dSa, mhat, var, mg,
                     dmz, dSz, ws, (int)N, (int)C, (int)HW, sp, eps);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(bn_bwd_finalize_kernel, dim3((unsigned)cdiv(C, 256)), dim3(256), 0, s, (const float*)ws, Sg, Sb,
                     dmg, dSg, dmb, dSb, (int)C, sp);
  return check_launch(what);
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

static inline int rms_rows_per_block(int64_t rows) {
  int64_t r = cdiv(rows, 1024);
  return (int)(r < 16 ? 16 : r);
}

extern "C" int64_t tagi_rmsnorm_bwd_ws_bytes(int64_t rows, int64_t D) {
  if (rows <= 0 || D <= 0) return 0;
  return cdiv(rows, rms_rows_per_block(rows)) * 2 * D * (int64_t)sizeof(float);
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
  const int rpb = rms_rows_per_block(rows);
  const int nblk = (int)cdiv(rows, rpb);
  hipLaunchKernelGGL(rmsnorm_bwd_partial_kernel, dim3((unsigned)nblk), dim3(256), 0, s, dmz, dSz, ma, inv_rms, mw, dma,
                     dSa, ws, rows, (int)D, rpb);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(rmsnorm_bwd_finalize_kernel, dim3((unsigned)cdiv(D, 256)), dim3(256), 0, s, (const float*)ws, Sw,
                     dmw, dSw, (int)D, nblk);
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
  hipLaunchKernelGGL(embedding_fwd_kernel, dim3(ew_blocks(n_tokens * D, 256)), dim3(256), 0, s, tokens, mw, Sw, mz, Sz,
                     n_tokens, V, (int)D, padding_idx);
  return check_launch(what);
}

extern "C" int64_t tagi_embedding_bwd_ws_bytes(int64_t n_tokens, int64_t V, int64_t D) {
  if (n_tokens <= 0 || V <= 0 || D <= 0) return 0;
  int slab, chunk, nch;
  emb_plan(n_tokens, V, D, &slab, &chunk, &nch);
  return (int64_t)nch * 2 * V * D * (int64_t)sizeof(float);
}

extern "C" int tagi_embedding_bwd(const float* tokens, const float* dmz, const float* dSz, const float* Sw, float* dmw,
                                  float* dSw, int64_t n_tokens, int64_t V, int64_t D, int64_t padding_idx, float* ws,
                                  int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_embedding_bwd";
  TAGI_REQUIRE(tokens && dmz && dSz && Sw && dmw && dSw, "%s: null pointer", what);
  TAGI_REQUIRE(n_tokens > 0 && V > 0 && D > 0, "%s: bad sizes", what);
  if (V > 256) return fail(TAGI_ERR_UNSUPPORTED, "%s: vocabularies above 256 rows", what);
  TAGI_REQUIRE(ws && ws_bytes >= tagi_embedding_bwd_ws_bytes(n_tokens, V, D), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_EMBEDDING, s, 0.0, 4.0 * n_tokens + 8.0 * n_tokens * D + 8.0 * V * D);
  int slab, chunk, nch;
  emb_plan(n_tokens, V, D, &slab, &chunk, &nch);
  const size_t lds = (size_t)2 * V * slab * sizeof(float);
  hipLaunchKernelGGL(embedding_bwd_partial_kernel, dim3((unsigned)cdiv(D, slab), (unsigned)nch), dim3(slab), lds, s,
                     tokens, dmz, dSz, Sw, ws, n_tokens, (int)V, (int)D, padding_idx, slab, chunk);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(embedding_bwd_finalize_kernel, dim3(ew_blocks(V * D, 256)), dim3(256), 0, s, (const float*)ws,
                     dmw, dSw, (int)V, (int)D, nch);
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
