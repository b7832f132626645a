// Output heads beyond the dense Gaussian likelihood:
//   * hierarchical softmax (HRC): the sparse innovation on the tree nodes of each
//     sample's class path, and the class probabilities / predicted labels;
//   * heteroscedastic TAGI-V: the innovation of an interleaved (mean, noise) output and
//     the EvenSoftplus activation that keeps the noise outputs positive.
// All are bandwidth- or latency-bound and touch each output element once.
#include "tagi_common.h"

namespace tagi {

// ------------------------------------------------------------------ HRC innovation
// Row b of the (rows x n_out) output receives, for each encoded bit c, the innovation
// (y - mu)/(S + v) and -1/(S + v) at node idx[b, c] - 1, and zeros elsewhere
// (observation.py:171-224). One thread per output element gathers the bits that select
// it, in bit order: nodes selected twice add up as scatter_add does, and no memset or
// atomic is needed. Node indices outside [1, n_out] select nothing. The grid covers one
// element per thread up to 2^28 elements, so the dependent loads (label, class table,
// moments) of many elements are in flight at once.
//
// LABELS: the bits come from class tables, obs/idx[label[b] * n_obs + c], with the
// scalar noise v = sigma_v^2 (labels_to_hrc + torch.full_like at network.py:205-209
// folded in); a label outside [0, n_classes) makes its row NaN.
template <bool LABELS, typename IT>
__global__ void __launch_bounds__(256) hrc_innovation_kernel(const float* __restrict__ ma,
                                                             const float* __restrict__ Sa,
                                                             const float* __restrict__ y_obs,
                                                             const float* __restrict__ var_obs,
                                                             const int32_t* __restrict__ idx,
                                                             const int64_t* __restrict__ labels, int64_t n_classes,
                                                             float var_scalar, float* __restrict__ dm,
                                                             float* __restrict__ dS, int64_t rows, int n_out,
                                                             int n_obs) {
  const int64_t total = rows * (int64_t)n_out;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    // IT = uint32_t when every flat index fits: 32-bit division is a short sequence
    const int64_t b = (int64_t)((IT)e / (IT)n_out);
    const int j = (int)(e - b * n_out);
    // the moments are loaded up front so their latency overlaps the table lookups
    const float mu = ma[e], S = Sa[e];
    const int32_t* ib;
    const float* yb;
    if constexpr (LABELS) {
      const int64_t lab = labels[b];
      if (lab < 0 || lab >= n_classes) {
        dm[e] = __builtin_nanf("");
        dS[e] = __builtin_nanf("");
        continue;
      }
      ib = idx + lab * n_obs;
      yb = y_obs + lab * n_obs;
    } else {
      ib = idx + b * n_obs;
      yb = y_obs + b * n_obs;
    }
    float am = 0.f, aS = 0.f;
    for (int c = 0; c < n_obs; ++c) {
      if (ib[c] - 1 != j) continue;
      const float v = LABELS ? var_scalar : var_obs[b * n_obs + c];
      const float den = S + v;
      am += (yb[c] - mu) / den;
      aS += -1.0f / den;
    }
    dm[e] = am;
    dS[e] = aS;
  }
}

// Small trees (fewer than 32 nodes): one thread per sample row, kHrcRows rows per
// block. Each thread adds its row's bits, in bit order, into the row's slots in LDS (the
// same sums as the kernel above, in the same order), then the block writes its rows with
// coalesced stores.
constexpr int kHrcRows = 256;
constexpr int kHrcRowLds = 64 * kHrcRows;  // floats of dynamic LDS at most (64 KiB)

__host__ __device__ inline int odd_stride(int n) { return n | 1; }

template <bool LABELS>
__global__ void __launch_bounds__(kHrcRows) hrc_innovation_rows_kernel(const float* __restrict__ ma,
                                                                       const float* __restrict__ Sa,
                                                                       const float* __restrict__ y_obs,
                                                                       const float* __restrict__ var_obs,
                                                                       const int32_t* __restrict__ idx,
                                                                       const int64_t* __restrict__ labels,
                                                                       int64_t n_classes, float var_scalar,
                                                                       float* __restrict__ dm, float* __restrict__ dS,
                                                                       int64_t rows, int n_out, int n_obs) {
  extern __shared__ float lds[];
  const int ldz = odd_stride(n_out);
  float* om = lds;                   // [kHrcRows][ldz]
  float* oS = lds + kHrcRows * ldz;  // [kHrcRows][ldz]
  const int64_t b0 = (int64_t)blockIdx.x * kHrcRows;
  const int nr = (int)min((int64_t)kHrcRows, rows - b0);
  for (int e = threadIdx.x; e < kHrcRows * ldz; e += kHrcRows) {
    om[e] = 0.f;
    oS[e] = 0.f;
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < nr) {
    const int64_t b = b0 + t;
    float* rm = om + t * ldz;
    float* rS = oS + t * ldz;
    int64_t tab = b;  // the row of the bit tables
    bool bad = false;
    if constexpr (LABELS) {
      const int64_t lab = labels[b];
      bad = lab < 0 || lab >= n_classes;
      tab = bad ? 0 : lab;
    }
    const int32_t* ib = idx + tab * n_obs;
    const float* yb = y_obs + tab * n_obs;
    if (bad) {
      for (int j = 0; j < n_out; ++j) {
        rm[j] = __builtin_nanf("");
        rS[j] = __builtin_nanf("");
      }
    } else {
      const float* mb = ma + b * n_out;
      const float* sb = Sa + b * n_out;
      // up to kU bits at a time: their loads are issued together, then the sums are added
      // in bit order
      constexpr int kU = 8;
      for (int c0 = 0; c0 < n_obs; c0 += kU) {
        int node[kU];
        float mu[kU], S[kU], y[kU], v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int c = c0 + u;
          node[u] = c < n_obs ? ib[c] - 1 : -1;
          const bool ok = node[u] >= 0 && node[u] < n_out;
          mu[u] = ok ? mb[node[u]] : 0.f;
          S[u] = ok ? sb[node[u]] : 0.f;
          y[u] = ok ? yb[c] : 0.f;
          v[u] = ok ? (LABELS ? var_scalar : var_obs[b * n_obs + c]) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          if (node[u] < 0 || node[u] >= n_out) continue;
          const float den = S[u] + v[u];
          rm[node[u]] += (y[u] - mu[u]) / den;
          rS[node[u]] += -1.0f / den;
        }
      }
    }
  }
  __syncthreads();
  const int64_t base = b0 * n_out;
  for (int e = threadIdx.x; e < nr * n_out; e += kHrcRows) {
    const int r = e / n_out, j = e - r * n_out;
    dm[base + e] = om[r * ldz + j];
    dS[base + e] = oS[r * ldz + j];
  }
}

// ------------------------------------------------------------ HRC class probabilities
// P_z[i] = Phi(mu[i] / sqrt(1/alpha^2 + S[i])) per tree node, then for each class the
// product along its path of P_z (bit +1) or 1 - P_z (bit -1) (hrc_softmax.py:164-208).
// Large trees: one block per sample row; node probabilities are formed once into LDS (up
// to kHrcLds nodes; larger trees evaluate them per use), then threads take classes. With
// `pred`, each kernel also writes the first index of the largest probability (a NaN
// counts as the largest, as torch's argmax treats it).
constexpr int kHrcLds = 8192;

__device__ __forceinline__ float node_prob(float m, float S, float inv_a2) {
  return 0.5f * erfcf(-(m / sqrtf(inv_a2 + S)) * 0.70710678118654752f);
}

// (value, index) order for the argmax: NaN first, then larger value, then lower index.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

// Small trees (odd-padded node and class widths summing to at most 64): one thread per
// sample row, kHrcRows rows per block. The block reads its rows' node moments
// with coalesced loads, forms each node probability once into LDS (row stride odd, so the
// per-thread row reads do not conflict), and every thread walks the classes in order:
// the table entries are the same for all lanes. Class probabilities go back through LDS so
// the stores are coalesced too.
__global__ void __launch_bounds__(kHrcRows) hrc_class_probs_rows_kernel(const float* __restrict__ ma,
                                                                        const float* __restrict__ Sa,
                                                                        const float* __restrict__ obs,
                                                                        const int32_t* __restrict__ idx,
                                                                        float inv_a2, float* __restrict__ probs,
                                                                        int64_t* __restrict__ pred, int64_t rows,
                                                                        int n_out, int n_obs, int n_classes) {
  extern __shared__ float lds[];
  const int ldz = odd_stride(n_out), ldp = odd_stride(n_classes);
  float* pz = lds;                      // [kHrcRows][ldz]
  float* pc = lds + kHrcRows * ldz;     // [kHrcRows][ldp]
  const int64_t b0 = (int64_t)blockIdx.x * kHrcRows;
  const int nr = (int)min((int64_t)kHrcRows, rows - b0);
  const int64_t base = b0 * n_out;
  for (int e = threadIdx.x; e < nr * n_out; e += kHrcRows) {
    const int r = e / n_out, j = e - r * n_out;
    pz[r * ldz + j] = node_prob(ma[base + e], Sa[base + e], inv_a2);
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < nr) {
    const float* z = pz + t * ldz;
    float* out = pc + t * ldp;
    float best_v = -__builtin_inff();
    int64_t best_i = 0x7fffffffffffffffll;
    for (int r = 0; r < n_classes; ++r) {
      float p = 1.0f;
      for (int c = 0; c < n_obs; ++c) {
        const int node = idx[r * n_obs + c] - 1;
        const float q = (node >= 0 && node < n_out) ? z[node] : 0.f;
        p *= obs[r * n_obs + c] > 0.f ? q : 1.0f - q;
      }
      out[r] = p;
      if (better(p, r, best_v, best_i)) {
        best_v = p;
        best_i = r;
      }
    }
    if (pred != nullptr) pred[b0 + t] = best_i;
  }
  __syncthreads();
  const int64_t obase = b0 * n_classes;
  for (int e = threadIdx.x; e < nr * n_classes; e += kHrcRows) {
    const int r = e / n_classes, k = e - r * n_classes;
    probs[obase + e] = pc[r * ldp + k];
  }
}

// Trees of at most 64 nodes and 64 classes: one wavefront per row, four rows per block.
// Lane j holds the probability of node j; class r (lane r) multiplies the probabilities
// of its path's nodes, fetched from the lanes that hold them by cross-lane permutes.
__global__ void __launch_bounds__(256) hrc_class_probs_wave_kernel(const float* __restrict__ ma,
                                                                   const float* __restrict__ Sa,
                                                                   const float* __restrict__ obs,
                                                                   const int32_t* __restrict__ idx, float inv_a2,
                                                                   float* __restrict__ probs,
                                                                   int64_t* __restrict__ pred, int64_t rows,
                                                                   int n_out, int n_obs, int n_classes) {
  const int lane = threadIdx.x & 63;
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= rows) return;  // whole wavefronts leave together
  const float pz = lane < n_out ? node_prob(ma[b * n_out + lane], Sa[b * n_out + lane], inv_a2) : 0.f;
  const bool mine = lane < n_classes;
  float p = 1.0f;
  for (int c = 0; c < n_obs; ++c) {
    int node = mine ? idx[lane * n_obs + c] - 1 : 0;
    const bool ok = node >= 0 && node < n_out;
    const float q = __shfl(pz, ok ? node : 0, 64);
    if (mine) p *= obs[lane * n_obs + c] > 0.f ? (ok ? q : 0.f) : 1.0f - (ok ? q : 0.f);
  }
  if (mine) probs[b * n_classes + lane] = p;
  if (pred == nullptr) return;
  float bv = mine ? p : -__builtin_inff();
  int64_t bi = mine ? lane : 0x7fffffffffffffffll;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int64_t oi = __shfl_xor(bi, off, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) pred[b] = bi;
}

__global__ void __launch_bounds__(256) hrc_class_probs_kernel(const float* __restrict__ ma,
                                                              const float* __restrict__ Sa,
                                                              const float* __restrict__ obs,
                                                              const int32_t* __restrict__ idx, float inv_a2,
                                                              float* __restrict__ probs, int64_t* __restrict__ pred,
                                                              int n_out, int n_obs, int n_classes) {
  __shared__ float pz[kHrcLds];
  __shared__ float wv[4];
  __shared__ int64_t wi[4];
  const int64_t b = blockIdx.x;
  const float* mb = ma + b * n_out;
  const float* sb = Sa + b * n_out;
  const bool in_lds = n_out <= kHrcLds;
  if (in_lds) {
    for (int j = threadIdx.x; j < n_out; j += blockDim.x) pz[j] = node_prob(mb[j], sb[j], inv_a2);
    __syncthreads();
  }
  float best_v = -__builtin_inff();
  int64_t best_i = 0x7fffffffffffffffll;
  for (int r = threadIdx.x; r < n_classes; r += blockDim.x) {
    float p = 1.0f;
    for (int c = 0; c < n_obs; ++c) {
      const int node = idx[(int64_t)r * n_obs + c] - 1;
      float q = 0.f;
      if (node >= 0 && node < n_out) q = in_lds ? pz[node] : node_prob(mb[node], sb[node], inv_a2);
      p *= obs[(int64_t)r * n_obs + c] > 0.f ? q : 1.0f - q;
    }
    probs[b * n_classes + r] = p;
    if (better(p, r, best_v, best_i)) {
      best_v = p;
      best_i = r;
    }
  }
  if (pred == nullptr) return;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best_v, off, 64);
    const int64_t oi = __shfl_xor(best_i, off, 64);
    if (better(ov, oi, best_v, best_i)) {
      best_v = ov;
      best_i = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    wv[w] = best_v;
    wi[w] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = wv[0];
    int64_t i = wi[0];
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k)
      if (better(wv[k], wi[k], v, i)) {
        v = wv[k];
        i = wi[k];
      }
    pred[b] = i;
  }
}

// ------------------------------------------------------- heteroscedastic innovation
// Output pairs (mean, noise) interleaved: mu[2i], S[2i] are the prediction of
// observation i and mu[2i+1], S[2i+1] the moments of the noise-variance output V2_bar.
// V ~ N(0, E[V2_bar]) is the observation noise: Y = A + V. The update conditions (A, V)
// on y, moves V^2 to its posterior moments and carries that to V2_bar through their
// covariance Var[V2_bar] (observation.py:49-111).
__device__ __forceinline__ void heteros_one(float y, float mu_a, float var_a, float mu_v2b, float var_v2b,
                                            float& d_mu, float& d_var, float& d_mu_v2, float& d_var_v2) {
  const float mu_v2 = mu_v2b;                                   // E[V^2]
  const float var_v2 = 3.0f * var_v2b + 2.0f * mu_v2b * mu_v2b;  // Var[V^2]
  const float cov_yv = mu_v2;
  const float var_sum = var_a + mu_v2;
  const float inv = 1.0f / var_sum;
  const float diff = y - mu_a;
  d_mu = inv * diff;
  d_var = -inv;
  const float mv_post = cov_yv / var_sum * diff;
  const float vv_post = mu_v2 - cov_yv / var_sum * cov_yv;
  const float mv2_post = mv_post * mv_post + vv_post;
  const float vv2_post = 2.0f * vv_post * vv_post + 4.0f * vv_post * mv_post * mv_post;
  const float k = var_v2b / var_v2;
  const float m_post = mu_v2b + k * (mv2_post - mu_v2);
  const float v_post = var_v2b + k * k * (vv2_post - var_v2);
  d_mu_v2 = m_post - mu_v2b;
  d_var_v2 = v_post - var_v2b;
}

template <bool VEC>
__global__ void heteros_innovation_kernel(const float* __restrict__ y, const float* __restrict__ mu,
                                          const float* __restrict__ var, float* __restrict__ dm,
                                          float* __restrict__ dS, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float m0, m1, s0, s1;
    if constexpr (VEC) {
      const float2 m = reinterpret_cast<const float2*>(mu)[i];
      const float2 s = reinterpret_cast<const float2*>(var)[i];
      m0 = m.x, m1 = m.y, s0 = s.x, s1 = s.y;
    } else {
      m0 = mu[2 * i], m1 = mu[2 * i + 1], s0 = var[2 * i], s1 = var[2 * i + 1];
    }
    float a, b, c, d;
    heteros_one(y[i], m0, s0, m1, s1, a, b, c, d);
    if constexpr (VEC) {
      reinterpret_cast<float2*>(dm)[i] = make_float2(a, c);
      reinterpret_cast<float2*>(dS)[i] = make_float2(b, d);
    } else {
      dm[2 * i] = a, dm[2 * i + 1] = c, dS[2 * i] = b, dS[2 * i + 1] = d;
    }
  }
}

// ------------------------------------------------------------------- EvenSoftplus
// Odd flat positions (the noise outputs of interleaved pairs) get the second-order
// moments of softplus, even positions pass through (even_softplus.py:38-90):
//   s = sigmoid(mu), mu_a = max(softplus(mu) + S s(1-s)/2, 1e-9),
//   S_a = max(s^2 S, 1e-9), J = s;   even: mu_a = mu, S_a = S, J = 1.
// softplus(mu) = mu above 20 and log1p(exp(mu)) below.
__device__ __forceinline__ void softplus_moments(float m, float S, float& ma, float& Sa, float& J) {
  const float sig = 1.0f / (1.0f + expf(-m));
  const float sp = m > 20.0f ? m : log1pf(expf(m));
  ma = fmaxf(sp + 0.5f * S * sig * (1.0f - sig), 1e-9f);
  Sa = fmaxf(sig * sig * S, 1e-9f);
  J = sig;
}

template <bool VEC>
__global__ void even_softplus_kernel(const float* __restrict__ mz, const float* __restrict__ Sz,
                                     float* __restrict__ ma, float* __restrict__ Sa, float* __restrict__ J,
                                     int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if constexpr (VEC) {
    // one (even, odd) pair per thread; n is even
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n / 2; i += stride) {
      const float2 m = reinterpret_cast<const float2*>(mz)[i];
      const float2 s = reinterpret_cast<const float2*>(Sz)[i];
      float a, b, j;
      softplus_moments(m.y, s.y, a, b, j);
      reinterpret_cast<float2*>(ma)[i] = make_float2(m.x, a);
      reinterpret_cast<float2*>(Sa)[i] = make_float2(s.x, b);
      reinterpret_cast<float2*>(J)[i] = make_float2(1.0f, j);
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
      if (i & 1) {
        softplus_moments(mz[i], Sz[i], ma[i], Sa[i], J[i]);
      } else {
        ma[i] = mz[i];
        Sa[i] = Sz[i];
        J[i] = 1.0f;
      }
    }
  }
}

static inline bool al(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace tagi

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

static unsigned hrc_blocks(int64_t total) { return (unsigned)std::min<int64_t>(cdiv(total, 256), 1ll << 20); }

// The row-per-thread innovation kernel holds two (256 x odd-padded width) float tables in LDS.
static bool hrc_rows_fit(int64_t rows, int64_t n_out) {
  return rows < (1ll << 31) && n_out < 32 && 2ll * kHrcRows * odd_stride((int)n_out) <= kHrcRowLds;
}

template <bool LABELS>
static void launch_hrc_rows(const float* ma, const float* Sa, const float* y_obs, const float* var_obs,
                            const int32_t* idx, const int64_t* labels, int64_t n_classes, float var_scalar, float* dm,
                            float* dS, int64_t rows, int64_t n_out, int64_t n_obs, hipStream_t s) {
  const size_t lds = 2ull * kHrcRows * odd_stride((int)n_out) * sizeof(float);
  hipLaunchKernelGGL((hrc_innovation_rows_kernel<LABELS>), dim3((unsigned)cdiv(rows, kHrcRows)), dim3(kHrcRows), lds,
                     s, ma, Sa, y_obs, var_obs, idx, labels, n_classes, var_scalar, dm, dS, rows, (int)n_out,
                     (int)n_obs);
}

extern "C" int tagi_innovation_indexed(const float* ma, const float* Sa, const float* y_obs, const float* var_obs,
                                       const int32_t* idx, float* dm, float* dS, int64_t rows, int64_t n_out,
                                       int64_t n_obs, tagi_stream_t stream) {
  const char* what = "tagi_innovation_indexed";
  TAGI_REQUIRE(rows >= 0 && n_out > 0 && n_obs >= 0, "%s: bad sizes", what);
  TAGI_REQUIRE(n_out < (1ll << 31) && n_obs < (1ll << 31), "%s: sizes above 2^31", what);
  if (rows == 0) return TAGI_OK;
  TAGI_REQUIRE(ma && Sa && dm && dS && (n_obs == 0 || (y_obs && var_obs && idx)), "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_INNOVATION, s, 0.0, 8.0 * rows * n_out + 12.0 * rows * n_obs + 8.0 * rows * n_out);
  if (hrc_rows_fit(rows, n_out))
    launch_hrc_rows<false>(ma, Sa, y_obs, var_obs, idx, nullptr, 0, 0.0f, dm, dS, rows, n_out, n_obs, s);
  else if (rows * n_out < (1ll << 32))
    hipLaunchKernelGGL((hrc_innovation_kernel<false, uint32_t>), dim3(hrc_blocks(rows * n_out)), dim3(256), 0, s,
                       ma, Sa, y_obs, var_obs, idx, (const int64_t*)nullptr, (int64_t)0, 0.0f, dm, dS, rows,
                       (int)n_out, (int)n_obs);
  else
    hipLaunchKernelGGL((hrc_innovation_kernel<false, int64_t>), dim3(hrc_blocks(rows * n_out)), dim3(256), 0, s,
                       ma, Sa, y_obs, var_obs, idx, (const int64_t*)nullptr, (int64_t)0, 0.0f, dm, dS, rows,
                       (int)n_out, (int)n_obs);
  return check_launch(what);
}

extern "C" int tagi_hrc_innovation(const float* ma, const float* Sa, const int64_t* labels, const float* obs,
                                   const int32_t* idx, float sigma_v2, float* dm, float* dS, int64_t rows,
                                   int64_t n_out, int64_t n_obs, int64_t n_classes, tagi_stream_t stream) {
  const char* what = "tagi_hrc_innovation";
  TAGI_REQUIRE(rows >= 0 && n_out > 0 && n_obs > 0 && n_classes > 0, "%s: bad sizes", what);
  TAGI_REQUIRE(n_out < (1ll << 31) && n_obs < (1ll << 31), "%s: sizes above 2^31", what);
  if (rows == 0) return TAGI_OK;
  TAGI_REQUIRE(ma && Sa && labels && obs && idx && dm && dS, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_INNOVATION, s, 0.0, 16.0 * rows * n_out + 8.0 * rows);
  if (hrc_rows_fit(rows, n_out))
    launch_hrc_rows<true>(ma, Sa, obs, nullptr, idx, labels, n_classes, sigma_v2, dm, dS, rows, n_out, n_obs, s);
  else if (rows * n_out < (1ll << 32))
    hipLaunchKernelGGL((hrc_innovation_kernel<true, uint32_t>), dim3(hrc_blocks(rows * n_out)), dim3(256), 0, s,
                       ma, Sa, obs, (const float*)nullptr, idx, labels, n_classes, sigma_v2, dm, dS, rows, (int)n_out,
                       (int)n_obs);
  else
    hipLaunchKernelGGL((hrc_innovation_kernel<true, int64_t>), dim3(hrc_blocks(rows * n_out)), dim3(256), 0, s,
                       ma, Sa, obs, (const float*)nullptr, idx, labels, n_classes, sigma_v2, dm, dS, rows, (int)n_out,
                       (int)n_obs);
  return check_launch(what);
}

extern "C" int tagi_hrc_class_probs(const float* ma, const float* Sa, const float* obs, const int32_t* idx,
                                    float alpha, float* probs, int64_t* pred, int64_t rows, int64_t n_out,
                                    int64_t n_obs, int64_t n_classes, tagi_stream_t stream) {
  const char* what = "tagi_hrc_class_probs";
  TAGI_REQUIRE(rows >= 0 && n_out > 0 && n_obs > 0 && n_classes > 0, "%s: bad sizes", what);
  TAGI_REQUIRE(n_out < (1ll << 31) && n_classes < (1ll << 31) && n_obs < (1ll << 31), "%s: sizes above 2^31", what);
  TAGI_REQUIRE(alpha > 0.f, "%s: alpha must be positive", what);
  if (rows == 0) return TAGI_OK;
  TAGI_REQUIRE(rows < (1ll << 31), "%s: more than 2^31 rows", what);
  TAGI_REQUIRE(ma && Sa && obs && idx && probs, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_INNOVATION, s, 0.0, 8.0 * rows * n_out + 4.0 * rows * n_classes + (pred ? 8.0 * rows : 0.0));
  const int64_t lds_floats = (int64_t)kHrcRows * (odd_stride((int)n_out) + odd_stride((int)n_classes));
  if (lds_floats <= kHrcRowLds && (int64_t)n_classes * n_obs < (1ll << 31))
    hipLaunchKernelGGL(hrc_class_probs_rows_kernel, dim3((unsigned)cdiv(rows, kHrcRows)), dim3(kHrcRows),
                       (size_t)lds_floats * sizeof(float), s, ma, Sa, obs, idx, 1.0f / (alpha * alpha), probs, pred,
                       rows, (int)n_out, (int)n_obs, (int)n_classes);
  else if (n_out <= 64 && n_classes <= 64)
    hipLaunchKernelGGL(hrc_class_probs_wave_kernel, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, ma, Sa, obs, idx,
                       1.0f / (alpha * alpha), probs, pred, rows, (int)n_out, (int)n_obs, (int)n_classes);
  else
    hipLaunchKernelGGL(hrc_class_probs_kernel, dim3((unsigned)rows), dim3(256), 0, s, ma, Sa, obs, idx,
                       1.0f / (alpha * alpha), probs, pred, (int)n_out, (int)n_obs, (int)n_classes);
  return check_launch(what);
}

extern "C" int tagi_innovation_heteros(const float* y, const float* mu, const float* var, float* dm, float* dS,
                                       int64_t n, tagi_stream_t stream) {
  const char* what = "tagi_innovation_heteros";
  TAGI_REQUIRE(n >= 0, "%s: n < 0", what);
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(y && mu && var && dm && dS, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_INNOVATION, s, 0.0, 36.0 * n);
  const bool vec = al(mu, 8) && al(var, 8) && al(dm, 8) && al(dS, 8);
  if (vec)
    hipLaunchKernelGGL(heteros_innovation_kernel<true>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, y, mu, var, dm, dS,
                       n);
  else
    hipLaunchKernelGGL(heteros_innovation_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, y, mu, var, dm,
                       dS, n);
  return check_launch(what);
}

extern "C" int tagi_even_softplus_fwd(const float* mz, const float* Sz, float* ma, float* Sa, float* J, int64_t n,
                                      tagi_stream_t stream) {
  const char* what = "tagi_even_softplus_fwd";
  TAGI_REQUIRE(n >= 0, "%s: n < 0", what);
  if (n == 0) return TAGI_OK;
  TAGI_REQUIRE(mz && Sz && ma && Sa && J, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_SOFTPLUS, s, 0.0, 20.0 * n);
  const bool vec = (n % 2 == 0) && al(mz, 8) && al(Sz, 8) && al(ma, 8) && al(Sa, 8) && al(J, 8);
  if (vec)
    hipLaunchKernelGGL(even_softplus_kernel<true>, dim3(ew_blocks(n / 2, 256)), dim3(256), 0, s, mz, Sz, ma, Sa, J,
                       n);
  else
    hipLaunchKernelGGL(even_softplus_kernel<false>, dim3(ew_blocks(n, 256)), dim3(256), 0, s, mz, Sz, ma, Sa, J, n);
  return check_launch(what);
}
