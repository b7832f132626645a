// fp32-MFMA moment GEMMs for gfx950 (CDNA4): Linear, Conv2D (implicit GEMM) and the
// batched attention products all run through one templated kernel.
//
// A TAGI product carries two accumulators per output tile -- the mean and the variance --
// fed from shared LDS tiles of both operands, with the squared operands formed in
// registers right before the MFMA:
//   PROD_FWD      A=(mu,S) B=(mu,S):  mean += Amu Bmu ; var += Amu^2 BS + AS (Bmu^2 + BS)
//   PROD_SHARED_B A=(mu,S) B=b     :  mean += Amu b   ; var += AS b^2
//   PROD_SHARED_A A=a      B=(mu,S):  mean += a Bmu   ; var += a^2 BS
//
// Matrix core: v_mfma_f32_32x32x2f32 (64 lanes; lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; accumulator register v of lane l is D[8(v/4)+4(l/32)+v%4][l%32]).
// LDS tiles are stored reduction-major ([k][row] and [k][col]) so both operand reads are
// 32 consecutive floats per half-wave. Global tiles are prefetched into registers one
// k-tile ahead of the MFMA work on the current LDS tile.
//
// Operand loaders gather straight from the caller's tensors: strided views (Linear,
// attention heads, transposes) or the convolution index maps (patches, transposed
// patches, weight gathers) -- no im2col / col2im buffers exist anywhere.
#pragma once
#include <float.h>

#include "tagi_common.h"

namespace tagi {

typedef float floatx16 __attribute__((ext_vector_type(16)));

enum { PROD_FWD = 0, PROD_SHARED_B = 1, PROD_SHARED_A = 2 };

// Loader kinds. "MN" kinds map consecutive threads to consecutive rows/cols of the tile
// (global memory contiguous along the output dim); "K" kinds map consecutive threads to
// consecutive reduction indices (global memory contiguous along the reduction).
enum {
  LD_STRIDED_MN = 0,  // p[zoff + mn*s_mn + k*s_k]
  LD_STRIDED_K = 1,   // same element, k-fast thread map
  LD_CONV_PATCH_MN = 2,  // mn = output pixel (n,oh,ow), k = (c,kh,kw): x[n,c,oh*s-pt+kh,ow*s-pl+kw]
  LD_CONV_PATCH_K = 3,   // mn = (c,kh,kw) [+ ones row], k = output pixel: same element
  LD_CONV_DY_MN = 4,     // mn = input pixel (n,h,w), k = (kh,kw,co): dy[n,co,oh,ow] with oh*s = h+pt-kh
  LD_CONV_WT_K = 5,      // mn = c, k = (kh,kw,co): w[(c*kk*kk + kh*kk + kw)*Cout + co]
  LD_CONV_DYROW_K = 6    // mn = co, k = output pixel (n,p): dy[(n*Cout+co)*HoWo + p]
};

template <int KIND>
struct KindTraits {
  static inline constexpr bool mn_fast = (KIND == LD_STRIDED_MN || KIND == LD_CONV_PATCH_MN || KIND == LD_CONV_DY_MN);
};

struct Operand {
  const float* p0;
  const float* p1;
  int64_t zdiv, sz1, sz2;  // batch offset (z/zdiv)*sz1 + (z%zdiv)*sz2
  int64_t s_mn, s_k;       // strided kinds
  int MN, K;               // extents along the tile dim and the reduction
  int ones_row;            // tile index that reads as 1.0 for valid k (bias row), -1 = none
  // convolution geometry (conv kinds)
  int C, H, W, Cout, kk, stride, pt, pl, Ho, Wo;
};

struct Epi {
  int kind;  // 0: strided store (+bias, scale); 1: weight deltas (+bias row)
  float* om;
  float* ov;
  const float* bm;
  const float* bv;
  int64_t b_sr, b_sc;
  float sm, sv;
  int64_t zdiv, sz1, sz2, srow, cdiv, sc1, sc2;
  const float* Sw;
  const float* Sb;
  float* dmb;
  float* dSb;
  int wrows;
  int64_t ldw;
};

struct GemmArgs {
  Operand a, b;
  Epi epi;
  int R, C, Kred;
  int tiles_m, tiles_n;
  int splits, k_chunk;
  float* partial;  // split-K partial sums, or null to apply the epilogue in place
};

template <int BM_, int BN_, int WM_, int WN_>
struct Cfg {
  static inline constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = 16;
  static inline constexpr int NTH = (BM / WM) * (BN / WN) * 64;
};

// ------------------------------------------------------------------------------------
// Element gather for each loader kind. Returns the two tensor values at (mn, k).
// ------------------------------------------------------------------------------------
template <int KIND, int NT>
__device__ __forceinline__ void gather(const Operand& o, int64_t zoff, int mn, int k, float& v0, float& v1) {
  v0 = 0.f;
  v1 = 0.f;
  if (k >= o.K) return;
  if constexpr (KIND == LD_STRIDED_MN || KIND == LD_STRIDED_K) {
    if (mn < o.MN) {
      int64_t off = zoff + (int64_t)mn * o.s_mn + (int64_t)k * o.s_k;
      v0 = o.p0[off];
      if constexpr (NT == 2) v1 = o.p1[off];
    } else if (mn == o.ones_row) {
      v0 = 1.f;
      v1 = 1.f;
    }
  } else if constexpr (KIND == LD_CONV_PATCH_MN || KIND == LD_CONV_PATCH_K) {
    // (pixel, feature) of the implicit patch matrix
    int m, f;
    if constexpr (KIND == LD_CONV_PATCH_MN) {
      m = mn;
      f = k;
      if (m >= o.MN) return;
    } else {
      m = k;
      f = mn;
      if (f >= o.MN) {
        if (f == o.ones_row) { v0 = 1.f; v1 = 1.f; }
        return;
      }
    }
    const int howo = o.Ho * o.Wo;
    const int n = m / howo;
    const int p = m - n * howo;
    const int oh = p / o.Wo;
    const int ow = p - oh * o.Wo;
    const int kk2 = o.kk * o.kk;
    const int c = f / kk2;
    const int r = f - c * kk2;
    const int kh = r / o.kk;
    const int kw = r - kh * o.kk;
    const int ih = oh * o.stride - o.pt + kh;
    const int iw = ow * o.stride - o.pl + kw;
    if (ih < 0 || ih >= o.H || iw < 0 || iw >= o.W) return;
    int64_t off = ((int64_t)(n * o.C + c) * o.H + ih) * o.W + iw;
    v0 = o.p0[off];
    if constexpr (NT == 2) v1 = o.p1[off];
  } else if constexpr (KIND == LD_CONV_DY_MN) {
    if (mn >= o.MN) return;
    const int hw = o.H * o.W;
    const int n = mn / hw;
    const int q = mn - n * hw;
    const int h = q / o.W;
    const int w = q - h * o.W;
    const int kidx = k / o.Cout;
    const int co = k - kidx * o.Cout;
    const int kh = kidx / o.kk;
    const int kw = kidx - kh * o.kk;
    const int ohn = h + o.pt - kh;
    const int own = w + o.pl - kw;
    if (ohn < 0 || own < 0) return;
    const int oh = ohn / o.stride;
    const int ow = own / o.stride;
    if (oh * o.stride != ohn || ow * o.stride != own || oh >= o.Ho || ow >= o.Wo) return;
    int64_t off = ((int64_t)(n * o.Cout + co) * o.Ho + oh) * o.Wo + ow;
    v0 = o.p0[off];
    if constexpr (NT == 2) v1 = o.p1[off];
  } else if constexpr (KIND == LD_CONV_WT_K) {
    if (mn >= o.MN) return;
    const int kidx = k / o.Cout;
    const int co = k - kidx * o.Cout;
    int64_t off = ((int64_t)mn * (o.kk * o.kk) + kidx) * o.Cout + co;
    v0 = o.p0[off];
    if constexpr (NT == 2) v1 = o.p1[off];
  } else if constexpr (KIND == LD_CONV_DYROW_K) {
    if (mn >= o.MN) return;
    const int howo = o.Ho * o.Wo;
    const int n = k / howo;
    const int p = k - n * howo;
    int64_t off = (int64_t)(n * o.Cout + mn) * howo + p;
    v0 = o.p0[off];
    if constexpr (NT == 2) v1 = o.p1[off];
  }
}

// Fetch one BMN x BK tile of NT tensors into registers (E values per tensor per thread).
template <int KIND, int NT, int BMN, int BK, int NTH>
__device__ __forceinline__ void fetch_tile(const Operand& o, int64_t zoff, int mn0, int k0, int tid,
                                           float (&r)[NT][BMN * BK / NTH]) {
  constexpr int E = BMN * BK / NTH;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int e = tid + i * NTH;
    int mn, k;
    if constexpr (KindTraits<KIND>::mn_fast) {
      mn = e % BMN;
      k = e / BMN;
    } else {
      mn = e / BK;
      k = e % BK;
    }
    float v0, v1;
    gather<KIND, NT>(o, zoff, mn0 + mn, k0 + k, v0, v1);
    r[0][i] = v0;
    if constexpr (NT == 2) r[1][i] = v1;
  }
}

template <int KIND, int NT, int BMN, int BK, int NTH>
__device__ __forceinline__ void store_tile(float* s, int tid, const float (&r)[NT][BMN * BK / NTH]) {
  constexpr int E = BMN * BK / NTH;
  constexpr int LD = BMN + 4;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int e = tid + i * NTH;
    int mn, k;
    if constexpr (KindTraits<KIND>::mn_fast) {
      mn = e % BMN;
      k = e / BMN;
    } else {
      mn = e / BK;
      k = e % BK;
    }
    s[k * LD + mn] = r[0][i];
    if constexpr (NT == 2) s[BK * LD + k * LD + mn] = r[1][i];
  }
}

__device__ __forceinline__ void epi_apply(const Epi& e, int z, int row, int col, float m, float v) {
  if (e.kind == 0) {
    const int64_t off = (z / e.zdiv) * e.sz1 + (z % e.zdiv) * e.sz2 + (int64_t)row * e.srow +
                        (col / e.cdiv) * e.sc1 + (col % e.cdiv) * e.sc2;
    float rm = m * e.sm;
    float rv = v * e.sv;
    const int64_t bi = (int64_t)row * e.b_sr + (int64_t)col * e.b_sc;
    if (e.bm) rm += e.bm[bi];
    if (e.bv) rv += e.bv[bi];
    if (e.om) e.om[off] = rm;
    e.ov[off] = rv;
  } else {
    if (row < e.wrows) {
      const int64_t idx = (int64_t)row * e.ldw + col;
      const float s = e.Sw ? e.Sw[idx] : 1.f;
      e.om[idx] = s * m;
      e.ov[idx] = (s * s) * v;
    } else {
      const float s = e.Sb ? e.Sb[col] : 1.f;
      e.dmb[col] = s * m;
      e.dSb[col] = (s * s) * v;
    }
  }
}

template <int PROD, class CFG, int KA, int KB>
__global__ void __launch_bounds__(CFG::NTH) gemm_kernel(GemmArgs g) {
  constexpr int BM = CFG::BM, BN = CFG::BN, BK = CFG::BK, WM = CFG::WM, WN = CFG::WN, NTH = CFG::NTH;
  constexpr int NA = (PROD == PROD_SHARED_A) ? 1 : 2;
  constexpr int NB = (PROD == PROD_SHARED_B) ? 1 : 2;
  constexpr int LDA = BM + 4, LDB = BN + 4;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int EA = BM * BK / NTH, EB = BN * BK / NTH;
  static_assert(NTH % BM == 0 && NTH % BN == 0 && NTH % BK == 0, "thread map");
  static_assert(EA * NTH == BM * BK && EB * NTH == BN * BK, "tile split");

  __shared__ float sA[NA * BK * LDA];
  __shared__ float sB[NB * BK * LDB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / (BN / WN);
  const int wn = wave % (BN / WN);
  const int hl = lane >> 5;
  const int rl = lane & 31;

  // XCD-aware tile order: workgroups are dealt round-robin over the 8 XCDs, so map
  // consecutive block ids of one XCD onto consecutive tiles (shared operand panels stay
  // in that XCD's L2).
  const int nt = g.tiles_m * g.tiles_n;
  const int bid = blockIdx.x;
  const int per = nt >> 3;
  const int t = (bid < (per << 3)) ? ((bid & 7) * per + (bid >> 3)) : bid;
  const int tmi = t / g.tiles_n;
  const int tni = t - tmi * g.tiles_n;
  const int m0 = tmi * BM;
  const int n0 = tni * BN;
  const int zz = blockIdx.y;
  const int z = zz / g.splits;
  const int split = zz - z * g.splits;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.Kred, kbeg + g.k_chunk);

  const int64_t zoa = (z / g.a.zdiv) * g.a.sz1 + (z % g.a.zdiv) * g.a.sz2;
  const int64_t zob = (z / g.b.zdiv) * g.b.sz1 + (z % g.b.zdiv) * g.b.sz2;

  floatx16 accM[TM][TN], accV[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        accM[i][j][v] = 0.f;
        accV[i][j][v] = 0.f;
      }

  float ra[NA][EA];
  float rb[NB][EB];
  if (kbeg < kend) {
    fetch_tile<KA, NA, BM, BK, NTH>(g.a, zoa, m0, kbeg, tid, ra);
    fetch_tile<KB, NB, BN, BK, NTH>(g.b, zob, n0, kbeg, tid, rb);
  }

  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    store_tile<KA, NA, BM, BK, NTH>(sA, tid, ra);
    store_tile<KB, NB, BN, BK, NTH>(sB, tid, rb);
    __syncthreads();
    if (k0 + BK < kend) {
      fetch_tile<KA, NA, BM, BK, NTH>(g.a, zoa, m0, k0 + BK, tid, ra);
      fetch_tile<KB, NB, BN, BK, NTH>(g.b, zob, n0, k0 + BK, tid, rb);
    }
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
      const int kr = 2 * s + hl;
      float a0[TM], a1[TM], b0[TN], b1[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int c = kr * LDA + wm * WM + i * 32 + rl;
        a0[i] = sA[c];
        if constexpr (NA == 2) a1[i] = sA[BK * LDA + c];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int c = kr * LDB + wn * WN + j * 32 + rl;
        b0[j] = sB[c];
        if constexpr (NB == 2) b1[j] = sB[BK * LDB + c];
      }
      if constexpr (PROD == PROD_FWD) {
        float asq[TM], bvar[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) asq[i] = a0[i] * a0[i];
#pragma unroll
        for (int j = 0; j < TN; ++j) bvar[j] = b0[j] * b0[j] + b1[j];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            accM[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[i], b0[j], accM[i][j], 0, 0, 0);
            accV[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(asq[i], b1[j], accV[i][j], 0, 0, 0);
            accV[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[i], bvar[j], accV[i][j], 0, 0, 0);
          }
      } else if constexpr (PROD == PROD_SHARED_B) {
        float bsq[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) bsq[j] = b0[j] * b0[j];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            accM[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[i], b0[j], accM[i][j], 0, 0, 0);
            accV[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[i], bsq[j], accV[i][j], 0, 0, 0);
          }
      } else {
        float asq[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) asq[i] = a0[i] * a0[i];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            accM[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[i], b0[j], accM[i][j], 0, 0, 0);
            accV[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(asq[i], b1[j], accV[i][j], 0, 0, 0);
          }
      }
    }
    __syncthreads();
  }

  // Epilogue: direct store, or split-K partials.
  const int64_t plane = (int64_t)g.R * g.C;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
        const int col = n0 + wn * WN + j * 32 + rl;
        if (row < g.R && col < g.C) {
          if (g.partial) {
            const int64_t base = ((int64_t)zz * 2) * plane + (int64_t)row * g.C + col;
            g.partial[base] = accM[i][j][v];
            g.partial[base + plane] = accV[i][j][v];
          } else {
            epi_apply(g.epi, z, row, col, accM[i][j][v], accV[i][j][v]);
          }
        }
      }
}

// Deterministic split-K reduction (fixed split order) followed by the epilogue.
template <int UNUSED = 0>
__global__ void splitk_reduce_kernel(const float* __restrict__ partial, Epi epi, int batch, int splits, int R,
                                     int C) {
  const int64_t plane = (int64_t)R * C;
  const int64_t total = plane * batch;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int z = (int)(idx / plane);
    const int64_t rc = idx - (int64_t)z * plane;
    const int row = (int)(rc / C);
    const int col = (int)(rc - (int64_t)row * C);
    float m = 0.f, v = 0.f;
    const float* p = partial + ((int64_t)z * splits * 2) * plane + rc;
    for (int s = 0; s < splits; ++s) {
      m += p[(2 * s) * plane];
      v += p[(2 * s + 1) * plane];
    }
    epi_apply(epi, z, row, col, m, v);
  }
}

// ------------------------------------------------------------------------------------
// Host side: tile-config choice, split-K choice and launch.
// ------------------------------------------------------------------------------------
using C128x128 = Cfg<128, 128, 64, 64>;
using C64x256 = Cfg<64, 256, 64, 64>;
using C128x64 = Cfg<128, 64, 64, 32>;
using C64x128 = Cfg<64, 128, 32, 64>;
using C64x64 = Cfg<64, 64, 32, 32>;
using C32x32 = Cfg<32, 32, 32, 32>;

struct CfgDesc {
  int BM, BN;
};
static const CfgDesc kCfg[] = {{128, 128}, {64, 256}, {128, 64}, {64, 128}, {64, 64}, {32, 32}};
static const int kNumCfg = 6;

struct Plan {
  int cfg;
  int splits;
  int k_chunk;
  int tiles_m, tiles_n;
};

// Pick the tile shape and split-K factor minimising a simple time model: MFMA time of
// the busiest wave of blocks (two resident blocks per CU) inflated by the per-tile load
// overhead, plus the HBM time of the split-K partial round trip.
static inline Plan choose_plan(int64_t R, int64_t C, int64_t Kred, int64_t batch, int products, bool allow_split,
                        int64_t max_splits) {
  Plan best{5, 1, (int)Kred, 1, 1};
  double best_t = DBL_MAX;
  const double flops_per_block_s = 157.3e12 / 256.0 / 2.0;
  for (int ci = 0; ci < kNumCfg; ++ci) {
    const int BM = kCfg[ci].BM, BN = kCfg[ci].BN;
    const int64_t tm = cdiv(R, BM), tn = cdiv(C, BN);
    for (int64_t sp = 1; sp <= 64; sp *= 2) {
      if (sp > 1 && (!allow_split || sp > max_splits)) break;
      int64_t kc = cdiv(cdiv(Kred, sp), 16) * 16;
      if (kc < 1) kc = 16;
      const int64_t actual = cdiv(Kred, kc);
      if (sp > 1 && actual < sp) break;
      const int64_t blocks = tm * tn * batch * actual;
      const int64_t waves = cdiv(blocks, 512);
      const double eff = 1.0 + 32.0 / BM + 32.0 / BN;
      double t = waves * (2.0 * BM * BN * kc * products * eff) / flops_per_block_s;
      if (actual > 1) t += (double)(actual * 2 + 2) * R * C * batch * 4.0 / 5.0e12 + 4e-6;
      if (t < best_t * 0.999) {
        best_t = t;
        best = Plan{ci, (int)actual, (int)kc, (int)tm, (int)tn};
      }
    }
  }
  return best;
}

static inline int64_t plan_ws_bytes(const Plan& p, int64_t R, int64_t C, int64_t batch) {
  return p.splits > 1 ? (int64_t)p.splits * 2 * R * C * batch * (int64_t)sizeof(float) : 0;
}

template <int PROD, class CFG, int KA, int KB>
static inline void launch_cfg(const GemmArgs& g, int64_t grid_x, int64_t grid_y, hipStream_t s) {
  hipLaunchKernelGGL((gemm_kernel<PROD, CFG, KA, KB>), dim3((unsigned)grid_x, (unsigned)grid_y), dim3(CFG::NTH), 0, s, g);
}

template <int PROD, int KA, int KB>
static inline int run_gemm(GemmArgs g, int64_t batch, const Plan& p, float* ws, int64_t ws_bytes, hipStream_t s,
                    const char* what) {
  g.tiles_m = p.tiles_m;
  g.tiles_n = p.tiles_n;
  g.splits = p.splits;
  g.k_chunk = p.k_chunk;
  g.partial = nullptr;
  if (p.splits > 1) {
    TAGI_REQUIRE(ws != nullptr && ws_bytes >= plan_ws_bytes(p, g.R, g.C, batch),
                 "%s: workspace of %lld bytes needed (got %lld)", what, (long long)plan_ws_bytes(p, g.R, g.C, batch),
                 (long long)ws_bytes);
    g.partial = ws;
  }
  const int64_t gx = (int64_t)p.tiles_m * p.tiles_n;
  const int64_t gy = batch * p.splits;
  TAGI_REQUIRE(gx < (1ll << 31) && gy < 65536, "%s: grid too large (%lld x %lld)", what, (long long)gx, (long long)gy);
  switch (p.cfg) {
    case 0: launch_cfg<PROD, C128x128, KA, KB>(g, gx, gy, s); break;
    case 1: launch_cfg<PROD, C64x256, KA, KB>(g, gx, gy, s); break;
    case 2: launch_cfg<PROD, C128x64, KA, KB>(g, gx, gy, s); break;
    case 3: launch_cfg<PROD, C64x128, KA, KB>(g, gx, gy, s); break;
    case 4: launch_cfg<PROD, C64x64, KA, KB>(g, gx, gy, s); break;
    default: launch_cfg<PROD, C32x32, KA, KB>(g, gx, gy, s); break;
  }
  int rc = check_launch(what);
  if (rc != TAGI_OK) return rc;
  if (p.splits > 1) {
    const int64_t total = (int64_t)g.R * g.C * batch;
    hipLaunchKernelGGL(splitk_reduce_kernel<0>, dim3(ew_blocks(total, 256)), dim3(256), 0, s, (const float*)ws, g.epi,
                       (int)batch, p.splits, g.R, g.C);
    rc = check_launch(what);
  }
  return rc;
}

static inline Operand strided_operand(const float* p0, const float* p1, int64_t zdiv, int64_t sz1, int64_t sz2,
                               int64_t s_mn, int64_t s_k, int64_t MN, int64_t K) {
  Operand o{};
  o.p0 = p0;
  o.p1 = p1;
  o.zdiv = zdiv > 0 ? zdiv : 1;
  o.sz1 = sz1;
  o.sz2 = sz2;
  o.s_mn = s_mn;
  o.s_k = s_k;
  o.MN = (int)MN;
  o.K = (int)K;
  o.ones_row = -1;
  return o;
}

static inline Epi epi_store(float* om, float* ov, const float* bm, const float* bv, int64_t b_sr, int64_t b_sc, float sm,
                     float sv, int64_t zdiv, int64_t sz1, int64_t sz2, int64_t srow, int64_t cdiv_, int64_t sc1,
                     int64_t sc2) {
  Epi e{};
  e.kind = 0;
  e.om = om;
  e.ov = ov;
  e.bm = bm;
  e.bv = bv;
  e.b_sr = b_sr;
  e.b_sc = b_sc;
  e.sm = sm;
  e.sv = sv;
  e.zdiv = zdiv > 0 ? zdiv : 1;
  e.sz1 = sz1;
  e.sz2 = sz2;
  e.srow = srow;
  e.cdiv = cdiv_ > 0 ? cdiv_ : 1;
  e.sc1 = sc1;
  e.sc2 = sc2;
  return e;
}

static inline Epi epi_wgrad(float* dmw, float* dSw, float* dmb, float* dSb, const float* Sw, const float* Sb, int64_t wrows,
                     int64_t ldw) {
  Epi e{};
  e.kind = 1;
  e.om = dmw;
  e.ov = dSw;
  e.dmb = dmb;
  e.dSb = dSb;
  e.Sw = Sw;
  e.Sb = Sb;
  e.wrows = (int)wrows;
  e.ldw = ldw;
  e.zdiv = 1;
  e.cdiv = 1;
  return e;
}

static inline bool fits_i32(int64_t v) { return v >= 0 && v < (1ll << 31); }

// Plans are shared by the entry points and their workspace queries.
static inline Plan linear_fwd_plan(int64_t M, int64_t K, int64_t N) { return choose_plan(M, N, K, 1, 3, true, 16); }
static inline Plan linear_wgrad_plan(int64_t M, int64_t K, int64_t N) { return choose_plan(K + 1, N, M, 1, 2, true, 64); }

static inline Operand conv_operand(const float* p0, const float* p1, const tagi_conv_geom* g, int64_t MN, int64_t K) {
  Operand o{};
  o.p0 = p0;
  o.p1 = p1;
  o.zdiv = 1;
  o.MN = (int)MN;
  o.K = (int)K;
  o.ones_row = -1;
  o.C = (int)g->C;
  o.H = (int)g->H;
  o.W = (int)g->W;
  o.Cout = (int)g->Cout;
  o.kk = (int)g->k;
  o.stride = (int)g->stride;
  o.pt = (int)g->pad_top;
  o.pl = (int)g->pad_left;
  o.Ho = (int)g->Ho;
  o.Wo = (int)g->Wo;
  return o;
}

static inline int check_geom(const tagi_conv_geom* g, const char* what) {
  TAGI_REQUIRE(g != nullptr, "%s: null geometry", what);
  TAGI_REQUIRE(g->N > 0 && g->C > 0 && g->H > 0 && g->W > 0 && g->Cout > 0 && g->k > 0 && g->stride > 0,
               "%s: sizes must be positive", what);
  // every gathered element is bounds-checked against H and W, so any output extent is
  // memory-safe; only the caller's output buffers must match Ho and Wo
  TAGI_REQUIRE(g->pad_top >= 0 && g->pad_left >= 0 && g->Ho > 0 && g->Wo > 0, "%s: bad padding/output size", what);
  TAGI_REQUIRE(fits_i32(g->N * g->C * g->H * g->W) && fits_i32(g->N * g->Cout * g->Ho * g->Wo) &&
                   fits_i32(g->C * g->k * g->k * g->Cout),
               "%s: tensor too large for 32-bit indexing", what);
  return TAGI_OK;
}

static inline Plan conv_fwd_plan(const tagi_conv_geom* g) {
  return choose_plan(g->Cout, g->N * g->Ho * g->Wo, g->C * g->k * g->k, 1, 3, true, 16);
}
static inline Plan conv_wgrad_plan(const tagi_conv_geom* g) {
  return choose_plan(g->C * g->k * g->k + 1, g->Cout, g->N * g->Ho * g->Wo, 1, 2, true, 64);
}

}  // namespace tagi

