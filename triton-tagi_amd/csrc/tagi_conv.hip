// Conv2D entry points on NHWC (channels-last) activations:
//   forward      implicit GEMM  rows = output pixels, cols = C_out, reduction (kh, kw, c)
//   input delta  transposed implicit GEMM split by stride phase (only the kernel taps that
//                reach a phase's pixels are multiplied; no col2im, no zero taps)
//   deltas       split-K GEMM over output pixels, rows (kh, kw, c) + a ones row for the bias
#include "tagi_gemm_core.h"

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

static ConvG to_g(const tagi_conv_geom* g) {
  ConvG c;
  c.N = (int)g->N;
  c.C = (int)g->C;
  c.H = (int)g->H;
  c.W = (int)g->W;
  c.Cout = (int)g->Cout;
  c.kk = (int)g->k;
  c.stride = (int)g->stride;
  c.pt = (int)g->pad_top;
  c.pl = (int)g->pad_left;
  c.Ho = (int)g->Ho;
  c.Wo = (int)g->Wo;
  c.dC = make_fastdiv(c.C);
  c.dCout = make_fastdiv(c.Cout);
  c.dkk = make_fastdiv(c.kk);
  c.dHW = make_fastdiv(c.Ho * c.Wo);
  c.dWo = make_fastdiv(c.Wo);
  return c;
}

// elems: the tensor's element count (its reach from p0)
static Operand conv_operand(const float* p0, const float* p1, const tagi_conv_geom* g, int64_t MN, int64_t K,
                            int64_t elems) {
  Operand o{};
  o.nbytes = 4 * elems;
  o.p0 = p0;
  o.p1 = p1;
  o.zdiv = 1;
  o.MN = (int)MN;
  o.K = (int)K;
  o.ones_row = -1;
  o.g = to_g(g);
  return o;
}

static int check_geom(const tagi_conv_geom* g, const char* what) {
  TAGI_REQUIRE(g != nullptr, "%s: null geometry", what);
  TAGI_REQUIRE(g->N > 0 && g->C > 0 && g->H > 0 && g->W > 0 && g->Cout > 0 && g->k > 0 && g->stride > 0,
               "%s: sizes must be positive", what);
  // every gathered element is bounds-checked against H and W, so any output extent is
  // memory-safe; only the caller's output buffers must match Ho and Wo
  TAGI_REQUIRE(g->pad_top >= 0 && g->pad_left >= 0 && g->Ho > 0 && g->Wo > 0, "%s: bad padding/output size", what);
  TAGI_REQUIRE(g->stride <= 8 && g->k <= 16, "%s: stride/kernel out of range", what);
  TAGI_REQUIRE(fits_i32(g->N * g->C * g->H * g->W) && fits_i32(g->N * g->Cout * g->Ho * g->Wo) &&
                   fits_i32(g->C * g->k * g->k * g->Cout + g->Cout),
               "%s: tensor too large for 32-bit indexing", what);
  return TAGI_OK;
}

// zero_var: a deterministic input (Sa NULL), run as the shared-A product (mean ma mw,
// variance ma^2 Sw; the Sa (mw^2 + Sw) terms it leaves out are exact zeros)
static Plan conv_fwd_plan(const tagi_conv_geom* g, bool zero_var = false) {
  return choose_plan(g->N * g->Ho * g->Wo, g->Cout, g->C * g->k * g->k, 1, zero_var ? PROD_SHARED_A : PROD_FWD, true,
                     16);
}

// Largest row count (phase 0) and largest reduction over the stride phases of the
// input-delta GEMM; the launch is sized for both.
static void bwd_phase0(const tagi_conv_geom* g, int64_t* R, int64_t* K) {
  const ConvG cg = to_g(g);
  const Phase p0 = make_phase(cg, 0);
  *R = g->N * (int64_t)p0.Hq * p0.Wq;
  int64_t kmax = 0;
  for (int ph = 0; ph < cg.stride * cg.stride; ++ph) {
    const Phase p = make_phase(cg, ph);
    const int64_t k = (int64_t)p.nkh * p.nkw * g->Cout;
    if (k > kmax) kmax = k;
  }
  *K = kmax;
}

static Plan conv_bwd_plan(const tagi_conv_geom* g) {
  int64_t R, K;
  bwd_phase0(g, &R, &K);
  if (K <= 0) K = 1;
  const ConvG cg = to_g(g);
  const int nph = cg.stride * cg.stride;
  int64_t pk[64];
  if (nph > 64) return choose_plan(R, g->C, K, nph, PROD_SHARED_B, true, 16);
  for (int ph = 0; ph < nph; ++ph) {
    const Phase p = make_phase(cg, ph);
    pk[ph] = (int64_t)p.nkh * p.nkw * g->Cout;
  }
  return choose_plan(R, g->C, K, nph, PROD_SHARED_B, true, 16, pk);
}

// rows: the weight rows (c, kh, kw), plus the ones row of the bias sums when the GEMM forms them
static Plan conv_wgrad_plan(const tagi_conv_geom* g, bool bias) {
  return choose_plan(g->C * g->k * g->k + (bias ? 1 : 0), g->Cout, g->N * g->Ho * g->Wo, 1, PROD_SHARED_A, true, 512);
}

static int64_t wt_floats(const tagi_conv_geom* g) { return ((g->C * g->k * g->k * g->Cout) + 3) / 4 * 4; }

// Plain transpose of a rows x cols matrix (LDS-tiled 32 x 32, coalesced both ways).
__global__ void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, int rows, int cols) {
  __shared__ float tile[32][33];
  const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 8 rows per pass
  for (int j = ty; j < 32; j += 8) {
    const int r = by + j, c = bx + tx;
    if (r < rows && c < cols) tile[j][tx] = in[(int64_t)r * cols + c];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int r = bx + j, c = by + tx;  // out is cols x rows
    if (r < cols && c < rows) out[(int64_t)r * rows + c] = tile[tx][j];
  }
}

__global__ void zero2_kernel(float* __restrict__ a, float* __restrict__ b, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    a[i] = 0.f;
    b[i] = 0.f;
  }
}

// ====================================================================== forward
extern "C" int64_t tagi_conv2d_fwd_ws_bytes(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->Ho <= 0 || g->Wo <= 0 || g->C <= 0 || g->k <= 0) return 0;
  const int64_t a = plan_ws_bytes(conv_fwd_plan(g), g->N * g->Ho * g->Wo, g->Cout, 1);
  const int64_t b = plan_ws_bytes(conv_fwd_plan(g, true), g->N * g->Ho * g->Wo, g->Cout, 1);
  return a > b ? a : b;
}

// Forward GEMM; with st_J/st_ws set (and no split-K) the epilogue also forms the ReLU
// Jacobian and the per-tile column sums of the rectified moments.
static int conv_fwd_impl(const char* what, const float* ma, const float* Sa, const float* mw, const float* Sw,
                         const float* mb, const float* Sb, float* mz, float* Sz, const tagi_conv_geom* g,
                         const Plan& p, float* st_J, float* st_ws, float* ws, int64_t ws_bytes, hipStream_t s) {
  const int64_t R = g->N * g->Ho * g->Wo, C = g->Cout, K = g->C * g->k * g->k;
  const bool zero_var = Sa == nullptr;
  ProfScope ps(FAM_CONV_FWD, s, 2.0 * (zero_var ? 2 : 3) * R * C * K,
               4.0 * ((zero_var ? 1 : 2) * g->N * g->C * g->H * g->W + 2 * K * C + 2 * R * C));
  GemmArgs a{};
  a.a = conv_operand(ma, Sa, g, R, K, g->N * g->C * g->H * g->W);
  a.b = conv_operand(mw, Sw, g, C, K, K * g->Cout);
  a.epi = epi_store(mz, Sz, mb, Sb, 0, 1, 1.f, 1.f, 1, 0, 0, C, 1);
  if (st_ws) {
    TAGI_REQUIRE(p.splits == 1 && st_J, "%s: internal: statistics epilogue needs an unsplit launch", what);
    a.epi.st_J = st_J;
    a.epi.st_ws = st_ws;
    a.epi.st_nblk = p.tiles_m;
  }
  a.R = (int)R;
  a.C = (int)C;
  a.Kred = (int)K;
  const bool va = g->C % 4 == 0 && al16(ma) && (zero_var || al16(Sa));
  const bool vb = g->Cout % 4 == 0 && al16(mw) && al16(Sw);
  if (zero_var) {
    if (va && vb && g->C % 16 == 0 && g->k <= 5)
      return run_gemm<PROD_SHARED_A, LD_CFWD_A4T, LD_CFWD_B4T>(a, 1, p, ws, ws_bytes, s, what);
    if (va && vb) return run_gemm<PROD_SHARED_A, LD_CFWD_A4, LD_CFWD_B4>(a, 1, p, ws, ws_bytes, s, what);
    if (vb) return run_gemm<PROD_SHARED_A, LD_CFWD_A_S, LD_CFWD_B4>(a, 1, p, ws, ws_bytes, s, what);
    return run_gemm<PROD_SHARED_A, LD_CFWD_A_S, LD_CFWD_B_S>(a, 1, p, ws, ws_bytes, s, what);
  }
  // 16 channels per k tile and at most 25 taps: the tile-aligned loaders
  if (va && vb && g->C % 16 == 0 && g->k <= 5)
    return run_gemm<PROD_FWD, LD_CFWD_A4T, LD_CFWD_B4T>(a, 1, p, ws, ws_bytes, s, what);
  if (va && vb) return run_gemm<PROD_FWD, LD_CFWD_A4, LD_CFWD_B4>(a, 1, p, ws, ws_bytes, s, what);
  if (vb) return run_gemm<PROD_FWD, LD_CFWD_A_S, LD_CFWD_B4>(a, 1, p, ws, ws_bytes, s, what);
  return run_gemm<PROD_FWD, LD_CFWD_A_S, LD_CFWD_B_S>(a, 1, p, ws, ws_bytes, s, what);
}

extern "C" int tagi_conv2d_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw, const float* mb,
                               const float* Sb, float* mz, float* Sz, const tagi_conv_geom* g, float* ws,
                               int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_conv2d_fwd";
  int rc = check_geom(g, what);
  if (rc) return rc;
  TAGI_REQUIRE(ma && mw && Sw && mz && Sz, "%s: null pointer", what);
  const int64_t R = g->N * g->Ho * g->Wo, C = g->Cout, K = g->C * g->k * g->k;
  Plan p = conv_fwd_plan(g, Sa == nullptr);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, R, C, 1)))
    p = choose_plan(R, C, K, 1, Sa ? PROD_FWD : PROD_SHARED_A, false, 1);
  return conv_fwd_impl(what, ma, Sa, mw, Sw, mb, Sb, mz, Sz, g, p, nullptr, nullptr, ws, ws_bytes,
                       as_stream(stream));
}

// Statistics partials of the fused form: one row per M tile of an unsplit launch; a
// split launch runs the separate statistics pass over the stored output instead.
static int64_t fwd_stats_floats(const tagi_conv_geom* g, const Plan& p) {
  const int64_t C = g->Cout;
  if (p.splits > 1) return (tagi_bn_stats_ws_bytes(g->N, C, g->Ho * g->Wo) + 3) / 4;
  return (int64_t)p.tiles_m * C * 3;
}

static int64_t fwd_stats_ws_bytes(const tagi_conv_geom* g, const Plan& p) {
  const int64_t conv = plan_ws_bytes(p, g->N * g->Ho * g->Wo, g->Cout, 1);
  return (conv + 255) / 256 * 256 + fwd_stats_floats(g, p) * (int64_t)sizeof(float);
}

extern "C" int64_t tagi_conv2d_fwd_relu_bn_stats_ws_bytes(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->Ho <= 0 || g->Wo <= 0 || g->C <= 0 || g->k <= 0) return 0;
  const int64_t a = fwd_stats_ws_bytes(g, conv_fwd_plan(g)), b = fwd_stats_ws_bytes(g, conv_fwd_plan(g, true));
  return a > b ? a : b;
}

extern "C" int tagi_conv2d_fwd_relu_bn_stats(const float* ma, const float* Sa, const float* mw, const float* Sw,
                                             const float* mb, const float* Sb, float* mz, float* Sz,
                                             const tagi_conv_geom* g, float* J, float* batch_mean, float* batch_var,
                                             float* running_mean, float* running_var, float* mg, float momentum,
                                             float eps, int first_call, int preserve_var, float* ws,
                                             int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_conv2d_fwd_relu_bn_stats";
  int rc = check_geom(g, what);
  if (rc) return rc;
  TAGI_REQUIRE(ma && mw && Sw && mz && Sz && J && batch_mean && batch_var, "%s: null pointer", what);
  const int64_t R = g->N * g->Ho * g->Wo, C = g->Cout;
  TAGI_REQUIRE(R > 1, "%s: BatchNorm2D needs more than one value per channel", what);
  TAGI_REQUIRE(ws && ws_bytes >= tagi_conv2d_fwd_relu_bn_stats_ws_bytes(g) && al16(ws),
               "%s: workspace of %lld bytes (16-byte aligned) needed", what,
               (long long)tagi_conv2d_fwd_relu_bn_stats_ws_bytes(g));
  hipStream_t s = as_stream(stream);
  const Plan p = conv_fwd_plan(g, Sa == nullptr);
  const int64_t conv = (plan_ws_bytes(p, R, C, 1) + 255) / 256 * 256;
  float* sws = ws + conv / (int64_t)sizeof(float);
  const int64_t sbytes = ws_bytes - conv;
  if (p.splits > 1) {
    rc = conv_fwd_impl(what, ma, Sa, mw, Sw, mb, Sb, mz, Sz, g, p, nullptr, nullptr, ws, conv, s);
    if (rc) return rc;
    return tagi_relu_bn_stats(mz, Sz, J, batch_mean, batch_var, running_mean, running_var, mg, g->N, C,
                              g->Ho * g->Wo, momentum, eps, first_call, preserve_var, sws, sbytes, stream);
  }
  rc = conv_fwd_impl(what, ma, Sa, mw, Sw, mb, Sb, mz, Sz, g, p, J, sws, ws, conv, s);
  if (rc) return rc;
  return bn_stats_finalize(what, sws, p.tiles_m, R, C, batch_mean, batch_var, running_mean, running_var, mg, momentum,
                           eps, first_call, preserve_var, s);
}

// ================================================================== input delta
extern "C" int64_t tagi_conv2d_bwd_delta_ws_bytes(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->C <= 0 || g->k <= 0 || g->stride <= 0) return 0;
  int64_t R, K;
  bwd_phase0(g, &R, &K);
  return wt_floats(g) * (int64_t)sizeof(float) + plan_ws_bytes(conv_bwd_plan(g), R, g->C, g->stride * g->stride);
}

// The BatchNorm2D -> ReLU backward folded into the input-delta GEMM's epilogue: the pair's
// saved state and the per-tile partial sums' destination.
struct BnBwdFuse {
  const float* mhat;
  const float* J;
  const float* var;
  const float* mg;
  float eps;
  float* part;
  // with an addend: where the fold's outputs go (the product + addend goes to dma/dSa)
  float* out_m;
  float* out_S;
};

// Tiles along the rows of the fused launch (the partial sums per channel), or 0 when the
// fold does not apply: stride 1 (one phase) and an unsplit plan.
static int64_t bn_fuse_tiles(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->C <= 0 || g->k <= 0 || g->stride != 1 || g->Cout % 4 != 0) return 0;
  const Plan p = conv_bwd_plan(g);
  return p.splits == 1 && bnf_cfg(p.cfg) ? p.tiles_m : 0;
}

static int conv_bwd_delta_impl(const char* what, const float* dmz, const float* dSz, const float* mw,
                               const float* add_m, const float* add_S, float* dma, float* dSa, const tagi_conv_geom* g,
                               float* ws, int64_t ws_bytes, tagi_stream_t stream, const BnBwdFuse* bnf = nullptr) {
  TAGI_REQUIRE((add_m == nullptr) == (add_S == nullptr), "%s: add_m and add_S must both be given or both be NULL",
               what);
  int rc = check_geom(g, what);
  if (rc) return rc;
  TAGI_REQUIRE(dmz && dSz && mw && dma && dSa, "%s: null pointer", what);
  TAGI_REQUIRE(ws && ws_bytes >= wt_floats(g) * (int64_t)sizeof(float), "%s: workspace too small", what);
  hipStream_t s = as_stream(stream);
  const int64_t Kw = g->C * g->k * g->k;
  // algorithmic work of the patch-space product (what an explicit col2im path computes)
  const double alg = 2.0 * 2 * (g->N * g->Ho * g->Wo) * Kw * g->Cout;
  ProfScope ps(FAM_CONV_BWD_DELTA, s, alg,
               4.0 * (2 * g->N * g->Cout * g->Ho * g->Wo + Kw * g->Cout + 2 * g->N * g->C * g->H * g->W));
  // With Cout % 4 == 0 the weights are read in place, float4 along co (the reduction
  // index); otherwise they are first transposed, (c, kh, kw) x co -> (kh, kw, co) x c,
  // for float4 (or scalar) reads along c.
  const bool in_place = g->Cout % 4 == 0 && al16(mw);
  float* wt = ws;
  if (!in_place) {
    const int rows = (int)g->C, cols = (int)(g->k * g->k * g->Cout);
    hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32)), dim3(256), 0, s, mw,
                       wt, rows, cols);
    if ((rc = check_launch(what))) return rc;
  }
  // any input pixel a stride phase leaves without taps gets zero deltas (k < stride)
  const int nph = (int)(g->stride * g->stride);
  bool holes = false;
  for (int ph = 0; ph < nph; ++ph) {
    const Phase p = make_phase(to_g(g), ph);
    if (p.Hq > 0 && p.Wq > 0 && (p.nkh == 0 || p.nkw == 0)) holes = true;
  }
  if (holes) {
    const int64_t n = g->N * g->C * g->H * g->W;
    hipLaunchKernelGGL(zero2_kernel, dim3(ew_blocks(n, 256)), dim3(256), 0, s, dma, dSa, n);
    if ((rc = check_launch(what))) return rc;
  }
  int64_t R0, K0;
  bwd_phase0(g, &R0, &K0);
  GemmArgs a{};
  a.a = conv_operand(dmz, dSz, g, R0, K0, g->N * g->Cout * g->Ho * g->Wo);
  a.b = conv_operand(in_place ? mw : wt, nullptr, g, g->C, K0, g->C * g->k * g->k * g->Cout);
  a.epi = Epi{};
  a.epi.kind = 2;
  a.epi.om = dma;
  a.epi.ov = dSa;
  a.epi.zdiv = 1;
  a.epi.g = to_g(g);
  a.epi.am = add_m;
  a.epi.av = add_S;
  if (bnf) {
    a.epi.bn_mhat = bnf->mhat;
    a.epi.bn_J = bnf->J;
    a.epi.bn_var = bnf->var;
    a.epi.bn_g = bnf->mg;
    a.epi.bn_eps = bnf->eps;
    a.epi.st_ws = bnf->part;
    a.epi.bn_om = bnf->out_m;
    a.epi.bn_ov = bnf->out_S;
  }
  a.R = (int)R0;
  a.C = (int)g->C;
  a.Kred = (int)K0;
  a.phased = 1;
  {
    // longest phase reductions first (stable for equal lengths)
    int64_t kz[64];
    for (int ph = 0; ph < nph; ++ph) {
      const Phase q = make_phase(to_g(g), ph);
      kz[ph] = (int64_t)q.nkh * q.nkw;
      a.phase_order[ph] = (unsigned char)ph;
    }
    for (int i = 1; i < nph; ++i)
      for (int j = i; j > 0 && kz[a.phase_order[j]] > kz[a.phase_order[j - 1]]; --j) {
        const unsigned char t = a.phase_order[j];
        a.phase_order[j] = a.phase_order[j - 1];
        a.phase_order[j - 1] = t;
      }
  }
  Plan p = conv_bwd_plan(g);
  float* part = ws + wt_floats(g);
  const int64_t part_bytes = ws_bytes - wt_floats(g) * (int64_t)sizeof(float);
  if (p.splits > 1 && part_bytes < plan_ws_bytes(p, R0, g->C, nph)) p = choose_plan(R0, g->C, K0, nph, PROD_SHARED_B, false, 1);
  if (bnf) {
    TAGI_REQUIRE(nph == 1 && p.splits == 1 && bnf_cfg(p.cfg),
                 "%s: the folded BatchNorm2D backward needs stride 1 and an unsplit one-tile-per-wave plan", what);
    // the folded epilogues address the (N, H, W, C) tensors with 32-bit offsets
    TAGI_REQUIRE(R0 * g->C < (int64_t)1 << 31, "%s: %lld x %lld deltas exceed the fold's 2^31 elements", what,
                 (long long)R0, (long long)g->C);
    a.epi.st_nblk = p.tiles_m;
  }
  const int64_t gx = (int64_t)p.tiles_m * p.tiles_n;  // phase 0 is the largest
  const bool va = g->Cout % 4 == 0 && al16(dmz) && al16(dSz);
  const bool vb = g->C % 4 == 0;
  if (bnf) {
    TAGI_REQUIRE(va && in_place, "%s: the folded BatchNorm2D backward needs Cout %% 4 == 0 and 16-byte aligned "
                 "deltas and weights", what);
    if (add_m) {
      TAGI_REQUIRE(bnf->out_m && bnf->out_S, "%s: null pointer", what);
      if (g->Cout % 16 == 0 && g->k <= 5)
        return run_gemm<PROD_SHARED_B, LD_CBWD_A4T, LD_CBWD_BK4T, 3>(a, nph, p, part, part_bytes, s, what, gx);
      return run_gemm<PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_BK4, 3>(a, nph, p, part, part_bytes, s, what, gx);
    }
    if (g->Cout % 16 == 0 && g->k <= 5)
      return run_gemm<PROD_SHARED_B, LD_CBWD_A4T, LD_CBWD_BK4T, 1>(a, nph, p, part, part_bytes, s, what, gx);
    return run_gemm<PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_BK4, 1>(a, nph, p, part, part_bytes, s, what, gx);
  }
  if (va && in_place && g->Cout % 16 == 0 && g->k <= 5)
    return run_gemm<PROD_SHARED_B, LD_CBWD_A4T, LD_CBWD_BK4T>(a, nph, p, part, part_bytes, s, what, gx);
  if (va && in_place) return run_gemm<PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_BK4>(a, nph, p, part, part_bytes, s, what, gx);
  if (va && vb) return run_gemm<PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_B4>(a, nph, p, part, part_bytes, s, what, gx);
  if (va) return run_gemm<PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_B_S>(a, nph, p, part, part_bytes, s, what, gx);
  return run_gemm<PROD_SHARED_B, LD_CBWD_A_S, LD_CBWD_B_S>(a, nph, p, part, part_bytes, s, what, gx);
}

extern "C" int tagi_conv2d_bwd_delta(const float* dmz, const float* dSz, const float* mw, float* dma, float* dSa,
                                     const tagi_conv_geom* g, float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  return conv_bwd_delta_impl("tagi_conv2d_bwd_delta", dmz, dSz, mw, nullptr, nullptr, dma, dSa, g, ws, ws_bytes,
                             stream);
}

extern "C" int tagi_conv2d_bwd_delta_add(const float* dmz, const float* dSz, const float* mw, const float* add_m,
                                         const float* add_S, float* dma, float* dSa, const tagi_conv_geom* g,
                                         float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  return conv_bwd_delta_impl("tagi_conv2d_bwd_delta_add", dmz, dSz, mw, add_m, add_S, dma, dSa, g, ws, ws_bytes,
                             stream);
}

extern "C" int64_t tagi_conv2d_bwd_delta_bn_relu_part_bytes(const tagi_conv_geom* g) {
  return bn_fuse_tiles(g) * 6 * (g ? g->C : 0) * (int64_t)sizeof(float);
}

extern "C" int tagi_conv2d_bwd_delta_bn_relu(const float* dmz, const float* dSz, const float* mw, const float* mhat,
                                             const float* J, const float* var, const float* mg, float eps,
                                             float* dma, float* dSa, float* part, int64_t part_bytes,
                                             const tagi_conv_geom* g, float* ws, int64_t ws_bytes,
                                             tagi_stream_t stream) {
  const char* what = "tagi_conv2d_bwd_delta_bn_relu";
  TAGI_REQUIRE(mhat && J && var && mg && part, "%s: null pointer", what);
  const int64_t need = tagi_conv2d_bwd_delta_bn_relu_part_bytes(g);
  if (need == 0)
    return fail(TAGI_ERR_UNSUPPORTED, "%s: needs stride 1 and an unsplit input-delta plan (use "
                "tagi_conv2d_bwd_delta and tagi_bn_relu_bwd_partials_bias)", what);
  TAGI_REQUIRE(part_bytes >= need, "%s: partial sums need %lld bytes (got %lld)", what, (long long)need,
               (long long)part_bytes);
  const BnBwdFuse f{mhat, J, var, mg, eps, part, nullptr, nullptr};
  return conv_bwd_delta_impl(what, dmz, dSz, mw, nullptr, nullptr, dma, dSa, g, ws, ws_bytes, stream, &f);
}

extern "C" int tagi_conv2d_bwd_delta_add_bn_relu(const float* dmz, const float* dSz, const float* mw,
                                                 const float* add_m, const float* add_S, float* dma, float* dSa,
                                                 const float* mhat, const float* J, const float* var,
                                                 const float* mg, float eps, float* dmz_prev, float* dSz_prev,
                                                 float* part, int64_t part_bytes, const tagi_conv_geom* g,
                                                 float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_conv2d_bwd_delta_add_bn_relu";
  TAGI_REQUIRE(add_m && add_S && mhat && J && var && mg && part && dmz_prev && dSz_prev, "%s: null pointer", what);
  const int64_t need = tagi_conv2d_bwd_delta_bn_relu_part_bytes(g);
  if (need == 0)
    return fail(TAGI_ERR_UNSUPPORTED, "%s: needs stride 1 and an unsplit input-delta plan (use "
                "tagi_conv2d_bwd_delta_add and tagi_bn_relu_bwd_partials_bias)", what);
  TAGI_REQUIRE(part_bytes >= need, "%s: partial sums need %lld bytes (got %lld)", what, (long long)need,
               (long long)part_bytes);
  const BnBwdFuse f{mhat, J, var, mg, eps, part, dmz_prev, dSz_prev};
  return conv_bwd_delta_impl(what, dmz, dSz, mw, add_m, add_S, dma, dSa, g, ws, ws_bytes, stream, &f);
}

// ============================================================== parameter deltas
extern "C" int64_t tagi_conv2d_wgrad_ws_bytes(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->Ho <= 0 || g->Wo <= 0 || g->C <= 0 || g->k <= 0) return 0;
  // enough for either form (with or without the bias row)
  const int64_t K = g->C * g->k * g->k;
  const int64_t a = plan_ws_bytes(conv_wgrad_plan(g, true), K + 1, g->Cout, 1);
  const int64_t b = plan_ws_bytes(conv_wgrad_plan(g, false), K, g->Cout, 1);
  return a > b ? a : b;
}

extern "C" int tagi_conv2d_wgrad(const float* ma, const float* dmz, const float* dSz, const float* Sw, const float* Sb,
                                 float* dmw, float* dSw, float* dmb, float* dSb, const tagi_conv_geom* g, float* ws,
                                 int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_conv2d_wgrad";
  int rc = check_geom(g, what);
  if (rc) return rc;
  TAGI_REQUIRE(ma && dmz && dSz && dmw && dSw, "%s: null pointer", what);
  TAGI_REQUIRE((dmb == nullptr) == (dSb == nullptr), "%s: dmb and dSb must both be given or both be NULL", what);
  hipStream_t s = as_stream(stream);
  const int64_t K = g->C * g->k * g->k, N = g->Cout, M = g->N * g->Ho * g->Wo;
  const bool bias = dmb != nullptr;
  ProfScope ps(FAM_CONV_WGRAD, s, 2.0 * 2 * M * K * N, 4.0 * (g->N * g->C * g->H * g->W + 2 * M * N + 3 * K * N));
  GemmArgs a{};
  a.a = conv_operand(ma, nullptr, g, K, M, g->N * g->C * g->H * g->W);
  if (bias) a.a.ones_row = (int)K;
  a.b = strided_operand(dmz, dSz, 1, 0, 0, 1, N, N, M);
  a.epi = epi_wgrad(dmw, dSw, dmb, dSb, Sw, Sb, K, N);
  a.epi.perm_C = (int)g->C;
  a.epi.perm_kk2 = (int)(g->k * g->k);
  a.epi.dperm = make_fastdiv((int)g->C);
  a.R = (int)(K + (bias ? 1 : 0));
  a.C = (int)N;
  a.Kred = (int)M;
  Plan p = conv_wgrad_plan(g, bias);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, a.R, N, 1)))
    p = choose_plan(a.R, N, M, 1, PROD_SHARED_A, false, 1);
  p.tiles_m = (int)cdiv(a.R, kCfg[p.cfg].BM);
  const bool va = g->C % 4 == 0 && al16(ma);
  const bool vb = g->Cout % 4 == 0 && al16(dmz) && al16(dSz);
  // every 16-pixel run of the reduction inside one image, in whole rows or within one row
  const int64_t howo = g->Ho * g->Wo;
  if (va && vb && howo % 16 == 0 && (g->Wo % 16 == 0 || 16 % g->Wo == 0))
    return run_gemm<PROD_SHARED_A, LD_CWG_A4T, LD_STR_MN4>(a, 1, p, ws, ws_bytes, s, what);
  if (va && vb) return run_gemm<PROD_SHARED_A, LD_CWG_A4, LD_STR_MN4>(a, 1, p, ws, ws_bytes, s, what);
  if (vb) return run_gemm<PROD_SHARED_A, LD_CWG_A_S, LD_STR_MN4>(a, 1, p, ws, ws_bytes, s, what);
  return run_gemm<PROD_SHARED_A, LD_CWG_A_S, LD_STR_MN_S>(a, 1, p, ws, ws_bytes, s, what);
}
