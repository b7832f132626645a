// Conv2D entry points: implicit-GEMM forward, transposed implicit GEMM for input deltas,
// split-K parameter deltas.
#include "tagi_gemm_core.h"

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

// ====================================================================== Conv2D
extern "C" int64_t tagi_conv2d_fwd_ws_bytes(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->Ho <= 0 || g->Wo <= 0) return 0;
  return plan_ws_bytes(conv_fwd_plan(g), g->Cout, g->N * g->Ho * g->Wo, 1);
}

extern "C" int tagi_conv2d_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw, const float* mb,
                               const float* Sb, float* mz, float* Sz, const tagi_conv_geom* g, float* ws,
                               int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_conv2d_fwd";
  int rc = check_geom(g, what);
  if (rc) return rc;
  TAGI_REQUIRE(ma && Sa && mw && Sw && mz && Sz, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  const int64_t R = g->Cout, C = g->N * g->Ho * g->Wo, K = g->C * g->k * g->k;
  ProfScope ps(FAM_CONV_FWD, s, 2.0 * 3 * R * C * K,
               4.0 * (2 * g->N * g->C * g->H * g->W + 2 * K * R + 2 * R * C));
  GemmArgs a{};
  a.a = strided_operand(mw, Sw, 1, 0, 0, 1, R, R, K);
  a.b = conv_operand(ma, Sa, g, C, K);
  const int64_t howo = g->Ho * g->Wo;
  a.epi = epi_store(mz, Sz, mb, Sb, 1, 0, 1.f, 1.f, 1, 0, 0, howo, howo, R * howo, 1);
  a.R = (int)R;
  a.C = (int)C;
  a.Kred = (int)K;
  Plan p = conv_fwd_plan(g);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, R, C, 1))) p = choose_plan(R, C, K, 1, 3, false, 1);
  return run_gemm<PROD_FWD, LD_STRIDED_MN, LD_CONV_PATCH_MN>(a, 1, p, ws, ws_bytes, s, what);
}

extern "C" int tagi_conv2d_bwd_delta(const float* dmz, const float* dSz, const float* mw, float* dma, float* dSa,
                                     const tagi_conv_geom* g, tagi_stream_t stream) {
  const char* what = "tagi_conv2d_bwd_delta";
  int rc = check_geom(g, what);
  if (rc) return rc;
  TAGI_REQUIRE(dmz && dSz && mw && dma && dSa, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  const int64_t hw = g->H * g->W;
  const int64_t R = g->C, C = g->N * hw, K = g->k * g->k * g->Cout;
  // algorithmic work of the patch-space product (what an explicit col2im path computes)
  const double alg = 2.0 * 2 * (g->N * g->Ho * g->Wo) * (g->C * g->k * g->k) * g->Cout;
  ProfScope ps(FAM_CONV_BWD_DELTA, s, alg, 4.0 * (2 * g->N * g->Cout * g->Ho * g->Wo + K * R + 2 * R * C));
  GemmArgs a{};
  a.a = conv_operand(mw, nullptr, g, R, K);
  a.b = conv_operand(dmz, dSz, g, C, K);
  a.epi = epi_store(dma, dSa, nullptr, nullptr, 0, 0, 1.f, 1.f, 1, 0, 0, hw, hw, R * hw, 1);
  a.R = (int)R;
  a.C = (int)C;
  a.Kred = (int)K;
  Plan p = choose_plan(R, C, K, 1, 2, false, 1);
  return run_gemm<PROD_SHARED_A, LD_CONV_WT_K, LD_CONV_DY_MN>(a, 1, p, nullptr, 0, s, what);
}

extern "C" int64_t tagi_conv2d_wgrad_ws_bytes(const tagi_conv_geom* g) {
  if (!g || g->N <= 0 || g->Cout <= 0 || g->Ho <= 0 || g->Wo <= 0 || g->C <= 0 || g->k <= 0) return 0;
  return plan_ws_bytes(conv_wgrad_plan(g), g->C * g->k * g->k + 1, g->Cout, 1);
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
  a.a = conv_operand(ma, nullptr, g, K, M);
  if (bias) a.a.ones_row = (int)K;
  a.b = conv_operand(dmz, dSz, g, N, M);
  a.epi = epi_wgrad(dmw, dSw, dmb, dSb, Sw, Sb, K, N);
  a.R = (int)(K + (bias ? 1 : 0));
  a.C = (int)N;
  a.Kred = (int)M;
  Plan p = conv_wgrad_plan(g);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, K + 1, N, 1)))
    p = choose_plan(K + 1, N, M, 1, 2, false, 1);
  p.tiles_m = (int)cdiv(a.R, kCfg[p.cfg].BM);
  return run_gemm<PROD_SHARED_A, LD_CONV_PATCH_K, LD_CONV_DYROW_K>(a, 1, p, ws, ws_bytes, s, what);
}
