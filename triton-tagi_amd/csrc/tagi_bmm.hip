// Batched attention products with strided operand views.
#include "tagi_gemm_core.h"

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

// ============================================================ batched products
static int view_kind(int64_t s_mn, int64_t s_k) { return (s_k == 1 && s_mn != 1) ? LD_STRIDED_K : LD_STRIDED_MN; }

template <int PROD>
static int bmm_dispatch(GemmArgs& g, int ka, int kb, int64_t batch, const Plan& p, hipStream_t s, const char* what) {
  if (ka == LD_STRIDED_K && kb == LD_STRIDED_K) return run_gemm<PROD, LD_STRIDED_K, LD_STRIDED_K>(g, batch, p, nullptr, 0, s, what);
  if (ka == LD_STRIDED_K && kb == LD_STRIDED_MN) return run_gemm<PROD, LD_STRIDED_K, LD_STRIDED_MN>(g, batch, p, nullptr, 0, s, what);
  if (ka == LD_STRIDED_MN && kb == LD_STRIDED_K) return run_gemm<PROD, LD_STRIDED_MN, LD_STRIDED_K>(g, batch, p, nullptr, 0, s, what);
  return run_gemm<PROD, LD_STRIDED_MN, LD_STRIDED_MN>(g, batch, p, nullptr, 0, s, what);
}

static int check_view(const tagi_view* v, const char* what, const char* name) {
  TAGI_REQUIRE(v != nullptr, "%s: null view %s", what, name);
  TAGI_REQUIRE(v->zdiv >= 1, "%s: view %s needs zdiv >= 1", what, name);
  return TAGI_OK;
}

extern "C" int tagi_bmm_tagi(const float* mu_a, const float* var_a, const float* mu_b, const float* var_b, float* mean,
                             float* var, int64_t batch, int64_t M, int64_t K, int64_t L, const tagi_view* va,
                             const tagi_view* vb, const tagi_view* vo, float scale, float scale_sq,
                             tagi_stream_t stream) {
  const char* what = "tagi_bmm_tagi";
  TAGI_REQUIRE(mu_a && var_a && mu_b && var_b && var, "%s: null pointer", what);
  TAGI_REQUIRE(batch > 0 && M > 0 && K > 0 && L > 0 && batch < 65536, "%s: bad sizes", what);
  int rc;
  if ((rc = check_view(va, what, "a")) || (rc = check_view(vb, what, "b")) || (rc = check_view(vo, what, "out")))
    return rc;
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BMM_FWD, s, 2.0 * (mean ? 3 : 2) * batch * M * K * L,
               4.0 * batch * (2 * M * K + 2 * K * L + (mean ? 2 : 1) * M * L));
  GemmArgs g{};
  g.a = strided_operand(mu_a, var_a, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
  g.b = strided_operand(mu_b, var_b, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
  g.epi = epi_store(mean, var, nullptr, nullptr, 0, 0, scale, scale_sq, vo->zdiv, vo->sz1, vo->sz2, vo->si, L, 0,
                    vo->sj);
  g.R = (int)M;
  g.C = (int)L;
  g.Kred = (int)K;
  Plan p = choose_plan(M, L, K, batch, 3, false, 1);
  return bmm_dispatch<PROD_FWD>(g, view_kind(va->si, va->sj), view_kind(vb->sj, vb->si), batch, p, s, what);
}

extern "C" int tagi_bmm_shared(const float* p0, const float* p1, const float* p2, float* mean, float* var,
                               int64_t batch, int64_t M, int64_t K, int64_t L, const tagi_view* va, const tagi_view* vb,
                               const tagi_view* vo, float scale, float scale_sq, int shared_left,
                               tagi_stream_t stream) {
  const char* what = "tagi_bmm_shared";
  TAGI_REQUIRE(p0 && p1 && p2 && mean && var, "%s: null pointer", what);
  TAGI_REQUIRE(batch > 0 && M > 0 && K > 0 && L > 0 && batch < 65536, "%s: bad sizes", what);
  int rc;
  if ((rc = check_view(va, what, "a")) || (rc = check_view(vb, what, "b")) || (rc = check_view(vo, what, "out")))
    return rc;
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BMM_SHARED, s, 2.0 * 2 * batch * M * K * L,
               4.0 * batch * ((shared_left ? 1 : 2) * M * K + (shared_left ? 2 : 1) * K * L + 2 * M * L));
  GemmArgs g{};
  g.epi = epi_store(mean, var, nullptr, nullptr, 0, 0, scale, scale_sq, vo->zdiv, vo->sz1, vo->sz2, vo->si, L, 0,
                    vo->sj);
  g.R = (int)M;
  g.C = (int)L;
  g.Kred = (int)K;
  Plan p = choose_plan(M, L, K, batch, 2, false, 1);
  if (!shared_left) {
    g.a = strided_operand(p0, p1, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
    g.b = strided_operand(p2, nullptr, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
    return bmm_dispatch<PROD_SHARED_B>(g, view_kind(va->si, va->sj), view_kind(vb->sj, vb->si), batch, p, s, what);
  }
  g.a = strided_operand(p2, nullptr, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
  g.b = strided_operand(p0, p1, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
  return bmm_dispatch<PROD_SHARED_A>(g, view_kind(va->si, va->sj), view_kind(vb->sj, vb->si), batch, p, s, what);
}

