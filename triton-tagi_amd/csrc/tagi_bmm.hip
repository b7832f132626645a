// Batched attention products with strided operand views.
#include "tagi_gemm_core.h"

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

// Loader kind of a strided operand: float4 along its unit-stride dim when every other
// stride, the extent of that dim and the base pointer allow it; scalar otherwise.
static int view_kind(const void* p, int64_t zdiv, int64_t sz1, int64_t sz2, int64_t s_mn, int64_t s_k, int64_t MN,
                     int64_t K) {
  const bool al = al16(p) && sz1 % 4 == 0 && sz2 % 4 == 0;
  if (s_k == 1 && K % 4 == 0 && s_mn % 4 == 0 && al) return LD_STR_K4;
  if (s_mn == 1 && MN % 4 == 0 && s_k % 4 == 0 && al) return LD_STR_MN4;
  (void)zdiv;
  return LD_STR_MN_S;
}

template <int PROD>
static int bmm_dispatch(GemmArgs& g, int ka, int kb, int64_t batch, const Plan& p, hipStream_t s, const char* what) {
  if (ka == LD_STR_MN_S || kb == LD_STR_MN_S)
    return run_gemm<PROD, LD_STR_MN_S, LD_STR_MN_S>(g, batch, p, nullptr, 0, s, what);
  if (ka == LD_STR_K4 && kb == LD_STR_K4) return run_gemm<PROD, LD_STR_K4, LD_STR_K4>(g, batch, p, nullptr, 0, s, what);
  if (ka == LD_STR_K4 && kb == LD_STR_MN4)
    return run_gemm<PROD, LD_STR_K4, LD_STR_MN4>(g, batch, p, nullptr, 0, s, what);
  if (ka == LD_STR_MN4 && kb == LD_STR_K4)
    return run_gemm<PROD, LD_STR_MN4, LD_STR_K4>(g, batch, p, nullptr, 0, s, what);
  return run_gemm<PROD, LD_STR_MN4, LD_STR_MN4>(g, batch, p, nullptr, 0, s, what);
}

static int check_view(const tagi_view* v, const char* what, const char* name) {
  TAGI_REQUIRE(v != nullptr, "%s: null view %s", what, name);
  TAGI_REQUIRE(v->zdiv >= 1, "%s: view %s needs zdiv >= 1", what, name);
  return TAGI_OK;
}

static bool view_fits(const tagi_view* v, int64_t batch, int64_t I, int64_t J) {
  const int64_t zmax = batch - 1;
  const int64_t span = (zmax / v->zdiv) * v->sz1 + (zmax % v->zdiv) * v->sz2 + (I - 1) * v->si + (J - 1) * v->sj;
  return span >= 0 && span < (1ll << 40);
}

extern "C" int tagi_bmm_tagi(const float* mu_a, const float* var_a, const float* mu_b, const float* var_b, float* mean,
                             float* var, int64_t batch, int64_t M, int64_t K, int64_t L, const tagi_view* va,
                             const tagi_view* vb, const tagi_view* vo, float scale, float scale_sq,
                             tagi_stream_t stream) {
  const char* what = "tagi_bmm_tagi";
  TAGI_REQUIRE(mu_a && var_a && mu_b && var_b && var, "%s: null pointer", what);
  TAGI_REQUIRE(batch > 0 && M > 0 && K > 0 && L > 0 && batch < 65536, "%s: bad sizes", what);
  TAGI_REQUIRE(fits_i32(M * L) && fits_i32(M * K) && fits_i32(K * L), "%s: matrices too large", what);
  int rc;
  if ((rc = check_view(va, what, "a")) || (rc = check_view(vb, what, "b")) || (rc = check_view(vo, what, "out")))
    return rc;
  TAGI_REQUIRE(view_fits(va, batch, M, K) && view_fits(vb, batch, K, L) && view_fits(vo, batch, M, L),
               "%s: negative or huge strides", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BMM_FWD, s, 2.0 * (mean ? 3 : 2) * batch * M * K * L,
               4.0 * batch * (2 * M * K + 2 * K * L + (mean ? 2 : 1) * M * L));
  GemmArgs g{};
  g.a = strided_operand(mu_a, var_a, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
  g.b = strided_operand(mu_b, var_b, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
  g.epi = epi_store(mean, var, nullptr, nullptr, 0, 0, scale, scale_sq, vo->zdiv, vo->sz1, vo->sz2, vo->si, vo->sj);
  g.R = (int)M;
  g.C = (int)L;
  g.Kred = (int)K;
  Plan p = choose_plan(M, L, K, batch, PROD_FWD, false, 1);
  int ka = view_kind(mu_a, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
  if (!al16(var_a)) ka = LD_STR_MN_S;
  int kb = view_kind(mu_b, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
  if (!al16(var_b)) kb = LD_STR_MN_S;
  return bmm_dispatch<PROD_FWD>(g, ka, kb, batch, p, s, what);
}

static int bmm_shared_impl(const char* what, const float* p0, const float* p1, const float* p2, const float* J,
                           float* mean, float* var, int64_t batch, int64_t M, int64_t K, int64_t L,
                           const tagi_view* va, const tagi_view* vb, const tagi_view* vo, float scale,
                           float scale_sq, int shared_left, tagi_stream_t stream) {
  TAGI_REQUIRE(p0 && p1 && p2 && mean && var, "%s: null pointer", what);
  TAGI_REQUIRE(batch > 0 && M > 0 && K > 0 && L > 0 && batch < 65536, "%s: bad sizes", what);
  TAGI_REQUIRE(fits_i32(M * L) && fits_i32(M * K) && fits_i32(K * L), "%s: matrices too large", what);
  int rc;
  if ((rc = check_view(va, what, "a")) || (rc = check_view(vb, what, "b")) || (rc = check_view(vo, what, "out")))
    return rc;
  TAGI_REQUIRE(view_fits(va, batch, M, K) && view_fits(vb, batch, K, L) && view_fits(vo, batch, M, L),
               "%s: negative or huge strides", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_BMM_SHARED, s, 2.0 * 2 * batch * M * K * L,
               4.0 * batch * ((shared_left ? 1 : 2) * M * K + (shared_left ? 2 : 1) * K * L + 2 * M * L));
  GemmArgs g{};
  g.epi = epi_store(mean, var, nullptr, nullptr, 0, 0, scale, scale_sq, vo->zdiv, vo->sz1, vo->sz2, vo->si, vo->sj);
  g.epi.jm = J;
  g.R = (int)M;
  g.C = (int)L;
  g.Kred = (int)K;
  Plan p = choose_plan(M, L, K, batch, shared_left ? PROD_SHARED_A : PROD_SHARED_B, false, 1);
  const float* a0 = shared_left ? p2 : p0;
  const float* a1 = shared_left ? nullptr : p1;
  const float* b0 = shared_left ? p0 : p2;
  const float* b1 = shared_left ? p1 : nullptr;
  g.a = strided_operand(a0, a1, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
  g.b = strided_operand(b0, b1, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
  int ka = view_kind(a0, va->zdiv, va->sz1, va->sz2, va->si, va->sj, M, K);
  if (a1 && !al16(a1)) ka = LD_STR_MN_S;
  int kb = view_kind(b0, vb->zdiv, vb->sz1, vb->sz2, vb->sj, vb->si, L, K);
  if (b1 && !al16(b1)) kb = LD_STR_MN_S;
  if (!shared_left) return bmm_dispatch<PROD_SHARED_B>(g, ka, kb, batch, p, s, what);
  return bmm_dispatch<PROD_SHARED_A>(g, ka, kb, batch, p, s, what);
}

extern "C" int tagi_bmm_shared(const float* p0, const float* p1, const float* p2, float* mean, float* var,
                               int64_t batch, int64_t M, int64_t K, int64_t L, const tagi_view* va, const tagi_view* vb,
                               const tagi_view* vo, float scale, float scale_sq, int shared_left,
                               tagi_stream_t stream) {
  return bmm_shared_impl("tagi_bmm_shared", p0, p1, p2, nullptr, mean, var, batch, M, K, L, va, vb, vo, scale,
                         scale_sq, shared_left, stream);
}

extern "C" int tagi_bmm_shared_jacobian(const float* p0, const float* p1, const float* p2, const float* J,
                                        float* mean, float* var, int64_t batch, int64_t M, int64_t K, int64_t L,
                                        const tagi_view* va, const tagi_view* vb, const tagi_view* vo, float scale,
                                        float scale_sq, int shared_left, tagi_stream_t stream) {
  const char* what = "tagi_bmm_shared_jacobian";
  TAGI_REQUIRE(J != nullptr, "%s: null Jacobian", what);
  return bmm_shared_impl(what, p0, p1, p2, J, mean, var, batch, M, K, L, va, vb, vo, scale, scale_sq, shared_left,
                         stream);
}
