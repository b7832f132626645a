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

// =================================================== attention scores + Remax, fused
// multihead_attention.py:174-190: the scores' moments Q K^T for one head and 32 query rows
// (the TAGI product of tagi_bmm_tagi, with its reduction order: k-tile t of 16, k-step s,
// lane half hl taking k = 16t + 8hl + s, so the scores are bit-identical to that path's),
// held in LDS and passed through the Remax row by row (the row math of tagi_remax_fwd).
// The raw scores never reach HBM: per head, 2 S x S tensors are neither written nor read
// back. Eight waves (4 waves per SIMD at two blocks per CU, to hide the Remax's dependent
// VALU chains): wave w forms column tile w (S <= 256), then applies the Remax to rows
// 4w .. 4w + 3 of the block. The LDS tile is 2 x 32 x 257 floats = 65,792 bytes, more than
// the 64 KiB a workgroup may use on earlier CDNA parts: these kernels rely on gfx950's
// 160 KiB of LDS per CU (two blocks per CU), and the library is built for gfx950 only.
namespace {
constexpr int kScoreLd = 257;  // padded LDS row (S <= 256): conflict-free row reads
constexpr int kScorePlane = 32 * kScoreLd;
static_assert(2 * 2 * kScorePlane * sizeof(float) <= 160 * 1024, "two score tiles must fit one CU's LDS");

// Scores of query rows r0 .. r0+31 of head (b, h) against all S keys into sm: means in
// rows 0..31, variances in rows 32..63 (row stride kScoreLd). hbase: offset of the head's
// first element plus the lane half's 8 reduction indices; E: row stride of q and k.
template <int HD, bool STAGED = false>
__device__ __forceinline__ void attn_scores_to_lds(const float* __restrict__ mq, const float* __restrict__ vq,
                                                   const float* __restrict__ mk, const float* __restrict__ vk,
                                                   float* sm, int64_t hbase, int r0, int S, int E, float scale,
                                                   float scale_sq, int wave, int hl, int rl,
                                                   const float* qst = nullptr) {
  constexpr int NKT = HD / 16;
  // query row r0 + rl: the lane's 8 reduction indices of each k-tile
  float aq[NKT][8], av[NKT][8];
  if constexpr (STAGED) {
    // from the block's rows staged in LDS ([moment][row][HD + 4], rows past S zero)
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = rl * (HD + 4) + 8 * hl + 16 * t + 4 * u;
        const float4 x = *reinterpret_cast<const float4*>(qst + c);
        const float4 y = *reinterpret_cast<const float4*>(qst + 32 * (HD + 4) + c);
        aq[t][4 * u + 0] = x.x, aq[t][4 * u + 1] = x.y, aq[t][4 * u + 2] = x.z, aq[t][4 * u + 3] = x.w;
        av[t][4 * u + 0] = y.x, av[t][4 * u + 1] = y.y, av[t][4 * u + 2] = y.z, av[t][4 * u + 3] = y.w;
      }
  } else {
    const int qi = r0 + rl;
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
        if (qi < S) {
          const int64_t o = hbase + (int64_t)qi * E + 16 * t + 4 * u;
          x = *reinterpret_cast<const float4*>(mq + o);
          y = *reinterpret_cast<const float4*>(vq + o);
        }
        aq[t][4 * u + 0] = x.x, aq[t][4 * u + 1] = x.y, aq[t][4 * u + 2] = x.z, aq[t][4 * u + 3] = x.w;
        av[t][4 * u + 0] = y.x, av[t][4 * u + 1] = y.y, av[t][4 * u + 2] = y.z, av[t][4 * u + 3] = y.w;
      }
  }
  if (wave * 32 >= S) return;  // column tiles past S are neither formed nor read
  const int kn = wave * 32 + rl;  // key row
  float bm[NKT][8], bv[NKT][8];
#pragma unroll
  for (int t = 0; t < NKT; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
      if (kn < S) {
        const int64_t o = hbase + (int64_t)kn * E + 16 * t + 4 * u;
        x = *reinterpret_cast<const float4*>(mk + o);
        y = *reinterpret_cast<const float4*>(vk + o);
      }
      bm[t][4 * u + 0] = x.x, bm[t][4 * u + 1] = x.y, bm[t][4 * u + 2] = x.z, bm[t][4 * u + 3] = x.w;
      bv[t][4 * u + 0] = y.x, bv[t][4 * u + 1] = y.y, bv[t][4 * u + 2] = y.z, bv[t][4 * u + 3] = y.w;
    }
  floatx16 accM, accV;
#pragma unroll
  for (int v = 0; v < 16; ++v) accM[v] = accV[v] = 0.f;
#pragma unroll
  for (int t = 0; t < NKT; ++t)
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float a0 = aq[t][s], a1 = av[t][s], b0 = bm[t][s], b1 = bv[t][s];
      const float asq = a0 * a0, bvar = b0 * b0 + b1;
      accM = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, accM, 0, 0, 0);
      accV = __builtin_amdgcn_mfma_f32_32x32x2f32(asq, b1, accV, 0, 0, 0);
      accV = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, bvar, accV, 0, 0, 0);
    }
  // accumulator v of lane l: row 8(v/4) + 4hl + v%4, column j*32 + rl (scaled as the
  // batched product's epilogue does); columns kn >= S hold zeros
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = 8 * (v >> 2) + 4 * hl + (v & 3);
    sm[row * kScoreLd + kn] = accM[v] * scale + 0.f;
    sm[kScorePlane + row * kScoreLd + kn] = accV[v] * scale_sq + 0.f;
  }
}

// The Remax of rows 4w .. 4w+3 of the block (wave w), written to mu_a / J (and var_a
// when non-null) at (z, r0 + row); with BACK, mu_a and var_a also replace the scores in LDS.
template <bool BACK>
__device__ __forceinline__ void attn_remax_rows(float* sm, float* __restrict__ ma, float* __restrict__ Sa,
                                                float* __restrict__ Jo, int64_t z, int r0, int S, int wave,
                                                int lane) {
#pragma unroll 1
  for (int rr = 0; rr < 4; ++rr) {
    const int row = wave * 4 + rr;
    const int i = r0 + row;
    if (i >= S) break;
    float m[4], v[4], oa[4], os[4], oj[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = lane + 64 * e;
      const bool ok = c < S;
      m[e] = ok ? sm[row * kScoreLd + c] : 0.f;
      v[e] = ok ? sm[kScorePlane + row * kScoreLd + c] : 1.f;
    }
    remax_row<4>(m, v, lane, S, oa, os, oj);
    const int64_t ob = (z * S + i) * S;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = lane + 64 * e;
      if (c < S) {
        ma[ob + c] = oa[e];
        if (Sa) Sa[ob + c] = os[e];
        Jo[ob + c] = oj[e];
        if constexpr (BACK) {
          sm[row * kScoreLd + c] = oa[e];
          sm[kScorePlane + row * kScoreLd + c] = os[e];
        }
      }
    }
  }
}

template <int HD>
__global__ void __launch_bounds__(512) attn_scores_remax_kernel(const float* __restrict__ mq,
                                                                const float* __restrict__ vq,
                                                                const float* __restrict__ mk,
                                                                const float* __restrict__ vk, float* __restrict__ ma,
                                                                float* __restrict__ Sa, float* __restrict__ Jo, int H,
                                                                int S, int E, float scale, float scale_sq) {
  // E: row stride of q and k (their rows hold the heads side by side, head h at h*HD)
  __shared__ float sm[2 * kScorePlane];
  const int z = blockIdx.y;
  const int b = z / H, h = z - b * H;
  const int r0 = blockIdx.x * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, rl = lane & 31;
  const int64_t hbase = (int64_t)b * S * E + (int64_t)h * HD + 8 * hl;
  attn_scores_to_lds<HD>(mq, vq, mk, vk, sm, hbase, r0, S, E, scale, scale_sq, wave, hl, rl);
  __syncthreads();
  attn_remax_rows<false>(sm, ma, Sa, Jo, z, r0, S, wave, lane);
}

// Scores, Remax and the score @ V product (multihead_attention.py:174-193) in one kernel
// for head dimensions up to 32: after the Remax, mu_a and var_a of the block's 32 rows sit
// in LDS and each wave multiplies its 32 keys' stretch of them by V (the TAGI product:
// mean mu_a mu_v, variance mu_a^2 S_v + S_a (mu_v^2 + S_v), MFMA k-step s taking key
// 32w + 2s + hl); the 8 partial 32 x 32 tiles are summed through LDS in wave order and
// written into the (B, S, ld_out) output at column h*HD. mu_a and J are written for the
// backward pass, var_a only when requested (the raw scores and var_a otherwise never
// reach HBM, and score @ V reads nothing of the S x S tensors back).
template <int HD>
__global__ void __launch_bounds__(512) attn_fwd_kernel(const float* __restrict__ mq, const float* __restrict__ vq,
                                                       const float* __restrict__ mk, const float* __restrict__ vk,
                                                       const float* __restrict__ mv, const float* __restrict__ vv,
                                                       float* __restrict__ ma, float* __restrict__ Sa,
                                                       float* __restrict__ Jo, float* __restrict__ om,
                                                       float* __restrict__ oS, int H, int S, int E, int ldo,
                                                       float scale, float scale_sq) {
  static_assert(HD <= 32, "one 32-column MFMA tile per head");
  constexpr int QLD = HD + 4;
  __shared__ float sm[2 * kScorePlane];
  __shared__ float qst[2 * 32 * QLD];  // the block's query rows, mean and variance
  const int z = blockIdx.y;
  const int b = z / H, h = z - b * H;
  const int r0 = blockIdx.x * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, rl = lane & 31;
  const int64_t hbase = (int64_t)b * S * E + (int64_t)h * HD + 8 * hl;
  if (threadIdx.x < 16 * HD) {
    // every wave reads all 32 query rows: one float4 per thread into LDS instead (L2 reads
    // of the rows 8 -> 1 per block; transformer block +0.4%)
    const int t = threadIdx.x;
    const int mom = t / (8 * HD), row = (t / (HD / 4)) & 31, c = 4 * (t % (HD / 4));
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r0 + row < S)
      x = *reinterpret_cast<const float4*>((mom ? vq : mq) + ((int64_t)b * S * E + (int64_t)h * HD +
                                                               (int64_t)(r0 + row) * E + c));
    *reinterpret_cast<float4*>(qst + mom * 32 * QLD + row * QLD + c) = x;
  }
  __syncthreads();
  attn_scores_to_lds<HD, true>(mq, vq, mk, vk, sm, hbase, r0, S, E, scale, scale_sq, wave, hl, rl, qst);
  __syncthreads();
  attn_remax_rows<true>(sm, ma, Sa, Jo, z, r0, S, wave, lane);
  __syncthreads();
  // score @ V over keys kb .. kb+31; LDS columns kb .. 32*ceil(S/32)-1 past S hold zeros
  // (scores formed from zero keys, left untouched by the Remax) and V reads as zero there
  const int kb = 32 * wave;
  floatx16 accM, accV;
#pragma unroll
  for (int v = 0; v < 16; ++v) accM[v] = accV[v] = 0.f;
  if (kb < S) {
    const int64_t vbase = (int64_t)b * S * E + (int64_t)h * HD + rl;
    float bm[16], bv[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int key = kb + 2 * s + hl;
      const bool ok = key < S && rl < HD;
      bm[s] = ok ? mv[vbase + (int64_t)key * E] : 0.f;
      bv[s] = ok ? vv[vbase + (int64_t)key * E] : 0.f;
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int key = kb + 2 * s + hl;
      const float a0 = sm[rl * kScoreLd + key], a1 = sm[kScorePlane + rl * kScoreLd + key];
      const float b0 = bm[s], b1 = bv[s];
      const float asq = a0 * a0, bvar = b0 * b0 + b1;
      accM = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, accM, 0, 0, 0);
      accV = __builtin_amdgcn_mfma_f32_32x32x2f32(asq, b1, accV, 0, 0, 0);
      accV = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, bvar, accV, 0, 0, 0);
    }
  }
  __syncthreads();  // every wave is done reading the scores
  float* red = sm;  // [wave][mean, variance][32 x 32]
  if (kb < S) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int o = (8 * (v >> 2) + 4 * hl + (v & 3)) * 32 + rl;
      red[wave * 2048 + o] = accM[v];
      red[wave * 2048 + 1024 + o] = accV[v];
    }
  }
  __syncthreads();
  const int nw = min(8, (S + 31) / 32);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int o = threadIdx.x + 512 * q;
    const int row = o >> 5, col = o & 31;
    float m = 0.f, v = 0.f;
    for (int w = 0; w < nw; ++w) {
      m += red[w * 2048 + o];
      v += red[w * 2048 + 1024 + o];
    }
    const int i = r0 + row;
    if (i < S && col < HD) {
      const int64_t off = ((int64_t)b * S + i) * ldo + (int64_t)h * HD + col;
      om[off] = m;
      oS[off] = v;
    }
  }
}
}  // namespace

extern "C" int tagi_attn_scores_remax(const float* mu_q, const float* var_q, const float* mu_k, const float* var_k,
                                      int64_t ld_qk, float* mu_a, float* var_a, float* J, int64_t B, int64_t H,
                                      int64_t S, int64_t D, float scale, float scale_sq, tagi_stream_t stream) {
  const char* what = "tagi_attn_scores_remax";
  TAGI_REQUIRE(mu_q && var_q && mu_k && var_k && mu_a && var_a && J, "%s: null pointer", what);
  TAGI_REQUIRE(B > 0 && H > 0 && S > 0 && D > 0, "%s: bad sizes", what);
  if (S > 256 || !(D == 16 || D == 32 || D == 64))
    return fail(TAGI_ERR_UNSUPPORTED, "%s: needs S <= 256 and head_dim 16, 32 or 64 (S=%lld, D=%lld)", what,
                (long long)S, (long long)D);
  TAGI_REQUIRE(ld_qk >= H * D && ld_qk % 4 == 0, "%s: row stride %lld below H*D or not a multiple of 4", what,
               (long long)ld_qk);
  TAGI_REQUIRE(al16(mu_q) && al16(var_q) && al16(mu_k) && al16(var_k), "%s: q/k must be 16-byte aligned", what);
  TAGI_REQUIRE(B * H < 65536 && fits_i32(B * S * ld_qk) && B * H * S * S < (1ll << 40), "%s: too large", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_ATTN_SCORES, s, 2.0 * 3 * B * H * S * S * D, 4.0 * (4 * B * S * H * D + 3 * B * H * S * S));
  const dim3 grid((unsigned)cdiv(S, 32), (unsigned)(B * H));
  const int E = (int)ld_qk;
  if (D == 16)
    hipLaunchKernelGGL(attn_scores_remax_kernel<16>, grid, dim3(512), 0, s, mu_q, var_q, mu_k, var_k, mu_a, var_a, J,
                       (int)H, (int)S, E, scale, scale_sq);
  else if (D == 32)
    hipLaunchKernelGGL(attn_scores_remax_kernel<32>, grid, dim3(512), 0, s, mu_q, var_q, mu_k, var_k, mu_a, var_a, J,
                       (int)H, (int)S, E, scale, scale_sq);
  else
    hipLaunchKernelGGL(attn_scores_remax_kernel<64>, grid, dim3(512), 0, s, mu_q, var_q, mu_k, var_k, mu_a, var_a, J,
                       (int)H, (int)S, E, scale, scale_sq);
  return check_launch(what);
}

extern "C" int tagi_attn_fwd(const float* mu_q, const float* var_q, const float* mu_k, const float* var_k,
                             const float* mu_v, const float* var_v, int64_t ld_qkv, float* mu_a, float* var_a,
                             float* J, float* out_m, float* out_S, int64_t ld_out, int64_t B, int64_t H, int64_t S,
                             int64_t D, float scale, float scale_sq, tagi_stream_t stream) {
  const char* what = "tagi_attn_fwd";
  TAGI_REQUIRE(mu_q && var_q && mu_k && var_k && mu_v && var_v && mu_a && J && out_m && out_S, "%s: null pointer",
               what);
  TAGI_REQUIRE(B > 0 && H > 0 && S > 0 && D > 0, "%s: bad sizes", what);
  if (S > 256 || !(D == 16 || D == 32))
    return fail(TAGI_ERR_UNSUPPORTED, "%s: needs S <= 256 and head_dim 16 or 32 (S=%lld, D=%lld)", what, (long long)S,
                (long long)D);
  TAGI_REQUIRE(ld_qkv >= H * D && ld_qkv % 4 == 0 && ld_out >= H * D, "%s: row strides %lld / %lld below H*D (or q/k "
               "stride not a multiple of 4)", what, (long long)ld_qkv, (long long)ld_out);
  TAGI_REQUIRE(al16(mu_q) && al16(var_q) && al16(mu_k) && al16(var_k), "%s: q/k must be 16-byte aligned", what);
  TAGI_REQUIRE(B * H < 65536 && fits_i32(B * S * ld_qkv) && fits_i32(ld_out) && B * H * S * S < (1ll << 40),
               "%s: too large", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_ATTN_SCORES, s, 2.0 * 6 * B * H * S * S * D,
               4.0 * (8 * B * S * H * D + (var_a ? 3 : 2) * B * H * S * S));
  const dim3 grid((unsigned)cdiv(S, 32), (unsigned)(B * H));
  const int E = (int)ld_qkv, LO = (int)ld_out;
  if (D == 16)
    hipLaunchKernelGGL(attn_fwd_kernel<16>, grid, dim3(512), 0, s, mu_q, var_q, mu_k, var_k, mu_v, var_v, mu_a,
                       var_a, J, out_m, out_S, (int)H, (int)S, E, LO, scale, scale_sq);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<32>, grid, dim3(512), 0, s, mu_q, var_q, mu_k, var_k, mu_v, var_v, mu_a,
                       var_a, J, out_m, out_S, (int)H, (int)S, E, LO, scale, scale_sq);
  return check_launch(what);
}

// ================================== attention score deltas -> dQ / dK products, fused
// multihead_attention.py:238-251: the score deltas d_out @ mu_v^T, scaled by the Remax
// Jacobian J (mean x J, variance x J^2), feed dQ = s * scaled @ mu_k and
// dK = s * scaled^T @ mu_q. Each block rebuilds in LDS the part of the scaled deltas its
// output needs -- 32 query rows for dQ, 32 key columns for dK (TRANS) -- with the
// score-delta product and Jacobian of tagi_bmm_shared_jacobian (same MFMA order and
// epilogue, so the same values), then runs the second product from LDS: the (B, H, S, S)
// scaled deltas are never written or read back. The second product's reduction over the
// S scores is split over the 8 waves (32 scores each); the 8 partial tiles are added in
// wave order, so results are deterministic and within rounding of the one-pass sum.
namespace {
// (at most 128 registers, so that two blocks -- four waves per SIMD -- fit beside the LDS)
template <int HD, bool TRANS>
__global__ void __launch_bounds__(512, 4) attn_dqk_kernel(const float* __restrict__ dmu, const float* __restrict__ dvar,
                                                       const float* __restrict__ mv, const float* __restrict__ Jg,
                                                       const float* __restrict__ mx, float* __restrict__ omu,
                                                       float* __restrict__ ovar, int H, int S, int ld_d, int ld_x,
                                                       int ld_o, float scale, float scale_sq) {
  constexpr int NKT = HD / 16;
  // phase 1-2: [moment][output row][score index]; phase 3: 8 waves x 2 moments x 32 x 32 partials
  __shared__ float sm[2 * 32 * kScoreLd];
  static_assert(8 * 2 * 32 * 32 <= 2 * 32 * kScoreLd, "partials must fit the score tile");
  const int z = blockIdx.y;
  const int b = z / H, h = z - b * H;
  const int o0 = blockIdx.x * 32;  // first output row: query (dQ) or key (dK)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, rl = lane & 31;
  // head h of batch b in the output deltas (row stride ld_d), mu_v / mu_x (ld_x), out (ld_o)
  const int64_t bd = (int64_t)b * S * ld_d + (int64_t)h * HD;
  const int64_t bx = (int64_t)b * S * ld_x + (int64_t)h * HD;
  const int64_t bo = (int64_t)b * S * ld_o + (int64_t)h * HD;
  const int64_t jz = (int64_t)z * S * S;
  const bool active = wave * 32 < S;  // this wave's 32 score indices exist

  // the Jacobian tile is loaded first, so its latency overlaps phase 1's loads and MFMAs
  float jr[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int tr = 8 * (q >> 2) + 4 * hl + (q & 3);
    const int qi = TRANS ? 32 * wave + tr : o0 + tr;
    const int kj = TRANS ? o0 + rl : 32 * wave + rl;
    jr[q] = (active && qi < S && kj < S) ? Jg[jz + (int64_t)qi * S + kj] : 0.f;
  }
  // phase 1: scaled score deltas of query rows x key columns, one 32 x 32 tile per wave
  if (active) {
    const int ai = TRANS ? 32 * wave + rl : o0 + rl;  // query row (A = output deltas)
    const int bj = TRANS ? o0 + rl : 32 * wave + rl;  // key row (B = mu_v, shared)
    float am[NKT][8], av[NKT][8], bm[NKT][8];
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x, w = x;
        const int ko = 8 * hl + 16 * t + 4 * u;
        if (ai < S) {
          x = *reinterpret_cast<const float4*>(dmu + bd + ko + (int64_t)ai * ld_d);
          y = *reinterpret_cast<const float4*>(dvar + bd + ko + (int64_t)ai * ld_d);
        }
        if (bj < S) w = *reinterpret_cast<const float4*>(mv + bx + ko + (int64_t)bj * ld_x);
        am[t][4 * u + 0] = x.x, am[t][4 * u + 1] = x.y, am[t][4 * u + 2] = x.z, am[t][4 * u + 3] = x.w;
        av[t][4 * u + 0] = y.x, av[t][4 * u + 1] = y.y, av[t][4 * u + 2] = y.z, av[t][4 * u + 3] = y.w;
        bm[t][4 * u + 0] = w.x, bm[t][4 * u + 1] = w.y, bm[t][4 * u + 2] = w.z, bm[t][4 * u + 3] = w.w;
      }
    floatx16 accM, accV;
#pragma unroll
    for (int v = 0; v < 16; ++v) accM[v] = accV[v] = 0.f;
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float b0 = bm[t][s], bsq = b0 * b0;
        accM = __builtin_amdgcn_mfma_f32_32x32x2f32(am[t][s], b0, accM, 0, 0, 0);
        accV = __builtin_amdgcn_mfma_f32_32x32x2f32(av[t][s], bsq, accV, 0, 0, 0);
      }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int tr = 8 * (v >> 2) + 4 * hl + (v & 3);  // tile row (query side of A)
      const float jj = jr[v];
      float m = accM[v] * 1.f + 0.f, vv = accV[v] * 1.f + 0.f;
      m *= jj;
      vv *= jj * jj;
      const int orow = TRANS ? rl : tr;
      const int ocol = TRANS ? 32 * wave + tr : 32 * wave + rl;
      sm[orow * kScoreLd + ocol] = m;
      sm[32 * kScoreLd + orow * kScoreLd + ocol] = vv;
    }
  }
  __syncthreads();

  // phase 2: the output rows times mu_x over this wave's 32 score indices
  floatx16 pM, pV;
#pragma unroll
  for (int v = 0; v < 16; ++v) pM[v] = pV[v] = 0.f;
  if (active) {
    float xr[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int k = 32 * wave + 16 * (q >> 3) + 8 * hl + (q & 7);
      xr[q] = (k < S && rl < HD) ? mx[bx + (int64_t)k * ld_x + rl] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int k = 32 * wave + 16 * t + 8 * hl + s;  // score index
        const float a0 = sm[rl * kScoreLd + k], a1 = sm[32 * kScoreLd + rl * kScoreLd + k];
        const float x = xr[8 * t + s];
        const float xsq = x * x;
        pM = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, x, pM, 0, 0, 0);
        pV = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, xsq, pV, 0, 0, 0);
      }
  }
  __syncthreads();
  // phase 3: partials (output row, column d) in wave order, then the fixed-order sum
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int tr = 8 * (v >> 2) + 4 * hl + (v & 3);
    sm[(wave * 2 + 0) * 1024 + tr * 32 + rl] = pM[v];
    sm[(wave * 2 + 1) * 1024 + tr * 32 + rl] = pV[v];
  }
  __syncthreads();
  const int nw = (S + 31) / 32;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int idx = threadIdx.x + 512 * q;  // 2 moments x 32 rows x 32 columns
    const int mom = idx >> 10, row = (idx >> 5) & 31, d = idx & 31;
    float acc = 0.f;
    for (int w = 0; w < nw; ++w) acc += sm[(w * 2 + mom) * 1024 + row * 32 + d];
    if (o0 + row < S && d < HD) {
      const int64_t o = bo + (int64_t)(o0 + row) * ld_o + d;
      if (mom == 0) omu[o] = acc * scale + 0.f;
      else ovar[o] = acc * scale_sq + 0.f;
    }
  }
}

// The query and key deltas of one head in one block (multihead_attention.py:239-260): for
// each block of 32 query rows in order, the scaled score deltas (phase 1, as in
// attn_dqk_kernel) are formed once into LDS; wave w then multiplies the tile's rows over its
// 32 keys by mu_k (partial query deltas, summed over the waves in wave order and stored, as
// attn_dqk_kernel does, so the query deltas are the same bits) and the transposed tile's
// columns -- its own 32 keys -- by mu_q into key-delta accumulators held in registers across
// all query blocks (summed query block by query block in order: deterministic). Against the
// two kernels above, the score-delta product and the Jacobian are formed and read once
// instead of twice. The query block's output deltas and mu_q rows, which every wave reads,
// are staged in LDS once per block: the next block's rows are requested at the start of
// phase 2 and stored once their buffers' last readers are past a barrier (the 8 waves
// read them from LDS instead of each loading them; 198 -> 163 us at b64 x 8 heads x 256).
// LDS: 65,792 + 9,216 + 4,736 bytes, two blocks per CU within gfx950's 160 KiB.
template <int HD>
__global__ void __launch_bounds__(512, 4) attn_dqk_joint_kernel(
    const float* __restrict__ dmu, const float* __restrict__ dvar, const float* __restrict__ mv,
    const float* __restrict__ Jg, const float* __restrict__ mq, const float* __restrict__ mk,
    float* __restrict__ oq_mu, float* __restrict__ oq_var, float* __restrict__ ok_mu, float* __restrict__ ok_var,
    int H, int S, int ld_d, int ld_x, int ld_o, float scale, float scale_sq) {
  constexpr int NKT = HD / 16;
  constexpr int RLD = HD + 4;  // padded row of the staged output deltas
  __shared__ float sm[2 * 32 * kScoreLd];
  __shared__ float rows[2 * 32 * RLD];  // the query block's output deltas, mean and variance
  // the query block's mu_q rows (+32: lanes past a head dimension of 16 read on into the
  // next row, and from the last row past it)
  __shared__ float qrows[32 * RLD + 32];
  static_assert(2 * sizeof(float) * (2 * 32 * kScoreLd + 2 * 32 * RLD + 32 * RLD + 32) <= 160 * 1024,
                "two blocks must fit one CU's LDS");
  static_assert(8 * 2 * 32 * 32 <= 2 * 32 * kScoreLd, "partials must fit the score tile");
  const int z = blockIdx.x;
  const int b = z / H, h = z - b * H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, rl = lane & 31;
  // per-head base pointers (uniform) and 32-bit lane offsets from them
  const float* hdm = dmu + (int64_t)b * S * ld_d + (int64_t)h * HD;
  const float* hdv = dvar + (int64_t)b * S * ld_d + (int64_t)h * HD;
  const float* hv = mv + (int64_t)b * S * ld_x + (int64_t)h * HD;
  // mu_q, mu_k and J through buffer resources (scalar registers) and 32-bit byte offsets in
  // the vector offset, the one the hardware checks against the range: rows at or past S lie
  // beyond the head's range and read as zeros (no per-element masks, no 64-bit addresses);
  // the scalar offset is left 0 because it is not range-checked
  const int64_t head_bytes = 4 * ((int64_t)(S - 1) * ld_x + HD);
  const tagi_i32x4 rq = make_buffer_rsrc(mq + (int64_t)b * S * ld_x + (int64_t)h * HD, head_bytes);
  const tagi_i32x4 rk = make_buffer_rsrc(mk + (int64_t)b * S * ld_x + (int64_t)h * HD, head_bytes);
  const tagi_i32x4 rJ = make_buffer_rsrc(Jg + (int64_t)z * S * S, 4 * (int64_t)S * S);
  const int64_t bo = (int64_t)b * S * ld_o + (int64_t)h * HD;
  float* hqm = oq_mu + bo;
  float* hqv = oq_var + bo;
  float* hkm = ok_mu + bo;
  float* hkv = ok_var + bo;
  const bool active = wave * 32 < S;  // this wave's 32 keys exist
  const int nw = (S + 31) / 32;
  floatx16 kM, kV;  // key deltas of keys 32 wave + (accumulator row), columns d = rl
#pragma unroll
  for (int v = 0; v < 16; ++v) kM[v] = kV[v] = 0.f;
  // staging of a query block's output-delta rows: thread t < 16 HD takes one float4
  // (moment t / (8 HD), row (t / (HD / 4)) % 32, columns 4 (t % (HD / 4)) ..)
  const int st_t = threadIdx.x;
  const bool st_on = st_t < 16 * HD;
  const int st_mom = st_t / (8 * HD), st_row = (st_t / (HD / 4)) & 31, st_c = 4 * (st_t % (HD / 4));
  auto stage_load = [&](int ob) -> float4 {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (st_on && ob + st_row < S)
      x = *reinterpret_cast<const float4*>((st_mom ? hdv : hdm) + ((ob + st_row) * ld_d + st_c));
    return x;
  };
  auto stage_store = [&](float4 x) {
    if (st_on) *reinterpret_cast<float4*>(rows + st_mom * 32 * RLD + st_row * RLD + st_c) = x;
  };
  // the query block's mu_q rows: thread t < 8 HD takes one float4 (row t / (HD / 4))
  const bool sq_on = st_t < 8 * HD;
  const int sq_row = st_t / (HD / 4), sq_c = 4 * (st_t % (HD / 4));
  const float* hq = mq + (int64_t)b * S * ld_x + (int64_t)h * HD;
  auto q_load = [&](int ob) -> float4 {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sq_on && ob + sq_row < S) x = *reinterpret_cast<const float4*>(hq + ((ob + sq_row) * ld_x + sq_c));
    return x;
  };
  auto q_store = [&](float4 x) {
    if (sq_on) *reinterpret_cast<float4*>(qrows + sq_row * RLD + sq_c) = x;
  };
  stage_store(stage_load(0));
  q_store(q_load(0));
  __syncthreads();

#pragma unroll 1
  for (int o0 = 0; o0 < S; o0 += 32) {
    // phase 1: scaled score deltas of query rows o0.. x this wave's keys (attn_dqk_kernel's
    // products and order; the operands of one 16-wide k-tile at a time and the Jacobian read
    // at the scaling, which keeps the key-delta accumulators in registers without spilling)
    if (active) {
      const int ai = o0 + rl, bj = 32 * wave + rl;
      floatx16 accM, accV;
#pragma unroll
      for (int v = 0; v < 16; ++v) accM[v] = accV[v] = 0.f;
#pragma unroll
      for (int t = 0; t < NKT; ++t) {
        float am[8], av[8], bm[8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          float4 w = make_float4(0.f, 0.f, 0.f, 0.f);
          const int ko = 8 * hl + 16 * t + 4 * u;
          // rows past S were staged as zeros
          const float4 x = *reinterpret_cast<const float4*>(rows + rl * RLD + ko);
          const float4 y = *reinterpret_cast<const float4*>(rows + 32 * RLD + rl * RLD + ko);
          if (bj < S) w = *reinterpret_cast<const float4*>(hv + (ko + bj * ld_x));
          am[4 * u + 0] = x.x, am[4 * u + 1] = x.y, am[4 * u + 2] = x.z, am[4 * u + 3] = x.w;
          av[4 * u + 0] = y.x, av[4 * u + 1] = y.y, av[4 * u + 2] = y.z, av[4 * u + 3] = y.w;
          bm[4 * u + 0] = w.x, bm[4 * u + 1] = w.y, bm[4 * u + 2] = w.z, bm[4 * u + 3] = w.w;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float b0 = bm[s], bsq = b0 * b0;
          accM = __builtin_amdgcn_mfma_f32_32x32x2f32(am[s], b0, accM, 0, 0, 0);
          accV = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s], bsq, accV, 0, 0, 0);
        }
      }
      // J of query rows o0 + 4 hl + c_v, c_v = 8 (v / 4) + v % 4; rows past S read 0, and key
      // columns past S (last tile) hold score deltas that are exactly 0 (their mu_v was 0)
      int jvo = 4 * ((o0 + 4 * hl) * S + bj);
      __asm__ volatile("" : "+v"(jvo));  // one offset per lane; the 16 sums below stay transient
      float* sw = sm + 4 * hl * kScoreLd + 32 * wave + rl;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int cv = 8 * (v >> 2) + (v & 3);
        const float jj = tagi_raw_buffer_load_f32(rJ, jvo + 4 * cv * S, 0, 0);
        float m = accM[v] * 1.f + 0.f, vv = accV[v] * 1.f + 0.f;
        m *= jj;
        vv *= jj * jj;
        sw[cv * kScoreLd] = m;
        sw[32 * kScoreLd + cv * kScoreLd] = vv;
      }
    }
    __syncthreads();
    // the next query block's output-delta rows: requested now, staged after phase 2 (the
    // rows buffer was last read in phase 1)
    const float4 nxt = stage_load(o0 + 32);
    const float4 nxq = q_load(o0 + 32);
    // phase 2: query rows times mu_k over this wave's keys (partials), and this wave's keys
    // times mu_q over the block's query rows (into the key-delta accumulators)
    floatx16 pM, pV;
#pragma unroll
    for (int v = 0; v < 16; ++v) pM[v] = pV[v] = 0.f;
    if (active) {
      // key 32 wave + 8 hl + c_q (query o0 + 8 hl + c_q), c_q = 16 (q / 8) + q % 8, column d = rl;
      // for head dimension 16 the lanes rl >= 16 read other columns, which only reach
      // accumulator columns that are never stored
      float xk[16], xq[16];
      int xko = 4 * ((32 * wave + 8 * hl) * ld_x + rl);
      __asm__ volatile("" : "+v"(xko));  // kept per query block: hoisted sums would spill
#pragma unroll
      for (int q = 0; q < 16; ++q)
        xk[q] = tagi_raw_buffer_load_f32(rk, xko + 4 * (16 * (q >> 3) + (q & 7)) * ld_x, 0, 0);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int k = 32 * wave + 16 * t + 8 * hl + s;  // key index (reduction of the query deltas)
          const float a0 = sm[rl * kScoreLd + k], a1 = sm[32 * kScoreLd + rl * kScoreLd + k];
          const float x = xk[8 * t + s];
          const float xsq = x * x;
          pM = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, x, pM, 0, 0, 0);
          pV = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, xsq, pV, 0, 0, 0);
        }
      // staged rows past S are zeros; columns rl >= HD (head dimension 16) read the next
      // row's first columns, which only reach accumulator columns that are never stored
#pragma unroll
      for (int q = 0; q < 16; ++q) xq[q] = qrows[(8 * hl + 16 * (q >> 3) + (q & 7)) * RLD + rl];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int q = 16 * t + 8 * hl + s;  // query row in the block (reduction of the key deltas)
          const float a0 = sm[q * kScoreLd + 32 * wave + rl], a1 = sm[32 * kScoreLd + q * kScoreLd + 32 * wave + rl];
          const float x = xq[8 * t + s];
          const float xsq = x * x;
          kM = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, x, kM, 0, 0, 0);
          kV = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, xsq, kV, 0, 0, 0);
        }
    }
    stage_store(nxt);
    __syncthreads();
    q_store(nxq);  // every wave is past phase 2, the last reader of the mu_q rows
    // phase 3: query-delta partials in wave order, then the fixed-order sum (attn_dqk_kernel)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int tr = 8 * (v >> 2) + 4 * hl + (v & 3);
      sm[(wave * 2 + 0) * 1024 + tr * 32 + rl] = pM[v];
      sm[(wave * 2 + 1) * 1024 + tr * 32 + rl] = pV[v];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = threadIdx.x + 512 * q;
      const int mom = idx >> 10, row = (idx >> 5) & 31, d = idx & 31;
      float acc = 0.f;
      for (int w = 0; w < nw; ++w) acc += sm[(w * 2 + mom) * 1024 + row * 32 + d];
      if (o0 + row < S && d < HD) {
        const int o = (o0 + row) * ld_o + d;
        if (mom == 0) hqm[o] = acc * scale + 0.f;
        else hqv[o] = acc * scale_sq + 0.f;
      }
    }
    __syncthreads();  // the tile area is written again by the next query block's phase 1
  }
  if (active) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = 32 * wave + 8 * (v >> 2) + 4 * hl + (v & 3);
      if (key < S && rl < HD) {
        const int o = key * ld_o + rl;
        hkm[o] = kM[v] * scale + 0.f;
        hkv[o] = kV[v] * scale_sq + 0.f;
      }
    }
  }
}
}  // namespace

extern "C" int tagi_attn_score_deltas_qk(const float* d_mu, const float* d_var, int64_t ld_d, const float* mu_v,
                                         const float* mu_x, int64_t ld_x, const float* J, float* out_mu,
                                         float* out_var, int64_t ld_out, int64_t B, int64_t H, int64_t S, int64_t D,
                                         float scale, float scale_sq, int transpose, tagi_stream_t stream) {
  const char* what = "tagi_attn_score_deltas_qk";
  TAGI_REQUIRE(d_mu && d_var && mu_v && J && mu_x && out_mu && out_var, "%s: null pointer", what);
  TAGI_REQUIRE(B > 0 && H > 0 && S > 0 && D > 0, "%s: bad sizes", what);
  if (S > 256 || !(D == 16 || D == 32))
    return fail(TAGI_ERR_UNSUPPORTED, "%s: needs S <= 256 and head_dim 16 or 32 (S=%lld, D=%lld)", what,
                (long long)S, (long long)D);
  TAGI_REQUIRE(ld_d >= H * D && ld_x >= H * D && ld_out >= H * D && ld_d % 4 == 0 && ld_x % 4 == 0,
               "%s: row strides below H*D (or d/x strides not multiples of 4)", what);
  TAGI_REQUIRE(al16(d_mu) && al16(d_var) && al16(mu_v), "%s: d_mu, d_var and mu_v must be 16-byte aligned", what);
  TAGI_REQUIRE(B * H < 65536 && fits_i32(B * S * ld_d) && fits_i32(B * S * ld_x) && fits_i32(B * S * ld_out) &&
                   B * H * S * S < (1ll << 40),
               "%s: too large", what);
  hipStream_t s = as_stream(stream);
  // algorithmic work: this product (2 moments) plus half of the score-delta product (2
  // moments), which the dQ and dK kernels each form again for their own blocks
  ProfScope ps(FAM_BMM_SHARED, s, 2.0 * 3 * B * H * S * S * D, 4.0 * (B * H * S * S + 6 * B * S * H * D));
  const dim3 grid((unsigned)cdiv(S, 32), (unsigned)(B * H));
#define TAGI_DQK(HD_, T_)                                                                                      \
  hipLaunchKernelGGL((attn_dqk_kernel<HD_, T_>), grid, dim3(512), 0, s, d_mu, d_var, mu_v, J, mu_x, out_mu, out_var, \
                     (int)H, (int)S, (int)ld_d, (int)ld_x, (int)ld_out, scale, scale_sq)
  if (D == 16) {
    if (transpose) TAGI_DQK(16, true);
    else TAGI_DQK(16, false);
  } else {
    if (transpose) TAGI_DQK(32, true);
    else TAGI_DQK(32, false);
  }
#undef TAGI_DQK
  return check_launch(what);
}

extern "C" int tagi_attn_score_deltas_qk_joint(const float* d_mu, const float* d_var, int64_t ld_d, const float* mu_v,
                                               const float* mu_q, const float* mu_k, int64_t ld_x, const float* J,
                                               float* dq_mu, float* dq_var, float* dk_mu, float* dk_var,
                                               int64_t ld_out, int64_t B, int64_t H, int64_t S, int64_t D,
                                               float scale, float scale_sq, tagi_stream_t stream) {
  const char* what = "tagi_attn_score_deltas_qk_joint";
  TAGI_REQUIRE(d_mu && d_var && mu_v && mu_q && mu_k && J && dq_mu && dq_var && dk_mu && dk_var, "%s: null pointer",
               what);
  TAGI_REQUIRE(B > 0 && H > 0 && S > 0 && D > 0, "%s: bad sizes", what);
  if (S > 256 || !(D == 16 || D == 32))
    return fail(TAGI_ERR_UNSUPPORTED, "%s: needs S <= 256 and head_dim 16 or 32 (S=%lld, D=%lld)", what,
                (long long)S, (long long)D);
  TAGI_REQUIRE(ld_d >= H * D && ld_x >= H * D && ld_out >= H * D && ld_d % 4 == 0 && ld_x % 4 == 0,
               "%s: row strides below H*D (or d/x strides not multiples of 4)", what);
  TAGI_REQUIRE(al16(d_mu) && al16(d_var) && al16(mu_v), "%s: d_mu, d_var and mu_v must be 16-byte aligned", what);
  TAGI_REQUIRE(B * H < (1ll << 31) && fits_i32(B * S * ld_d) && fits_i32(B * S * ld_x) && fits_i32(B * S * ld_out) &&
                   (S + 32) * ld_x * 4 < (1ll << 31) && B * H * S * S < (1ll << 40),
               "%s: too large", what);
  hipStream_t s = as_stream(stream);
  // algorithmic work: the score-delta product and the query and key products (2 moments each)
  ProfScope ps(FAM_BMM_SHARED, s, 2.0 * 6 * B * H * S * S * D, 4.0 * (B * H * S * S + 7 * B * S * H * D));
  const dim3 grid((unsigned)(B * H));
#define TAGI_DQKJ(HD_)                                                                                             \
  hipLaunchKernelGGL((attn_dqk_joint_kernel<HD_>), grid, dim3(512), 0, s, d_mu, d_var, mu_v, J, mu_q, mu_k, dq_mu, \
                     dq_var, dk_mu, dk_var, (int)H, (int)S, (int)ld_d, (int)ld_x, (int)ld_out, scale, scale_sq)
  if (D == 16) TAGI_DQKJ(16);
  else TAGI_DQKJ(32);
#undef TAGI_DQKJ
  return check_launch(what);
}
