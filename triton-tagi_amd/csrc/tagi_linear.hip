// Linear layer entry points (forward moments, backward deltas, parameter deltas).
#include "tagi_linear_internal.h"

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

Plan tagi::linear_fwd_plan(int64_t M, int64_t K, int64_t N) { return choose_plan(M, N, K, 1, PROD_FWD, true, 16); }
static Plan linear_bwd_plan(int64_t M, int64_t K, int64_t N) { return choose_plan(M, K, N, 1, PROD_SHARED_B, true, 16); }
static Plan linear_wgrad_plan(int64_t M, int64_t K, int64_t N) { return choose_plan(K + 1, N, M, 1, PROD_SHARED_A, true, 512); }

// A deterministic input (no variance, Sa NULL): mean = ma mw, variance = ma^2 Sw, the
// shared-A product (two MFMAs per k-step instead of three; the terms Sa (mw^2 + Sw) it
// leaves out are exact zeros)
static Plan linear_fwd0_plan(int64_t M, int64_t K, int64_t N) { return choose_plan(M, N, K, 1, PROD_SHARED_A, true, 16); }

extern "C" int64_t tagi_linear_fwd_ws_bytes(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  const int64_t a = plan_ws_bytes(linear_fwd_plan(M, K, N), M, N, 1), b = plan_ws_bytes(linear_fwd0_plan(M, K, N), M, N, 1);
  return a > b ? a : b;
}

int tagi::linear_fwd_check(const char* what, const float* ma, const float* Sa, const float* mw, const float* Sw,
                           const float* Sz, int64_t M, int64_t K, int64_t N) {
  TAGI_REQUIRE(ma && Sa && mw && Sw && Sz, "%s: null pointer", what);
  TAGI_REQUIRE(M > 0 && K > 0 && N > 0, "%s: sizes must be positive (M=%lld K=%lld N=%lld)", what, (long long)M,
               (long long)K, (long long)N);
  TAGI_REQUIRE(fits_i32(M * K) && fits_i32(K * N) && fits_i32(M * N), "%s: too large for 32-bit tiles", what);
  return TAGI_OK;
}

int tagi::linear_fwd_run(const char* what, const float* ma, const float* Sa, const float* mw, const float* Sw,
                         const float* mb, const float* Sb, float* mz, float* Sz, int64_t M, int64_t K, int64_t N,
                         const Plan& p, float* ws, int64_t ws_bytes, hipStream_t s, float* relu_J) {
  ProfScope ps(FAM_LINEAR_FWD, s, 2.0 * 3 * M * K * N,
               4.0 * (2 * M * K + 2 * K * N + (relu_J ? 3 : 2) * M * N));
  GemmArgs g{};
  g.a = strided_operand(ma, Sa, 1, 0, 0, K, 1, M, K);
  g.b = strided_operand(mw, Sw, 1, 0, 0, 1, N, N, K);
  g.epi = epi_store(mz, Sz, mb, Sb, 0, 1, 1.f, 1.f, 1, 0, 0, N, 1);
  g.epi.relu_J = relu_J;
  g.R = (int)M;
  g.C = (int)N;
  g.Kred = (int)K;
  const bool v4 = K % 4 == 0 && N % 4 == 0 && al16(ma) && al16(Sa) && al16(mw) && al16(Sw);
  if (relu_J) {
    if (v4) return run_gemm<PROD_FWD, LD_STR_K4, LD_STR_MN4, 4>(g, 1, p, ws, ws_bytes, s, what);
    return run_gemm<PROD_FWD, LD_STR_K_S, LD_STR_MN_S, 4>(g, 1, p, ws, ws_bytes, s, what);
  }
  if (v4) return run_gemm<PROD_FWD, LD_STR_K4, LD_STR_MN4>(g, 1, p, ws, ws_bytes, s, what);
  return run_gemm<PROD_FWD, LD_STR_K_S, LD_STR_MN_S>(g, 1, p, ws, ws_bytes, s, what);
}

// The forward of a zero-variance input (Sa == NULL): two products, mean ma mw and variance
// ma^2 Sw (the Sa terms are exact zeros). With relu_J, ReLU(z)'s moments and Jacobian.
static int linear_fwd0(const char* what, const float* ma, const float* mw, const float* Sw, const float* mb,
                       const float* Sb, float* mz, float* Sz, int64_t M, int64_t K, int64_t N, float* ws,
                       int64_t ws_bytes, hipStream_t s, float* relu_J) {
  TAGI_REQUIRE(ma && mw && Sw && Sz, "%s: null pointer", what);
  TAGI_REQUIRE(M > 0 && K > 0 && N > 0, "%s: sizes must be positive (M=%lld K=%lld N=%lld)", what, (long long)M,
               (long long)K, (long long)N);
  TAGI_REQUIRE(fits_i32(M * K) && fits_i32(K * N) && fits_i32(M * N), "%s: too large for 32-bit tiles", what);
  Plan p = linear_fwd0_plan(M, K, N);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, M, N, 1)))
    p = choose_plan(M, N, K, 1, PROD_SHARED_A, false, 1);
  ProfScope ps(FAM_LINEAR_FWD, s, 2.0 * 2 * M * K * N, 4.0 * (M * K + 2 * K * N + (relu_J ? 3 : 2) * M * N));
  GemmArgs g{};
  g.a = strided_operand(ma, nullptr, 1, 0, 0, K, 1, M, K);
  g.b = strided_operand(mw, Sw, 1, 0, 0, 1, N, N, K);
  g.epi = epi_store(mz, Sz, mb, Sb, 0, 1, 1.f, 1.f, 1, 0, 0, N, 1);
  g.epi.relu_J = relu_J;
  g.R = (int)M;
  g.C = (int)N;
  g.Kred = (int)K;
  const bool v4 = K % 4 == 0 && N % 4 == 0 && al16(ma) && al16(mw) && al16(Sw);
  if (relu_J) {
    if (v4) return run_gemm<PROD_SHARED_A, LD_STR_K4, LD_STR_MN4, 4>(g, 1, p, ws, ws_bytes, s, what);
    return run_gemm<PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S, 4>(g, 1, p, ws, ws_bytes, s, what);
  }
  if (v4) return run_gemm<PROD_SHARED_A, LD_STR_K4, LD_STR_MN4>(g, 1, p, ws, ws_bytes, s, what);
  return run_gemm<PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S>(g, 1, p, ws, ws_bytes, s, what);
}

static int linear_fwd_impl(const char* what, const float* ma, const float* Sa, const float* mw, const float* Sw,
                           const float* mb, const float* Sb, float* mz, float* Sz, float* relu_J, int64_t M,
                           int64_t K, int64_t N, float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  if (!Sa) return linear_fwd0(what, ma, mw, Sw, mb, Sb, mz, Sz, M, K, N, ws, ws_bytes, as_stream(stream), relu_J);
  int rc = linear_fwd_check(what, ma, Sa, mw, Sw, Sz, M, K, N);
  if (rc != TAGI_OK) return rc;
  Plan p = linear_fwd_plan(M, K, N);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, M, N, 1))) p = choose_plan(M, N, K, 1, PROD_FWD, false, 1);
  return linear_fwd_run(what, ma, Sa, mw, Sw, mb, Sb, mz, Sz, M, K, N, p, ws, ws_bytes, as_stream(stream), relu_J);
}

extern "C" int tagi_linear_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw, const float* mb,
                               const float* Sb, float* mz, float* Sz, int64_t M, int64_t K, int64_t N, float* ws,
                               int64_t ws_bytes, tagi_stream_t stream) {
  return linear_fwd_impl("tagi_linear_fwd", ma, Sa, mw, Sw, mb, Sb, mz, Sz, nullptr, M, K, N, ws, ws_bytes, stream);
}

extern "C" int tagi_linear_fwd_relu(const float* ma, const float* Sa, const float* mw, const float* Sw,
                                    const float* mb, const float* Sb, float* ma_out, float* Sa_out, float* J,
                                    int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                                    tagi_stream_t stream) {
  const char* what = "tagi_linear_fwd_relu";
  TAGI_REQUIRE(ma_out && Sa_out && J, "%s: null pointer", what);
  return linear_fwd_impl(what, ma, Sa, mw, Sw, mb, Sb, ma_out, Sa_out, J, M, K, N, ws, ws_bytes, stream);
}

extern "C" int64_t tagi_linear_bwd_delta_ws_bytes(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  return plan_ws_bytes(linear_bwd_plan(M, K, N), M, K, 1);
}

static int linear_bwd_delta_impl(const char* what, const float* dmz, const float* dSz, const float* mw,
                                 const float* add_m, const float* add_S, const float* J, float* dma, float* dSa,
                                 int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                                 tagi_stream_t stream) {
  TAGI_REQUIRE(dmz && dSz && mw && dma && dSa, "%s: null pointer", what);
  TAGI_REQUIRE((add_m == nullptr) == (add_S == nullptr), "%s: add_m and add_S must both be given or both be NULL",
               what);
  TAGI_REQUIRE(M > 0 && K > 0 && N > 0, "%s: sizes must be positive", what);
  TAGI_REQUIRE(fits_i32(M * K) && fits_i32(K * N) && fits_i32(M * N), "%s: too large for 32-bit tiles", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_LINEAR_BWD_DELTA, s, 2.0 * 2 * M * K * N, 4.0 * (2 * M * N + K * N + 2 * M * K));
  GemmArgs g{};
  g.a = strided_operand(dmz, dSz, 1, 0, 0, N, 1, M, N);
  g.b = strided_operand(mw, nullptr, 1, 0, 0, N, 1, K, N);
  g.epi = epi_store(dma, dSa, nullptr, nullptr, 0, 0, 1.f, 1.f, 1, 0, 0, K, 1);
  g.epi.am = add_m;
  g.epi.av = add_S;
  g.epi.jm = J;
  g.R = (int)M;
  g.C = (int)K;
  g.Kred = (int)N;
  Plan p = linear_bwd_plan(M, K, N);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, M, K, 1))) p = choose_plan(M, K, N, 1, PROD_SHARED_B, false, 1);
  const bool v4 = N % 4 == 0 && al16(dmz) && al16(dSz) && al16(mw);
  if (v4) return run_gemm<PROD_SHARED_B, LD_STR_K4, LD_STR_K4>(g, 1, p, ws, ws_bytes, s, what);
  return run_gemm<PROD_SHARED_B, LD_STR_K_S, LD_STR_K_S>(g, 1, p, ws, ws_bytes, s, what);
}

extern "C" int tagi_linear_bwd_delta(const float* dmz, const float* dSz, const float* mw, float* dma, float* dSa,
                                     int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                                     tagi_stream_t stream) {
  return linear_bwd_delta_impl("tagi_linear_bwd_delta", dmz, dSz, mw, nullptr, nullptr, nullptr, dma, dSa, M, K, N,
                               ws, ws_bytes, stream);
}

extern "C" int tagi_linear_bwd_delta_jacobian(const float* dmz, const float* dSz, const float* mw, const float* J,
                                              float* dma, float* dSa, int64_t M, int64_t K, int64_t N, float* ws,
                                              int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_linear_bwd_delta_jacobian";
  TAGI_REQUIRE(J, "%s: null pointer", what);
  return linear_bwd_delta_impl(what, dmz, dSz, mw, nullptr, nullptr, J, dma, dSa, M, K, N, ws, ws_bytes, stream);
}

extern "C" int tagi_linear_bwd_delta_add(const float* dmz, const float* dSz, const float* mw, const float* add_m,
                                         const float* add_S, float* dma, float* dSa, int64_t M, int64_t K, int64_t N,
                                         float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  return linear_bwd_delta_impl("tagi_linear_bwd_delta_add", dmz, dSz, mw, add_m, add_S, nullptr, dma, dSa, M, K, N,
                               ws, ws_bytes, stream);
}

extern "C" int64_t tagi_linear_wgrad_ws_bytes(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  return plan_ws_bytes(linear_wgrad_plan(M, K, N), K + 1, N, 1);
}

namespace {
// The parameter-delta product of tagi_linear_wgrad; with mw non-null, also the capped
// update of mw, Sw (and of mb, Sb with the bias) in the epilogue.
int linear_wgrad_impl(const char* what, const float* ma, const float* dmz, const float* dSz, const float* Sw,
                      const float* Sb, float* dmw, float* dSw, float* dmb, float* dSb, float* mw, float* mb,
                      float cap, int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  // with the update (mw given) the delta outputs may all be NULL: applied, not stored
  const bool keep = dmw != nullptr;
  TAGI_REQUIRE(ma && dmz && dSz && (keep || mw) && (dSw != nullptr) == keep, "%s: null pointer", what);
  TAGI_REQUIRE((dmb == nullptr) == (dSb == nullptr), "%s: dmb and dSb must both be given or both be NULL", what);
  TAGI_REQUIRE(keep || dmb == nullptr, "%s: bias deltas without the weight deltas", what);
  TAGI_REQUIRE(M > 0 && K > 0 && N > 0, "%s: sizes must be positive", what);
  TAGI_REQUIRE(fits_i32(M * K) && fits_i32((K + 1) * N) && fits_i32(M * N), "%s: too large for 32-bit tiles", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_LINEAR_WGRAD, s, 2.0 * 2 * M * K * N,
               4.0 * (M * K + 2 * M * N + (keep ? 3 : 1) * K * N + (mw ? 3 * K * N : 0)));
  const bool bias = mw ? mb != nullptr : dmb != nullptr;
  GemmArgs g{};
  g.a = strided_operand(ma, nullptr, 1, 0, 0, 1, K, K, M);
  if (bias) g.a.ones_row = (int)K;
  g.b = strided_operand(dmz, dSz, 1, 0, 0, 1, N, N, M);
  g.epi = epi_wgrad(dmw, dSw, dmb, dSb, Sw, Sb, K, N);
  if (mw) {
    g.epi.upd_mw = mw;
    g.epi.upd_Sw = const_cast<float*>(Sw);
    g.epi.upd_mb = mb;
    g.epi.upd_Sb = const_cast<float*>(Sb);
    g.epi.cap = cap;
  }
  g.R = (int)(K + (bias ? 1 : 0));
  g.C = (int)N;
  g.Kred = (int)M;
  Plan p = linear_wgrad_plan(M, K, N);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_ws_bytes(p, K + 1, N, 1)))
    p = choose_plan(K + 1, N, M, 1, PROD_SHARED_A, false, 1);
  p.tiles_m = (int)cdiv(g.R, kCfg[p.cfg].BM);
  const bool v4 = K % 4 == 0 && N % 4 == 0 && al16(ma) && al16(dmz) && al16(dSz);
  if (mw) {
    if (v4) return run_gemm<PROD_SHARED_A, LD_STR_MN4, LD_STR_MN4, 2>(g, 1, p, ws, ws_bytes, s, what);
    return run_gemm<PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S, 2>(g, 1, p, ws, ws_bytes, s, what);
  }
  if (v4) return run_gemm<PROD_SHARED_A, LD_STR_MN4, LD_STR_MN4>(g, 1, p, ws, ws_bytes, s, what);
  return run_gemm<PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S>(g, 1, p, ws, ws_bytes, s, what);
}
}  // namespace

extern "C" int tagi_linear_wgrad(const float* ma, const float* dmz, const float* dSz, const float* Sw, const float* Sb,
                                 float* dmw, float* dSw, float* dmb, float* dSb, int64_t M, int64_t K, int64_t N,
                                 float* ws, int64_t ws_bytes, tagi_stream_t stream) {
  return linear_wgrad_impl("tagi_linear_wgrad", ma, dmz, dSz, Sw, Sb, dmw, dSw, dmb, dSb, nullptr, nullptr, 0.f, M,
                           K, N, ws, ws_bytes, stream);
}

extern "C" int tagi_linear_wgrad_update(const float* ma, const float* dmz, const float* dSz, float* mw, float* Sw,
                                        float* mb, float* Sb, float* dmw, float* dSw, float* dmb, float* dSb,
                                        float cap_factor, int64_t M, int64_t K, int64_t N, float* ws,
                                        int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_linear_wgrad_update";
  TAGI_REQUIRE(mw && Sw, "%s: null pointer", what);
  TAGI_REQUIRE((mb == nullptr) == (Sb == nullptr) && (dmw == nullptr || (dmb == nullptr) == (mb == nullptr)),
               "%s: the bias needs mb, Sb, dmb and dSb together (or none of them; dmb, dSb NULL when the deltas "
               "are not stored)", what);
  TAGI_REQUIRE(cap_factor > 0.f && cap_factor <= 3.4e38f, "%s: cap_factor must be positive and finite", what);
  return linear_wgrad_impl(what, ma, dmz, dSz, Sw, Sb, dmw, dSw, dmb, dSb, mw, mb, cap_factor, M, K, N, ws, ws_bytes,
                           stream);
}

// ------------------------------------------------------------------- Embedding
// Backward (embedding.py:111-145): delta_mw[cat, d] = sum over the category's tokens of
// dmz[t, d] Sw[cat, d], and delta_Sw with dSz and Sw^2. Sw[cat, d] is the same for every
// token of a category, so the raw sums are formed first and weighted once (equal in exact
// arithmetic). One block per category, 16 waves, over windows of 16384 tokens:
//   * each wave takes a 1024-token stretch of the window (ids loaded up front), finds the
//     category's tokens by a ballot per 64-token chunk and appends them to its own LDS list
//     in token order -- the window's matches are the wave lists one after the other;
//   * match j of that sequence is added by wave j % 16 (up to 4 rows' loads in flight per
//     wave, each lane holding 4 columns of a 256-column group);
//   * the 16 waves' sums are added in wave order through LDS.
// The sum order is fixed by the token ids alone: deterministic. Every delta row is read
// once; the ids are read once per category (cache-resident, 4 bytes per token). Tokens of
// padding_idx or outside [0, V) add nothing, and a delta row reaches only its category.
namespace {
constexpr int kEmbWaves = 16;
constexpr int kEmbPerWave = 1024;                    // tokens a wave scans per window
constexpr int kEmbWin = kEmbWaves * kEmbPerWave;     // tokens per window

__device__ __forceinline__ int64_t emb_token_id(float t) { return (int64_t)t; }  // truncation, as .long()

template <bool V4>
__global__ void __launch_bounds__(1024) embedding_bwd_kernel(const float* __restrict__ tokens,
                                                             const float* __restrict__ dmz,
                                                             const float* __restrict__ dSz,
                                                             const float* __restrict__ Sw, float* __restrict__ dmw,
                                                             float* __restrict__ dSw, int64_t n, int D,
                                                             int64_t padding_idx) {
  // the match lists (window-relative token indices), then the waves' sums (float
  // [wave][moment][256]) in the same 32 KB
  __shared__ __attribute__((aligned(16))) unsigned char buf[kEmbWin * sizeof(unsigned short)];
  __shared__ int wcnt[kEmbWaves];
  static_assert(kEmbWaves * 2 * 256 * sizeof(float) <= sizeof(buf), "sums must fit the list space");
  unsigned short* list = reinterpret_cast<unsigned short*>(buf);
  float* red = reinterpret_cast<float*>(buf);
  const int64_t cat = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool skip = cat == padding_idx;
  for (int g0 = 0; g0 < D; g0 += 256) {
    float am[4] = {0.f, 0.f, 0.f, 0.f}, as[4] = {0.f, 0.f, 0.f, 0.f};
    const int col = g0 + 4 * lane;
    for (int64_t w0 = 0; w0 < n && !skip; w0 += kEmbWin) {
      // scan: this wave's stretch of the window, matches appended in token order
      const int64_t s0 = w0 + (int64_t)wave * kEmbPerWave;
      constexpr int NCH = kEmbPerWave / 64;
      bool hit[NCH];
#pragma unroll
      for (int q = 0; q < NCH; ++q) {
        const int64_t t = s0 + 64 * q + lane;
        hit[q] = t < n && emb_token_id(tokens[t]) == cat;
      }
      int cnt = 0;
      unsigned short* mylist = list + wave * kEmbPerWave;
#pragma unroll
      for (int q = 0; q < NCH; ++q) {
        const uint64_t m = __ballot(hit[q]);
        if (hit[q]) mylist[cnt + __popcll(m & ((1ull << lane) - 1))] = (unsigned short)(wave * kEmbPerWave + 64 * q + lane);
        cnt += __popcll(m);
      }
      if (lane == 0) wcnt[wave] = cnt;
      __syncthreads();
      // sum: match j (in wave-list order) goes to wave j % kEmbWaves
      int total = 0;
      for (int w = 0; w < kEmbWaves; ++w) total += wcnt[w];
      for (int j0 = wave; j0 < total; j0 += 4 * kEmbWaves) {
        int64_t tt[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = j0 + u * kEmbWaves;
          tt[u] = -1;
          if (j < total) {
            // locate match j: wave list w holds matches [sum of earlier counts, + wcnt[w])
            int w = 0, base = 0;
            while (j >= base + wcnt[w]) base += wcnt[w++];
            tt[u] = w0 + list[w * kEmbPerWave + (j - base)];
          }
        }
        float xm[4][4], xs[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if constexpr (V4) {
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
            if (tt[u] >= 0 && col < D) {
              a = *reinterpret_cast<const float4*>(dmz + tt[u] * D + col);
              b = *reinterpret_cast<const float4*>(dSz + tt[u] * D + col);
            }
            xm[u][0] = a.x, xm[u][1] = a.y, xm[u][2] = a.z, xm[u][3] = a.w;
            xs[u][0] = b.x, xs[u][1] = b.y, xs[u][2] = b.z, xs[u][3] = b.w;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool ok = tt[u] >= 0 && col + e < D;
              xm[u][e] = ok ? dmz[tt[u] * D + col + e] : 0.f;
              xs[u][e] = ok ? dSz[tt[u] * D + col + e] : 0.f;
            }
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (tt[u] >= 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              am[e] += xm[u][e];
              as[e] += xs[u][e];
            }
          }
      }
      __syncthreads();  // the lists and counts are rewritten by the next window
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      red[(wave * 2 + 0) * 256 + 4 * lane + e] = am[e];
      red[(wave * 2 + 1) * 256 + 4 * lane + e] = as[e];
    }
    __syncthreads();
    if (threadIdx.x < 256) {
      const int d = g0 + (int)threadIdx.x;
      float sm = red[threadIdx.x], ss = red[256 + threadIdx.x];
#pragma unroll
      for (int w = 1; w < kEmbWaves; ++w) {
        sm += red[(w * 2 + 0) * 256 + threadIdx.x];
        ss += red[(w * 2 + 1) * 256 + threadIdx.x];
      }
      if (d < D) {
        const float sw = Sw[cat * D + d];
        dmw[cat * D + d] = sm * sw;
        dSw[cat * D + d] = ss * (sw * sw);
      }
    }
    __syncthreads();
  }
}
}  // namespace

extern "C" int64_t tagi_embedding_bwd_ws_bytes(int64_t n_tokens, int64_t V, int64_t D) {
  (void)n_tokens, (void)V, (void)D;
  return 0;
}

extern "C" int tagi_embedding_bwd(const float* tokens, const float* dmz, const float* dSz, const float* Sw, float* dmw,
                                  float* dSw, int64_t n_tokens, int64_t V, int64_t D, int64_t padding_idx, float* ws,
                                  int64_t ws_bytes, tagi_stream_t stream) {
  const char* what = "tagi_embedding_bwd";
  (void)ws, (void)ws_bytes;
  TAGI_REQUIRE(tokens && dmz && dSz && Sw && dmw && dSw, "%s: null pointer", what);
  TAGI_REQUIRE(n_tokens > 0 && V > 0 && D > 0, "%s: bad sizes", what);
  TAGI_REQUIRE(V < (1ll << 31) && D < (1 << 30) && n_tokens * D < (1ll << 40), "%s: too large", what);
  hipStream_t s = as_stream(stream);
  ProfScope ps(FAM_EMBEDDING, s, 0.0, 4.0 * n_tokens + 8.0 * n_tokens * D + 12.0 * V * D);
  const bool v4 = D % 4 == 0 && al16(dmz) && al16(dSz);
  if (v4)
    hipLaunchKernelGGL(embedding_bwd_kernel<true>, dim3((unsigned)V), dim3(1024), 0, s, tokens, dmz, dSz, Sw, dmw, dSw,
                       n_tokens, (int)D, padding_idx);
  else
    hipLaunchKernelGGL(embedding_bwd_kernel<false>, dim3((unsigned)V), dim3(1024), 0, s, tokens, dmz, dSz, Sw, dmw,
                       dSw, n_tokens, (int)D, padding_idx);
  return check_launch(what);
}
