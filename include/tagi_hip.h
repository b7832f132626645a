/*
 * libtagi_hip — C ABI of the MI355X (gfx950) TAGI step engine.
 *
 * One TAGI training step (forward moments -> output innovation -> backward deltas ->
 * capped parameter update) is built from the entry points below. Every entry point:
 *   - takes raw device pointers to fp32 buffers, int64 sizes and a hipStream_t
 *     (passed as void*; NULL means the null stream);
 *   - queues its kernels on that stream and returns without synchronising;
 *   - never allocates or frees device memory: outputs and workspaces are the caller's;
 *   - returns TAGI_OK (0) or a TAGI_ERR_* code, with a message in tagi_last_error().
 * All tensors are contiguous row-major unless a stride descriptor says otherwise.
 *
 * Each declaration names the reference interface it replaces (file:line in
 * miquelflorensa/triton-tagi).
 */
#ifndef TAGI_HIP_H
#define TAGI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TAGI_ABI_VERSION 5

enum {
  TAGI_OK = 0,
  TAGI_ERR_ARG = 1,         /* bad size, null pointer, or too-small workspace   */
  TAGI_ERR_LAUNCH = 2,      /* hipGetLastError reported a failure after launch  */
  TAGI_ERR_UNSUPPORTED = 3  /* shape outside what the kernels implement         */
};

typedef void* tagi_stream_t; /* a hipStream_t */

/* ---------------------------------------------------------------- housekeeping */
int tagi_abi_version(void);
/* Message of the last failing call on this host thread ("" if none). */
const char* tagi_last_error(void);

/* Orders stream `waiter` after the work queued on `producer` so far (both on one GPU):
 * what is queued on `waiter` after the call starts once that work has finished. The event
 * behind it carries no timing and no system-scope fence, so a fork or join between two
 * streams costs no cache writeback. Also valid while the streams are being captured into
 * a HIP graph (the wait becomes a graph edge). Replaces torch.cuda.Stream.wait_stream for
 * the side stream of the parameter deltas; no counterpart in the reference, whose step
 * runs on one stream (network.py:119-152). */
int tagi_stream_wait(tagi_stream_t waiter, tagi_stream_t producer);

/* Live per-kernel-family timer (HIP events around each launch, on the launch stream).
 * family_mask: bit f enables family f (TAGI_FAM_*). Events are created at begin. */
int tagi_prof_begin(uint64_t family_mask);
/* Waits for the recorded events; fills per-family totals (arrays of TAGI_FAM_COUNT):
 * milliseconds, launches, algorithmic FLOPs and algorithmic bytes. Turns the timer off. */
int tagi_prof_end(double* ms, int64_t* launches, double* flops, double* bytes);
enum {
  TAGI_FAM_CONV_FWD = 0, TAGI_FAM_CONV_BWD_DELTA = 1, TAGI_FAM_CONV_WGRAD = 2,
  TAGI_FAM_LINEAR_FWD = 3, TAGI_FAM_LINEAR_BWD_DELTA = 4, TAGI_FAM_LINEAR_WGRAD = 5,
  TAGI_FAM_BMM_FWD = 6, TAGI_FAM_BMM_SHARED = 7, TAGI_FAM_RELU = 8, TAGI_FAM_REMAX = 9,
  TAGI_FAM_BN_STATS = 10, TAGI_FAM_BN_FWD = 11, TAGI_FAM_BN_BWD = 12, TAGI_FAM_UPDATE = 13,
  TAGI_FAM_INNOVATION = 14, TAGI_FAM_ADD = 15, TAGI_FAM_AVGPOOL = 16, TAGI_FAM_JACOBIAN = 17,
  TAGI_FAM_RMSNORM = 18, TAGI_FAM_EMBEDDING = 19, TAGI_FAM_PE = 20, TAGI_FAM_SPLITK_REDUCE = 21,
  TAGI_FAM_MAXPOOL = 22, TAGI_FAM_LAYERNORM = 23, TAGI_FAM_SOFTPLUS = 24, TAGI_FAM_COUNT = 25
};

/* Ceiling probe (no counterpart in the reference; measurement only): `blocks` blocks of
 * four 64-lane waves, each wave running `iters` rounds of four independent fp32
 * 32x32x2 MFMAs with no memory traffic (16384 flops per wave per round). out receives
 * blocks*256 floats. blocks = 256*w on a 256-CU GPU gives w waves per SIMD. */
int tagi_probe_mfma_loop(float* out, int64_t blocks, int64_t iters, tagi_stream_t stream);

/* Co-issue probe (no counterpart in the reference; measurement only): the loop of
 * tagi_probe_mfma_loop with `per_mfma` (1, 2, 4 or 8) further instructions after every
 * MFMA, independent v_fma_f32 chains (kind 0) or LDS reads (kind 1); the drop in MFMA
 * rate against tagi_probe_mfma_loop is what each such instruction costs the matrix core. */
int tagi_probe_mfma_mix(float* out, int64_t blocks, int64_t iters, int kind, int per_mfma, tagi_stream_t stream);

/* HBM ceiling probe (no counterpart in the reference; measurement only): mode 0 copies n
 * floats src -> dst with float4 loads and stores, mode 1 reads n floats and writes one
 * partial sum per thread (dst holds blocks*256 floats). Grid-stride over `blocks` blocks
 * of 256 threads, 4 float4 loads in flight per thread. n % 4 == 0, 16-byte aligned. */
int tagi_probe_stream(const float* src, float* dst, int64_t n, int64_t blocks, int mode,
                      tagi_stream_t stream);

/* Measurement probe, no counterpart in the reference: variants of tagi_probe_stream to
 * find the best HBM streaming form on this GPU. mode 0 copies n floats src -> dst, 1 reads
 * them (per-thread sums into dst, which must hold blocks * 256 floats), 2 writes dst;
 * unroll 4, 8 or 16 float4 in flight per lane; flags bit 0 nontemporal loads, bit 1
 * nontemporal stores, bit 2 one contiguous chunk per block instead of a grid-stride walk.
 * dst_n is the number of floats dst holds (checked). */
int tagi_probe_stream_variant(const float* src, float* dst, int64_t n, int64_t dst_n, int64_t blocks, int mode,
                              int unroll, int flags, tagi_stream_t stream);

/* ------------------------------------------------------------------ Linear ---- */
/* Fused Linear forward moments, one MFMA pass sharing the A/B tiles:
 *   mz = ma @ mw + mb
 *   Sz = ma^2 @ Sw + Sa @ (mw^2 + Sw) + Sb
 * ma, Sa (M,K); mw, Sw (K,N); mb, Sb (N) or NULL (no bias); mz, Sz (M,N).
 * mz may be NULL: then only Sz is produced (triton_fused_var_forward). Sa may be NULL for a
 * deterministic input (the network input, whose variance the reference passes as zeros,
 * network.py:92-114): the same values with two products instead of three.
 * Replaces linear.py:99-100 (torch.matmul + triton_fused_var_forward, common.py:170). */
int tagi_linear_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw,
                    const float* mb, const float* Sb, float* mz, float* Sz,
                    int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                    tagi_stream_t stream);
int64_t tagi_linear_fwd_ws_bytes(int64_t M, int64_t K, int64_t N);

/* tagi_linear_fwd followed by a ReLU, in one launch: ma_out, Sa_out and J (M,N) receive
 * the moments of ReLU(z) and its Jacobian in place of z's moments, which are not stored;
 * the same bits as tagi_linear_fwd then tagi_relu_fwd. Sa may be NULL as in
 * tagi_linear_fwd. The workspace query is tagi_linear_fwd_ws_bytes. Replaces
 * Linear.forward followed by ReLU.forward (linear.py:83-103, relu.py:94-122). */
int tagi_linear_fwd_relu(const float* ma, const float* Sa, const float* mw, const float* Sw,
                         const float* mb, const float* Sb, float* ma_out, float* Sa_out, float* J,
                         int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                         tagi_stream_t stream);

/* Bytes of the fixed device scratch behind tagi_linear_fwd_noalloc, per GPU. */
#define TAGI_LINEAR_FWD_NOALLOC_SCRATCH_BYTES (128ll << 20)

/* tagi_linear_fwd with no workspace argument that allocates nothing. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The split-K
 * partial sums go to a fixed device array of TAGI_LINEAR_FWD_NOALLOC_SCRATCH_BYTES, alone
 * in a code object of its own: the HIP runtime allocates it on a GPU when it loads that
 * code object there, which with its default deferred loading is this entry point's first
 * call on that GPU (with HIP_ENABLE_DEFERRED_LOADING=0, when the library is loaded), and
 * the GPU keeps it until the process ends. Same plan and kernels
 * as tagi_linear_fwd given its full workspace, so the same results bit for bit; a shape
 * whose partials exceed the scratch returns TAGI_ERR_ARG before launching anything. The
 * stream's device must be the current device. Calls that overlap on one GPU (several
 * streams or host threads) share the scratch and race: serialise them. */
int tagi_linear_fwd_noalloc(const float* ma, const float* Sa, const float* mw, const float* Sw,
                            const float* mb, const float* Sb, float* mz, float* Sz,
                            int64_t M, int64_t K, int64_t N, tagi_stream_t stream);

/* Backward delta propagation:  dma = dmz @ mw^T ;  dSa = dSz @ (mw^2)^T.
 * dmz, dSz (M,N); mw (K,N); dma, dSa (M,K). ws: split-K partials (size from the query).
 * Replaces triton_fused_backward_delta (common.py:287). */
int tagi_linear_bwd_delta(const float* dmz, const float* dSz, const float* mw,
                          float* dma, float* dSa, int64_t M, int64_t K, int64_t N,
                          float* ws, int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_linear_bwd_delta_ws_bytes(int64_t M, int64_t K, int64_t N);

/* tagi_linear_bwd_delta with the Jacobian of the elementwise layer in front (a ReLU's J,
 * laid out like dma) applied in the epilogue: dma = (dmz @ mw^T) * J and
 * dSa = (dSz @ (mw^2)^T) * J^2, the deltas at that layer's input. Equal to
 * tagi_linear_bwd_delta then tagi_jacobian_bwd up to the rounding of the variance's J^2
 * (v * (J * J) here, (v * J) * J there). The workspace query is
 * tagi_linear_bwd_delta_ws_bytes. Replaces triton_fused_backward_delta followed by
 * ReLU.backward (common.py:287, relu.py:152-169). */
int tagi_linear_bwd_delta_jacobian(const float* dmz, const float* dSz, const float* mw, const float* J,
                                   float* dma, float* dSa, int64_t M, int64_t K, int64_t N,
                                   float* ws, int64_t ws_bytes, tagi_stream_t stream);

/* tagi_linear_bwd_delta plus an addend in the epilogue: dma = dmz @ mw^T + add_m,
 * dSa = dSz @ (mw^2)^T + add_S (add_* laid out like dma; they may alias dma/dSa, each
 * element is read and then written by one thread). The workspace query is
 * tagi_linear_bwd_delta_ws_bytes. Replaces one projection's triton_fused_backward_delta
 * plus the sum of the projections' input deltas in MultiheadAttentionV2.backward
 * (multihead_attention.py:262-267). */
int tagi_linear_bwd_delta_add(const float* dmz, const float* dSz, const float* mw,
                              const float* add_m, const float* add_S, float* dma, float* dSa,
                              int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                              tagi_stream_t stream);

/* Parameter deltas of a Linear layer (reduction over the M rows):
 *   gmw = ma^T @ dmz, gSw = (ma^2)^T @ dSz, gmb = sum_rows dmz, gSb = sum_rows dSz
 *   dmw = Sw * gmw, dSw = Sw^2 * gSw, dmb = Sb * gmb, dSb = Sb^2 * gSb
 * Sw == NULL gives the raw gmw/gSw (triton_fused_weight_grad, common.py:410);
 * dmb == NULL skips the bias. ws: split-K partials, size from tagi_linear_wgrad_ws_bytes.
 * Replaces linear.py:138-151. */
int tagi_linear_wgrad(const float* ma, const float* dmz, const float* dSz, const float* Sw,
                      const float* Sb, float* dmw, float* dSw, float* dmb, float* dSb,
                      int64_t M, int64_t K, int64_t N, float* ws, int64_t ws_bytes,
                      tagi_stream_t stream);
int64_t tagi_linear_wgrad_ws_bytes(int64_t M, int64_t K, int64_t N);

/* tagi_linear_wgrad followed by the capped update of the layer's parameters, in one
 * pass: the epilogue that forms each delta also applies
 *   m += sign(dm) min(|dm|, sqrt(max(S, 1e-10)) / cap_factor),
 *   S += sign(dS) min(|dS|, same bound), S <= 0 -> 1e-5
 * to mw, Sw (and mb, Sb with the bias) in place, with the variance before the update in
 * the bound and in the deltas. The deltas are also written to dmw, dSw (dmb, dSb), unless
 * those are all NULL: then they are applied without being stored (half the epilogue's
 * writes). The bias needs mb and Sb together, and dmb, dSb with them when the deltas are
 * stored. mw, Sw, mb, Sb must not overlap the
 * inputs or the delta outputs, and no other work may read them until the call completes
 * (the layer's input-delta product reads mw: run it first). ws: tagi_linear_wgrad_ws_bytes.
 * Replaces linear.py:138-151 followed by the layer's update (parameters.py:58-96,
 * network.py:146-150) for one Linear layer. */
int tagi_linear_wgrad_update(const float* ma, const float* dmz, const float* dSz, float* mw,
                             float* Sw, float* mb, float* Sb, float* dmw, float* dSw, float* dmb,
                             float* dSb, float cap_factor, int64_t M, int64_t K, int64_t N,
                             float* ws, int64_t ws_bytes, tagi_stream_t stream);

/* ------------------------------------------------------- batched products ---- */
/* A strided batched operand: element (z, i, j) of batch z sits at
 *   base + (z / zdiv) * sz1 + (z % zdiv) * sz2 + i * si + j * sj
 * which covers (B,H,S,D) head views of a (B,S,E) tensor and transposed views. */
typedef struct {
  int64_t zdiv, sz1, sz2, si, sj;
} tagi_view;

/* TAGI product of two Gaussian batched matrices, mean and variance in one pass:
 *   mean[z,m,l] = scale    * sum_k mu_a[z,m,k] mu_b[z,k,l]
 *   var [z,m,l] = scale_sq * sum_k ( var_a (mu_b^2 + var_b) + mu_a^2 var_b )
 * mean may be NULL (bmm_tagi_var). Views: a (i=m, j=k), b (i=k, j=l), out (i=m, j=l).
 * Replaces bmm_tagi_var (attention.py:149) plus the mean torch.matmul
 * (multihead_attention.py:180,192). */
int tagi_bmm_tagi(const float* mu_a, const float* var_a, const float* mu_b, const float* var_b,
                  float* mean, float* var, int64_t batch, int64_t M, int64_t K, int64_t L,
                  const tagi_view* va, const tagi_view* vb, const tagi_view* vo, float scale,
                  float scale_sq, tagi_stream_t stream);

/* Batched product with one deterministic operand.
 * shared_left == 0 (bmm_shared_right, attention.py:286):
 *   mean = scale * a_mean @ b ;  var = scale_sq * a_var @ b^2   (a: mean/var, b: shared)
 * shared_left == 1 (bmm_shared_left, attention.py:339):
 *   mean = scale * a @ b_mean ;  var = scale_sq * a^2 @ b_var   (a: shared, b: mean/var)
 * p0/p1 are the mean/var pair of the non-shared side, p2 the shared operand. */
int tagi_bmm_shared(const float* p0, const float* p1, const float* p2, float* mean, float* var,
                    int64_t batch, int64_t M, int64_t K, int64_t L, const tagi_view* va,
                    const tagi_view* vb, const tagi_view* vo, float scale, float scale_sq,
                    int shared_left, tagi_stream_t stream);

/* tagi_bmm_shared followed by an elementwise Jacobian J laid out like the output (view vo):
 *   mean *= J ;  var *= J^2
 * Replaces bmm_shared_right (attention.py:286) and the Remax Jacobian applied to the
 * score deltas in MultiheadAttentionV2.backward (multihead_attention.py:239-243). */
int tagi_bmm_shared_jacobian(const float* p0, const float* p1, const float* p2, const float* J,
                             float* mean, float* var, int64_t batch, int64_t M, int64_t K,
                             int64_t L, const tagi_view* va, const tagi_view* vb,
                             const tagi_view* vo, float scale, float scale_sq, int shared_left,
                             tagi_stream_t stream);

/* The attention scores' moments passed through the Remax in one kernel
 * (multihead_attention.py:174-190: Q K^T by bmm_tagi_var and the scaled mean matmul, then
 * triton_remax over each score row). q/k: rows of ld_qk floats (batch b, position s at row
 * b*S + s), head h at columns h*D .. h*D+D-1 from the given pointers (so the Q, K and V
 * projections may share one (B*S, 3*H*D) buffer), 16-byte aligned, ld_qk % 4 == 0;
 * outputs mu_a, var_a, J: (B, H, S, S) contiguous. The scores are the ones
 * tagi_bmm_tagi forms (scale, scale_sq applied) and the outputs those of
 * tagi_remax_fwd on them, bit for bit, but the scores never reach memory. Needs S <= 256
 * and D in {16, 32, 64} (else TAGI_ERR_UNSUPPORTED: use the two calls). */
int tagi_attn_scores_remax(const float* mu_q, const float* var_q, const float* mu_k, const float* var_k,
                           int64_t ld_qk, float* mu_a, float* var_a, float* J, int64_t B, int64_t H, int64_t S,
                           int64_t D, float scale, float scale_sq, tagi_stream_t stream);

/* The attention forward of one layer in one kernel (multihead_attention.py:174-193): the
 * scores and their Remax as tagi_attn_scores_remax forms them (bit for bit), then
 *   out = mu_a @ mu_v,   out_var = mu_a^2 @ var_v + var_a @ (mu_v^2 + var_v)
 * (the score @ V TAGI product of tagi_bmm_tagi with scale 1), written into out_m / out_S:
 * rows of ld_out floats (batch b, position s at row b*S + s), head h at columns h*D ...
 * q/k/v as in tagi_attn_scores_remax (row stride ld_qkv; v needs no alignment). mu_a and J
 * (B, H, S, S) are written for the backward pass; var_a may be NULL (then the score
 * variances never reach memory; tagi_attn_scores_remax rebuilds them). Needs S <= 256
 * and D in {16, 32} (else TAGI_ERR_UNSUPPORTED: use tagi_attn_scores_remax and
 * tagi_bmm_tagi). The score @ V sums run in another order than tagi_bmm_tagi's (per
 * 32-key stretch, then over the stretches), so out / out_var agree with it to rounding. */
int tagi_attn_fwd(const float* mu_q, const float* var_q, const float* mu_k, const float* var_k, const float* mu_v,
                  const float* var_v, int64_t ld_qkv, float* mu_a, float* var_a, float* J, float* out_m,
                  float* out_S, int64_t ld_out, int64_t B, int64_t H, int64_t S, int64_t D, float scale,
                  float scale_sq, tagi_stream_t stream);

/* The attention's query or key deltas from the output deltas in one kernel
 * (multihead_attention.py:238-251): with scaled = (d_out @ mu_v^T) x J (mean; the variance
 * is (d_var @ (mu_v^2)^T) x J^2, as tagi_bmm_shared_jacobian forms it),
 *   transpose == 0:  out = scale * scaled @ mu_x,   out_var = scale_sq * scaled_var @ mu_x^2  (dQ, mu_x = mu_k)
 *   transpose == 1:  out = scale * scaled^T @ mu_x, ...                                      (dK, mu_x = mu_q)
 * Rows as in tagi_attn_scores_remax: d_mu, d_var with row stride ld_d, mu_v and mu_x ld_x,
 * out ld_out (head h at columns h*D ..); J: (B, H, S, S). The scaled deltas are formed
 * per block in LDS and never reach memory. Needs S <= 256, D in {16, 32}, 16-byte
 * aligned d_mu, d_var, mu_v and ld_d, ld_x multiples of 4 (else TAGI_ERR_UNSUPPORTED /
 * TAGI_ERR_ARG: use tagi_bmm_shared_jacobian and tagi_bmm_shared). */
int tagi_attn_score_deltas_qk(const float* d_mu, const float* d_var, int64_t ld_d, const float* mu_v,
                              const float* mu_x, int64_t ld_x, const float* J, float* out_mu, float* out_var,
                              int64_t ld_out, int64_t B, int64_t H, int64_t S, int64_t D, float scale,
                              float scale_sq, int transpose, tagi_stream_t stream);

/* The query and the key deltas of tagi_attn_score_deltas_qk in one launch
 * (multihead_attention.py:239-260, replacing its two bmm_shared_right calls after the
 * score-delta product): one block per (batch, head) forms the Jacobian-scaled score deltas
 * of each block of 32 query rows once, writes that block's query deltas and accumulates the
 * key deltas over the query blocks in order. dq_* = tagi_attn_score_deltas_qk(transpose 0)
 * bit for bit; dk_* its transpose-1 values up to the order of the fp32 sums. mu_q and mu_k
 * have row stride ld_x; the outputs row stride ld_out. S <= 256, D in {16, 32}. */
int tagi_attn_score_deltas_qk_joint(const float* d_mu, const float* d_var, int64_t ld_d, const float* mu_v,
                                    const float* mu_q, const float* mu_k, int64_t ld_x, const float* J,
                                    float* dq_mu, float* dq_var, float* dk_mu, float* dk_var, int64_t ld_out,
                                    int64_t B, int64_t H, int64_t S, int64_t D, float scale, float scale_sq,
                                    tagi_stream_t stream);

/* ------------------------------------------------------------------ Conv2D ---- */
/* 4-D activations and deltas of the conv path (Conv2D, BatchNorm2D, AvgPool2D) are
 * channels-last: element (n, c, h, w) of an (N, C, H, W) tensor sits at ((n*H + h)*W + w)*C + c
 * (torch.channels_last). Weights keep the reference layout.
 *
 * Geometry of a square-kernel 2-D convolution. pad_top/pad_left are the
 * zero rows/cols before the image; rows/cols past H/W read as zero. padding_type 1
 * (symmetric p) is pad_top = pad_left = p, Ho = (H + 2p - k)/s + 1; padding_type 2
 * (right/bottom only, conv2d.py:280-291) is pad_top = pad_left = 0, Ho = (H + p - k)/s + 1. */
typedef struct {
  int64_t N, C, H, W, Cout, k, stride, pad_top, pad_left, Ho, Wo;
} tagi_conv_geom;

/* Implicit-GEMM forward: patches are gathered into LDS, never materialised.
 *   mz = P(ma) @ mw + mb ; Sz = P(ma)^2 @ Sw + P(Sa) @ (mw^2 + Sw) + Sb (channels-last).
 * mw, Sw (C*k*k, Cout) with rows ordered (c, kh, kw); mb, Sb (Cout). Sa may be NULL for a
 * deterministic input (zero variance, as the network input): two products instead of three.
 * Replaces Conv2D.forward (conv2d.py:254-309: im2col + matmul + fused var + permute). */
int tagi_conv2d_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw,
                    const float* mb, const float* Sb, float* mz, float* Sz,
                    const tagi_conv_geom* g, float* ws, int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_conv2d_fwd_ws_bytes(const tagi_conv_geom* g);

/* tagi_conv2d_fwd followed by the first pass of ReLU -> BatchNorm2D on its output
 * (conv2d.py:254-309, relu.py:135-140, batchnorm2d.py:307-355): mz, Sz as tagi_conv2d_fwd,
 * then J, the batch statistics and the running-stat / gamma bookkeeping as
 * tagi_relu_bn_stats on (mz, Sz). Where the GEMM runs unsplit its epilogue forms J and
 * the per-tile channel sums, so the output is not read back. Sa may be NULL as for
 * tagi_conv2d_fwd. ws: 16-byte aligned, size from tagi_conv2d_fwd_relu_bn_stats_ws_bytes. */
int tagi_conv2d_fwd_relu_bn_stats(const float* ma, const float* Sa, const float* mw, const float* Sw,
                                  const float* mb, const float* Sb, float* mz, float* Sz,
                                  const tagi_conv_geom* g, float* J, float* batch_mean,
                                  float* batch_var, float* running_mean, float* running_var,
                                  float* mg, float momentum, float eps, int first_call,
                                  int preserve_var, float* ws, int64_t ws_bytes,
                                  tagi_stream_t stream);
int64_t tagi_conv2d_fwd_relu_bn_stats_ws_bytes(const tagi_conv_geom* g);

/* Transposed implicit GEMM for the input deltas (no patch matrix, no col2im):
 *   dma = fold(dmz_rows @ mw^T), dSa = fold(dSz_rows @ (mw^2)^T), channels-last (N,C,H,W).
 * Split by stride phase: each phase multiplies only the kernel taps that reach it.
 * ws holds the transposed weights (+ split-K partials); size from the query.
 * Replaces conv2d.py:357-370 (fused backward delta + col2im + crop). */
int tagi_conv2d_bwd_delta(const float* dmz, const float* dSz, const float* mw, float* dma,
                          float* dSa, const tagi_conv_geom* g, float* ws, int64_t ws_bytes,
                          tagi_stream_t stream);
int64_t tagi_conv2d_bwd_delta_ws_bytes(const tagi_conv_geom* g);

/* tagi_conv2d_bwd_delta plus an addend of the output's layout and shape:
 *   dma = fold(...) + add_m, dSa = fold(...) + add_S
 * (the input deltas of a residual block's first convolution merged with the deltas of the
 * shortcut branch in the same pass). Workspace as tagi_conv2d_bwd_delta.
 * Replaces conv2d.py:357-370 followed by triton_delta_merge (resblock.py:157, 421-423). */
int tagi_conv2d_bwd_delta_add(const float* dmz, const float* dSz, const float* mw, const float* add_m,
                              const float* add_S, float* dma, float* dSa, const tagi_conv_geom* g,
                              float* ws, int64_t ws_bytes, tagi_stream_t stream);
/* tagi_conv2d_bwd_delta followed by the backward of the BatchNorm2D and the ReLU in front
 * of the convolution (the layer order conv_prev -> ReLU -> BatchNorm2D -> this conv), in the
 * GEMM's epilogue: the products (deltas at the BatchNorm2D output) never reach memory.
 * dma/dSa receive the deltas at the ReLU input, the values tagi_bn_relu_bwd_partials_bias
 * writes for them (batchnorm2d.py:465-513, relu.py:152-169); part receives per-tile sums of
 * the six quantities that call's ws holds, for tagi_bn_bwd_finalize_multi (with nblk =
 * part_bytes / (24 C) and the conv_prev bias fields). mhat, J: the BatchNorm2D's saved
 * normalised input and the ReLU's Jacobian, laid out like dma; var, mg: the normalisation
 * variance and gamma means (C). Needs stride 1 and an unsplit plan:
 * tagi_conv2d_bwd_delta_bn_relu_part_bytes returns the partial-sum bytes, 0 when the fold
 * does not apply (then TAGI_ERR_UNSUPPORTED: use the two calls). ws as for
 * tagi_conv2d_bwd_delta. */
int tagi_conv2d_bwd_delta_bn_relu(const float* dmz, const float* dSz, const float* mw, const float* mhat,
                                  const float* J, const float* var, const float* mg, float eps, float* dma,
                                  float* dSa, float* part, int64_t part_bytes, const tagi_conv_geom* g, float* ws,
                                  int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_conv2d_bwd_delta_bn_relu_part_bytes(const tagi_conv_geom* g);
/* tagi_conv2d_bwd_delta_add followed by the same fold, across a residual block boundary:
 * dma/dSa = product + addend as tagi_conv2d_bwd_delta_add stores them (the deltas at the
 * output of the block in front, which its shortcut reads again), and dmz_prev/dSz_prev the
 * deltas at the input of that block's closing ReLU (or the stem's), the values
 * tagi_bn_relu_bwd_partials_bias writes for dma/dSa; part, mhat, J, var, mg as for
 * tagi_conv2d_bwd_delta_bn_relu, with the same size query and the same
 * TAGI_ERR_UNSUPPORTED where it does not apply. dma may alias add_m (dSa add_S).
 * Replaces conv2d.py:357-370, triton_delta_merge (resblock.py:421-423) and the next
 * block's BatchNorm2D -> ReLU backward (batchnorm2d.py:465-513, relu.py:152-169). */
int tagi_conv2d_bwd_delta_add_bn_relu(const float* dmz, const float* dSz, const float* mw, const float* add_m,
                                      const float* add_S, float* dma, float* dSa, const float* mhat,
                                      const float* J, const float* var, const float* mg, float eps,
                                      float* dmz_prev, float* dSz_prev, float* part, int64_t part_bytes,
                                      const tagi_conv_geom* g, float* ws, int64_t ws_bytes,
                                      tagi_stream_t stream);

/* Parameter deltas of a Conv2D layer (reduction over N*Ho*Wo patches, split-K):
 *   dmw = Sw * P^T @ dmz, dSw = Sw^2 * (P^2)^T @ dSz, dmb = Sb * sum dmz, dSb = Sb^2 * sum dSz.
 * Replaces conv2d.py:341-354. */
int tagi_conv2d_wgrad(const float* ma, const float* dmz, const float* dSz, const float* Sw,
                      const float* Sb, float* dmw, float* dSw, float* dmb, float* dSb,
                      const tagi_conv_geom* g, float* ws, int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_conv2d_wgrad_ws_bytes(const tagi_conv_geom* g);

/* ------------------------------------------------------------- elementwise ---- */
/* Rectified-Gaussian moments: ma, Sa, J = Phi(alpha) (Phi ~ pdf/(-alpha) for alpha < -5).
 * Replaces bayesian_relu / _bayesian_relu_kernel (relu.py:43-122). */
int tagi_relu_fwd(const float* mz, const float* Sz, float* ma, float* Sa, float* J, int64_t n,
                  tagi_stream_t stream);

/* Jacobian backward shared by ReLU and Remax: dm_out = dm * J, dS_out = dS * J^2.
 * Replaces relu.py:152-169 and remax.py:185-188. */
int tagi_jacobian_bwd(const float* dm, const float* dS, const float* J, float* dm_out,
                      float* dS_out, int64_t n, tagi_stream_t stream);

/* Remax over the last dim of a (rows, K) tensor: mu_a, var_a, J.
 * Replaces triton_remax / _remax_kernel (remax.py:33-159). */
int tagi_remax_fwd(const float* mz, const float* Sz, float* ma, float* Sa, float* J,
                   int64_t rows, int64_t K, tagi_stream_t stream);

/* Dense output innovation: dm = (y - mu)/(var + sv2), dS = -1/(var + sv2).
 * Replaces compute_innovation / _output_innovation_kernel (observation.py:24-46,119-163). */
int tagi_innovation(const float* y, const float* mu, const float* var, float sigma_v2,
                    float* dm, float* dS, int64_t n, tagi_stream_t stream);

/* In-place capped update (both caps use the pre-update S):
 *   bar = sqrt(max(S,1e-10))/cap; m += sign(dm) min(|dm|,bar);
 *   S' = S + sign(dS) min(|dS|,bar); S = S' <= 0 ? 1e-5 : S'.
 * Replaces update_parameters / _capped_param_update_kernel (parameters.py:58-128). */
int tagi_capped_update(float* m, float* S, const float* dm, const float* dS, float cap_factor,
                       int64_t n, tagi_stream_t stream);

/* Many capped updates in one launch: tensor t has n[t] elements at m[t], S[t], dm[t], dS[t].
 * The pointer/size tables live in host memory and are copied into the kernel arguments
 * (at most 64 tensors per call). Same arithmetic as tagi_capped_update. */
int tagi_capped_update_multi(float* const* m, float* const* S, const float* const* dm,
                             const float* const* dS, const int64_t* n, int64_t count,
                             float cap_factor, tagi_stream_t stream);

/* In-place moment add: mu_a += mu_s ; var_a += var_s.
 * Replaces triton_add_shortcut and triton_delta_merge (resblock.py:138,157). */
int tagi_add_inplace(const float* mu_s, const float* var_s, float* mu_a, float* var_a, int64_t n,
                     tagi_stream_t stream);

/* Non-overlapping k x k average pool of channels-last moments: mean scaled by 1/k^2,
 * variance by var_scale (1/k^4 default, 1/k^2 with spatial_correlation); input pixels past
 * the last full window get zero deltas. Replaces avgpool2d.py:38-130. */
int tagi_avgpool2d_fwd(const float* ma, const float* Sa, float* ma_out, float* Sa_out, int64_t N,
                       int64_t C, int64_t H, int64_t W, int64_t k, float var_scale,
                       tagi_stream_t stream);
int tagi_avgpool2d_bwd(const float* dm, const float* dS, float* dm_out, float* dS_out, int64_t N,
                       int64_t C, int64_t H, int64_t W, int64_t k, float var_scale,
                       tagi_stream_t stream);

/* ReLU followed by the average pool above, in one pass over the channels-last (N, C, H, W)
 * input moments mz, Sz: writes the ReLU Jacobian J (N, C, H, W) and the pooled moments
 * (N, C, H/k, W/k), channels-last, or row-major NCHW with pooled_nchw != 0 (what a
 * following Flatten, flatten.py:25-53, reads as a plain view); the ReLU output is not
 * written. The same values, bit for bit, as tagi_relu_fwd followed by tagi_avgpool2d_fwd.
 * H and W multiples of k (else TAGI_ERR_UNSUPPORTED). Replaces relu.py:94-122 followed
 * by avgpool2d.py:38-90. */
int tagi_relu_avgpool2d_fwd(const float* mz, const float* Sz, float* J, float* ma_out,
                            float* Sa_out, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k,
                            float var_scale, int pooled_nchw, tagi_stream_t stream);
/* The backward of that pair: pooled deltas dm, dS (N, C, H/k, W/k; channels-last, or
 * row-major NCHW with pooled_nchw != 0) and the stored J give the deltas at the ReLU input
 * (N, C, H, W, channels-last), bit for bit tagi_avgpool2d_bwd followed by
 * tagi_jacobian_bwd. Replaces avgpool2d.py:92-130 followed by relu.py:152-169. */
int tagi_avgpool2d_relu_bwd(const float* dm, const float* dS, const float* J, float* dm_out,
                            float* dS_out, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k,
                            float var_scale, int pooled_nchw, tagi_stream_t stream);

/* ----------------------------------------------------------- BatchNorm2D ---- */
/* Per-channel batch statistics of channels-last moments (batchnorm2d.py:307-339):
 *   mean_c = E[mu], var_c = (E[S] + E[mu^2] - mean_c^2) * n/(n-1), n = N*H*W,
 * and the running-stat / gamma bookkeeping of batchnorm2d.py:341-355:
 *   first_call: running := batch, and if preserve_var: mg := sqrt(var + eps);
 *   otherwise running := (1-momentum) running + momentum batch.
 * ws: per-block partial sums, size from tagi_bn_stats_ws_bytes. */
int tagi_bn_stats(const float* mz, const float* Sz, float* batch_mean, float* batch_var,
                  float* running_mean, float* running_var, float* mg, int64_t N, int64_t C,
                  int64_t HW, float momentum, float eps, int first_call, int preserve_var,
                  float* ws, int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_bn_stats_ws_bytes(int64_t N, int64_t C, int64_t HW);

/* Normalise + Gaussian affine (batchnorm2d.py:59-126):
 *   mhat = (mu - mean)/sqrt(var+eps), Shat = S/(var+eps),
 *   ma = mg mhat + mb, Sa = mg^2 Shat + Sg (mhat^2 + Shat) + Sb.  Shat may be NULL. */
int tagi_bn_fwd(const float* mz, const float* Sz, const float* mean, const float* var,
                const float* mg, const float* Sg, const float* mb, const float* Sb, float* ma,
                float* Sa, float* mhat, float* Shat, int64_t N, int64_t C, int64_t HW, float eps,
                tagi_stream_t stream);

/* Backward (batchnorm2d.py:134-192, 465-513): dmz = dma mg/sqrt(var+eps),
 * dSz = dSa mg^2/(var+eps), and the parameter deltas
 * dmg = Sg sum(dma mhat), dSg = Sg^2 sum(dSa mhat^2), dmb = Sb sum dma, dSb = Sb^2 sum dSa. */
int tagi_bn_bwd(const float* dma, const float* dSa, const float* mhat, const float* var,
                const float* mg, const float* Sg, const float* Sb, float* dmz, float* dSz,
                float* dmg, float* dSg, float* dmb, float* dSb, int64_t N, int64_t C, int64_t HW,
                float eps, float* ws, int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_bn_bwd_ws_bytes(int64_t N, int64_t C, int64_t HW);

/* ReLU followed by BatchNorm2D (relu.py:135-140, then batchnorm2d.py:307-355), first pass:
 * the batch statistics of the rectified moments of (mz, Sz), with the same running-stat /
 * gamma bookkeeping as tagi_bn_stats, and J = Phi(alpha) for the ReLU backward. The
 * rectified moments themselves are not stored. ws: size from tagi_bn_stats_ws_bytes. */
int tagi_relu_bn_stats(const float* mz, const float* Sz, float* J, float* batch_mean, float* batch_var,
                       float* running_mean, float* running_var, float* mg, int64_t N, int64_t C,
                       int64_t HW, float momentum, float eps, int first_call, int preserve_var,
                       float* ws, int64_t ws_bytes, tagi_stream_t stream);

/* ReLU followed by BatchNorm2D, second pass: recomputes the rectified moments of (mz, Sz)
 * and normalises them as tagi_bn_fwd (Shat not stored). When add_m/add_S are given the
 * Gaussian stream (add_m, add_S) is added to the output: the residual add that closes a
 * block (resblock.py:380, triton_add_shortcut resblock.py:138). */
int tagi_relu_bn_fwd(const float* mz, const float* Sz, const float* mean, const float* var,
                     const float* mg, const float* Sg, const float* mb, const float* Sb,
                     const float* add_m, const float* add_S, float* ma, float* Sa, float* mhat,
                     int64_t N, int64_t C, int64_t HW, float eps, tagi_stream_t stream);

/* BatchNorm2D backward followed by the Jacobian of the ReLU in front of it
 * (batchnorm2d.py:134-192 then relu.py:152-169):
 *   dmz = (dma mg/sqrt(var+eps)) J,  dSz = (dSa mg^2/(var+eps)) J^2,
 * parameter deltas as tagi_bn_bwd. ws: size from tagi_bn_bwd_ws_bytes. */
int tagi_bn_relu_bwd(const float* dma, const float* dSa, const float* mhat, const float* J,
                     const float* var, const float* mg, const float* Sg, const float* Sb, float* dmz,
                     float* dSz, float* dmg, float* dSg, float* dmb, float* dSb, int64_t N, int64_t C,
                     int64_t HW, float eps, float* ws, int64_t ws_bytes, tagi_stream_t stream);

/* tagi_bn_relu_bwd without the parameter-delta pass: dmz/dSz are written and the
 * per-channel partial sums are left in ws (size from tagi_bn_bwd_ws_bytes), which must
 * stay untouched until tagi_bn_bwd_finalize_multi has consumed them. Together the two
 * replace batchnorm2d.py:465-513 + relu.py:152-169 for a whole network's BatchNorm2D
 * layers with one parameter-delta launch. */
int tagi_bn_relu_bwd_partials(const float* dma, const float* dSa, const float* mhat,
                              const float* J, const float* var, const float* mg, float* dmz,
                              float* dSz, int64_t N, int64_t C, int64_t HW, float eps, float* ws,
                              int64_t ws_bytes, tagi_stream_t stream);

/* tagi_bn_relu_bwd_partials that also leaves the per-channel sums of its outputs dmz and
 * dSz in ws: the bias sums of the Conv2D whose output feeds the ReLU (conv2d.py:341-354,
 * the column sums of its output deltas), so that Conv2D's parameter-delta GEMM needs no
 * bias row. ws: size from tagi_bn_relu_bwd_bias_ws_bytes (six sums per channel). */
int tagi_bn_relu_bwd_partials_bias(const float* dma, const float* dSa, const float* mhat,
                                   const float* J, const float* var, const float* mg, float* dmz,
                                   float* dSz, int64_t N, int64_t C, int64_t HW, float eps, float* ws,
                                   int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_bn_relu_bwd_bias_ws_bytes(int64_t N, int64_t C, int64_t HW);

/* One layer left pending by tagi_bn_relu_bwd_partials(_bias) or
 * tagi_conv2d_bwd_delta_bn_relu: its partial sums (ws) and sizes, the gamma/beta variances
 * and the four parameter-delta outputs of length C; for a layer left by the _bias variant
 * or the conv fold also the conv's bias variances cSb and its two bias delta outputs (all
 * three NULL otherwise); nblk: partial sums per channel and quantity (0: the count
 * tagi_bn_relu_bwd_partials uses for N*HW rows; the conv fold's is its part_bytes / (24 C)). */
typedef struct {
  const float* ws;
  const float* Sg;
  const float* Sb;
  float* dmg;
  float* dSg;
  float* dmb;
  float* dSb;
  int64_t N, C, HW;
  const float* cSb;
  float* cdmb;
  float* cdSb;
  int64_t nblk;
} tagi_bn_bwd_pending;

/* The parameter deltas of count pending layers, in one launch per 32 layers:
 *   dmg = Sg * sum(dmu mhat), dSg = Sg^2 * sum(dS mhat^2), dmb = Sb * sum(dmu), dSb = Sb^2 * sum(dS);
 * with conv bias outputs also cdmb = cSb * sum(dmz), cdSb = cSb^2 * sum(dSz). */
int tagi_bn_bwd_finalize_multi(const tagi_bn_bwd_pending* items, int64_t count, tagi_stream_t stream);

/* -------------------------------------------------- RMSNorm / Embedding / PE ---- */
/* RMSNorm forward over rows of length D (rms_norm.py:93-110); inv_rms (rows) is cached. */
int tagi_rmsnorm_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw,
                     float* mz, float* Sz, float* inv_rms, int64_t rows, int64_t D, float eps,
                     tagi_stream_t stream);
/* RMSNorm backward (rms_norm.py:115-134): propagated deltas and gamma deltas. */
int tagi_rmsnorm_bwd(const float* dmz, const float* dSz, const float* ma, const float* inv_rms,
                     const float* mw, const float* Sw, float* dma, float* dSa, float* dmw,
                     float* dSw, int64_t rows, int64_t D, float* ws, int64_t ws_bytes,
                     tagi_stream_t stream);
int64_t tagi_rmsnorm_bwd_ws_bytes(int64_t rows, int64_t D);

/* Embedding lookup (embedding.py:88-106): tokens are float ids (cast toward zero).
 * Rows equal to padding_idx (>= 0) emit zeros. */
int tagi_embedding_fwd(const float* tokens, const float* mw, const float* Sw, float* mz,
                       float* Sz, int64_t n_tokens, int64_t V, int64_t D, int64_t padding_idx,
                       tagi_stream_t stream);
/* Embedding deltas (embedding.py:111-150): dmw[cat] = sum dm Sw[cat], dSw[cat] = sum dS Sw[cat]^2
 * over the tokens of each category; dmw/dSw (V,D) are overwritten. One block per category
 * finds its tokens from ballots of the ids and sums their delta rows in an order fixed by
 * the ids (deterministic). ws is not used (tagi_embedding_bwd_ws_bytes returns 0; kept so
 * that callers sizing a workspace keep working). */
int tagi_embedding_bwd(const float* tokens, const float* dmz, const float* dSz, const float* Sw,
                       float* dmw, float* dSw, int64_t n_tokens, int64_t V, int64_t D,
                       int64_t padding_idx, float* ws, int64_t ws_bytes, tagi_stream_t stream);
int64_t tagi_embedding_bwd_ws_bytes(int64_t n_tokens, int64_t V, int64_t D);

/* Sinusoidal positional encoding add (positional_encoding.py:62): out = ma + pe[:S]. */
int tagi_pe_add(const float* ma, const float* pe, float* out, int64_t B, int64_t S, int64_t E,
                tagi_stream_t stream);

/* ------------------------------------------------- output heads and further layers */
/* Sparse (hierarchical-softmax) innovation. Replaces compute_innovation_with_indices
 * (observation.py:171-224). ma, Sa, dm, dS: (rows, n_out); y_obs, var_obs: (rows, n_obs)
 * fp32; idx: (rows, n_obs) int32, 1-indexed nodes. dm/dS are overwritten: zero except at
 * the selected nodes, where (y - ma)/(Sa + v) and -1/(Sa + v) are added per bit (a node
 * selected twice receives both). Indices outside [1, n_out] select nothing. */
int tagi_innovation_indexed(const float* ma, const float* Sa, const float* y_obs, const float* var_obs,
                            const int32_t* idx, float* dm, float* dS, int64_t rows, int64_t n_out,
                            int64_t n_obs, tagi_stream_t stream);
/* The same from integer class labels: row b uses the class tables obs/idx (n_classes, n_obs)
 * at labels[b] and the noise variance sigma_v2. Replaces labels_to_hrc + full_like +
 * compute_innovation_with_indices inside Sequential.step_hrc (network.py:157-224,
 * hrc_softmax.py:131-150). A label outside [0, n_classes) makes its row of dm/dS NaN. */
int tagi_hrc_innovation(const float* ma, const float* Sa, const int64_t* labels, const float* obs,
                        const int32_t* idx, float sigma_v2, float* dm, float* dS, int64_t rows,
                        int64_t n_out, int64_t n_obs, int64_t n_classes, tagi_stream_t stream);
/* Class probabilities of a hierarchical-softmax output (hrc_softmax.py:164-208):
 * probs[b, r] = prod_c (obs[r,c] > 0 ? P : 1 - P), P = Phi(ma/sqrt(1/alpha^2 + Sa)) at node
 * idx[r,c]-1 of row b. probs: (rows, n_classes). pred (optional, may be NULL): int64 (rows,)
 * first index of the largest probability (get_predicted_labels, hrc_softmax.py:211-231). */
int tagi_hrc_class_probs(const float* ma, const float* Sa, const float* obs, const int32_t* idx,
                         float alpha, float* probs, int64_t* pred, int64_t rows, int64_t n_out,
                         int64_t n_obs, int64_t n_classes, tagi_stream_t stream);
/* Heteroscedastic (TAGI-V) innovation: y has n elements; mu/var/dm/dS have 2n, interleaved
 * (mean, noise-variance) pairs. Replaces _output_innovation_kernel_heteros
 * (observation.py:49-111) and the 2x-wide dispatch of compute_innovation (:137). */
int tagi_innovation_heteros(const float* y, const float* mu, const float* var, float* dm,
                            float* dS, int64_t n, tagi_stream_t stream);
/* EvenSoftplus forward (even_softplus.py:38-124): softplus moments at odd flat positions,
 * identity at even ones; J = sigmoid(mu) or 1. The backward pass is tagi_jacobian_bwd. */
int tagi_even_softplus_fwd(const float* mz, const float* Sz, float* ma, float* Sa, float* J,
                           int64_t n, tagi_stream_t stream);
/* MaxPool2D, hard argmax of the means (maxpool2d.py:62-126). Tensors (N, C, H, W), all
 * NCHW or all channels-last (channels_last != 0); output (N, C, Ho, Wo), Ho = (H + 2 pad -
 * k)/stride + 1; pool_idx int32 (output layout) holds h*W + w of each pick. Needs
 * 0 <= pad <= k/2. */
int tagi_maxpool2d_fwd(const float* ma, const float* Sa, float* mz, float* Sz, int32_t* pool_idx,
                       int64_t N, int64_t C, int64_t H, int64_t W, int64_t k, int64_t stride,
                       int64_t pad, int channels_last, tagi_stream_t stream);
/* MaxPool2D deltas: each input position receives the sum of the output deltas whose window
 * picked it (scatter_add at maxpool2d.py:100-126); dma/dSa (N, C, H, W) are overwritten. */
int tagi_maxpool2d_bwd(const float* dmz, const float* dSz, const int32_t* pool_idx, float* dma,
                       float* dSa, int64_t N, int64_t C, int64_t H, int64_t W, int64_t k,
                       int64_t stride, int64_t pad, int channels_last, tagi_stream_t stream);
/* LayerNorm forward over the last dimension (layernorm.py:101-135): rows x D; writes the
 * per-row mean mu_ra and Bessel-corrected variance var_ra (rows,) used by the backward. */
int tagi_layernorm_fwd(const float* ma, const float* Sa, const float* mw, const float* Sw,
                       const float* mb, const float* Sb, float* mz, float* Sz, float* mu_ra,
                       float* var_ra, int64_t rows, int64_t D, float eps, tagi_stream_t stream);
/* LayerNorm deltas (layernorm.py:140-175): dma = J dmz, dSa = J^2 dSz with J = mw/sqrt(var_ra +
 * eps); dmw/dSw/dmb/dSb (D,) overwritten with the parameter deltas. ws from
 * tagi_layernorm_bwd_ws_bytes (deterministic two-stage column sums). */
int tagi_layernorm_bwd(const float* dmz, const float* dSz, const float* ma, const float* mu_ra,
                       const float* var_ra, const float* mw, const float* Sw, const float* Sb,
                       float* dma, float* dSa, float* dmw, float* dSw, float* dmb, float* dSb,
                       int64_t rows, int64_t D, float eps, float* ws, int64_t ws_bytes,
                       tagi_stream_t stream);
int64_t tagi_layernorm_bwd_ws_bytes(int64_t rows, int64_t D);

#ifdef __cplusplus
}
#endif
#endif /* TAGI_HIP_H */
