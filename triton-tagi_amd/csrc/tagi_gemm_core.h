// fp32-MFMA moment GEMMs for gfx950 (CDNA4): Linear, Conv2D (implicit GEMM on NHWC
// activations) and the batched attention products all run through one templated kernel.
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
// LDS tiles are double-buffered and the global loads run two k-tiles ahead: while the
// MFMAs consume tile t, tile t+2 is in flight and tile t+1 is stored to the other LDS
// buffer; one barrier per k-tile.
//
// Operand loaders read the caller's tensors in place -- strided views (Linear, attention
// heads, transposes) or the NHWC convolution index maps (patches, transposed patches,
// pre-transposed weights) -- with float4 accesses along whichever dim is contiguous.
// No im2col / col2im buffer exists anywhere.
#pragma once
#include <float.h>

#include <type_traits>

#include "tagi_common.h"
#include "tagi_moments.h"

namespace tagi {

typedef float floatx16 __attribute__((ext_vector_type(16)));

enum { PROD_FWD = 0, PROD_SHARED_B = 1, PROD_SHARED_A = 2 };

// Loader kinds ("MN": consecutive threads walk the tile's row/col dim, float4 along it;
// "K": consecutive threads walk the reduction, float4 along it; "S": scalar element gather).
enum {
  LD_STR_MN4 = 0,     // p[zoff + mn + k*s_k]                   (s_mn == 1)
  LD_STR_K4 = 1,      // p[zoff + mn*s_mn + k]                  (s_k == 1)
  LD_STR_MN_S = 2,    // p[zoff + mn*s_mn + k*s_k], scalar, mn-fast
  LD_STR_K_S = 3,     // same, k-fast
  LD_CFWD_A4 = 4,     // conv fwd patches: mn = out pixel m, k = (kh,kw,c)  (NHWC, C%4==0)
  LD_CFWD_A_S = 5,    //   scalar version (any C)
  LD_CFWD_B4 = 6,     // conv fwd weights: mn = co, k = (kh,kw,c): w[(c*kk2 + kh*kk + kw)*Cout + co]
  LD_CBWD_A4 = 7,     // conv input delta: mn = phase pixel q, k = (ikh,ikw,co): dy[n,oh,ow,co]
  LD_CBWD_A_S = 8,    //   scalar version
  LD_CBWD_B4 = 9,     // transposed weights wt[((kh*kk+kw)*Cout + co)*C + c]: mn = c, k = (ikh,ikw,co)
  LD_CBWD_B_S = 10,   //   scalar version
  LD_CWG_A4 = 11,     // conv weight delta patches: mn = (kh,kw,c) [+ ones row], k = out pixel m
  LD_CWG_A_S = 12,    //   scalar version
  LD_CFWD_B_S = 13,   // conv fwd weights, scalar (any Cout)
  LD_CBWD_BK4 = 14,   // input-delta weights read in place, w[((c*kk + kh)*kk + kw)*Cout + co]:
                      //   mn = c, k = (ikh,ikw,co), float4 along co (Cout % 4 == 0)
  // Tile-aligned conv kinds: the same index maps as LD_CFWD_A4 / LD_CFWD_B4 / LD_CBWD_A4 /
  // LD_CBWD_BK4 / LD_CWG_A4 for geometries where a 16-wide k tile never straddles a kernel
  // tap (C % 16 == 0, or Cout % 16 == 0 for the input delta) or an image (the weight
  // delta: Ho*Wo % 16 == 0 and Wo a multiple or a divisor of 16). The tile's tap (or
  // image and output position) is then the same for every lane, so it is decoded once in
  // scalar registers and each lane adds a constant formed at block start; a lane's
  // padding test is one bit of a per-lane mask over the taps (kk <= 5).
  LD_CFWD_A4T = 17,
  LD_CFWD_B4T = 18,
  LD_CBWD_A4T = 19,
  LD_CBWD_BK4T = 20,
  LD_CWG_A4T = 21,
};

template <int KIND>
struct KindTraits {
  static constexpr bool mn_fast = (KIND == LD_STR_MN4 || KIND == LD_STR_MN_S || KIND == LD_CFWD_B4 ||
                                   KIND == LD_CBWD_B4 || KIND == LD_CBWD_B_S || KIND == LD_CWG_A4 ||
                                   KIND == LD_CWG_A_S || KIND == LD_CFWD_B_S || KIND == LD_CFWD_B4T ||
                                   KIND == LD_CWG_A4T);
  static constexpr bool vec4 = (KIND == LD_STR_MN4 || KIND == LD_STR_K4 || KIND == LD_CFWD_A4 || KIND == LD_CFWD_B4 ||
                                KIND == LD_CBWD_A4 || KIND == LD_CBWD_B4 || KIND == LD_CWG_A4 || KIND == LD_CBWD_BK4 ||
                                KIND >= LD_CFWD_A4T);
  static constexpr bool tiled = KIND >= LD_CFWD_A4T;
};

// Exact division by an invariant d >= 1 for dividends 0 <= n < 2^31 (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994, the
// round-up multiplier with the add-back step): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1 (which fits 32 bits), floor(n / d) =
// (umulhi(n, m) + n) >> l. The sum stays below 2^32 because umulhi(n, m) <= n < 2^31.
// Three full-rate 32-bit instructions (multiply-high, add, shift).
struct FastDiv {
  uint32_t m;
  int l;
};

__host__ __device__ inline FastDiv make_fastdiv(int d) {
  int l = 0;
  while ((1ll << l) < (long long)d) ++l;
  const uint64_t num = ((1ull << l) - (uint64_t)d) << 32;
  return FastDiv{(uint32_t)(num / (uint64_t)d + 1), l};
}

__device__ __forceinline__ int fdiv(int n, FastDiv f) {
  return (int)((__umulhi((uint32_t)n, f.m) + (uint32_t)n) >> f.l);
}

struct ConvG {
  int N, C, H, W, Cout, kk, stride, pt, pl, Ho, Wo;
  FastDiv dC, dCout, dkk, dHW, dWo;  // dividers for C, Cout, kk, Ho*Wo and Wo
};

// Phase of the stride-s input-delta GEMM: input pixels (h, w) with h % s == a, w % s == b;
// only kernel taps kh = kh0 + i*s (kw = kw0 + j*s) reach them.
struct Phase {
  int a, b, kh0, kw0, nkh, nkw, Hq, Wq;
};

__host__ __device__ inline Phase make_phase(const ConvG& g, int phase) {
  Phase p;
  const int s = g.stride;
  p.a = phase / s;
  p.b = phase % s;
  p.kh0 = (p.a + g.pt) % s;
  p.kw0 = (p.b + g.pl) % s;
  p.nkh = p.kh0 < g.kk ? (g.kk - p.kh0 + s - 1) / s : 0;
  p.nkw = p.kw0 < g.kk ? (g.kk - p.kw0 + s - 1) / s : 0;
  p.Hq = p.a < g.H ? (g.H - p.a + s - 1) / s : 0;
  p.Wq = p.b < g.W ? (g.W - p.b + s - 1) / s : 0;
  return p;
}

struct Operand {
  const float* p0;
  const float* p1;
  int64_t zdiv, sz1, sz2;  // batch offset (z/zdiv)*sz1 + (z%zdiv)*sz2 (strided kinds)
  int64_t s_mn, s_k;       // strided kinds
  int MN, K;               // extents along the tile dim and the reduction
  int ones_row;            // tile index that reads as 1.0 for valid k (bias row), -1 = none
  ConvG g;                 // conv kinds
  int64_t nbytes;          // bytes reachable from the operand's (per-batch) base; < 2^31
};

// Buffer loads (MUBUF, raw, offset in a VGPR): the operand tensors are read through a
// buffer resource held in scalar registers, so the per-lane address is a 32-bit byte
// offset (no 64-bit address arithmetic) and a chunk outside the operand or in the conv
// zero padding is given an offset past the resource's range, for which the hardware
// returns zeros (no exec-mask branch and no select per element).
typedef int tagi_i32x4 __attribute__((ext_vector_type(4)));
typedef float tagi_f32x4 __attribute__((ext_vector_type(4)));
__device__ tagi_f32x4 tagi_raw_buffer_load_f32x4(tagi_i32x4 rsrc, int voffset, int soffset,
                                                 int aux) __asm("llvm.amdgcn.raw.buffer.load.v4f32");
__device__ float tagi_raw_buffer_load_f32(tagi_i32x4 rsrc, int voffset, int soffset,
                                          int aux) __asm("llvm.amdgcn.raw.buffer.load.f32");

constexpr uint32_t kBufOutOfRange = 0x80000000u;  // byte offset past every operand's range

// Resource of `nbytes` bytes at `base`: 48-bit base address, stride 0, the range in bytes,
// and the gfx9 raw-buffer format word.
__device__ __forceinline__ tagi_i32x4 make_buffer_rsrc(const float* base, int64_t nbytes) {
  const uint64_t a = (uint64_t)base;
  tagi_i32x4 r;
  r.x = (int)(uint32_t)a;
  r.y = (int)((a >> 32) & 0xffffu);
  r.z = (int)nbytes;
  r.w = 0x00020000;
  return r;
}

struct Epi {
  int kind;  // 0: strided store (+bias, scale); 1: weight deltas (+bias row); 2: conv input-delta rows
  float* om;
  float* ov;
  const float* bm;
  const float* bv;
  int64_t b_sr, b_sc;
  float sm, sv;
  int64_t zdiv, sz1, sz2, srow, scol;
  // kind 1
  const float* Sw;
  const float* Sb;
  float* dmb;
  float* dSb;
  int wrows;
  int64_t ldw;
  int perm_C, perm_kk2;  // conv: row r = (kh*kk+kw)*C + c maps to weight row c*kk2 + kh*kk + kw
  FastDiv dperm;         // divider for perm_C
  // kind 1, optional: the capped update applied in place as the deltas are formed
  // (upd_mw/upd_Sw the weights, upd_mb/upd_Sb the bias, Sw/Sb their variances before the
  // update: the same arrays as upd_Sw/upd_Sb); each element is read and written by the
  // one thread that forms its deltas. With the update, om/ov and dmb/dSb may be null:
  // the deltas are then applied without being stored
  float* upd_mw;
  float* upd_Sw;
  float* upd_mb;
  float* upd_Sb;
  float cap;
  // kind 2
  ConvG g;
  // kinds 0 and 2: optional addend laid out like the output (out = result + addend; may
  // alias the output, each element is read and written by one thread)
  const float* am;
  const float* av;
  // kind 0: optional multiplier laid out like the output (mean * j, variance * j^2: the
  // Jacobian of an elementwise layer applied to the product's deltas)
  const float* jm;
  // kind 0, plain store only: statistics of ReLU(output) for a BatchNorm2D after it.
  // st_J receives the ReLU Jacobian (laid out like the output) and st_ws the per-tile
  // column sums of mu_a, S_a and mu_a^2, st_ws[(q * C + col) * st_nblk + tile row].
  float* st_J;
  float* st_ws;
  int st_nblk;
  // kind 2, unsplit single-phase launches: the backward of a BatchNorm2D and the ReLU in
  // front of it applied to the product (the deltas at the BatchNorm2D output), whose
  // outputs are then the deltas at the ReLU input: m mg/sqrt(var+eps) J and
  // v mg^2/(var+eps) J^2; st_ws receives the per-tile column sums of m mhat, v mhat^2, m,
  // v and of the two outputs, st_ws[(q * C + col) * st_nblk + tile row]
  const float* bn_mhat;
  const float* bn_J;
  const float* bn_var;
  const float* bn_g;
  float bn_eps;
  // EPI 3: the same fold applied to product + addend, which is still stored to om/ov (the
  // deltas at the BatchNorm2D output, read again by the block's shortcut); the fold's
  // outputs go to bn_om/bn_ov
  float* bn_om;
  float* bn_ov;
  // kind 0 (EPI 4 in the GEMM kernel, and the split-K reduction): the outputs are the
  // moments of ReLU(product) instead -- om the mean, ov the variance, relu_J the ReLU
  // Jacobian, all laid out like the output (the product's own moments are not stored)
  float* relu_J;
};

struct GemmArgs {
  Operand a, b;
  Epi epi;
  int R, C, Kred;  // rows, cols, reduction (per phase for the conv input delta)
  int tiles_m, tiles_n;
  int splits, k_chunk;
  int phased;      // conv input delta: z indexes the stride phase
  float* partial;  // split-K partial sums, or null to apply the epilogue in place
  // phased launches: blockIdx.y / splits -> phase, longest reductions first so the short
  // phases fill in behind them
  unsigned char phase_order[64];
};

template <int BM_, int BN_, int WM_, int WN_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = 16;
  static constexpr int NTH = (BM / WM) * (BN / WN) * 64;
  // blocks per CU the register budget is sized for (2 x 256-thread blocks = 2 waves/SIMD)
  static constexpr int MINB = NTH >= 512 ? 1 : 2;
};

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E-1, in order.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// ------------------------------------------------------------------------------------
// Operand loaders. Each thread owns NC chunks (float4 or scalar) of the BMN x BK tile;
// the chunk -> (mn, k) map is fixed per thread, so per-row / per-k invariants are
// computed once in init().
// ------------------------------------------------------------------------------------
template <int KIND, int NT, int BMN, int BK, int NTH, int PF = 1>
struct Loader {
  static constexpr bool V4 = KindTraits<KIND>::vec4;
  static constexpr bool MNF = KindTraits<KIND>::mn_fast;
  static constexpr int W = V4 ? 4 : 1;  // elements per chunk
  static constexpr int NCH = BMN * BK / W;  // chunks in the tile
  // fewer chunks than threads (a 32-wide operand of a 4-wave block): threads past NCH idle
  static constexpr bool PART = NCH < NTH;
  static constexpr int NC = PART ? 1 : NCH / NTH;
  static_assert(PART ? (NCH * W == BMN * BK && NTH % NCH == 0) : (NC * W * NTH == BMN * BK),
                "tile does not split evenly over threads");
  static constexpr int LD = BMN + 4;
  // LDS tile of one tensor. Reduction-major [BK][LD] (rows of the tile dim padded by 4),
  // except for float4 loaders that walk the reduction ("K4" kinds): those keep the tile
  // row-major, [BMN][BK], so a fetched chunk (4 consecutive k of one row) is stored with
  // one 16-byte write instead of four scattered ones, and a lane reads the 8 k values of
  // its fragments with two 16-byte reads. The 4 chunks of a row are XOR-swizzled by
  // ((row >> 1) ^ (row >> 2)) & 3 so that 8 (or 16) lanes of one 16-byte access hit
  // distinct bank groups with 32 (or 64) banks, for the stores (4 lanes per row) and for
  // the fragment reads (one row per lane).
  static constexpr bool KMAJ = V4 && !MNF;
  static constexpr int TILE = KMAJ ? BMN * BK : BK * LD;
  static_assert(!KMAJ || BK == 16, "the row-major tile swizzle assumes 4 chunks per row");
  __device__ static __forceinline__ int kmaj_off(int row, int k) {
    return row * BK + ((((k >> 2) ^ (row >> 1) ^ (row >> 2)) & 3) << 2);
  }

  using Vt = typename std::conditional<V4, float4, float>::type;
  static constexpr bool CONV_ROWS = (KIND == LD_CFWD_A4 || KIND == LD_CFWD_A_S || KIND == LD_CBWD_A4 ||
                                     KIND == LD_CBWD_A_S);
  static constexpr bool CONV_R = CONV_ROWS || KIND == LD_CBWD_B4 || KIND == LD_CBWD_B_S || KIND == LD_CBWD_BK4 ||
                                 KIND == LD_CWG_A4 || KIND == LD_CWG_A_S;
  static constexpr int NRB = CONV_ROWS ? NC : 1;  // per-chunk row bases only where rows differ
  static constexpr int NR = CONV_R ? NC : 1;

  Vt v[PF][NT][NC];  // PF register stages of fetched chunks
  // kinds with a ones row (the bias sums of a parameter-delta product): the chunk holds
  // that row, whose first element is written as 1.0 when the chunk is stored to LDS (a
  // select on the loaded value at fetch time would wait for the load right there)
  static constexpr bool ONES = (KIND == LD_STR_MN4 || KIND == LD_STR_MN_S || KIND == LD_STR_K_S ||
                                KIND == LD_CWG_A4 || KIND == LD_CWG_A_S || KIND == LD_CWG_A4T);
  static constexpr bool TILED = KindTraits<KIND>::tiled;
  bool onef[ONES ? PF : 1][ONES ? NC : 1];
  FastDiv dnkw;              // divider for the phase's taps per row (conv input delta)
  int mnmax, kmax;           // extents checked by fetch (per phase for the conv input delta)
  int cmn[NC], ck[NC];       // chunk origin within the tile
  bool active;               // this thread loads a chunk (always, unless PART)
  int rowbase[NRB];          // per-chunk image base (conv rows), elements from the operand base
  int r0[NR], r1[NR], r2[NR];
  tagi_i32x4 rs0, rs1;       // buffer resources of the operand's tensors (block-uniform)
  // tile-aligned kinds: per-chunk byte offset of the chunk at the tile's origin (modulo
  // 2^32; the tile's scalar part is added per fetch), tap masks, and the weight delta's
  // input-row / input-column offsets of the chunk's pixel and kernel tap
  uint32_t lb[TILED ? NC : 1], tapm[TILED ? NC : 1];
  int lih[TILED ? NC : 1], liw[TILED ? NC : 1];
  bool okl[TILED ? NC : 1], onel[TILED ? NC : 1];
  int tkh0, tkw0, tnkw;      // input delta: the phase's first tap and taps per row
  uint32_t oobv;             // kBufOutOfRange, held in a register

  __device__ __forceinline__ void map(int tid) {
    active = !PART || tid < NCH;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + i * NTH;
      if constexpr (MNF) {
        cmn[i] = (c % (BMN / W)) * W;
        ck[i] = c / (BMN / W);
      } else {
        cmn[i] = c / (BK / W);
        ck[i] = (c % (BK / W)) * W;
      }
    }
  }

  // per-block / per-thread invariants
  // klim: end of the block's stretch of the reduction (its split-K chunk); tiles past it
  // read as zeros
  __device__ __forceinline__ void init(const Operand& o, int z, int mn0, int tid, int klim) {
    map(tid);
    mnmax = o.MN;
    kmax = o.K;
    if constexpr (KIND == LD_CBWD_A4 || KIND == LD_CBWD_A_S || KIND == LD_CBWD_B4 || KIND == LD_CBWD_B_S ||
                  KIND == LD_CBWD_BK4 || KIND == LD_CBWD_A4T || KIND == LD_CBWD_BK4T) {
      const Phase ph = make_phase(o.g, z);
      kmax = ph.nkh * ph.nkw * o.g.Cout;
      dnkw = make_fastdiv(ph.nkw > 0 ? ph.nkw : 1);
      if constexpr (KIND == LD_CBWD_A4 || KIND == LD_CBWD_A_S || KIND == LD_CBWD_A4T) mnmax = o.g.N * ph.Hq * ph.Wq;
      tkh0 = ph.kh0;
      tkw0 = ph.kw0;
      tnkw = ph.nkw;
    }
    kmax = min(kmax, klim);
    oobv = kBufOutOfRange;
    asm volatile("" : "+v"(oobv));  // one register for every chunk's out-of-range offset
    if constexpr (TILED) init_tiled(o, z, mn0);
    if constexpr (KIND == LD_CFWD_A4 || KIND == LD_CFWD_A_S) {
      // rows are output pixels: base of image n and the top-left input corner
      const int howo = o.g.Ho * o.g.Wo;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int m = mn0 + cmn[i];
        if (m < o.MN) {
          const int n = m / howo, p = m - n * howo;
          const int oh = p / o.g.Wo, ow = p - oh * o.g.Wo;
          rowbase[i] = n * o.g.H * o.g.W * o.g.C;
          r0[i] = oh * o.g.stride - o.g.pt;
          r1[i] = ow * o.g.stride - o.g.pl;
        } else {
          rowbase[i] = 0;
          r0[i] = -(1 << 28);
          r1[i] = -(1 << 28);
        }
      }
    } else if constexpr (KIND == LD_CBWD_A4 || KIND == LD_CBWD_A_S) {
      // rows are the phase's input pixels: image base and output coordinates of tap kh0,kw0
      const Phase ph = make_phase(o.g, z);
      const int hq = ph.Hq * ph.Wq;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int q = mn0 + cmn[i];
        if (q < mnmax && hq > 0) {
          const int n = q / hq, rr = q - n * hq;
          const int hh = rr / ph.Wq, ww = rr - hh * ph.Wq;
          const int h = hh * o.g.stride + ph.a, w = ww * o.g.stride + ph.b;
          rowbase[i] = n * o.g.Ho * o.g.Wo * o.g.Cout;
          r0[i] = (h + o.g.pt - ph.kh0) / o.g.stride;
          r1[i] = (w + o.g.pl - ph.kw0) / o.g.stride;
        } else {
          rowbase[i] = 0;
          r0[i] = -(1 << 28);
          r1[i] = -(1 << 28);
        }
        r2[i] = ph.nkw;
      }
    } else if constexpr (KIND == LD_CBWD_B4 || KIND == LD_CBWD_B_S || KIND == LD_CBWD_BK4) {
      // tap offsets of this phase
      const Phase ph = make_phase(o.g, z);
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        r0[i] = ph.kh0;
        r1[i] = ph.kw0;
        r2[i] = ph.nkw;
      }
    } else if constexpr (KIND == LD_CWG_A4 || KIND == LD_CWG_A_S) {
      // rows are weight rows r = (kh*kk + kw)*C + c: split once
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int r = mn0 + cmn[i];
        const int kidx = r / o.g.C;
        const int c = r - kidx * o.g.C;
        const int kh = kidx / o.g.kk;
        r0[i] = kh;
        r1[i] = kidx - kh * o.g.kk;
        r2[i] = c;
      }
    }
    if constexpr (CONV_R || TILED || KIND == LD_CFWD_B4 || KIND == LD_CFWD_B_S) {
      rs0 = make_buffer_rsrc(o.p0, o.nbytes);
      rs1 = make_buffer_rsrc(NT == 2 ? o.p1 : o.p0, o.nbytes);
    } else {
      // strided kinds: the batch offset goes into the resources' base
      const int64_t zb = (z / o.zdiv) * o.sz1 + (z % o.zdiv) * o.sz2;
      rs0 = make_buffer_rsrc(o.p0 + zb, o.nbytes);
      rs1 = make_buffer_rsrc((NT == 2 ? o.p1 : o.p0) + zb, o.nbytes);
    }
  }

  // bits j of [0, n) with lo <= j < hi (n <= 25)
  __device__ static __forceinline__ uint32_t range_bits(int lo, int hi, int n) {
    lo = max(lo, 0);
    hi = min(hi, n);
    return hi > lo ? ((1u << hi) - 1u) & ~((1u << lo) - 1u) : 0u;
  }
  // tap mask over (i, j) in [0, nh) x [0, nw), bit i*nw + j: row bit i and column bit j
  __device__ static __forceinline__ uint32_t spread_bits(uint32_t hm, uint32_t wm, int nh, int nw) {
    uint32_t m = 0;
    for (int i = 0; i < nh; ++i)
      if ((hm >> i) & 1u) m |= wm << (i * nw);
    return m;
  }

  __device__ __forceinline__ void init_tiled(const Operand& o, int z, int mn0) {
    using U = uint32_t;
    const ConvG& g = o.g;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int mn = mn0 + cmn[i];
      if constexpr (KIND == LD_CFWD_A4T) {
        // row = output pixel (n, oh, ow); chunk = 4 channels at k offset ck of tap (kh, kw)
        uint32_t base = 0, msk = 0;
        if (mn < o.MN) {
          const int howo = g.Ho * g.Wo;
          const int n = mn / howo, p = mn - n * howo;
          const int oh = p / g.Wo, ow = p - oh * g.Wo;
          const int ih0 = oh * g.stride - g.pt, iw0 = ow * g.stride - g.pl;
          base = ((U(n) * U(g.H) + U(ih0)) * U(g.W) + U(iw0)) * U(g.C) + U(ck[i]);
          msk = spread_bits(range_bits(-ih0, g.H - ih0, g.kk), range_bits(-iw0, g.W - iw0, g.kk), g.kk, g.kk);
        }
        lb[i] = base * 4u;
        tapm[i] = msk;
      } else if constexpr (KIND == LD_CFWD_B4T) {
        // weights w[(c*kk2 + kidx)*Cout + co]: chunk = 4 co at reduction offset ck (channel c0 + ck)
        lb[i] = (U(ck[i]) * U(g.kk * g.kk) * U(g.Cout) + U(mn)) * 4u;
        okl[i] = mn < o.MN;
      } else if constexpr (KIND == LD_CBWD_A4T) {
        // row = input pixel of stride phase z; (r0, r1) = output pixel of tap (kh0, kw0)
        const Phase ph = make_phase(g, z);
        const int hq = ph.Hq * ph.Wq;
        uint32_t base = 0, msk = 0;
        if (mn < mnmax && hq > 0) {
          const int n = mn / hq, rr = mn - n * hq;
          const int hh = rr / ph.Wq, ww = rr - hh * ph.Wq;
          const int h = hh * g.stride + ph.a, w = ww * g.stride + ph.b;
          const int r0 = (h + g.pt - ph.kh0) / g.stride, r1 = (w + g.pl - ph.kw0) / g.stride;
          base = ((U(n) * U(g.Ho) + U(r0)) * U(g.Wo) + U(r1)) * U(g.Cout) + U(ck[i]);
          // output row r0 - ikh in [0, Ho) and column r1 - ikw in [0, Wo)
          msk = spread_bits(range_bits(r0 - g.Ho + 1, r0 + 1, ph.nkh), range_bits(r1 - g.Wo + 1, r1 + 1, ph.nkw),
                            ph.nkh, ph.nkw);
        }
        lb[i] = base * 4u;
        tapm[i] = msk;
      } else if constexpr (KIND == LD_CBWD_BK4T) {
        // weights w[((c*kk + kh)*kk + kw)*Cout + co] in place: row c, chunk = 4 co at offset ck
        lb[i] = (U(mn) * U(g.kk * g.kk) * U(g.Cout) + U(ck[i])) * 4u;
        okl[i] = mn < mnmax;
      } else if constexpr (KIND == LD_CWG_A4T) {
        // row = weight row (kh, kw, c) (+ the ones row); the chunk's pixel is at offset ck
        // of a 16-pixel run inside one image, (dh, dw) rows/columns past the run's start
        const int kidx = mn / g.C, c = mn - kidx * g.C;
        const int kh = kidx / g.kk, kw = kidx - kh * g.kk;
        const int dh = g.Wo >= 16 ? 0 : ck[i] / g.Wo, dw = ck[i] - dh * g.Wo;
        int ih = dh * g.stride - g.pt + kh;
        const int iw = dw * g.stride - g.pl + kw;
        if (mn >= o.MN) ih = -(1 << 28);  // past the weight rows: reads zeros
        lih[i] = ih;
        liw[i] = iw;
        lb[i] = ((U(ih) * U(g.W) + U(iw)) * U(g.C) + U(c)) * 4u;
        onel[i] = mn == o.ones_row;
      }
    }
  }

  template <int ST>
  __device__ __forceinline__ void load_chunk(int i, uint32_t vo) {
    if constexpr (V4) {
      const tagi_f32x4 a = tagi_raw_buffer_load_f32x4(rs0, (int)vo, 0, 0);
      v[ST][0][i] = make_float4(a.x, a.y, a.z, a.w);
      if constexpr (NT == 2) {
        const tagi_f32x4 b = tagi_raw_buffer_load_f32x4(rs1, (int)vo, 0, 0);
        v[ST][1][i] = make_float4(b.x, b.y, b.z, b.w);
      }
    } else {
      v[ST][0][i] = tagi_raw_buffer_load_f32(rs0, (int)vo, 0, 0);
      if constexpr (NT == 2) v[ST][1][i] = tagi_raw_buffer_load_f32(rs1, (int)vo, 0, 0);
    }
  }

  // Tile-aligned kinds: the tile's tap / pixel run is decoded in scalar registers
  // (k0 is the same for every lane), then one add and a mask bit per chunk.
  template <int ST>
  __device__ __forceinline__ void fetch_tiled(const Operand& o, int k0) {
    using U = uint32_t;
    const ConvG& g = o.g;
    const bool kin = k0 < kmax;  // whole tile in range (the reduction length is a multiple of 16)
    if constexpr (KIND == LD_CFWD_A4T || KIND == LD_CFWD_B4T) {
      const int kidx = fdiv(k0, g.dC), c0 = k0 - kidx * g.C;
      if constexpr (KIND == LD_CFWD_A4T) {
        const int kh = fdiv(kidx, g.dkk), kw = kidx - kh * g.kk;
        const uint32_t s4 = ((U(kh) * U(g.W) + U(kw)) * U(g.C) + U(c0)) * 4u;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
          const bool ok = kin && ((tapm[i] >> (kidx & 31)) & 1u);
          load_chunk<ST>(i, ok ? lb[i] + s4 : oobv);
        }
      } else {
        const uint32_t s4 = (U(c0) * U(g.kk * g.kk) + U(kidx)) * U(g.Cout) * 4u;
#pragma unroll
        for (int i = 0; i < NC; ++i) load_chunk<ST>(i, (kin && okl[i]) ? lb[i] + s4 : oobv);
      }
    } else if constexpr (KIND == LD_CBWD_A4T || KIND == LD_CBWD_BK4T) {
      const int kidx = fdiv(k0, g.dCout), co0 = k0 - kidx * g.Cout;
      const int ikh = fdiv(kidx, dnkw), ikw = kidx - ikh * tnkw;
      if constexpr (KIND == LD_CBWD_A4T) {
        const uint32_t s4 = ((U(ikh) * U(g.Wo) + U(ikw)) * U(g.Cout) - U(co0)) * 4u;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
          const bool ok = kin && ((tapm[i] >> (kidx & 31)) & 1u);
          load_chunk<ST>(i, ok ? lb[i] - s4 : oobv);
        }
      } else {
        const int kh = tkh0 + ikh * g.stride, kw = tkw0 + ikw * g.stride;
        const uint32_t s4 = ((U(kh) * U(g.kk) + U(kw)) * U(g.Cout) + U(co0)) * 4u;
#pragma unroll
        for (int i = 0; i < NC; ++i) load_chunk<ST>(i, (kin && okl[i]) ? lb[i] + s4 : oobv);
      }
    } else if constexpr (KIND == LD_CWG_A4T) {
      const int n = fdiv(k0, g.dHW), p0 = k0 - n * (g.Ho * g.Wo);
      const int oh0 = fdiv(p0, g.dWo), ow0 = p0 - oh0 * g.Wo;
      const int sih = oh0 * g.stride, siw = ow0 * g.stride;
      const uint32_t s4 = ((U(n) * U(g.H) + U(sih)) * U(g.W) + U(siw)) * U(g.C) * 4u;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int ih = sih + lih[i], iw = siw + liw[i];
        const bool ok = kin && U(ih) < U(g.H) && U(iw) < U(g.W);
        onef[ST][i] = kin && onel[i];
        load_chunk<ST>(i, ok ? lb[i] + s4 : oobv);
      }
    }
  }

  // Gather of one k tile: each chunk's reduction index is decoded with exact
  // multiply-high divisions; chunks outside the operand or in the zero padding read as 0.
  template <int ST = 0>
  __device__ __forceinline__ void fetch(const Operand& o, int z, int mn0, int k0) {
    if constexpr (PART) {
      if (!active) return;
    }
    if constexpr (TILED) {
      fetch_tiled<ST>(o, k0);
      return;
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int mn = mn0 + cmn[i];
      const int k = k0 + ck[i];
      bool ok = false, one = false;
      // element offset from the resource base (< 2^29 when ok, checked on the host); formed
      // in unsigned arithmetic because chunks that are not ok may compute anything
      uint32_t off = 0;
      using U = uint32_t;
      if constexpr (KIND == LD_STR_MN4 || KIND == LD_STR_MN_S || KIND == LD_STR_K_S) {
        ok = k < kmax && mn < o.MN;
        one = k < kmax && mn == o.ones_row;
        if constexpr (KIND == LD_STR_MN4) off = U(mn) + U(k) * U(o.s_k);
        else off = U(mn) * U(o.s_mn) + U(k) * U(o.s_k);
      } else if constexpr (KIND == LD_STR_K4) {
        ok = mn < o.MN && k < kmax;
        off = U(mn) * U(o.s_mn) + U(k);
      } else if constexpr (KIND == LD_CFWD_A4 || KIND == LD_CFWD_A_S) {
        // k = (kh*kk + kw)*C + c
        const int kidx = fdiv(k, o.g.dC), c = k - kidx * o.g.C;
        const int kh = fdiv(kidx, o.g.dkk), kw = kidx - kh * o.g.kk;
        const int ih = r0[i] + kh, iw = r1[i] + kw;
        ok = k < kmax && ih >= 0 && ih < o.g.H && iw >= 0 && iw < o.g.W;
        off = U(rowbase[i]) + (U(ih) * U(o.g.W) + U(iw)) * U(o.g.C) + U(c);
      } else if constexpr (KIND == LD_CFWD_B4 || KIND == LD_CFWD_B_S) {
        // k = kidx*C + c; weight row (c, kh, kw)
        const int kidx = fdiv(k, o.g.dC), c = k - kidx * o.g.C;
        ok = k < kmax && mn < o.MN;
        off = (U(c) * U(o.g.kk * o.g.kk) + U(kidx)) * U(o.g.Cout) + U(mn);
      } else if constexpr (KIND == LD_CBWD_A4 || KIND == LD_CBWD_A_S) {
        // k = (ikh*nkw + ikw)*Cout + co over the phase's taps
        const int kidx = fdiv(k, o.g.dCout), co = k - kidx * o.g.Cout;
        const int ikh = fdiv(kidx, dnkw), ikw = kidx - ikh * r2[i];
        const int oh = r0[i] - ikh, ow = r1[i] - ikw;
        ok = k < kmax && oh >= 0 && oh < o.g.Ho && ow >= 0 && ow < o.g.Wo;
        off = U(rowbase[i]) + (U(oh) * U(o.g.Wo) + U(ow)) * U(o.g.Cout) + U(co);
      } else if constexpr (KIND == LD_CBWD_B4 || KIND == LD_CBWD_B_S) {
        const int kidx = fdiv(k, o.g.dCout), co = k - kidx * o.g.Cout;
        const int ikh = fdiv(kidx, dnkw), ikw = kidx - ikh * r2[i];
        const int kh = r0[i] + ikh * o.g.stride;
        const int kw = r1[i] + ikw * o.g.stride;
        ok = k < kmax && mn < mnmax;
        off = ((U(kh) * U(o.g.kk) + U(kw)) * U(o.g.Cout) + U(co)) * U(o.g.C) + U(mn);
      } else if constexpr (KIND == LD_CBWD_BK4) {
        // the same (kh, kw, co) as LD_CBWD_B4, read from the weights in their own layout: the
        // chunk's 4 reduction indices are 4 consecutive co of one tap
        const int kidx = fdiv(k, o.g.dCout), co = k - kidx * o.g.Cout;
        const int ikh = fdiv(kidx, dnkw), ikw = kidx - ikh * r2[i];
        const int kh = r0[i] + ikh * o.g.stride;
        const int kw = r1[i] + ikw * o.g.stride;
        ok = k < kmax && mn < mnmax;
        off = ((U(mn) * U(o.g.kk) + U(kh)) * U(o.g.kk) + U(kw)) * U(o.g.Cout) + U(co);
      } else if constexpr (KIND == LD_CWG_A4 || KIND == LD_CWG_A_S) {
        // k = (n*Ho + oh)*Wo + ow
        const int n = fdiv(k, o.g.dHW), pix = k - n * (o.g.Ho * o.g.Wo);
        const int oh = fdiv(pix, o.g.dWo), ow = pix - oh * o.g.Wo;
        const int ih = oh * o.g.stride - o.g.pt + r0[i];
        const int iw = ow * o.g.stride - o.g.pl + r1[i];
        ok = k < kmax && mn < o.MN && ih >= 0 && ih < o.g.H && iw >= 0 && iw < o.g.W;
        one = k < kmax && mn == o.ones_row;
        off = U(n) * U(o.g.H * o.g.W * o.g.C) + (U(ih) * U(o.g.W) + U(iw)) * U(o.g.C) + U(r2[i]);
      }
      if constexpr (ONES) onef[ST][i] = one;
      (void)one;
      load_chunk<ST>(i, ok ? off * 4u : oobv);
    }
  }

  template <int ST = 0>
  __device__ __forceinline__ void store(float* s) const {
    if constexpr (PART) {
      if (!active) return;
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      Vt x[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) x[t] = v[ST][t][i];
      if constexpr (ONES) {
        // ones-row chunks are out of range (loaded as zeros): their first element is 1
        if (onef[ST][i]) {
          if constexpr (V4) x[0].x = 1.f;
          else x[0] = 1.f;
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float* st = s + t * TILE;
        if constexpr (!V4) {
          st[ck[i] * LD + cmn[i]] = x[t];
        } else if constexpr (MNF) {
          *reinterpret_cast<float4*>(st + ck[i] * LD + cmn[i]) = x[t];
        } else {
          *reinterpret_cast<float4*>(st + kmaj_off(cmn[i], ck[i])) = x[t];
        }
      }
    }
  }
};

// ------------------------------------------------------------------------------------
// Epilogue
// ------------------------------------------------------------------------------------
// OPT_DELTAS: the kind-1 deltas are stored only where om (dmb) is given -- the split-K
// reduction's form; the GEMM kernel's, whose kind-1 outputs always exist, keeps the plain
// stores (the extra branch, inlined per output, costs its 128-row tiles a stack frame).
template <bool OPT_DELTAS = false>
__device__ __forceinline__ void epi_apply(const Epi& e, int z, int row, int col, float m, float v) {
  if (e.kind == 0) {
    const int64_t off = (z / e.zdiv) * e.sz1 + (z % e.zdiv) * e.sz2 + (int64_t)row * e.srow + (int64_t)col * e.scol;
    float rm = m * e.sm;
    float rv = v * e.sv;
    const int64_t bi = (int64_t)row * e.b_sr + (int64_t)col * e.b_sc;
    if (e.bm) rm += e.bm[bi];
    if (e.bv) rv += e.bv[bi];
    if (e.jm) {
      const float j = e.jm[off];
      rm *= j;
      rv *= j * j;
    }
    if (e.am) {
      rm += e.am[off];
      rv += e.av[off];
    }
    if (e.relu_J) {
      float ra, rS, rJ;
      relu_moments(rm, rv, ra, rS, rJ);
      e.om[off] = ra;
      e.ov[off] = rS;
      e.relu_J[off] = rJ;
    } else {
      if (e.om) e.om[off] = rm;
      e.ov[off] = rv;
    }
  } else if (e.kind == 1) {
    if (row < e.wrows) {
      int wr = row;
      if (e.perm_C > 0) {
        const int kidx = fdiv(row, e.dperm);
        wr = (row - kidx * e.perm_C) * e.perm_kk2 + kidx;
      }
      const int64_t idx = (int64_t)wr * e.ldw + col;
      const float s = e.Sw ? e.Sw[idx] : 1.f;
      const float dm = s * m, dS = (s * s) * v;
      if (!OPT_DELTAS || e.om) {
        e.om[idx] = dm;
        e.ov[idx] = dS;
      }
      if (e.upd_mw) {
        float pm = e.upd_mw[idx], pS = s;
        capped(pm, pS, dm, dS, e.cap);
        e.upd_mw[idx] = pm;
        e.upd_Sw[idx] = pS;
      }
    } else {
      const float s = e.Sb ? e.Sb[col] : 1.f;
      const float dm = s * m, dS = (s * s) * v;
      if (!OPT_DELTAS || e.dmb) {
        e.dmb[col] = dm;
        e.dSb[col] = dS;
      }
      if (e.upd_mb) {
        float pm = e.upd_mb[col], pS = s;
        capped(pm, pS, dm, dS, e.cap);
        e.upd_mb[col] = pm;
        e.upd_Sb[col] = pS;
      }
    }
  } else {
    // conv input delta: row = pixel q of phase z, col = input channel
    const Phase ph = make_phase(e.g, z);
    const int hq = ph.Hq * ph.Wq;
    if (row >= e.g.N * hq) return;  // rows past this phase's pixels (split-K reduction covers phase 0's rows)
    const int n = row / hq, rr = row - n * hq;
    const int hh = rr / ph.Wq, ww = rr - hh * ph.Wq;
    const int h = hh * e.g.stride + ph.a, w = ww * e.g.stride + ph.b;
    const int64_t off = (((int64_t)n * e.g.H + h) * e.g.W + w) * e.g.C + col;
    if (e.am) {
      m = m + e.am[off];
      v = v + e.av[off];
    }
    e.om[off] = m;
    e.ov[off] = v;
  }
}

// Four consecutive columns of one output row (the split-K reduction's float4 groups) with
// vector loads and stores where the layout allows it; false sends the caller to the
// per-element path.
__device__ __forceinline__ bool epi_apply4(const Epi& e, int z, int row, int col, const float* m, const float* v) {
  if (e.kind == 2) {
    const Phase ph = make_phase(e.g, z);
    const int hq = ph.Hq * ph.Wq;
    if (row >= e.g.N * hq) return true;  // rows past this phase's pixels
    const int n = row / hq, rr = row - n * hq;
    const int hh = rr / ph.Wq, ww = rr - hh * ph.Wq;
    const int h = hh * e.g.stride + ph.a, w = ww * e.g.stride + ph.b;
    const int64_t off = (((int64_t)n * e.g.H + h) * e.g.W + w) * e.g.C + col;
    uintptr_t al = (uintptr_t)(e.om + off) | (uintptr_t)(e.ov + off);
    if (e.am) al |= (uintptr_t)(e.am + off) | (uintptr_t)(e.av + off);
    if (al & 15u) return false;
    float4 om4 = make_float4(m[0], m[1], m[2], m[3]), ov4 = make_float4(v[0], v[1], v[2], v[3]);
    if (e.am) {
      const float4 a = *reinterpret_cast<const float4*>(e.am + off);
      const float4 b = *reinterpret_cast<const float4*>(e.av + off);
      om4 = make_float4(om4.x + a.x, om4.y + a.y, om4.z + a.z, om4.w + a.w);
      ov4 = make_float4(ov4.x + b.x, ov4.y + b.y, ov4.z + b.z, ov4.w + b.w);
    }
    *reinterpret_cast<float4*>(e.om + off) = om4;
    *reinterpret_cast<float4*>(e.ov + off) = ov4;
    return true;
  }
  if (e.kind == 1) {
    // parameter deltas: 4 consecutive columns of one weight row (or of the bias row)
    const bool wrow = row < e.wrows;
    int64_t idx = col;
    if (wrow) {
      int wr = row;
      if (e.perm_C > 0) {
        const int kidx = fdiv(row, e.dperm);
        wr = (row - kidx * e.perm_C) * e.perm_kk2 + kidx;
      }
      idx = (int64_t)wr * e.ldw + col;
    }
    const float* sp = wrow ? e.Sw : e.Sb;
    float* om = wrow ? e.om : e.dmb;
    float* ov = wrow ? e.ov : e.dSb;
    float* um = wrow ? e.upd_mw : e.upd_mb;
    float* uS = wrow ? e.upd_Sw : e.upd_Sb;
    uintptr_t al = om ? ((uintptr_t)(om + idx) | (uintptr_t)(ov + idx)) : 0;
    if (sp) al |= (uintptr_t)(sp + idx);
    if (um) al |= (uintptr_t)(um + idx) | (uintptr_t)(uS + idx);
    if (al & 15u) return false;
    const float4 s4 = sp ? *reinterpret_cast<const float4*>(sp + idx) : make_float4(1.f, 1.f, 1.f, 1.f);
    const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
    float dm[4], dS[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dm[j] = sv[j] * m[j];
      dS[j] = (sv[j] * sv[j]) * v[j];
    }
    if (om) {
      *reinterpret_cast<float4*>(om + idx) = make_float4(dm[0], dm[1], dm[2], dm[3]);
      *reinterpret_cast<float4*>(ov + idx) = make_float4(dS[0], dS[1], dS[2], dS[3]);
    }
    if (um) {
      const float4 m4 = *reinterpret_cast<const float4*>(um + idx);
      float pm[4] = {m4.x, m4.y, m4.z, m4.w}, pS[4] = {sv[0], sv[1], sv[2], sv[3]};
#pragma unroll
      for (int j = 0; j < 4; ++j) capped(pm[j], pS[j], dm[j], dS[j], e.cap);
      *reinterpret_cast<float4*>(um + idx) = make_float4(pm[0], pm[1], pm[2], pm[3]);
      *reinterpret_cast<float4*>(uS + idx) = make_float4(pS[0], pS[1], pS[2], pS[3]);
    }
    return true;
  }
  if (e.kind == 0 && e.scol == 1 && !e.jm && !e.am) {
    const int64_t off = (z / e.zdiv) * e.sz1 + (z % e.zdiv) * e.sz2 + (int64_t)row * e.srow + col;
    uintptr_t al = (uintptr_t)(e.ov + off);
    if (e.om) al |= (uintptr_t)(e.om + off);
    if (e.relu_J) al |= (uintptr_t)(e.relu_J + off);
    if (al & 15u) return false;
    float rm[4], rv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t bi = (int64_t)row * e.b_sr + (int64_t)(col + j) * e.b_sc;
      rm[j] = m[j] * e.sm + (e.bm ? e.bm[bi] : 0.f);
      rv[j] = v[j] * e.sv + (e.bv ? e.bv[bi] : 0.f);
    }
    if (e.relu_J) {
      float rJ[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) relu_moments(rm[j], rv[j], rm[j], rv[j], rJ[j]);
      *reinterpret_cast<float4*>(e.relu_J + off) = make_float4(rJ[0], rJ[1], rJ[2], rJ[3]);
    }
    if (e.om) *reinterpret_cast<float4*>(e.om + off) = make_float4(rm[0], rm[1], rm[2], rm[3]);
    *reinterpret_cast<float4*>(e.ov + off) = make_float4(rv[0], rv[1], rv[2], rv[3]);
    return true;
  }
  return false;
}

// Rows of the output tile in GEMM z (phase-dependent for the conv input delta).
__device__ __forceinline__ int rows_of(const GemmArgs& g, int z) {
  if (!g.phased) return g.R;
  const Phase ph = make_phase(g.a.g, z);
  return g.a.g.N * ph.Hq * ph.Wq;
}

__device__ __forceinline__ int kred_of(const GemmArgs& g, int z) {
  if (!g.phased) return g.Kred;
  const Phase ph = make_phase(g.a.g, z);
  return ph.nkh * ph.nkw * g.a.g.Cout;
}

// EPI 1: the kind-2 epilogue with the BatchNorm2D -> ReLU backward folded in; EPI 2: the
// kind-1 epilogue with the capped parameter update applied in place; EPI 3: EPI 1 applied
// to product + addend, storing both; EPI 4: the kind-0 plain store of ReLU(product)'s
// moments and Jacobian (separate instantiations: their extra registers would otherwise
// cost every kernel occupancy)
// (the folded BatchNorm2D epilogues keep 4 waves per SIMD: their prefetched operands would
// otherwise take the register count just past the 128 that allows it)
template <int PROD, class CFG, int KA, int KB, int EPI = 0>
__global__ void __launch_bounds__(CFG::NTH, ((EPI == 1 || EPI == 3) && CFG::NTH == 256) ? 4 : CFG::MINB)
    gemm_kernel(GemmArgs g) {
  constexpr int BM = CFG::BM, BN = CFG::BN, BK = CFG::BK, WM = CFG::WM, WN = CFG::WN, NTH = CFG::NTH;
  constexpr int NA = (PROD == PROD_SHARED_A) ? 1 : 2;
  constexpr int NB = (PROD == PROD_SHARED_B) ? 1 : 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  // register stages of operand prefetch: k-tiles are fetched two tiles ahead, except in
  // the forward product's 8-wave tiles, where a second stage would cost the tile its
  // second resident block per CU
  // register stages of operand prefetch: k-tile t+2 is fetched while tile t is consumed,
  // and tile t+1 (fetched one step earlier) is stored to the other LDS buffer halfway
  // through tile t's MFMAs, so the LDS stores overlap the matrix work instead of
  // bunching up before the barrier
  constexpr int PF = 2;
  using LA = Loader<KA, NA, BM, BK, NTH, PF>;
  using LB = Loader<KB, NB, BN, BK, NTH, PF>;
  constexpr int LDA = LA::LD, LDB = LB::LD;
  constexpr int SA = NA * LA::TILE, SB = NB * LB::TILE;

  __shared__ __attribute__((aligned(16))) float smem[2 * (SA + SB)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / (BN / WN);
  const int wn = wave % (BN / WN);
  const int hl = lane >> 5;
  const int rl = lane & 31;

  // Split-K launches with at least 8 split groups: every tile of one split group (the
  // tiles that read the same stretch of the reduction) goes to one XCD. Workgroups are
  // dealt round-robin over the 8 XCDs in linear-id order, so the linear id L is read as
  // (XCD x = L mod 8, k-th block of that XCD) and group 8*(k / nt) + x, tile k mod nt
  // are assigned; groups past the last multiple of 8 keep the plain order. Without this,
  // the tiles of a group land on different XCDs and each XCD's L2 fetches the shared
  // operand panels again (the parameter-delta GEMMs' 9 tap tiles share one pixel range).
  int zq, split, bid;
  bool xcd_tiles = true;
  if (!g.phased && g.splits > 1 && gridDim.y >= 8 && (uint64_t)gridDim.x * gridDim.y < (1ull << 31)) {
    const int nt0 = g.tiles_m * g.tiles_n;
    const int L = blockIdx.x + blockIdx.y * gridDim.x;
    const int g8 = (int)(gridDim.y & ~7u);
    int grp, tile;
    if (L < g8 * nt0) {
      const int k = L >> 3, q = k / nt0;
      grp = q * 8 + (L & 7);
      tile = k - q * nt0;
    } else {
      const int L2 = L - g8 * nt0, q = L2 / nt0;
      grp = g8 + q;
      tile = L2 - q * nt0;
    }
    zq = grp / g.splits;
    split = grp - zq * g.splits;
    bid = tile;
    xcd_tiles = false;
  } else {
    zq = blockIdx.y / g.splits;
    split = blockIdx.y - zq * g.splits;
    bid = blockIdx.x;
  }
  const int z = g.phased ? (int)g.phase_order[zq] : zq;
  const int zz = z * g.splits + split;  // partial-sum slot
  const int R = rows_of(g, z);
  const int Kred = kred_of(g, z);
  const int tiles_m = g.phased ? (R + BM - 1) / BM : g.tiles_m;

  // XCD-aware tile order: workgroups are dealt round-robin over the 8 XCDs, so map
  // consecutive block ids of one XCD onto consecutive tiles (shared operand panels stay
  // in that XCD's L2).
  const int nt = tiles_m * g.tiles_n;
  if (bid >= nt) return;  // phased launches size the grid for the largest phase
  const int per = nt >> 3;
  const int t = (xcd_tiles && bid < (per << 3)) ? ((bid & 7) * per + (bid >> 3)) : bid;
  const int tmi = t / g.tiles_n;
  const int tni = t - tmi * g.tiles_n;
  const int m0 = tmi * BM;
  const int n0 = tni * BN;
  const int kbeg = split * g.k_chunk;
  const int kend = min(Kred, kbeg + g.k_chunk);

  LA la;
  LB lb;
  la.init(g.a, z, m0, tid, kend);
  lb.init(g.b, z, n0, tid, kend);

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

  const int nk = kbeg < kend ? (kend - kbeg + BK - 1) / BK : 0;
  // a split past this phase's reduction contributes nothing; the reduction skips it
  if (g.phased && g.partial && nk == 0) return;
  // The k-loop below runs a whole number of its periods and issues every fetch and LDS
  // store without a condition: tiles past the block's reduction (the padding tile of an
  // odd count, the prefetches past the end) read as zeros and add nothing. With no
  // conditional loads, the compiler can count the loads still in flight exactly and waits
  // only for the stage it stores, keeping the next tiles' loads in flight.
  if (nk > 0) {
    la.fetch(g.a, z, m0, kbeg);
    lb.fetch(g.b, z, n0, kbeg);
    la.store(smem);
    lb.store(smem + SA);
    // tiles 1 .. PF-1 go to register stages 1 .. PF-1
    static_for<1, PF>([&](auto U) {
      constexpr int u = decltype(U)::value;
      la.template fetch<u>(g.a, z, m0, kbeg + u * BK);
      lb.template fetch<u>(g.b, z, n0, kbeg + u * BK);
    });
  }
  __syncthreads();

  // one k-tile of MFMAs on LDS buffer sA
  auto compute_tile = [&](const float* sA, auto&& mid) {
    const float* sB = sA + SA;
    {
      // MFMA k-step s takes reduction indices s (lanes 0-31) and NS + s (lanes 32-63) of
      // the tile, the same assignment for both operands. Row-major (K4) tiles give a lane
      // its 8 values with two 16-byte reads at the start of the tile; for the others the
      // fragments of k-step s+2 are read while the MFMAs of k-step s run (in the forward
      // product, scheduling barriers keep the compiler from sinking the reads next to
      // their use).
      constexpr int NS = BK / 2;
      constexpr int PD = 2;
      // fa[t] / fb[t]: fragments of the operand's tensor t (mean, then variance)
      float fa[NA][NS][TM], fb[NB][NS][TN];
      auto load = [&](int s) {
        const int kr = hl * NS + s;
        if constexpr (!LA::KMAJ) {
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            const int c = kr * LDA + wm * WM + i * 32 + rl;
#pragma unroll
            for (int t = 0; t < NA; ++t) fa[t][s][i] = sA[t * LA::TILE + c];
          }
        }
        if constexpr (!LB::KMAJ) {
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int c = kr * LDB + wn * WN + j * 32 + rl;
#pragma unroll
            for (int t = 0; t < NB; ++t) fb[t][s][j] = sB[t * LB::TILE + c];
          }
        }
      };
      if constexpr (LA::KMAJ) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int row = wm * WM + i * 32 + rl;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int o = LA::kmaj_off(row, hl * NS + 4 * h);
#pragma unroll
            for (int t = 0; t < NA; ++t) {
              const float4 x = *reinterpret_cast<const float4*>(sA + t * LA::TILE + o);
              fa[t][4 * h + 0][i] = x.x;
              fa[t][4 * h + 1][i] = x.y;
              fa[t][4 * h + 2][i] = x.z;
              fa[t][4 * h + 3][i] = x.w;
            }
          }
        }
      }
      if constexpr (LB::KMAJ) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int row = wn * WN + j * 32 + rl;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int o = LB::kmaj_off(row, hl * NS + 4 * h);
#pragma unroll
            for (int t = 0; t < NB; ++t) {
              const float4 x = *reinterpret_cast<const float4*>(sB + t * LB::TILE + o);
              fb[t][4 * h + 0][j] = x.x;
              fb[t][4 * h + 1][j] = x.y;
              fb[t][4 * h + 2][j] = x.z;
              fb[t][4 * h + 3][j] = x.w;
            }
          }
        }
      }
      auto mma = [&](int s) {
        const float* a0 = fa[0][s];
        const float* b0 = fb[0][s];
        if constexpr (PROD == PROD_FWD) {
          const float* a1 = fa[1][s];
          const float* b1 = fb[1][s];
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
          const float* a1 = fa[1][s];
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
          const float* b1 = fb[1][s];
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
      };
#pragma unroll
      for (int s = 0; s < PD; ++s) load(s);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (s + PD < NS) load(s + PD);
        // the forward product keeps its fragment reads ahead of the MFMAs (a barrier after
        // them as well is 0.4% slower); the two-product kernels run 1-3% faster with the
        // compiler's own interleaving
        if constexpr (PROD == PROD_FWD) __builtin_amdgcn_sched_barrier(0);
        mma(s);
        if (s == NS / 2 - 1) {
          mid();
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };
  // Tile t is in LDS buffer t & 1 and tile t+1 in register stage (t+1) % 2. Step t
  // fetches tile t+2 into stage t % 2 (whose tile went to LDS during step t-1), runs tile
  // t's MFMAs and, halfway through them, stores tile t+1 to buffer (t+1) & 1, which no
  // wave reads after the barrier that ended step t-1. The loop runs in periods of two
  // steps so that every buffer and stage index is a compile-time constant.
  constexpr int PERIOD = 2;
  // EPI 2 with one 32 x 32 tile per wave: the epilogue's operands (each output's
  // variance and mean before the update) are loaded during the last period's MFMAs, in
  // place of that period's fetches, which would only read past the reduction. Without
  // it every block of a round reaches its epilogue at about the same time and waits
  // there for those loads with the matrix cores idle (K = 256: a quarter of the time).
  constexpr bool EPF = EPI == 2 && TM == 1 && TN == 1 && KA == LD_STR_MN4;
  float epf_s[EPF ? 16 : 1];
  auto epf_load = [&] {
    if constexpr (EPF) {
      const Epi& e = g.epi;
      const int col = n0 + wn * WN + rl;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + 8 * (v >> 2) + 4 * hl + (v & 3);
        epf_s[v] = 1.f;
        if (row < R && col < g.C) {
          if (row < e.wrows) {
            int wr = row;
            if (e.perm_C > 0) {
              const int kidx = fdiv(row, e.dperm);
              wr = (row - kidx * e.perm_C) * e.perm_kk2 + kidx;
            }
            const int64_t wi = (int64_t)wr * e.ldw + col;
            epf_s[v] = e.Sw[wi];
          } else {
            epf_s[v] = e.Sb[col];
          }
        }
      }
    }
  };
  // EPI 1 and 3 (stride 1: GEMM row r is input pixel r): the BatchNorm2D's saved m_hat
  // and the ReLU Jacobian of the lane's 16 outputs, loaded the same way (the host keeps
  // R * C below 2^31, so 32-bit offsets); in the 64 x 64 tiles, the ones the ResNet
  // stages use (in the others the registers would cost occupancy or spill)
  constexpr bool EPFB = (EPI == 1 || EPI == 3) && BM == 64 && BN == 64 && TM == 1 && TN == 1;
  float epb_h[EPFB ? 16 : 1], epb_j[EPFB ? 16 : 1];
  auto epb_load = [&] {
    if constexpr (EPFB) {
      const Epi& e = g.epi;
      const int col = n0 + wn * WN + rl;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + 8 * (v >> 2) + 4 * hl + (v & 3);
        const bool ok = row < R && col < g.C;
        const int off = row * g.C + col;
        epb_h[v] = ok ? e.bn_mhat[off] : 0.f;
        epb_j[v] = ok ? e.bn_J[off] : 0.f;
      }
    }
  };
  constexpr bool PEEL = EPF || EPFB;
  const int kt_end = (PEEL && nk > 0) ? ((nk - 1) / PERIOD) * PERIOD : nk;
  for (int kt = 0; kt < kt_end; kt += PERIOD) {
    static_for<0, PERIOD>([&](auto U) {
      constexpr int u = decltype(U)::value;
      const int t = kt + u;
      la.template fetch<u % PF>(g.a, z, m0, kbeg + (t + PF) * BK);
      lb.template fetch<u % PF>(g.b, z, n0, kbeg + (t + PF) * BK);
      float* nA = smem + ((u + 1) & 1) * (SA + SB);
      compute_tile(smem + (u & 1) * (SA + SB), [&] {
        la.template store<(u + 1) % PF>(nA);
        lb.template store<(u + 1) % PF>(nA + SA);
      });
      __syncthreads();
    });
  }
  if constexpr (PEEL) {
    static_assert(PERIOD == 2 && PF == 2, "the last period below is written for two steps and two stages");
    if (nk > 0) {
      // the last period: tile kt_end (buffer 0), then tile kt_end + 1 (buffer 1, fetched
      // into stage 1 during the previous period; zeros when nk is odd); nothing is fetched
      compute_tile(smem, [&] {
        la.template store<1>(smem + (SA + SB));
        lb.template store<1>(smem + (SA + SB) + SA);
        epf_load();
        epb_load();
      });
      __syncthreads();
      compute_tile(smem + (SA + SB), [] {});
      __syncthreads();
    } else {
      epf_load();
      epb_load();
    }
  }

  // Epilogue: split-K partial sums, or the layer's epilogue. The epilogue kind is the same
  // for the whole launch, so each kind gets its own unrolled loop with the per-block
  // invariants (bias columns, the stride phase and its pixel dividers) hoisted out.
  const Epi& e = g.epi;
  if (g.partial) {
    const int64_t plane = (int64_t)g.R * g.C;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          const int col = n0 + wn * WN + j * 32 + rl;
          if (row < R && col < g.C) {
            const int64_t base = ((int64_t)zz * 2) * plane + (int64_t)row * g.C + col;
            g.partial[base] = accM[i][j][v];
            g.partial[base + plane] = accV[i][j][v];
          }
        }
  } else if (e.kind == 0 && e.b_sr == 0) {
    // plain store with an optional per-column bias (Linear, Conv2D forward, bmm)
    const int64_t zoff = (z / e.zdiv) * e.sz1 + (z % e.zdiv) * e.sz2;
    const bool st = e.st_ws != nullptr;
    float* red = smem;  // [BM / WM][3][BN] column sums per wave row (LDS is free here)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WN + j * 32 + rl;
      const bool cok = col < g.C;
      const float bmj = (e.bm && cok) ? e.bm[(int64_t)col * e.b_sc] : 0.f;
      const float bvj = (e.bv && cok) ? e.bv[(int64_t)col * e.b_sc] : 0.f;
      const int64_t coff = zoff + (int64_t)col * e.scol;
      float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        // Multiplier and addend of the lane's 16 outputs are loaded before any store: the
        // addend may alias the output, so loads issued after a store could not be moved
        // ahead of it and every element would wait for the previous one's store.
        // (linear and batched products only: in the conv kernels the extra registers cost
        // more occupancy than the loads gain)
        constexpr bool PRE = KA <= LD_STR_K_S;
        float jv[16], av0[16], av1[16];
        if (PRE && (e.jm || e.am)) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
            const bool ok = row < R && cok;
            const int64_t off = coff + (int64_t)row * e.srow;
            jv[v] = (e.jm && ok) ? e.jm[off] : 1.f;
            av0[v] = (e.am && ok) ? e.am[off] : 0.f;
            av1[v] = (e.am && ok) ? e.av[off] : 0.f;
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          if (row < R && cok) {
            const int64_t off = coff + (int64_t)row * e.srow;
            float m = accM[i][j][v] * e.sm + bmj, vv = accV[i][j][v] * e.sv + bvj;
            if (e.jm) {
              const float jj = PRE ? jv[v] : e.jm[off];
              m *= jj;
              vv *= jj * jj;
            }
            if (e.am) {
              m += PRE ? av0[v] : e.am[off];
              vv += PRE ? av1[v] : e.av[off];
            }
            if constexpr (EPI == 4) {
              float ra, rS, rJ;
              relu_moments(m, vv, ra, rS, rJ);
              e.om[off] = ra;
              e.ov[off] = rS;
              e.relu_J[off] = rJ;
              continue;
            }
            if (e.om) e.om[off] = m;
            e.ov[off] = vv;
            if (st) {
              float ra, rS, rJ;
              relu_moments(m, vv, ra, rS, rJ);
              e.st_J[off] = rJ;
              s0 += ra;
              s1 += rS;
              s2 += ra * ra;
            }
          }
        }
      }
      if (st) {
        // lanes l and l + 32 hold the same column
        s0 += __shfl_xor(s0, 32, 64);
        s1 += __shfl_xor(s1, 32, 64);
        s2 += __shfl_xor(s2, 32, 64);
        if (hl == 0) {
          const int cl = wn * WN + j * 32 + rl;
          red[(wm * 3 + 0) * BN + cl] = s0;
          red[(wm * 3 + 1) * BN + cl] = s1;
          red[(wm * 3 + 2) * BN + cl] = s2;
        }
      }
    }
    if (st) {
      __syncthreads();
      for (int cl = tid; cl < BN; cl += NTH) {
        const int col = n0 + cl;
        if (col < g.C) {
#pragma unroll
          for (int q = 0; q < 3; ++q) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < BM / WM; ++w) sum += red[(w * 3 + q) * BN + cl];
            e.st_ws[((int64_t)q * g.C + col) * e.st_nblk + tmi] = sum;
          }
        }
      }
    }
  } else if (e.kind == 2) {
    // conv input delta: row q of stride phase z is input pixel (n, hh*s + a, ww*s + b)
    const Phase ph = make_phase(e.g, z);
    const int hq = ph.Hq * ph.Wq;
    const FastDiv dhq = make_fastdiv(hq > 0 ? hq : 1), dwq = make_fastdiv(ph.Wq > 0 ? ph.Wq : 1);
    // With an addend (the shortcut deltas, possibly the output itself), a lane's 16 addends
    // of a column are loaded before any of its outputs is stored: a load issued after a
    // store to a possibly aliasing address would wait for it, element by element.
    constexpr bool bn = EPI == 1 || EPI == 3;
    float* red = smem;  // BatchNorm sums: [BM / WM][6][BN] column sums per wave row
    static_assert((BM / WM) * 6 * BN <= 2 * (SA + SB), "BatchNorm sums must fit the LDS tiles");
    float bsum[TN][6];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 6; ++q) bsum[j][q] = 0.f;
    if constexpr (EPFB) {
      // m_hat and J are in registers (loaded during the last k-period); EPI 3 loads its
      // addends 8 at a time, each group before its stores (which may alias them)
      const int col = n0 + wn * WN + rl;
      if (col < g.C) {
        const float rv = e.bn_var[col] + e.bn_eps;
        const float km = e.bn_g[col] * (1.0f / sqrtf(rv));
        const float kS = e.bn_g[col] * e.bn_g[col] * (1.0f / rv);
        float ad0[EPI == 3 ? 8 : 1], ad1[EPI == 3 ? 8 : 1];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm * WM + 8 * (v >> 2) + 4 * hl + (v & 3);
          if constexpr (EPI == 3) {
            if ((v & 7) == 0) {
#pragma unroll
              for (int u = 0; u < 8; ++u) {
                const int ru = m0 + wm * WM + 8 * ((v + u) >> 2) + 4 * hl + ((v + u) & 3);
                const int ou = ru * g.C + col;
                ad0[u] = ru < R ? e.am[ou] : 0.f;
                ad1[u] = ru < R ? e.av[ou] : 0.f;
              }
            }
          }
          if (row >= R) continue;
          const int off = row * g.C + col;
          float a = accM[0][0][v], b = accV[0][0][v];
          if constexpr (EPI == 3) {
            a = a + ad0[v & 7];
            b = b + ad1[v & 7];
            e.om[off] = a;
            e.ov[off] = b;
          }
          const float h = epb_h[v], jj = epb_j[v];
          bsum[0][0] += a * h;
          bsum[0][1] += b * h * h;
          bsum[0][2] += a;
          bsum[0][3] += b;
          float o0 = a * km, o1 = b * kS;
          o0 = o0 * jj;
          o1 = o1 * jj * jj;
          bsum[0][4] += o0;
          bsum[0][5] += o1;
          if constexpr (EPI == 3) {
            e.bn_om[off] = o0;
            e.bn_ov[off] = o1;
          } else {
            e.om[off] = o0;
            e.ov[off] = o1;
          }
        }
      }
    } else
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      int64_t pixc[16];  // pixel offset * C, or -1 past the phase's rows
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
        const int n = fdiv(row, dhq), rr = row - n * hq;
        const int hh = fdiv(rr, dwq), ww = rr - hh * ph.Wq;
        const int64_t pix = ((int64_t)n * e.g.H + (hh * e.g.stride + ph.a)) * e.g.W + (ww * e.g.stride + ph.b);
        pixc[v] = row < R ? pix * e.g.C : -1;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + rl;
        if (col >= g.C) continue;
        if constexpr (bn) {
          // the same operations, in the same order, as the separate BatchNorm2D -> ReLU
          // backward pass (bn_reduce_kernel MODE 4), so the outputs are identical
          const float rv = e.bn_var[col] + e.bn_eps;
          const float km = e.bn_g[col] * (1.0f / sqrtf(rv));
          const float kS = e.bn_g[col] * e.bn_g[col] * (1.0f / rv);
          // EPI 3 in two halves of 8 outputs (all four operands of 16 at once would cost
          // occupancy); each half's loads come before its stores, which may alias the addend
          constexpr int NH = EPI == 3 ? 2 : 1, HV = 16 / NH;
#pragma unroll
          for (int hh = 0; hh < NH; ++hh) {
            float hv[HV], jv[HV], ad0[HV], ad1[HV];
#pragma unroll
            for (int u = 0; u < HV; ++u) {
              const int v = hh * HV + u;
              hv[u] = pixc[v] >= 0 ? e.bn_mhat[pixc[v] + col] : 0.f;
              jv[u] = pixc[v] >= 0 ? e.bn_J[pixc[v] + col] : 0.f;
              if constexpr (EPI == 3) {
                ad0[u] = pixc[v] >= 0 ? e.am[pixc[v] + col] : 0.f;
                ad1[u] = pixc[v] >= 0 ? e.av[pixc[v] + col] : 0.f;
              }
            }
#pragma unroll
            for (int u = 0; u < HV; ++u) {
              const int v = hh * HV + u;
              if (pixc[v] < 0) continue;
              const int64_t off = pixc[v] + col;
              float a = accM[i][j][v], b = accV[i][j][v];
              if constexpr (EPI == 3) {
                a = a + ad0[u];
                b = b + ad1[u];
                e.om[off] = a;
                e.ov[off] = b;
              }
              const float h = hv[u], jj = jv[u];
              bsum[j][0] += a * h;
              bsum[j][1] += b * h * h;
              bsum[j][2] += a;
              bsum[j][3] += b;
              float o0 = a * km, o1 = b * kS;
              o0 = o0 * jj;
              o1 = o1 * jj * jj;
              bsum[j][4] += o0;
              bsum[j][5] += o1;
              if constexpr (EPI == 3) {
                e.bn_om[off] = o0;
                e.bn_ov[off] = o1;
              } else {
                e.om[off] = o0;
                e.ov[off] = o1;
              }
            }
          }
          continue;
        }
        float addm[16], addv[16];
        if (e.am) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            addm[v] = pixc[v] >= 0 ? e.am[pixc[v] + col] : 0.f;
            addv[v] = pixc[v] >= 0 ? e.av[pixc[v] + col] : 0.f;
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          if (pixc[v] < 0) continue;
          const int64_t off = pixc[v] + col;
          float m = accM[i][j][v], vv = accV[i][j][v];
          if (e.am) {
            m = m + addm[v];
            vv = vv + addv[v];
          }
          e.om[off] = m;
          e.ov[off] = vv;
        }
      }
    }
    if constexpr (bn) {
      // lanes l and l + 32 hold the same column; then the tile's wave rows in order
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int q = 0; q < 6; ++q) bsum[j][q] += __shfl_xor(bsum[j][q], 32, 64);
        if (hl == 0) {
          const int cl = wn * WN + j * 32 + rl;
#pragma unroll
          for (int q = 0; q < 6; ++q) red[(wm * 6 + q) * BN + cl] = bsum[j][q];
        }
      }
      __syncthreads();
      for (int cl = tid; cl < BN; cl += NTH) {
        const int col = n0 + cl;
        if (col < g.C) {
#pragma unroll
          for (int q = 0; q < 6; ++q) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < BM / WM; ++w) sum += red[(w * 6 + q) * BN + cl];
            e.st_ws[((int64_t)q * g.C + col) * e.st_nblk + tmi] = sum;
          }
        }
      }
    }
  } else if (e.kind == 1) {
    // parameter deltas (unsplit): the Sw (Sb) factors of a lane's 16 outputs are loaded
    // before any of them is stored -- the stores may alias them as far as the compiler
    // knows, so a load issued after a store would wait for it, element by element
    const bool keep = e.om != nullptr;  // the update without stored deltas: om, dmb null
    (void)keep;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + rl;
        if constexpr (EPF) {
          // the variances were loaded during the last k-period; the means are loaded one
          // group of 4 ahead of the stores (a load after a store that may alias it would
          // wait for it)
          auto widx = [&](int v) -> int64_t {
            const int row = m0 + wm * WM + 8 * (v >> 2) + 4 * hl + (v & 3);
            if (!(row < R && col < g.C)) return -2;
            if (row >= e.wrows) return -1;
            int wr = row;
            if (e.perm_C > 0) {
              const int kidx = fdiv(row, e.dperm);
              wr = (row - kidx * e.perm_C) * e.perm_kk2 + kidx;
            }
            return (int64_t)wr * e.ldw + col;
          };
          float pm[4][4];
          auto load_means = [&](int q) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int64_t w = widx(4 * q + u);
              pm[q][u] = w >= 0 ? e.upd_mw[w] : (w == -1 ? e.upd_mb[col] : 0.f);
            }
          };
          load_means(0);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (q < 3) load_means(q + 1);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int64_t w = widx(4 * q + u);
              if (w == -2) continue;
              const float sv = epf_s[4 * q + u];
              const float dm = sv * accM[0][0][4 * q + u], dS = (sv * sv) * accV[0][0][4 * q + u];
              float pmu = pm[q][u], pS = sv;
              capped(pmu, pS, dm, dS, e.cap);
              if (w >= 0) {
                if (keep) {
                  e.om[w] = dm;
                  e.ov[w] = dS;
                }
                e.upd_mw[w] = pmu;
                e.upd_Sw[w] = pS;
              } else {
                if (keep) {
                  e.dmb[col] = dm;
                  e.dSb[col] = dS;
                }
                e.upd_mb[col] = pmu;
                e.upd_Sb[col] = pS;
              }
            }
          }
          continue;
        } else if constexpr (EPI == 2) {
          // with the capped update in place: per group of 4 outputs, the variances and
          // means are loaded before the group's stores (16 at once would cost occupancy)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float sv4[4], pm4[4];
            int64_t wi[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int row = m0 + wm * WM + i * 32 + 8 * q + 4 * hl + u;
              sv4[u] = 1.f;
              pm4[u] = 0.f;
              wi[u] = -1;
              if (row < R && col < g.C) {
                if (row < e.wrows) {
                  int wr = row;
                  if (e.perm_C > 0) {
                    const int kidx = fdiv(row, e.dperm);
                    wr = (row - kidx * e.perm_C) * e.perm_kk2 + kidx;
                  }
                  wi[u] = (int64_t)wr * e.ldw + col;
                  sv4[u] = e.Sw[wi[u]];
                  pm4[u] = e.upd_mw[wi[u]];
                } else {
                  sv4[u] = e.Sb[col];
                  pm4[u] = e.upd_mb[col];
                }
              }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int row = m0 + wm * WM + i * 32 + 8 * q + 4 * hl + u;
              if (row < R && col < g.C) {
                const float sv = sv4[u];
                const float dm = sv * accM[i][j][4 * q + u], dS = (sv * sv) * accV[i][j][4 * q + u];
                float pm = pm4[u], pS = sv;
                capped(pm, pS, dm, dS, e.cap);
                if (row < e.wrows) {
                  if (keep) {
                    e.om[wi[u]] = dm;
                    e.ov[wi[u]] = dS;
                  }
                  e.upd_mw[wi[u]] = pm;
                  e.upd_Sw[wi[u]] = pS;
                } else {
                  if (keep) {
                    e.dmb[col] = dm;
                    e.dSb[col] = dS;
                  }
                  e.upd_mb[col] = pm;
                  e.upd_Sb[col] = pS;
                }
              }
            }
          }
          continue;
        }
        float sf[16];
        int64_t widx[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          sf[v] = 1.f;
          widx[v] = -1;
          if (row < R && col < g.C) {
            if (row < e.wrows) {
              int wr = row;
              if (e.perm_C > 0) {
                const int kidx = fdiv(row, e.dperm);
                wr = (row - kidx * e.perm_C) * e.perm_kk2 + kidx;
              }
              widx[v] = (int64_t)wr * e.ldw + col;
              if (e.Sw) sf[v] = e.Sw[widx[v]];
            } else if (e.Sb) {
              sf[v] = e.Sb[col];
            }
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          if (row < R && col < g.C) {
            const float sv = sf[v];
            if (row < e.wrows) {
              e.om[widx[v]] = sv * accM[i][j][v];
              e.ov[widx[v]] = (sv * sv) * accV[i][j][v];
            } else {
              e.dmb[col] = sv * accM[i][j][v];
              e.dSb[col] = (sv * sv) * accV[i][j][v];
            }
          }
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          const int col = n0 + wn * WN + j * 32 + rl;
          if (row < R && col < g.C) epi_apply(e, z, row, col, accM[i][j][v], accV[i][j][v]);
        }
  }
}

// Deterministic split-K reduction followed by the epilogue. A block owns 64*V consecutive
// output elements; its G waves each sum the splits s = g, g+G, g+2G, ... of those
// elements (V at a time), then wave 0 adds the G wave sums in order g = 0..G-1. The
// summation order depends only on (splits, G), so results repeat bit for bit.
// For the phased conv input delta (k_chunk > 0) phase z sums only the splits that
// cover its own reduction length.
template <int G, int V>
__global__ void __launch_bounds__(64 * G) splitk_reduce_kernel(const float* __restrict__ partial, Epi epi, int batch,
                                                                int splits, int R, int C, int k_chunk) {
  __shared__ float red[G > 1 ? 2 * (G - 1) * 64 * V : 1];
  const int64_t plane = (int64_t)R * C;
  const int64_t total = plane * batch;
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  const int64_t idx0 = ((int64_t)blockIdx.x * 64 + lane) * V;
  float m[V], v[V];
#pragma unroll
  for (int e = 0; e < V; ++e) m[e] = v[e] = 0.f;
  int z = 0;
  int64_t rc = 0;
  if (idx0 < total) {
    z = (int)(idx0 / plane);
    rc = idx0 - (int64_t)z * plane;
    const float* p = partial + ((int64_t)z * splits * 2) * plane + rc;
    int ns = splits;
    if (k_chunk > 0) {
      const Phase ph = make_phase(epi.g, z);
      const int kz = ph.nkh * ph.nkw * epi.g.Cout;
      ns = min(splits, (kz + k_chunk - 1) / k_chunk);
    }
    if constexpr (V == 4) {
      // plane % 4 == 0: the 4 elements lie in one plane, 16-byte aligned
      for (int s = g; s < ns; s += G) {
        const float4 a = *reinterpret_cast<const float4*>(p + (int64_t)(2 * s) * plane);
        const float4 b = *reinterpret_cast<const float4*>(p + (int64_t)(2 * s + 1) * plane);
        m[0] += a.x; m[1] += a.y; m[2] += a.z; m[3] += a.w;
        v[0] += b.x; v[1] += b.y; v[2] += b.z; v[3] += b.w;
      }
    } else {
      for (int s = g; s < ns; s += G) {
        m[0] += p[(int64_t)(2 * s) * plane];
        v[0] += p[(int64_t)(2 * s + 1) * plane];
      }
    }
  }
  if constexpr (G > 1) {
    if (g > 0) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        red[((g - 1) * 2) * 64 * V + lane * V + e] = m[e];
        red[((g - 1) * 2 + 1) * 64 * V + lane * V + e] = v[e];
      }
    }
    __syncthreads();
    if (g != 0) return;
#pragma unroll
    for (int h = 1; h < G; ++h)
#pragma unroll
      for (int e = 0; e < V; ++e) {
        m[e] += red[((h - 1) * 2) * 64 * V + lane * V + e];
        v[e] += red[((h - 1) * 2 + 1) * 64 * V + lane * V + e];
      }
  }
  if (idx0 >= total) return;
  if constexpr (V == 4) {
    if (C % 4 == 0) {
      // the 4 elements are consecutive columns of one row
      const int row = (int)(rc / C);
      if (epi_apply4(epi, z, row, (int)(rc - (int64_t)row * C), m, v)) return;
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int64_t r = rc + e;
    if (V > 1 && idx0 + e >= total) break;
    const int row = (int)(r / C);
    const int col = (int)(r - (int64_t)row * C);
    epi_apply<true>(epi, z, row, col, m[e], v[e]);
  }
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int V>
static inline void launch_reduce(const float* ws, const Epi& epi, int64_t batch, int splits, int R, int C,
                                 int k_chunk, hipStream_t s) {
  const int64_t total = (int64_t)R * C * batch;
  const int64_t blocks = cdiv(total, 64 * V);
  // enough waves in flight to cover HBM latency: aim for ~4096 waves over the chip
  int G = 1;
  while (G < 16 && G * 2 <= splits && blocks * G < 4096) G *= 2;
  const dim3 grid((unsigned)blocks);
  switch (G) {
    case 1: hipLaunchKernelGGL((splitk_reduce_kernel<1, V>), grid, dim3(64), 0, s, ws, epi, (int)batch, splits, R, C, k_chunk); break;
    case 2: hipLaunchKernelGGL((splitk_reduce_kernel<2, V>), grid, dim3(128), 0, s, ws, epi, (int)batch, splits, R, C, k_chunk); break;
    case 4: hipLaunchKernelGGL((splitk_reduce_kernel<4, V>), grid, dim3(256), 0, s, ws, epi, (int)batch, splits, R, C, k_chunk); break;
    case 8: hipLaunchKernelGGL((splitk_reduce_kernel<8, V>), grid, dim3(512), 0, s, ws, epi, (int)batch, splits, R, C, k_chunk); break;
    default: hipLaunchKernelGGL((splitk_reduce_kernel<16, V>), grid, dim3(1024), 0, s, ws, epi, (int)batch, splits, R, C, k_chunk); break;
  }
}

// ------------------------------------------------------------------------------------
// Host side: tile-config choice, split-K choice and launch.
// ------------------------------------------------------------------------------------
using C128x128 = Cfg<128, 128, 64, 32>;  // 8 waves, 64x32 per wave
using C128x64 = Cfg<128, 64, 64, 32>;    // 4 waves
using C64x128 = Cfg<64, 128, 32, 64>;    // 4 waves
using C64x64 = Cfg<64, 64, 32, 32>;      // 4 waves
using C32x32 = Cfg<32, 32, 32, 32>;      // 1 wave
using C128x32 = Cfg<128, 32, 32, 32>;    // 4 waves stacked along M (products with 32 columns)

struct CfgDesc {
  int BM, BN;
};
static const CfgDesc kCfg[] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}, {32, 32}, {128, 32}};
static const int kNumCfg = 6;

struct Plan {
  int cfg;
  int splits;
  int k_chunk;
  int tiles_m, tiles_n;
};

// Pick the tile shape and split-K factor minimising a time model of the launch:
//   * blocks run in rounds of 256 CUs x (resident blocks per CU); a partial last round
//     runs at the occupancy of the blocks it holds (a lone block per CU leaves the MFMA
//     pipes half idle);
//   * each tile shape and product sustains a fraction of the fp32 MFMA peak (operand
//     loads, LDS traffic and epilogue per flop), and fewer than ~3 waves per SIMD expose
//     latency;
//   * split-K adds the partial sums' round trip (8 bytes per element and split, written
//     and read back, mostly through the last-level cache) plus the reduction launch.
// Resident blocks per CU are what the built kernels' register and LDS use allow (the
// 8-wave 128x128 kernels need more than 128 VGPRs, so one block per CU). The sustained
// fractions, the occupancy factors and the split costs were fitted to a sweep of every
// tile shape and split count (each plan forced in turn and timed alone) over the
// ResNet-18, CNN, transformer (including its batched attention products) and Linear
// microbenchmark GEMMs on MI355X: mean loss against the best measured plan 1.5%. (Twice
// the cost per partial-sum byte, for reductions that share the GPU with the other
// stream's GEMMs, gives ResNet-18 +0.5% but the CNN's input deltas -20%.) The split
// counts tried are the swept ones.
//
// phase_k (optional, batch entries): per-GEMM reduction lengths when they differ (stride
// phases of the conv input delta); splits past a GEMM's own length launch no work.
static inline Plan choose_plan_uncached(int64_t R, int64_t C, int64_t Kred, int64_t batch, int prod, bool allow_split,
                                        int64_t max_splits, const int64_t* phase_k) {
  // [tile config][product: forward, shared B, shared A]
  static const int kBpc[6][3] = {{1, 1, 1}, {2, 3, 3}, {2, 3, 2}, {4, 4, 4}, {8, 10, 10}, {3, 4, 4}};
  static const double kEff[6][3] = {{0.624, 0.353, 0.483}, {0.595, 0.632, 0.608}, {0.465, 0.519, 0.492},
                                    {0.655, 0.639, 0.687}, {0.300, 0.398, 0.442}, {0.655, 0.374, 0.427}};
  static const int kWaves[] = {8, 4, 4, 4, 1, 4};
  // (up to 512: the parameter deltas of a conv on a 3-channel input reduce over all N*H*W
  // pixels into one or two tiles, so their splits are the whole launch)
  static const int kSplits[] = {1,  2,  3,  4,  5,  6,   8,   10,  12,  16,  20,  24,  32,
                                40, 48, 64, 80, 96, 128, 160, 192, 256, 320, 384, 512};
  const double kOcc2 = 0.924, kOcc1 = 0.667, kOcc0 = 0.35;
  const double kSplitSecPerByte = 1.82e-13, kSplitLaunch = 5.95e-6;
  // Small problems (fewer than 128 tiles of 64 x 64, the Linear layers of the MLP and CNN
  // heads): a block's k-loop waits on its loads' latency rather than on the matrix cores,
  // so a round takes at least kChainFixed + kChainTile per k-tile of the block, and the
  // reduction of their few partial sums costs less than a large one's. Fitted to a sweep
  // of every tile config and split count on those shapes (kernel-trace durations). Not for
  // the phased conv input deltas, whose unsplit plans carry the folded BatchNorm backward.
  static const double kChainTile[6] = {2.4e-6, 1.8e-6, 1.8e-6, 0.96e-6, 1.0e-6, 1.05e-6};
  const double kChainFixed = 3.5e-6, kSplitLaunchSmall = 3.0e-6;
  const bool small = !phase_k && cdiv(R, 64) * cdiv(C, 64) * batch < 128;
  const int products = prod == PROD_FWD ? 3 : 2;
  Plan best{3, 1, (int)Kred, 1, 1};
  double best_t = DBL_MAX;
  const double peak_cu = 157.3e12 / 256.0;
  const int64_t max_sp = allow_split ? (max_splits < 512 ? max_splits : 512) : 1;
  for (int ci = 0; ci < kNumCfg; ++ci) {
    const int BM = kCfg[ci].BM, BN = kCfg[ci].BN;
    const int64_t tm = cdiv(R, BM), tn = cdiv(C, BN);
    const int bpc = kBpc[ci][prod];
    int64_t prev_actual = -1;
    for (int si = 0; si < (int)(sizeof(kSplits) / sizeof(kSplits[0])) && kSplits[si] <= max_sp; ++si) {
      const int64_t sp = kSplits[si];
      int64_t kc = cdiv(cdiv(Kred, sp), 16) * 16;
      if (kc < 16) kc = 16;
      const int64_t actual = cdiv(Kred, kc);
      if (actual == prev_actual) continue;
      prev_actual = actual;
      // splits below 4 k-tiles (2 in small problems) only add reduction traffic
      if (actual > 1 && kc < (small ? 32 : 64)) break;
      int64_t blocks = tm * tn * batch * actual;
      if (phase_k) {
        // a phase with a shorter reduction (or the short last chunk of one) does that
        // fraction of a kc block's work; tap-less phases only write zeros
        double eq = 0.0;
        for (int64_t z = 0; z < batch; ++z) eq += (double)(tm * tn) * (phase_k[z] > 0 ? (double)phase_k[z] / kc : 0.1);
        blocks = (int64_t)ceil(eq);
      }
      const double block_s = (2.0 * BM * BN * kc * products) / (peak_cu * kEff[ci][prod]);
      // time for one CU to finish r co-resident blocks
      auto round_s = [&](int64_t r) {
        const double wps = (double)r * kWaves[ci] / 4.0;  // waves per SIMD
        const double occ = wps >= 3.0 ? 1.0 : (wps >= 2.0 ? kOcc2 : (wps >= 1.0 ? kOcc1 : kOcc0));
        const double t = (double)r * block_s / occ;
        return small ? fmax(t, kChainFixed + (double)(kc / 16) * kChainTile[ci]) : t;
      };
      const int64_t slots = 256 * (int64_t)bpc;
      const int64_t full = blocks / slots, rem = blocks - full * slots;
      double t = (double)full * round_s(bpc) + (rem > 0 ? round_s(cdiv(rem, 256)) : 0.0);
      if (actual > 1)
        t += (double)actual * 16.0 * R * C * batch * kSplitSecPerByte + (small ? kSplitLaunchSmall : kSplitLaunch);
      if (t < best_t * 0.999) {
        best_t = t;
        best = Plan{ci, (int)actual, (int)kc, (int)tm, (int)tn};
      }
    }
  }
  return best;
}

// Plans are pure functions of the problem shape; memoise them per host thread (the
// search above costs a few microseconds and the same shapes recur every step).
static inline Plan choose_plan(int64_t R, int64_t C, int64_t Kred, int64_t batch, int prod, bool allow_split,
                               int64_t max_splits, const int64_t* phase_k = nullptr) {
  struct Key {
    int64_t R, C, K, batch, max_splits, salt;
    int prod, allow;
  };
  int64_t salt = 0;
  if (phase_k)
    for (int64_t z = 0; z < batch; ++z) salt = salt * 1000003 + phase_k[z] + 1;
  struct Entry {
    Key k;
    Plan p;
  };
  static thread_local Entry cache[64];
  static thread_local int used = 0, next = 0;
  const Key key{R, C, Kred, batch, max_splits, salt, prod, allow_split ? 1 : 0};
  for (int i = 0; i < used; ++i) {
    const Key& k = cache[i].k;
    if (k.R == R && k.C == C && k.K == Kred && k.batch == batch && k.max_splits == max_splits && k.salt == salt &&
        k.prod == prod && k.allow == key.allow)
      return cache[i].p;
  }
  const Plan p = choose_plan_uncached(R, C, Kred, batch, prod, allow_split, max_splits, phase_k);
  cache[next] = Entry{key, p};
  next = (next + 1) % 64;
  if (used < 64) ++used;
  return p;
}

static inline int64_t plan_ws_bytes(const Plan& p, int64_t R, int64_t C, int64_t batch) {
  return p.splits > 1 ? (int64_t)p.splits * 2 * R * C * batch * (int64_t)sizeof(float) : 0;
}

// The (product, tile config, loader) combinations the entry points launch. Each
// combination's kernel is compiled once, in tagi_gemm_inst.hip (built once per tile
// config and product, so the kernels compile in parallel translation units); the entry
// points' translation units see launch_cfg's declaration only.
#define TAGI_GEMM_COMBOS_FWD(X)                                                          \
  X(PROD_FWD, LD_CFWD_A4T, LD_CFWD_B4T)                                                  \
  X(PROD_FWD, LD_CFWD_A4, LD_CFWD_B4) X(PROD_FWD, LD_CFWD_A_S, LD_CFWD_B4)               \
  X(PROD_FWD, LD_CFWD_A_S, LD_CFWD_B_S) X(PROD_FWD, LD_STR_K4, LD_STR_MN4)               \
  X(PROD_FWD, LD_STR_K_S, LD_STR_MN_S) X(PROD_FWD, LD_STR_MN_S, LD_STR_MN_S)             \
  X(PROD_FWD, LD_STR_K4, LD_STR_K4) X(PROD_FWD, LD_STR_MN4, LD_STR_K4)                   \
  X(PROD_FWD, LD_STR_MN4, LD_STR_MN4)
#define TAGI_GEMM_COMBOS_SHARED_B(X)                                                     \
  X(PROD_SHARED_B, LD_CBWD_A4T, LD_CBWD_BK4T)                                            \
  X(PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_B4) X(PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_BK4)     \
  X(PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_B_S) X(PROD_SHARED_B, LD_CBWD_A_S, LD_CBWD_B_S)   \
  X(PROD_SHARED_B, LD_STR_K4, LD_STR_K4) X(PROD_SHARED_B, LD_STR_K_S, LD_STR_K_S)        \
  X(PROD_SHARED_B, LD_STR_MN_S, LD_STR_MN_S) X(PROD_SHARED_B, LD_STR_K4, LD_STR_MN4)     \
  X(PROD_SHARED_B, LD_STR_MN4, LD_STR_K4) X(PROD_SHARED_B, LD_STR_MN4, LD_STR_MN4)
#define TAGI_GEMM_COMBOS_SHARED_A(X)                                                     \
  X(PROD_SHARED_A, LD_CFWD_A4T, LD_CFWD_B4T)                                             \
  X(PROD_SHARED_A, LD_CFWD_A4, LD_CFWD_B4) X(PROD_SHARED_A, LD_CFWD_A_S, LD_CFWD_B4)     \
  X(PROD_SHARED_A, LD_CFWD_A_S, LD_CFWD_B_S)                                             \
  X(PROD_SHARED_A, LD_CWG_A4T, LD_STR_MN4)                                               \
  X(PROD_SHARED_A, LD_CWG_A4, LD_STR_MN4) X(PROD_SHARED_A, LD_CWG_A_S, LD_STR_MN4)       \
  X(PROD_SHARED_A, LD_CWG_A_S, LD_STR_MN_S)                                              \
  X(PROD_SHARED_A, LD_STR_MN4, LD_STR_MN4) X(PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S)    \
  X(PROD_SHARED_A, LD_STR_K4, LD_STR_K4) X(PROD_SHARED_A, LD_STR_K4, LD_STR_MN4)         \
  X(PROD_SHARED_A, LD_STR_MN4, LD_STR_K4)

// The input-delta loader pairs that also get the folded BatchNorm2D epilogues (EPI 1 and
// 3), in the tile configs with one 32 x 32 tile per wave (64 x 64, 32 x 32, 128 x 32)
#define TAGI_GEMM_COMBOS_SHARED_B_BNF(X)                                                 \
  X(PROD_SHARED_B, LD_CBWD_A4T, LD_CBWD_BK4T) X(PROD_SHARED_B, LD_CBWD_A4, LD_CBWD_BK4)
static inline bool bnf_cfg(int cfg) { return cfg == 3 || cfg == 4 || cfg == 5; }
// The Linear parameter-delta loader pairs that also get the in-place update (EPI 2), in
// every tile config
#define TAGI_GEMM_COMBOS_SHARED_A_UPD(X)                                                 \
  X(PROD_SHARED_A, LD_STR_MN4, LD_STR_MN4) X(PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S)
// The Linear forward loader pairs that also store ReLU(product) (EPI 4), in every tile
// config: the three-product forward, and the two-product one of a zero-variance input
#define TAGI_GEMM_COMBOS_FWD_RELU(X)                                                     \
  X(PROD_FWD, LD_STR_K4, LD_STR_MN4) X(PROD_FWD, LD_STR_K_S, LD_STR_MN_S)
#define TAGI_GEMM_COMBOS_SHARED_A_RELU(X)                                                \
  X(PROD_SHARED_A, LD_STR_K4, LD_STR_MN4) X(PROD_SHARED_A, LD_STR_MN_S, LD_STR_MN_S)

template <int PROD, class CFG, int KA, int KB, int EPI = 0>
void launch_cfg(const GemmArgs& g, int64_t grid_x, int64_t grid_y, hipStream_t s)
#ifdef TAGI_GEMM_DEFINE_LAUNCH
{
  hipLaunchKernelGGL((gemm_kernel<PROD, CFG, KA, KB, EPI>), dim3((unsigned)grid_x, (unsigned)grid_y), dim3(CFG::NTH),
                     0, s, g);
}
#else
    ;
#endif

// Launch with plan p. For phased (conv input-delta) launches grid_x covers the largest
// phase and blocks past a phase's tiles exit at once.
template <int PROD, int KA, int KB, int EPI = 0>
static inline int run_gemm(GemmArgs g, int64_t batch, const Plan& p, float* ws, int64_t ws_bytes, hipStream_t s,
                           const char* what, int64_t grid_x_override = 0) {
  if constexpr (EPI == 1 || EPI == 3)
    TAGI_REQUIRE(bnf_cfg(p.cfg) && p.splits == 1, "%s: folded epilogue needs an unsplit one-tile-per-wave plan",
                 what);
  // operand byte offsets are 32-bit with the out-of-range sentinel above them
  TAGI_REQUIRE(g.a.nbytes >= 0 && g.a.nbytes < (int64_t)kBufOutOfRange && g.b.nbytes >= 0 &&
                   g.b.nbytes < (int64_t)kBufOutOfRange,
               "%s: an operand spans %lld / %lld bytes; at most 2 GiB per operand", what, (long long)g.a.nbytes,
               (long long)g.b.nbytes);
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
  const int64_t gx = grid_x_override > 0 ? grid_x_override : (int64_t)p.tiles_m * p.tiles_n;
  const int64_t gy = batch * p.splits;
  TAGI_REQUIRE(gx > 0 && gx < (1ll << 31) && gy < 65536, "%s: grid out of range (%lld x %lld)", what, (long long)gx,
               (long long)gy);
  if constexpr (EPI == 1 || EPI == 3) {
    switch (p.cfg) {
      case 3: launch_cfg<PROD, C64x64, KA, KB, EPI>(g, gx, gy, s); break;
      case 5: launch_cfg<PROD, C128x32, KA, KB, EPI>(g, gx, gy, s); break;
      default: launch_cfg<PROD, C32x32, KA, KB, EPI>(g, gx, gy, s); break;
    }
  } else {
    // EPI 2 and 4 apply their epilogue in the kernel only when unsplit (the reduction's
    // epilogue does it otherwise, from the same Epi fields)
    constexpr int E = (EPI == 2 || EPI == 4) ? EPI : 0;
    if (E != 0 && p.splits > 1) {
      switch (p.cfg) {
        case 0: launch_cfg<PROD, C128x128, KA, KB>(g, gx, gy, s); break;
        case 1: launch_cfg<PROD, C128x64, KA, KB>(g, gx, gy, s); break;
        case 2: launch_cfg<PROD, C64x128, KA, KB>(g, gx, gy, s); break;
        case 3: launch_cfg<PROD, C64x64, KA, KB>(g, gx, gy, s); break;
        case 5: launch_cfg<PROD, C128x32, KA, KB>(g, gx, gy, s); break;
        default: launch_cfg<PROD, C32x32, KA, KB>(g, gx, gy, s); break;
      }
    } else {
      switch (p.cfg) {
        case 0: launch_cfg<PROD, C128x128, KA, KB, E>(g, gx, gy, s); break;
        case 1: launch_cfg<PROD, C128x64, KA, KB, E>(g, gx, gy, s); break;
        case 2: launch_cfg<PROD, C64x128, KA, KB, E>(g, gx, gy, s); break;
        case 3: launch_cfg<PROD, C64x64, KA, KB, E>(g, gx, gy, s); break;
        case 5: launch_cfg<PROD, C128x32, KA, KB, E>(g, gx, gy, s); break;
        default: launch_cfg<PROD, C32x32, KA, KB, E>(g, gx, gy, s); break;
      }
    }
  }
  int rc = check_launch(what);
  if (rc != TAGI_OK) return rc;
  if (p.splits > 1) {
    if (((int64_t)g.R * g.C) % 4 == 0 && al16(ws))
      launch_reduce<4>(ws, g.epi, batch, p.splits, g.R, g.C, g.phased ? p.k_chunk : 0, s);
    else
      launch_reduce<1>(ws, g.epi, batch, p.splits, g.R, g.C, g.phased ? p.k_chunk : 0, s);
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
  // reach of one batch entry (strides are non-negative)
  o.nbytes = (MN > 0 && K > 0) ? 4 * ((MN - 1) * s_mn + (K - 1) * s_k + 1) : 0;
  return o;
}

static inline Epi epi_store(float* om, float* ov, const float* bm, const float* bv, int64_t b_sr, int64_t b_sc,
                            float sm, float sv, int64_t zdiv, int64_t sz1, int64_t sz2, int64_t srow, int64_t scol) {
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
  e.scol = scol;
  return e;
}

static inline Epi epi_wgrad(float* dmw, float* dSw, float* dmb, float* dSb, const float* Sw, const float* Sb,
                            int64_t wrows, int64_t ldw) {
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
  return e;
}

static inline bool fits_i32(int64_t v) { return v >= 0 && v < (1ll << 31); }


}  // namespace tagi
