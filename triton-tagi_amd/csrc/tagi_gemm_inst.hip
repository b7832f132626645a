// Kernel instantiations of the moment GEMM engine: the launch_cfg<product, tile config,
// loaders> combinations listed in tagi_gemm_core.h for one tile config and one product.
// build.py compiles this file once per (TAGI_INST_CFG, TAGI_INST_PROD) pair, so the
// ~200 kernels compile in parallel translation units.
#define TAGI_GEMM_DEFINE_LAUNCH
#include "tagi_gemm_core.h"

#ifndef TAGI_INST_CFG
#error "compile with -DTAGI_INST_CFG=<0..5> -DTAGI_INST_PROD=<0..2>"
#endif

namespace tagi {

#if TAGI_INST_CFG == 0
using InstCfg = C128x128;
#elif TAGI_INST_CFG == 1
using InstCfg = C128x64;
#elif TAGI_INST_CFG == 2
using InstCfg = C64x128;
#elif TAGI_INST_CFG == 3
using InstCfg = C64x64;
#elif TAGI_INST_CFG == 4
using InstCfg = C32x32;
#else
using InstCfg = C128x32;
#endif

#define TAGI_INST(P, KA, KB) template void launch_cfg<P, InstCfg, KA, KB>(const GemmArgs&, int64_t, int64_t, hipStream_t);
#define TAGI_INST_RELU(P, KA, KB) \
  template void launch_cfg<P, InstCfg, KA, KB, 4>(const GemmArgs&, int64_t, int64_t, hipStream_t);
#if TAGI_INST_PROD == 0
TAGI_GEMM_COMBOS_FWD(TAGI_INST)
TAGI_GEMM_COMBOS_FWD_RELU(TAGI_INST_RELU)
#elif TAGI_INST_PROD == 1
TAGI_GEMM_COMBOS_SHARED_B(TAGI_INST)
#if TAGI_INST_CFG >= 3
#define TAGI_INST_BNF(P, KA, KB) \
  template void launch_cfg<P, InstCfg, KA, KB, 1>(const GemmArgs&, int64_t, int64_t, hipStream_t); \
  template void launch_cfg<P, InstCfg, KA, KB, 3>(const GemmArgs&, int64_t, int64_t, hipStream_t);
TAGI_GEMM_COMBOS_SHARED_B_BNF(TAGI_INST_BNF)
#endif
#else
TAGI_GEMM_COMBOS_SHARED_A(TAGI_INST)
#define TAGI_INST_UPD(P, KA, KB) \
  template void launch_cfg<P, InstCfg, KA, KB, 2>(const GemmArgs&, int64_t, int64_t, hipStream_t);
TAGI_GEMM_COMBOS_SHARED_A_UPD(TAGI_INST_UPD)
TAGI_GEMM_COMBOS_SHARED_A_RELU(TAGI_INST_RELU)
#endif

}  // namespace tagi
