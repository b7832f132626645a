// The Linear forward's argument check, plan and launch, shared by tagi_linear.hip (the
// workspace entry point) and tagi_noalloc.hip (the entry point without allocation), so
// that both run the same plan and kernels and give the same bits.
#pragma once

#include "tagi_gemm_core.h"

namespace tagi {

Plan linear_fwd_plan(int64_t M, int64_t K, int64_t N);

int linear_fwd_check(const char* what, const float* ma, const float* Sa, const float* mw, const float* Sw,
                     const float* Sz, int64_t M, int64_t K, int64_t N);

// Launch of the forward product with plan p (split-K partials in ws when p splits). With
// relu_J, mz / Sz receive the moments of ReLU(z) and relu_J its Jacobian instead of z's
// moments.
int linear_fwd_run(const char* what, const float* ma, const float* Sa, const float* mw, const float* Sw,
                   const float* mb, const float* Sb, float* mz, float* Sz, int64_t M, int64_t K, int64_t N,
                   const Plan& p, float* ws, int64_t ws_bytes, hipStream_t s, float* relu_J = nullptr);

}  // namespace tagi
