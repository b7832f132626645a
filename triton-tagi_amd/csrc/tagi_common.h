// Shared host/device helpers for libtagi_hip: error reporting, launch checks and the
// per-kernel-family event timer used by the roofline report.
//
// Nothing in this library allocates device memory: every buffer (outputs, split-K
// partials, per-channel partial sums) is passed in by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tagi_hip.h"

namespace tagi {

// ---------------------------------------------------------------------------------
// Error state (thread-local message, integer status codes from tagi_hip.h).
// ---------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define TAGI_REQUIRE(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::tagi::fail(TAGI_ERR_ARG, __VA_ARGS__);  \
  } while (0)

// Check the launch that was just queued; returns TAGI_OK or TAGI_ERR_LAUNCH.
int check_launch(const char* what);

// ---------------------------------------------------------------------------------
// Kernel families, for the live timer (tagi_prof_begin / tagi_prof_end).
// ---------------------------------------------------------------------------------
enum Family {
  FAM_CONV_FWD = 0,
  FAM_CONV_BWD_DELTA = 1,
  FAM_CONV_WGRAD = 2,
  FAM_LINEAR_FWD = 3,
  FAM_LINEAR_BWD_DELTA = 4,
  FAM_LINEAR_WGRAD = 5,
  FAM_BMM_FWD = 6,
  FAM_BMM_SHARED = 7,
  FAM_RELU = 8,
  FAM_REMAX = 9,
  FAM_BN_STATS = 10,
  FAM_BN_FWD = 11,
  FAM_BN_BWD = 12,
  FAM_UPDATE = 13,
  FAM_INNOVATION = 14,
  FAM_ADD = 15,
  FAM_AVGPOOL = 16,
  FAM_JACOBIAN = 17,
  FAM_RMSNORM = 18,
  FAM_EMBEDDING = 19,
  FAM_PE = 20,
  FAM_SPLITK_REDUCE = 21,
  FAM_MAXPOOL = 22,
  FAM_LAYERNORM = 23,
  FAM_SOFTPLUS = 24,
  FAM_ATTN_SCORES = 25,
  FAM_COUNT = 26
};

// Record a start event for `fam` on `s` if the timer is on for that family.
// Returns a slot id (>= 0) or -1; pass it to prof_end with the launch's work.
int prof_start(int fam, hipStream_t s);
void prof_end(int slot, hipStream_t s, double flops, double bytes);

// RAII bracket used by every entry point.
struct ProfScope {
  int slot;
  hipStream_t s;
  double flops, bytes;
  ProfScope(int fam, hipStream_t st, double f, double b) : slot(prof_start(fam, st)), s(st), flops(f), bytes(b) {}
  ~ProfScope() { prof_end(slot, s, flops, bytes); }
};

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// BatchNorm2D batch statistics from per-row-range partial sums of (mu, S, mu^2),
// ws[(q * C + c) * nblk + b], with the running-stat / gamma bookkeeping of tagi_bn_stats
// (defined with the BatchNorm kernels; launched on s, returns a TAGI status).
int bn_stats_finalize(const char* what, const float* ws, int nblk, int64_t rows, int64_t C, float* batch_mean,
                      float* batch_var, float* running_mean, float* running_var, float* mg, float momentum, float eps,
                      int first_call, int preserve_var, hipStream_t s);

// Grid size for a grid-stride elementwise kernel: enough blocks to fill 256 CUs several
// times over, never more than needed.
inline unsigned ew_blocks(int64_t n_items, int threads) {
  int64_t b = cdiv(n_items, threads);
  if (b > 256 * 16) b = 256 * 16;
  if (b < 1) b = 1;
  return (unsigned)b;
}

}  // namespace tagi
