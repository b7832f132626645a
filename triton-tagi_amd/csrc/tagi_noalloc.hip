// tagi_linear_fwd_noalloc: the Linear forward for callers that cannot allocate device
// memory. It sits in a translation unit of its own so that its fixed scratch array lives
// in a code object of its own: the runtime allocates the array on a device when it loads
// that code object there, which happens on the first call of this entry point on that
// device (hipGetSymbolAddress below), not when any other kernel of the library loads.
#include <mutex>

#include "tagi_linear_internal.h"

using namespace tagi;

static inline hipStream_t as_stream(tagi_stream_t s) { return (hipStream_t)s; }

// tagi_linear_fwd_noalloc keeps the split-K partial sums of a call in this file-scope
// device array instead of a caller workspace. Each GPU holds its own copy, at its own
// address, from the first call on that GPU until the process ends. In host code the
// array's name is not a device address: the address is taken once per device with
// hipGetSymbolAddress (that device current) and only that pointer is handed to kernels.
// Every split writes all of its partial plane before the reduction reads it, so nothing
// in the array has to start at zero; the array keeps the last call's partials. Calls
// that overlap on one GPU (two streams, or two host threads) share the array and race.
static __device__ __align__(256) float scratch[TAGI_LINEAR_FWD_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// The calling thread's current device's copy of `scratch` (its address resolved on the
// first call for that device).
static int scratch_of_current_device(const char* what, hipStream_t s, float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TAGI_ERR_LAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  TAGI_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device index %d out of range", what, dev);
  if (s != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(s, &sdev);
    if (e != hipSuccess) return fail(TAGI_ERR_LAUNCH, "%s: hipStreamGetDevice failed: %s", what, hipGetErrorString(e));
    TAGI_REQUIRE((int)sdev == dev, "%s: the stream belongs to device %d but device %d is current", what, (int)sdev,
                 dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(TAGI_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return TAGI_OK;
}

extern "C" int tagi_linear_fwd_noalloc(const float* ma, const float* Sa, const float* mw, const float* Sw,
                                       const float* mb, const float* Sb, float* mz, float* Sz, int64_t M, int64_t K,
                                       int64_t N, tagi_stream_t stream) {
  const char* what = "tagi_linear_fwd_noalloc";
  int rc = linear_fwd_check(what, ma, Sa, mw, Sw, Sz, M, K, N);
  if (rc != TAGI_OK) return rc;
  // the plan tagi_linear_fwd runs with its full workspace, so results are the same bits
  const Plan p = linear_fwd_plan(M, K, N);
  const int64_t need = plan_ws_bytes(p, M, N, 1);
  TAGI_REQUIRE(need <= (int64_t)TAGI_LINEAR_FWD_NOALLOC_SCRATCH_BYTES,
               "%s: M=%lld K=%lld N=%lld needs %lld bytes of split-K scratch, above the fixed %lld; use "
               "tagi_linear_fwd with a workspace",
               what, (long long)M, (long long)K, (long long)N, (long long)need,
               (long long)TAGI_LINEAR_FWD_NOALLOC_SCRATCH_BYTES);
  hipStream_t s = as_stream(stream);
  float* ws = nullptr;
  rc = scratch_of_current_device(what, s, &ws);
  if (rc != TAGI_OK) return rc;
  return linear_fwd_run(what, ma, Sa, mw, Sw, mb, Sb, mz, Sz, M, K, N, p, ws, need, s);
}

