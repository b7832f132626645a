// Error state and the live per-family event timer of libtagi_hip.
#include <stdarg.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "tagi_common.h"

namespace tagi {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TAGI_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TAGI_OK;
}

// ---------------------------------------------------------------------------------
// Timer: a fixed pool of event pairs, created when the timer is switched on.
// ---------------------------------------------------------------------------------
namespace {
constexpr int kMaxSlots = 16384;
struct Prof {
  std::mutex mu;
  bool on = false;
  uint64_t mask = 0;
  std::vector<hipEvent_t> ev;  // 2 per slot
  std::vector<int> fam;
  std::vector<double> flops, bytes;
  int used = 0;
};
Prof& prof() {
  static Prof p;
  return p;
}
}  // namespace

int prof_start(int f, hipStream_t s) {
  Prof& p = prof();
  if (!p.on || !((p.mask >> f) & 1ull)) return -1;
  std::lock_guard<std::mutex> lk(p.mu);
  if (p.used >= kMaxSlots) return -1;
  int slot = p.used++;
  p.fam[slot] = f;
  hipEventRecord(p.ev[2 * slot], s);
  return slot;
}

void prof_end(int slot, hipStream_t s, double flops, double bytes) {
  if (slot < 0) return;
  Prof& p = prof();
  hipEventRecord(p.ev[2 * slot + 1], s);
  p.flops[slot] = flops;
  p.bytes[slot] = bytes;
}

}  // namespace tagi

using namespace tagi;

extern "C" int tagi_abi_version(void) { return TAGI_ABI_VERSION; }

extern "C" const char* tagi_last_error(void) { return g_err; }

// Stream ordering through one untimed event per device and host thread, recorded without
// the system-scope fence: a wait between two streams of one GPU needs the producer's work
// to have finished, and the kernels' own device-scope release already makes their writes
// visible to the device's other kernels. hipStreamWaitEvent orders the waiter after the
// record that precedes the call, so the event is recorded again for the next call.
extern "C" int tagi_stream_wait(tagi_stream_t waiter, tagi_stream_t producer) {
  hipStream_t w = (hipStream_t)waiter, pr = (hipStream_t)producer;
  if (w == pr) return TAGI_OK;
  int dev = 0;
  if (hipStreamGetDevice(pr, &dev) != hipSuccess) return fail(TAGI_ERR_ARG, "tagi_stream_wait: unknown producer stream");
  constexpr int kMaxDev = 64;
  thread_local hipEvent_t ev[kMaxDev] = {};
  if (dev < 0 || dev >= kMaxDev) return fail(TAGI_ERR_ARG, "tagi_stream_wait: device %d out of range", dev);
  if (!ev[dev]) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(dev) != hipSuccess)
      return fail(TAGI_ERR_LAUNCH, "tagi_stream_wait: cannot select device %d", dev);
    const hipError_t e = hipEventCreateWithFlags(&ev[dev], hipEventDisableTiming | hipEventDisableSystemFence);
    hipSetDevice(cur);
    if (e != hipSuccess) {
      ev[dev] = nullptr;
      return fail(TAGI_ERR_LAUNCH, "tagi_stream_wait: hipEventCreate failed");
    }
  }
  if (hipEventRecord(ev[dev], pr) != hipSuccess) return fail(TAGI_ERR_LAUNCH, "tagi_stream_wait: event record failed");
  if (hipStreamWaitEvent(w, ev[dev], 0) != hipSuccess) return fail(TAGI_ERR_LAUNCH, "tagi_stream_wait: wait failed");
  return TAGI_OK;
}

extern "C" int tagi_prof_begin(uint64_t family_mask) {
  Prof& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  if (p.ev.empty()) {
    p.ev.resize(2 * kMaxSlots);
    // timing-only events: no system-scope fence when they are recorded (that fence writes
    // back the L2 and holds the queue for about 5 us per record; their timestamps are read
    // after a device synchronisation)
    for (auto& e : p.ev) {
      if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess)
        return fail(TAGI_ERR_LAUNCH, "tagi_prof_begin: hipEventCreate failed");
    }
    p.fam.resize(kMaxSlots);
    p.flops.resize(kMaxSlots);
    p.bytes.resize(kMaxSlots);
  }
  p.used = 0;
  p.mask = family_mask;
  p.on = true;
  return TAGI_OK;
}

extern "C" int tagi_prof_end(double* ms, int64_t* launches, double* flops, double* bytes) {
  Prof& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  p.on = false;
  for (int f = 0; f < FAM_COUNT; ++f) {
    if (ms) ms[f] = 0;
    if (launches) launches[f] = 0;
    if (flops) flops[f] = 0;
    if (bytes) bytes[f] = 0;
  }
  for (int i = 0; i < p.used; ++i) {
    if (hipEventSynchronize(p.ev[2 * i + 1]) != hipSuccess) return fail(TAGI_ERR_LAUNCH, "tagi_prof_end: event sync failed");
    float t = 0.f;
    if (hipEventElapsedTime(&t, p.ev[2 * i], p.ev[2 * i + 1]) != hipSuccess) return fail(TAGI_ERR_LAUNCH, "tagi_prof_end: elapsed time failed");
    int f = p.fam[i];
    if (ms) ms[f] += t;
    if (launches) launches[f] += 1;
    if (flops) flops[f] += p.flops[i];
    if (bytes) bytes[f] += p.bytes[i];
  }
  p.used = 0;
  return TAGI_OK;
}

// ------------------------------------------------------------------ ceiling probe
// A loop of independent fp32 MFMAs with no memory traffic: each 64-lane wave keeps four
// 32x32 accumulators in flight. Its rate bounds what any fp32 MFMA kernel can sustain at
// the same number of waves per SIMD.
namespace {
typedef float probe_floatx16 __attribute__((ext_vector_type(16)));
__global__ void __launch_bounds__(256) mfma_loop_kernel(float* __restrict__ out, int iters) {
  probe_floatx16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;
  const float x = 1.0f + threadIdx.x * 1e-6f, y = 1.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[i][v];
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}
// The same loop with `V` other instructions after each MFMA: independent v_fma_f32
// chains (KIND 0) or LDS reads (KIND 1, waited for once per round). Written as inline
// assembly so that the compiler issues exactly V of them per MFMA. How much each costs
// the MFMA rate tells whether that kind of instruction issues beside the matrix core.
template <int KIND, int V>
__global__ void __launch_bounds__(256) mfma_mix_kernel(float* __restrict__ out, int iters) {
  __shared__ float lds[256];
  lds[threadIdx.x] = threadIdx.x * 1e-3f;
  __syncthreads();
  probe_floatx16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;
  const float x = 1.0f + threadIdx.x * 1e-6f, y = 1.0f;
  float f[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = threadIdx.x * 1e-3f + j;
  const float c0 = 0.999f, c1 = 0.5f;
  float r = 0.f;
  const unsigned addr = (unsigned)(threadIdx.x * 4);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[i], 0, 0, 0);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (KIND == 0) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(f[v & 7]) : "v"(c0), "v"(c1));
        else asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr));
      }
    }
    if constexpr (KIND == 1) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  float s = r;
#pragma unroll
  for (int j = 0; j < 8; ++j) s += f[j];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[i][v];
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}
// HBM streaming probes. Each thread moves U float4 per grid-stride step with all U loads
// issued before any store or add, so U * 16 bytes per lane are in flight.
constexpr int kStreamU = 4;

__global__ void __launch_bounds__(256) stream_copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                          int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * kStreamU;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x * kStreamU + threadIdx.x; base < n4; base += stride) {
    float4 v[kStreamU];
#pragma unroll
    for (int u = 0; u < kStreamU; ++u) {
      const int64_t i = base + (int64_t)u * blockDim.x;
      if (i < n4) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < kStreamU; ++u) {
      const int64_t i = base + (int64_t)u * blockDim.x;
      if (i < n4) dst[i] = v[u];
    }
  }
}

__global__ void __launch_bounds__(256) stream_read_kernel(const float4* __restrict__ src, float* __restrict__ out,
                                                          int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * kStreamU;
  float acc = 0.f;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x * kStreamU + threadIdx.x; base < n4; base += stride) {
    float4 v[kStreamU];
#pragma unroll
    for (int u = 0; u < kStreamU; ++u) {
      const int64_t i = base + (int64_t)u * blockDim.x;
      v[u] = i < n4 ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kStreamU; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;  // keeps the loads live
}

// Variants of the streaming probe, to settle how close to the HBM datasheet a kernel of
// this engine can get: MODE 0 copies, 1 reads (summed per thread), 2 writes a constant;
// U float4 per lane per step, all loads issued before any store; NTL / NTS mark the loads /
// stores nontemporal (__builtin_nontemporal_load/store: the "nt" cache policy); CHUNK gives
// each block one contiguous stretch of the array instead of a grid-stride walk.
typedef float probe_f4 __attribute__((ext_vector_type(4)));

template <int MODE, int U, bool NTL, bool NTS, bool CHUNK>
__global__ void __launch_bounds__(256) stream_variant_kernel(const probe_f4* __restrict__ src,
                                                             probe_f4* __restrict__ dst, int64_t n4) {
  const int64_t step = (int64_t)blockDim.x * U;
  int64_t begin, end, stride;
  if constexpr (CHUNK) {
    const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
    begin = (int64_t)blockIdx.x * per;
    end = begin + per < n4 ? begin + per : n4;
    stride = step;
  } else {
    begin = (int64_t)blockIdx.x * step;
    end = n4;
    stride = (int64_t)gridDim.x * step;
  }
  float acc = 0.f;
  for (int64_t base = begin + threadIdx.x; base < end; base += stride) {
    probe_f4 v[U];
    if constexpr (MODE != 2) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = base + (int64_t)u * blockDim.x;
        if (i < end) v[u] = NTL ? __builtin_nontemporal_load(src + i) : src[i];
        else v[u] = probe_f4{0.f, 0.f, 0.f, 0.f};
      }
    }
    if constexpr (MODE == 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = base + (int64_t)u * blockDim.x;
        if (i < end) {
          const probe_f4 w = MODE == 0 ? v[u] : probe_f4{1.f, 2.f, 3.f, 4.f};
          if (NTS) __builtin_nontemporal_store(w, dst + i);
          else dst[i] = w;
        }
      }
    }
  }
  if constexpr (MODE == 1) reinterpret_cast<float*>(dst)[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

template <int MODE, int U>
static void launch_stream_variant(int flags, dim3 grid, hipStream_t s, const probe_f4* src, probe_f4* dst, int64_t n4) {
#define TAGI_SV(L, S, C) hipLaunchKernelGGL((stream_variant_kernel<MODE, U, L, S, C>), grid, dim3(256), 0, s, src, dst, n4)
  switch (flags & 7) {
    case 0: TAGI_SV(false, false, false); break;
    case 1: TAGI_SV(true, false, false); break;
    case 2: TAGI_SV(false, true, false); break;
    case 3: TAGI_SV(true, true, false); break;
    case 4: TAGI_SV(false, false, true); break;
    case 5: TAGI_SV(true, false, true); break;
    case 6: TAGI_SV(false, true, true); break;
    default: TAGI_SV(true, true, true); break;
  }
#undef TAGI_SV
}

template <int MODE>
static void launch_stream_mode(int unroll, int flags, dim3 grid, hipStream_t s, const probe_f4* src, probe_f4* dst,
                               int64_t n4) {
  if (unroll == 4) launch_stream_variant<MODE, 4>(flags, grid, s, src, dst, n4);
  else if (unroll == 8) launch_stream_variant<MODE, 8>(flags, grid, s, src, dst, n4);
  else launch_stream_variant<MODE, 16>(flags, grid, s, src, dst, n4);
}
}  // namespace

extern "C" int tagi_probe_stream(const float* src, float* dst, int64_t n, int64_t blocks, int mode,
                                 tagi_stream_t stream) {
  const char* what = "tagi_probe_stream";
  TAGI_REQUIRE(src != nullptr && dst != nullptr && n > 0 && n % 4 == 0 && blocks > 0 && blocks <= (1 << 20) &&
                   (mode == 0 || mode == 1) && (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0,
               "%s: bad arguments (n must be a positive multiple of 4, buffers 16-byte aligned, mode 0 or 1)", what);
  hipStream_t s = (hipStream_t)stream;
  if (mode == 0)
    hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst), n / 4);
  else
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(src), dst, n / 4);
  return check_launch(what);
}

extern "C" int tagi_probe_mfma_mix(float* out, int64_t blocks, int64_t iters, int kind, int per_mfma,
                                   tagi_stream_t stream) {
  const char* what = "tagi_probe_mfma_mix";
  TAGI_REQUIRE(out != nullptr && blocks > 0 && blocks <= (1 << 20) && iters > 0 && iters < (1ll << 31),
               "%s: bad arguments", what);
  TAGI_REQUIRE((kind == 0 || kind == 1) && (per_mfma == 1 || per_mfma == 2 || per_mfma == 4 || per_mfma == 8),
               "%s: kind must be 0 (VALU) or 1 (LDS) and per_mfma 1, 2, 4 or 8", what);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), blk(256);
#define TAGI_MIX(K, V) hipLaunchKernelGGL((mfma_mix_kernel<K, V>), grid, blk, 0, s, out, (int)iters)
  if (kind == 0) {
    if (per_mfma == 1) TAGI_MIX(0, 1);
    else if (per_mfma == 2) TAGI_MIX(0, 2);
    else if (per_mfma == 4) TAGI_MIX(0, 4);
    else TAGI_MIX(0, 8);
  } else {
    if (per_mfma == 1) TAGI_MIX(1, 1);
    else if (per_mfma == 2) TAGI_MIX(1, 2);
    else if (per_mfma == 4) TAGI_MIX(1, 4);
    else TAGI_MIX(1, 8);
  }
#undef TAGI_MIX
  return check_launch(what);
}

extern "C" int tagi_probe_mfma_loop(float* out, int64_t blocks, int64_t iters, tagi_stream_t stream) {
  const char* what = "tagi_probe_mfma_loop";
  TAGI_REQUIRE(out != nullptr && blocks > 0 && blocks <= (1 << 20) && iters > 0 && iters < (1ll << 31),
               "%s: bad arguments", what);
  hipLaunchKernelGGL(mfma_loop_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, out, (int)iters);
  return check_launch(what);
}

extern "C" int tagi_probe_stream_variant(const float* src, float* dst, int64_t n, int64_t dst_n, int64_t blocks,
                                         int mode, int unroll, int flags, tagi_stream_t stream) {
  const char* what = "tagi_probe_stream_variant";
  TAGI_REQUIRE(src != nullptr && dst != nullptr && n > 0 && n % 4 == 0 && blocks > 0 && blocks <= (1 << 20) &&
                   mode >= 0 && mode <= 2 && (unroll == 4 || unroll == 8 || unroll == 16) && flags >= 0 &&
                   flags <= 7 && (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0,
               "%s: bad arguments (n a positive multiple of 4, mode 0-2, unroll 4/8/16, flags 0-7, buffers "
               "16-byte aligned)", what);
  TAGI_REQUIRE(mode == 1 ? dst_n >= blocks * 256 : dst_n >= n, "%s: dst holds %lld floats, needs %lld", what,
               (long long)dst_n, (long long)(mode == 1 ? blocks * 256 : n));
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks);
  const auto* src4 = reinterpret_cast<const probe_f4*>(src);
  auto* dst4 = reinterpret_cast<probe_f4*>(dst);
  if (mode == 0) launch_stream_mode<0>(unroll, flags, grid, s, src4, dst4, n / 4);
  else if (mode == 1) launch_stream_mode<1>(unroll, flags, grid, s, src4, dst4, n / 4);
  else launch_stream_mode<2>(unroll, flags, grid, s, src4, dst4, n / 4);
  return check_launch(what);
}
