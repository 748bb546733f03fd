// Library-level plumbing: version, per-thread error messages and the
// co-residency capacity of the persistent kernels.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "common.h"

namespace ma {

// Whether workgroup i of a launch runs on XCD (i + o) mod kXcds for one o (o
// changes from launch to launch), so that the workgroups with equal i mod
// kXcds share an XCD and its L2: one probe launch per device (256 workgroups
// of 512 threads) records every workgroup's XCD into a static array (no
// allocation), read back once.  It synchronises ``st``; while ``st`` is
// being captured into a graph it cannot run, so the answer is "no" and
// nothing is cached.
constexpr int kProbeWgs = 256;
__device__ uint32_t g_xcd_probe[kProbeWgs];

__global__ __launch_bounds__(512) void k_xcd_probe(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = static_cast<uint32_t>(xcc_id());
}

// Per device: 1 once the host has turned the XCD-split forms off
// (ma_xcd_forms_disable), after one of them found its workgroups not spread
// as probed.
static std::atomic<int> g_xcd_off[64];

int xcd_round_robin(hipStream_t st, bool* ok) {
  static std::mutex mu;
  static int known[64];  // 0 unknown, 1 yes, 2 no
  *ok = false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(MA_ERUNTIME, "no current HIP device");
  if (g_xcd_off[dev].load(std::memory_order_relaxed)) return MA_OK;
  std::lock_guard<std::mutex> lock(mu);
  if (!known[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return fail(MA_ERUNTIME, "XCD probe: stream query failed");
    if (cs != hipStreamCaptureStatusNone) return MA_OK;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return fail(MA_ERUNTIME, "XCD probe: device query failed");
    bool good = cus % kXcds == 0;
    if (good) {
      uint32_t* d = nullptr;
      uint32_t h[kProbeWgs];
      if (hipGetSymbolAddress(reinterpret_cast<void**>(&d), HIP_SYMBOL(g_xcd_probe)) != hipSuccess)
        return fail(MA_ERUNTIME, "XCD probe: symbol");
      hipLaunchKernelGGL(k_xcd_probe, dim3(kProbeWgs), dim3(512), 0, st, d);
      if (hipGetLastError() != hipSuccess || hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, st) != hipSuccess ||
          hipStreamSynchronize(st) != hipSuccess)
        return fail(MA_ERUNTIME, "XCD probe failed");
      const uint32_t o = h[0] % kXcds;  // XCD of workgroup 0
      for (int i = 0; i < kProbeWgs; ++i) good = good && h[i] == (i + o) % kXcds;
    }
    known[dev] = good ? 1 : 2;
  }
  *ok = known[dev] == 1;
  return MA_OK;
}

}  // namespace ma

// Turn the XCD-split forms (one-launch MoE layer, XCD-local decode attention)
// off (disable != 0) or back on for a device; later calls take the
// one-barrier / cross-XCD forms.  For the host's reaction to the layout check.
extern "C" int ma_xcd_forms_disable(int device, int disable) {
  if (device < 0 || device >= 64) return ma::fail(MA_EVALUE, "xcd_forms_disable: device %d", device);
  ma::g_xcd_off[device].store(disable ? 1 : 0, std::memory_order_relaxed);
  return MA_OK;
}

namespace ma {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MA_ERUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MA_OK;
}

// Workgroups of `kernel` (launched with `threads` threads and no dynamic LDS)
// the current device holds at once: compute units x resident workgroups per
// compute unit.  A host-side table of device properties, filled on first use
// per (device, kernel) and read-only afterwards.
int resident_capacity(const void* kernel, int threads, int64_t* capacity) {
  struct Entry {
    int dev;
    const void* fn;
    int threads;
    int64_t cap;
  };
  static std::mutex mu;
  static Entry table[64];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MA_ERUNTIME, "no current HIP device");
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (table[i].dev == dev && table[i].fn == kernel && table[i].threads == threads) {
      *capacity = table[i].cap;
      return MA_OK;
    }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess)
    return fail(MA_ERUNTIME, "occupancy query failed");
  const int64_t cap = static_cast<int64_t>(cus) * per_cu;
  if (used < 64) table[used++] = Entry{dev, kernel, threads, cap};
  *capacity = cap;
  return MA_OK;
}

}  // namespace ma

extern "C" int ma_version(void) { return 100; }

extern "C" const char* ma_last_error(void) { return ma::g_err; }
