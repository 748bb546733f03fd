// Library-level plumbing: version, per-thread error messages and the
// co-residency capacity of the persistent kernels.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "common.h"

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
