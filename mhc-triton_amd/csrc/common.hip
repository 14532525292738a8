// Host-side plumbing shared by every entry point: error reporting and device
// queries.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace mhc {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return MHC_OK;
  set_error("%s: %s", where, hipGetErrorString(e));
  return MHC_ERR_HIP;
}

int num_cus() {
  static thread_local int dev_cached = -1;
  static thread_local int cus = 256;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return cus;
  if (dev != dev_cached) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    dev_cached = dev;
  }
  return cus;
}

}  // namespace mhc

extern "C" int mhc_abi_version(void) { return 3; }

extern "C" const char* mhc_last_error(void) { return mhc::g_err; }
