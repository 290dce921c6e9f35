// Library-wide pieces of the C ABI: version and the per-thread error message.
#include <stdarg.h>
#include <stdio.h>

#include "capi_internal.h"

namespace {
thread_local char g_err[512] = "";
}

namespace solort {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

}  // namespace solort

extern "C" int solort_abi_version(void) { return 10; }

#ifndef SOLORT_SOURCE_ID
#define SOLORT_SOURCE_ID 0ULL
#endif
extern "C" uint64_t solort_source_id(void) { return SOLORT_SOURCE_ID; }

extern "C" int solort_init(void) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return solort::set_error((int)e, "init: no device: %s", hipGetErrorString(e));
  const int rc = solort::verify_xcd_placement(dev);
  return rc ? rc : solort::noalloc_scratch_setup(dev);
}

extern "C" const char* solort_last_error(void) { return g_err; }
