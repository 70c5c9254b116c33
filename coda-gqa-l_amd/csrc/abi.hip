// Library-wide entry points and error plumbing of the C ABI.
#include "common.h"

#include <stdarg.h>
#include <stdio.h>

namespace coda {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CODA_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return CODA_OK;
}

}  // namespace coda

extern "C" int coda_abi_version(void) { return CODA_ABI_VERSION; }

extern "C" const char* coda_last_error(void) { return coda::g_last_error.c_str(); }

// build.py defines it as the hash of the sources it compiled
#ifndef CODA_SOURCE_HASH
#define CODA_SOURCE_HASH "unknown"
#endif
extern "C" const char* coda_source_hash(void) { return CODA_SOURCE_HASH; }

extern "C" int coda_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}
