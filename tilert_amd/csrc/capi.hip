// Library-wide plumbing of the C ABI: thread-local error text, version string,
// launch checking.  Every entry point returns an int status (0 = ok) and leaves a
// message retrievable with tl_last_error() on failure.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "../../include/tilert_amd.h"

namespace tl {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return kErrHip;
  }
  return kOk;
}

}  // namespace tl

extern "C" const char* tl_last_error(void) { return tl::g_err; }

extern "C" const char* tl_version(void) { return "tilert_amd 0.1.0 gfx950"; }
