// Library-wide plumbing of the C ABI: thread-local error text, version string,
// launch checking.  Every entry point returns an int status (0 = ok) and leaves a
// message retrievable with tl_last_error() on failure.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <set>
#include <utility>

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

int allow_dynamic_lds(const void* kernel, int bytes, const char* who) {
  static std::mutex mu;
  static std::set<std::pair<int, const void*>> done;  // (device, kernel) already raised
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
    return kErrHip;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({dev, kernel})) return kOk;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) {
    set_error("%s: hipFuncSetAttribute failed: %s", who, hipGetErrorString(e));
    return kErrHip;
  }
  done.insert({dev, kernel});
  return kOk;
}

}  // namespace tl

extern "C" const char* tl_last_error(void) { return tl::g_err; }

extern "C" const char* tl_version(void) { return "tilert_amd 0.1.0 gfx950"; }
