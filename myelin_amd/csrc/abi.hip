// Error reporting for the C ABI: one message buffer per host thread.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace myelin {
namespace {
thread_local char g_error[512] = "";
}

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int invalid(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return MYELIN_EINVAL;
}

int launched(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return MYELIN_EHIP;
  }
  return MYELIN_OK;
}

}  // namespace myelin

extern "C" const char *myelin_last_error(void) { return myelin::g_error; }

extern "C" int myelin_abi_version(void) { return 1; }
