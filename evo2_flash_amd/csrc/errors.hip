// Error reporting for the C ABI: a per-thread message buffer and the
// version query.  No kernels here.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace evo2 {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(EVO2_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return EVO2_OK;
}

}  // namespace evo2

extern "C" const char *evo2_last_error(void) { return evo2::g_err; }

extern "C" int evo2_abi_version(void) { return 1; }
