// Status, version and error reporting of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "hsmoe_internal.h"

namespace hsmoe {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HSMOE_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return HSMOE_OK;
}

}  // namespace hsmoe

extern "C" int hsmoe_version(void) { return HSMOE_VERSION; }

extern "C" const char* hsmoe_last_error(void) { return hsmoe::g_last_error; }

extern "C" void hsmoe_clear_error(void) { hsmoe::g_last_error[0] = 0; }
