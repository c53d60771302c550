// aq_capi.hip -- ABI version, thread-local error reporting.
#include <stdarg.h>
#include <stdio.h>

#include "aq_common.h"

namespace aq {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return AQ_OK;
  return set_error(AQ_EHIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace aq

extern "C" int aq_abi_version(void) { return AQ_ABI_VERSION; }

extern "C" const char* aq_last_error(void) { return aq::g_last_error; }
