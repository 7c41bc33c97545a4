// Thread-local last-error storage behind pa_last_error().
#include "pa_errors.h"

namespace pa {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace pa

extern "C" const char* pa_last_error(void) { return pa::g_last_error; }

extern "C" int pa_abi_version(void) { return 2; }
