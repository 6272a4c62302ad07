// Error reporting and version query of the C ABI (include/gdn_amd.h).
#include <stdarg.h>
#include <stdio.h>

#include "gdn_host.h"

namespace gdn {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_abi_version(void) { return 3; }

extern "C" const char *gdn_last_error(void) { return gdn::g_last_error; }
