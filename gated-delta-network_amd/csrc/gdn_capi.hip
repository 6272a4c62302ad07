// Error reporting and version query of the C ABI (include/gdn_amd.h); the
// message store itself is in gdn_args.cpp.
#include "gdn_host.h"

namespace gdn {

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_abi_version(void) { return 4; }

extern "C" const char *gdn_last_error(void) { return gdn::last_error_text(); }
