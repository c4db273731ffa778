// Library-wide host plumbing: ABI version and the per-thread error message.
#include <cstdarg>

#include "gdn_common.hpp"

namespace {
thread_local char g_last_error[512] = {0};
}

namespace gdn_host {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(GDN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  g_last_error[0] = 0;
  return GDN_OK;
}

}  // namespace gdn_host

extern "C" int gdn_abi_version(void) { return GDN_ABI_VERSION; }

extern "C" const char* gdn_last_error(void) { return g_last_error; }
