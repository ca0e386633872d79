// Error state and version query of the C ABI.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "maxsim_host.h"

namespace maxsim {

static thread_local std::string g_error;

void clear_error() { g_error.clear(); }

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(MAXSIM_ERR_LAUNCH, "%s launch failed: %s", what,
                hipGetErrorString(e));
  return MAXSIM_OK;
}

}  // namespace maxsim

extern "C" {

int maxsim_amd_abi_version(void) { return 10; }

const char* maxsim_amd_last_error(void) { return maxsim::g_error.c_str(); }

}  // extern "C"
