// ABI plumbing: version and thread-local error text.
#include <stdarg.h>
#include <string.h>

#include "si_common.h"

namespace si {

static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return SI_ERR_HIP;
  }
  return SI_OK;
}

}  // namespace si

extern "C" int si_abi_version(void) { return SI_ABI_VERSION; }

extern "C" const char* si_last_error(void) { return si::g_error; }
