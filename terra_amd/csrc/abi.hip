// Library-wide C ABI entry points: version and last-error text.
#include "common.h"

#include <string.h>

namespace terra {

static thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = '\0'; }

const char* last_error() { return g_last_error; }

}  // namespace terra

extern "C" int terra_abi_version(void) { return TERRA_SWIN_ABI_VERSION; }

extern "C" const char* terra_last_error(void) { return terra::last_error(); }
