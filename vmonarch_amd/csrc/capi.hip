// C-ABI bookkeeping: version and per-thread error messages.
#include "vmo_host.h"

#include <string.h>

namespace vmo {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace vmo

extern "C" int vmo_abi_version(void) { return VMO_ABI_VERSION; }

extern "C" const char* vmo_last_error(void) { return vmo::g_last_error; }
