// Error reporting and version of liblema_hip.so.
#include "lema_internal.h"

namespace lema {
namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace lema

extern "C" const char* lema_last_error(void) { return lema::g_error; }

extern "C" int lema_abi_version(void) { return 1; }
