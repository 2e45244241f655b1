// Library-wide entry points: version and the thread-local last-error string.
#include <stdarg.h>

#include "common.hpp"

namespace svhip {

static thread_local char g_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace svhip

extern "C" int svhip_version(void) { return 200; }

extern "C" const char* svhip_last_error(void) { return svhip::g_error; }
