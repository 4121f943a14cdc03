// Library-wide entry points: error string and version.
#include <stdarg.h>

#include "sf_common.hpp"

namespace sf {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace sf

extern "C" const char* sf_last_error(void) { return sf::g_last_error; }

// Major * 10000 + minor * 100 + patch.
extern "C" int sf_version(void) { return 100; }
