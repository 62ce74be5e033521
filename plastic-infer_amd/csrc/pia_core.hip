// Library-level entry points: error reporting and ABI version.
#include "pia_internal.h"

namespace pia {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace pia

extern "C" const char* pia_last_error(void) { return pia::g_last_error; }

extern "C" int pia_abi_version(void) { return 3; }
