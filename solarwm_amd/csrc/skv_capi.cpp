// Host-side state of libsolarkv.so: per-thread error message and version.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/solarkv.h"

namespace skv {

static thread_local char g_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = 0; }

}  // namespace skv

extern "C" int skv_version(void) { return 100; /* 0.1.0 */ }

extern "C" const char* skv_last_error(void) { return skv::g_error; }
