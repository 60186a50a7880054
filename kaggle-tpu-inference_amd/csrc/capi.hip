// Library-level entry points: version and error reporting.
#include "capi_util.h"

#include <string.h>

namespace g4mi {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace g4mi

extern "C" {

int g4mi_version(void) { return G4MI_ABI_VERSION; }

const char* g4mi_last_error_string(void) { return g4mi::g_last_error; }

}  // extern "C"
