// Error state and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "capi_util.hpp"

namespace gtk {
static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
}  // namespace gtk

extern "C" const char* gtk_last_error(void) { return gtk::g_err; }
extern "C" int gtk_version(void) { return 100; }
