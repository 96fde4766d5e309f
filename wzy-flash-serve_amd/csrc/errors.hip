// errors.hip -- thread-local error message behind wzy_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "wzy_host.h"

namespace wzy {
static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
void clear_error() { g_err[0] = 0; }
}  // namespace wzy

extern "C" const char* wzy_last_error(void) { return wzy::g_err; }
extern "C" const char* wzy_version(void) { return "wzy-mi355x 0.1 (gfx950)"; }
