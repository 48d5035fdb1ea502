// status.cpp -- the calling thread's last-error text (qraf_hip_last_error).
#include "status.h"

#include <stdarg.h>
#include <stdio.h>

namespace qraf_hip {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}
void clear_error() { g_err[0] = 0; }

}  // namespace qraf_hip

extern "C" const char* qraf_hip_last_error(void) { return qraf_hip::g_err; }
