#include "gsp_status.h"

#include <cstdarg>
#include <cstdio>

#include "../../include/glacier_paged.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace gsp {

void clear_error() { g_last_error[0] = '\0'; }

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace gsp

extern "C" const char* gsp_last_error(void) { return g_last_error; }
