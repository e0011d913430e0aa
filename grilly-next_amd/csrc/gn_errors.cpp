// gn_errors.cpp — thread-local error message and version string of libgn_bwd.
#include <cstdarg>
#include <cstdio>

#include "gn_common.h"

namespace gn {

static thread_local char t_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_last_error, sizeof(t_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { t_last_error[0] = '\0'; }

}  // namespace gn

extern "C" const char* gn_last_error(void) { return gn::t_last_error; }

extern "C" const char* gn_version(void) { return "libgn_bwd 0.1 (gfx950, wave64, bf16/fp32 MFMA)"; }
