// C-ABI plumbing of libmdx: the thread-local error message and the ABI version.
#include <stdarg.h>
#include <stdio.h>

#include "mdx_common.hpp"

namespace mdx {
static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
}  // namespace mdx

extern "C" const char* mdx_last_error(void) { return mdx::g_err; }
extern "C" int mdx_version(void) { return 2; }
