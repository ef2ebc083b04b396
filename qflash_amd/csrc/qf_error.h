// Per-thread error message shared by every entry point of libqflash_hip.so
// (returned by qflash_hip_last_error).
#pragma once
#include <stdarg.h>
#include <stdio.h>

namespace qferr {
inline thread_local char g_err[512];

__attribute__((format(printf, 2, 3))) inline int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace qferr
