// The library's error state, host side: the C ABI's status codes (include/hymoe.h) and the thread-local message
// hy_last_error() returns.  Host-only, so that host code (the GGUF reader) builds with any C++ compiler.
#pragma once
#include "../../include/hymoe.h"

namespace hy {
void set_error(const char *fmt, ...);   // printf-style message for hy_last_error()
} // namespace hy
