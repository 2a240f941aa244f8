// ABI version and per-thread error reporting.
#include <cstdarg>

#include "common.hpp"

namespace koemi {

namespace {
thread_local char g_last_error[1024] = {0};
}

void set_error(const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
    va_end(args);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace koemi

extern "C" int koemi_abi_version(void) { return 1; }

extern "C" const char* koemi_last_error(void) { return koemi::g_last_error; }
