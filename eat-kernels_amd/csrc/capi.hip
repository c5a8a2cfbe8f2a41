// C-ABI bookkeeping of libkda355.so: thread-local error text and the version.
#include "common.h"

namespace kda355 {
namespace {
thread_local char g_err[512] = {0};
}
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
}  // namespace kda355

extern "C" const char* kda355_last_error(void) { return kda355::g_err; }
extern "C" int kda355_version(void) { return 100; }
