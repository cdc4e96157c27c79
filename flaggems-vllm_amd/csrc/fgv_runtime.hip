// Library-wide C-ABI entry points: version and per-thread error text.
#include <stdio.h>
#include <string.h>

#include "fgv_host.h"

namespace fgv {
namespace {
thread_local char g_last_error[256] = "";
}

int fail(int code, const char* msg) {
    snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
    return code;
}

}  // namespace fgv

extern "C" int fgv_version(void) { return 100; /* 0.1.0 */ }

extern "C" const char* fgv_last_error(void) { return fgv::g_last_error; }
