// ABI version and the thread-local error message of libmxdecode.
#include "common.h"

namespace mx {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace mx

extern "C" int mx_abi_version(void) { return MX_ABI_VERSION; }

extern "C" const char* mx_last_error(void) { return mx::g_last_error; }
