// Library-wide C-ABI entry points: version and last-error reporting.
#include <stdarg.h>

#include "abi_common.h"

namespace mxabi {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace mxabi

extern "C" int mxfp8_abi_version(void) { return MXFP8_MLP_ABI_VERSION; }

extern "C" const char* mxfp8_last_error(void) { return mxabi::g_err; }
