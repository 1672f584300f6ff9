// Version and error reporting of the q36 C-ABI.
#include <string.h>

#include "q36_host.h"

namespace q36 {
static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
}  // namespace q36

extern "C" int q36_abi_version(void) { return Q36_ABI_VERSION; }
extern "C" const char* q36_last_error(void) { return q36::g_err; }
