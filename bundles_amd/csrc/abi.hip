// Version and error reporting of the q36 C-ABI, and the shared launch helper for kernels that
// need more than 64 KiB of dynamic LDS.
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

// Raise the dynamic-LDS limit of kernel fn to the CU's 160 KiB once per device (a repeated call
// from a racing thread only repeats the same attribute write).
int ensure_lds(const void* fn, size_t bytes, const char* what) {
  if (bytes <= 65536) return Q36_OK;
  if (bytes > 160 * 1024) {
    set_error("%s: %zu bytes of LDS exceed the 160 KiB of a CU", what, bytes);
    return Q36_EINVAL;
  }
  static const void* done[64][16] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  for (int i = 0; i < 16; ++i)
    if (done[dev][i] == fn) return Q36_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) {
    set_error("%s: hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed", what);
    return Q36_ELAUNCH;
  }
  for (int i = 0; i < 16; ++i)
    if (done[dev][i] == nullptr) {
      done[dev][i] = fn;
      break;
    }
  return Q36_OK;
}
}  // namespace q36

extern "C" int q36_abi_version(void) { return Q36_ABI_VERSION; }
extern "C" const char* q36_last_error(void) { return q36::g_err; }
