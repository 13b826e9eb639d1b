// Error reporting and version entry points of libmce.so.
#include "mce_common.h"

#include <atomic>

namespace mce {

static thread_local char g_last_error[512] = {0};

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MCE_ERR_LAUNCH, "%s: launch failed: %s", what,
                     hipGetErrorString(e));
  return MCE_OK;
}

// CUs of the current device, looked up once per device (threads that race
// on the first lookup store the same value)
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace mce

extern "C" const char *mce_last_error(void) { return mce::g_last_error; }

extern "C" int mce_abi_version(void) { return MCE_ABI_VERSION; }
