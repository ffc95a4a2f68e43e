// Library-wide C ABI entry points: version and per-thread error reporting.
#include <atomic>

#include "aa_common.h"

namespace aa {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// Reports an error left by the launch just made (bad configuration, no
// device code for this GPU). Does not synchronise.
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(AA_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  }
  return AA_OK;
}

// Compute units of the current device (queried once per device).
int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace aa

extern "C" int aa_abi_version(void) { return AA_ABI_VERSION; }

extern "C" const char* aa_last_error(void) { return aa::g_last_error.c_str(); }
