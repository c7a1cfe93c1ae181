// Library-wide error state, device properties and version query.
#include <atomic>

#include "tpf_status.hpp"

namespace tpf {
char* error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}
}  // namespace tpf

extern "C" {

const char* tpf_last_error(void) { return tpf::error_buffer(); }

int tpf_abi_version(void) { return 8; }

}  // extern "C"
