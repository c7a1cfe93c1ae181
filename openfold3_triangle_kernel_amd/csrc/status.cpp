// Library-wide error state and version query.
#include "tpf_status.hpp"

namespace tpf {
char* error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}
}  // namespace tpf

extern "C" {

const char* tpf_last_error(void) { return tpf::error_buffer(); }

int tpf_abi_version(void) { return 4; }

}  // extern "C"
