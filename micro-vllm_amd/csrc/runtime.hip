// Error reporting and version entry points of the C ABI.
#include <cstring>
#include <string>

#include "common.h"

namespace mvllm {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* fmt, ...) {
  char buffer[1024];
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error.assign(buffer);
  return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace mvllm

extern "C" const char* mvllm_last_error(void) {
  return mvllm::g_last_error.c_str();
}

extern "C" int mvllm_abi_version(void) { return MVLLM_ABI_VERSION; }
