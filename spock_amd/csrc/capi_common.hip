// capi_common.hip -- error reporting shared by every C-ABI entry point.
#include "capi_common.hpp"

#include <cstdarg>
#include <cstdio>
#include <string>

namespace {
thread_local std::string g_last_error;
}

namespace spk {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SPK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return SPK_OK;
}

}  // namespace spk

extern "C" const char* spk_last_error(void) { return g_last_error.c_str(); }
extern "C" uint32_t spk_abi_version(void) { return (1u << 16) | 0u; }
