// Library-level C ABI: version and per-thread error reporting.
#include <string>

#include "ia_common.hpp"

namespace ia {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IA_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return IA_OK;
}

}  // namespace ia

extern "C" {

const char* ia_last_error(void) { return ia::g_last_error.c_str(); }

int ia_version(void) { return 1; }

}  // extern "C"
