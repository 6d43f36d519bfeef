// Library-wide exports: version string and per-thread error reporting.
#include "sb_common.h"

namespace sb {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

void clear_error() { g_last_error.clear(); }

int fail(const char* fn, const std::string& msg) {
  g_last_error = std::string(fn) + ": " + msg;
  return SB_ERR_INVALID_ARGUMENT;
}

int check_launch(const char* fn) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return SB_OK;
  g_last_error = std::string(fn) + ": kernel launch failed: " + hipGetErrorString(e);
  return static_cast<int>(e);
}

}  // namespace sb

extern "C" const char* sb_version(void) { return "semblend_hip 0.1.0 gfx950"; }

extern "C" const char* sb_last_error_string(void) { return sb::g_last_error.c_str(); }
