// Host-side plumbing of the C ABI: version and thread-local error messages.
#include "sa_internal.h"

namespace sa {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(SA_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return SA_OK;
}

}  // namespace sa

extern "C" int sa_abi_version(void) { return SA_ABI_VERSION; }

extern "C" const char* sa_last_error(void) { return sa::g_last_error.c_str(); }
