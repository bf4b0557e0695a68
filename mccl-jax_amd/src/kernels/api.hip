// Error plumbing and device queries shared by every mk_* entry point.
#include "mk_common.h"

namespace mk {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(MK_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return MK_OK;
}

}  // namespace mk

extern "C" const char* mk_last_error(void) { return mk::g_last_error.c_str(); }
extern "C" int mk_abi_version(void) { return 1; }
extern "C" int mk_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}
