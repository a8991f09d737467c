// Library-wide entry points of libghost_hip.so: ABI version, thread-local error text and
// the launch-status check shared by every kernel wrapper.
#include <string>

#include "gs_common.h"

namespace gs {

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
  if (e != hipSuccess) {
    return fail(GS_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return GS_OK;
}

}  // namespace gs

extern "C" int gs_abi_version(void) { return GS_ABI_VERSION; }

extern "C" const char* gs_last_error(void) { return gs::g_last_error.c_str(); }
