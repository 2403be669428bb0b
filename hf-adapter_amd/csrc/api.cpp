// Error bookkeeping and version query of the rwkv7mi C ABI.
#include "common.h"

namespace rwkv7mi {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(RWKV7MI_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return RWKV7MI_OK;
}

}  // namespace rwkv7mi

extern "C" const char* rwkv7mi_last_error(void) { return rwkv7mi::g_last_error.c_str(); }

extern "C" int rwkv7mi_abi_version(void) { return 100; }
