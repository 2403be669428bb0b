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

int raise_dynamic_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done, const char* who) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(RWKV7MI_ELAUNCH, std::string(who) + ": no current device");
  const uint64_t bit = 1ull << dev;
  if (done.load(std::memory_order_acquire) & bit) return RWKV7MI_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
    return fail(RWKV7MI_ELAUNCH, std::string(who) + ": cannot raise the dynamic LDS limit");
  done.fetch_or(bit, std::memory_order_acq_rel);
  return RWKV7MI_OK;
}

}  // namespace rwkv7mi

extern "C" const char* rwkv7mi_last_error(void) { return rwkv7mi::g_last_error.c_str(); }

extern "C" int rwkv7mi_abi_version(void) { return 100; }
