// C ABI housekeeping: per-thread error text and launch checks.
#include "fs_common.h"

namespace fs {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FS_ERR_RUNTIME, std::string(what) + ": " + hipGetErrorString(e));
  return FS_OK;
}

}  // namespace fs

extern "C" const char* fs_last_error(void) { return fs::g_last_error.c_str(); }

extern "C" int fs_abi_version(void) { return 2; }
