// Error reporting shared by every entry point of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace q3 {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() {
  g_last_error[0] = '\0';
  // Drop a stale status left by an earlier, unrelated HIP call so the check
  // after our launch reports only our own launch.
  (void)hipGetLastError();
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(static_cast<int>(e), "%s: kernel launch failed: %s", what,
                hipGetErrorString(e));
  }
  return QWEN3_OK;
}

}  // namespace q3

extern "C" const char* qwen3_attn_last_error(void) { return q3::g_last_error; }

extern "C" int qwen3_attn_abi_version(void) { return 9; }
