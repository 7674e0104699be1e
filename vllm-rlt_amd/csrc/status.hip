// Error reporting for the C ABI: a per-thread message buffer.
#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace {
thread_local char g_message[512] = "";
}

namespace rlt {

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* kernel) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(RLT_ELAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(err));
  g_message[0] = '\0';
  return RLT_OK;
}

}  // namespace rlt

extern "C" const char* rlt_last_error(void) { return g_message; }

extern "C" const char* rlt_version(void) { return "rlt_kv 0.1 gfx950"; }
