// Library-wide ABI helpers: version and thread-local error message.
#include "common.h"

namespace {
thread_local std::string g_last_error;
}

namespace st {

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ST_EDEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ST_OK;
}

}  // namespace st

extern "C" int st_abi_version(void) { return 1; }

extern "C" const char* st_last_error(void) { return g_last_error.c_str(); }
