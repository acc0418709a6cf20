// Error reporting and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "ws_common.h"

namespace ws {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(WS_ELAUNCH, "%s: launch failed: %s", what,
                     hipGetErrorString(e));
  return WS_OK;
}

}  // namespace ws

extern "C" const char* ws_last_error(void) { return ws::g_last_error; }

extern "C" const char* ws_version(void) { return "wsgpu 0.2 gfx950"; }
