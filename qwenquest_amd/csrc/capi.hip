// Library-level entry points: version and error reporting.
#include <stdarg.h>
#include <string.h>

#include "qq_common.h"

namespace qq {
namespace {
thread_local char g_last_error[1024] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(QQ_EHIP, "%s: %s", what, hipGetErrorString(e));
  return QQ_OK;
}

}  // namespace qq

extern "C" int qq_version(void) { return 100; }

extern "C" const char* qq_last_error(void) { return qq::g_last_error; }
