// Error reporting and version entry points of libzenith_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include "zk_common.hpp"

namespace zk {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(ZK_ERR_HIP, "%s: kernel launch failed: %s", what,
                hipGetErrorString(e));
  return ZK_OK;
}

}  // namespace zk

extern "C" const char *zk_last_error(void) { return zk::g_last_error; }

// Major * 10000 + minor * 100 + patch.
extern "C" int zk_version(void) { return 100; }
