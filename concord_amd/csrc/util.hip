// util.hip -- error reporting, version and workspace sizing of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "workspace.h"

namespace concord {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return CONCORD_ELAUNCH;
  }
  return CONCORD_OK;
}

}  // namespace concord

extern "C" const char* concord_last_error(void) { return concord::g_err; }

extern "C" int concord_version(void) { return 1; }

extern "C" size_t concord_workspace_bytes(int64_t N, int64_t K, int64_t M) {
  if (N < 1) N = 1;
  if (K < 1) K = 1;
  if (M < 0) M = 0;
  return concord::workspace_layout(N, K, M).total;
}
