// sdm_errors.hip -- the thread-local error message of the C ABI (sdm_rt_last_error).
#include "sdm_common.h"

namespace sdmrt {

thread_local char g_err[512] = "";

int set_err(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace sdmrt

extern "C" const char* sdm_rt_last_error(void) { return sdmrt::g_err; }
