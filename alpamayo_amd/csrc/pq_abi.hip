// Library-wide entry points: ABI version and the thread-local error message.
#include <cstdarg>
#include <cstdio>

#include "pq_common.h"

namespace pq {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return PQ_ERR_HIP;
  }
  return PQ_OK;
}

}  // namespace pq

extern "C" int pq_abi_version(void) { return PQ_ABI_VERSION; }

extern "C" const char* pq_last_error(void) { return pq::g_last_error; }
