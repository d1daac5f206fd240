// Thread-local last-error string of the C-ABI (the library's only mutable
// global state besides the per-device launch-shape cache).
#include <cstdio>
#include <cstring>
#include "capi_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace slo {

int fail(int code, const char* msg) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    std::snprintf(g_last_error, sizeof(g_last_error), "%s: launch failed: %s", what, hipGetErrorString(e));
    return SLO_ERR_HIP;
  }
  return SLO_OK;
}

}  // namespace slo

extern "C" const char* slo_last_error(void) { return g_last_error; }

extern "C" size_t slo_paged_attention_args_size(void) { return sizeof(slo_paged_attention_args); }
