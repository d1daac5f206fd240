// Error reporting shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/slo_attn.h"

namespace slo {

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const char* msg);

// Checks the launch that was just enqueued; never synchronises.
int check_launch(const char* what);

}  // namespace slo
