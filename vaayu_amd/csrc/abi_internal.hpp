// Error reporting shared by the entry points (thread-local last error).
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/vaayu_amd.h"

namespace vaayu {

int set_error(int code, const char* msg);
void clear_error();
// The launch status of the kernels just enqueued: 0, or the hipError_t (message kept).
int check_launch(const char* what);

}  // namespace vaayu
