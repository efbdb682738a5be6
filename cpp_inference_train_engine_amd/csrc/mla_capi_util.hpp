// Error capture shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace mla {

// Records msg as this thread's last error and returns code.
int fail(int code, const std::string& msg);
// MLA_OK for hipSuccess, else MLA_ERR_GPU / MLA_ERR_OUT_OF_MEMORY with the HIP message.
int gpu_status(hipError_t e, const char* what);

}  // namespace mla
