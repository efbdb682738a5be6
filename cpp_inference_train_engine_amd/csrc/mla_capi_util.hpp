// Error capture shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace mla {

// Records msg as this thread's last error and returns code.
int fail(int code, const std::string& msg);
// MLA_OK for hipSuccess, else MLA_ERR_GPU / MLA_ERR_OUT_OF_MEMORY with the HIP message.
int gpu_status(hipError_t e, const char* what);

struct DecodeArgs;
// Checks MLA_DECODE_FUSED_MERGE in `flags` against the batch and the device and fills the
// XCD count the fused kernel verifies (a.xcd_n); MLA_OK or an error status.
int fused_checks(DecodeArgs& a, int flags, const char* fn);
// The file-scope array of mla_decode_attention_noalloc on the current device.
int noalloc_scratch(void** out, size_t* bytes);

}  // namespace mla
