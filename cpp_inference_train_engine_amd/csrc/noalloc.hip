// mla_decode_attention_noalloc: the decode attention call for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  The split partials that mla_decode_attention keeps in the caller's
// workspace live here in a file-scope device array instead, one copy per GPU, held until
// the process ends.  Same kernels, same results as mla_decode_attention.
#include "mla_capi_util.hpp"
#include "mla_hip.h"
#include "mla_internal.hpp"

#include <mutex>
#include <string>

constexpr size_t kScratchBytes = (size_t)MLA_NOALLOC_SCRATCH_MIB << 20;

// The workspace of the decode: a head of merge counters and the status word (zero at
// load, and every fused call without a failed check leaves the counters zero), then the
// partials (o[kv_rank] and (m, l) per work item and head), which every merge reads only
// after its work items wrote them in the same call.  In host code this name is not a
// device address: kernels get the address from scratch_on().
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch` on each GPU

// The address of this GPU's `scratch` (resolved once per device, with it current).
int scratch_on(int device, void** out) {
    if (device < 0 || device >= kMaxDevices)
        return mla::fail(MLA_ERR_UNSUPPORTED, "mla_decode_attention_noalloc: device index " +
                                                  std::to_string(device) + " out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return mla::gpu_status(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                   "mla_decode_attention_noalloc: scratch address");
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return MLA_OK;
}

}  // namespace

namespace mla {

// The no-allocation array of the current device (its head holds the fused merge's
// counters and the decode status word, as a workspace's does).
int noalloc_scratch(void** out, size_t* bytes) {
    int device = -1;
    if (hipError_t e = hipGetDevice(&device); e != hipSuccess)
        return gpu_status(e, "mla_decode_status");
    *bytes = kScratchBytes;
    return scratch_on(device, out);
}

}  // namespace mla

extern "C" {

size_t mla_noalloc_scratch_bytes(void) { return kScratchBytes; }

int mla_decode_attention_noalloc(void* stream, int B, int n_heads, int kv_rank, int rope_dim,
                                 int page_size, int dtype, float scale,
                                 const int32_t* cu_seqlens_q, const int32_t* page_table,
                                 int max_pages, int num_pool_pages, const void* pages,
                                 const void* q_latent, const void* q_rope,
                                 const int32_t* num_splits, const int32_t* cu_splits,
                                 const int32_t* work_desc, const int32_t* work_pages,
                                 const int32_t* info, int max_work, float* out, float* lse,
                                 int flags) {
    const size_t need = mla_decode_workspace_bytes(max_work, B, n_heads, kv_rank);
    if (need > kScratchBytes)
        return mla::fail(MLA_ERR_INVALID_ARGUMENT,
                         "mla_decode_attention_noalloc: the split partials need " +
                             std::to_string(need) + " bytes, above the " +
                             std::to_string(kScratchBytes) +
                             "-byte scratch maximum (use mla_decode_attention with a workspace)");
    int device = -1;
    hipError_t e = hipGetDevice(&device);
    if (e == hipSuccess && stream) {
        int stream_device = -1;
        e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_device);
        if (e == hipSuccess && stream_device != device)
            return mla::fail(MLA_ERR_INVALID_ARGUMENT,
                             "mla_decode_attention_noalloc: the stream's device must be the "
                             "current device");
    }
    if (e != hipSuccess)
        return mla::gpu_status(e, "mla_decode_attention_noalloc");
    void* ws = nullptr;
    if (int st = scratch_on(device, &ws))
        return st;
    return mla_decode_attention(stream, B, n_heads, kv_rank, rope_dim, page_size, dtype, scale,
                                cu_seqlens_q, page_table, max_pages, num_pool_pages, pages,
                                q_latent, q_rope, num_splits, cu_splits, work_desc, work_pages,
                                info, max_work, out, lse, ws, kScratchBytes, flags);
}

}  // extern "C"
