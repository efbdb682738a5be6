// C ABI of the kernel-level entry points (include/mla_hip.h).  Host-side
// validation, error capture (thread-local message) and kernel launches.
#include "mla_capi_util.hpp"
#include "mla_hip.h"
#include "mla_internal.hpp"

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>

namespace mla {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int gpu_status(hipError_t e, const char* what) {
    if (e == hipSuccess)
        return MLA_OK;
    return fail(e == hipErrorOutOfMemory ? MLA_ERR_OUT_OF_MEMORY : MLA_ERR_GPU,
                std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace mla

using namespace mla;

static_assert(MLA_INFO_INTS == kInfoInts && MLA_DECODE_WORKSPACE_HEAD == kMergeCounterBytes &&
                  MLA_DECODE_STATUS_OFFSET == kStatusOffset &&
                  MLA_DECODE_STATUS_XCD == kStatusXcd &&
                  MLA_DECODE_STATUS_UNPLACED == kStatusUnplaced &&
                  MLA_PLACE_MAX_SESSIONS == kPlaceMaxSessions,
              "mla_hip.h and mla_internal.hpp agree");

extern "C" {

const char* mla_last_error(void) { return g_last_error.c_str(); }

int mla_abi_version(void) { return 2; }

}  // extern "C"

namespace {

// Shared by mla_build_metadata and mla_build_metadata_placed: n_xcd = 0 (session order)
// or the XCD count the work list is laid out for.
int build_metadata(const char* fn, void* stream, int B, const int32_t* ctx_len,
                   const int32_t* q_len, const int32_t* cu_pages, const int32_t* page_ids,
                   int page_size, int max_pages, int num_pool_pages, int split_pages,
                   int target_blocks, int max_work, int max_rows, int n_xcd,
                   int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int32_t* page_table,
                   int32_t* slot_mapping, int32_t* num_splits, int32_t* cu_splits,
                   int32_t* work_session, int32_t* work_split, int32_t* work_desc,
                   int32_t* work_pages, int32_t* info) {
    if (!info || !cu_seqlens_q || !cu_seqlens_k || !cu_splits || !cu_pages ||
        (B > 0 && (!ctx_len || !q_len || !num_splits || (max_pages > 0 && !page_table))) ||
        (max_work > 0 && (!work_session || !work_split || !work_desc || !work_pages)) ||
        (max_rows > 0 && !slot_mapping))
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": null buffer");
    if ((long long)B * max_pages > (1LL << 40))
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": page table too large");
    MetadataArgs a{B, ctx_len, q_len, cu_pages, page_ids, page_size, max_pages, num_pool_pages,
                   split_pages, target_blocks, max_work, max_rows, cu_seqlens_q, cu_seqlens_k,
                   page_table, slot_mapping, num_splits, cu_splits, work_session, work_split,
                   work_desc, work_pages, info, n_xcd};
    return gpu_status(launch_build_metadata(a, static_cast<hipStream_t>(stream)), fn);
}

bool scalars_ok(int B, int page_size, int max_pages, int num_pool_pages, int split_pages,
                int target_blocks, int max_work, int max_rows) {
    return B >= 0 && page_size >= 1 && max_pages >= 0 && num_pool_pages >= 0 &&
           split_pages >= 0 && target_blocks >= 1 && max_work >= 0 && max_work <= kMaxWork &&
           max_rows >= 0;
}

// Per device: 0 unknown, else 1 + the XCD count (1 = the probe failed), and the reason of
// a failure.
std::mutex g_place_mu;
int g_place_known[64];
std::string g_place_reason[64];

// Status reads still to be failed on purpose (mla_testing_fail_decode_status).
std::atomic<int> g_forced_failures{0};

}  // namespace

namespace mla {

int32_t decode_head_status(const int32_t* head) {
    int32_t st = head[kStatusOffset / sizeof(int32_t)];
    for (int i = 0; i < kPlaceMaxSessions; ++i)
        if (head[i] != 0) {  // a session nobody merged (or merged early from a stale count)
            st |= kStatusXcd;
            break;
        }
    for (int f = g_forced_failures.load(); f > 0;)
        if (g_forced_failures.compare_exchange_weak(f, f - 1)) {
            st |= kStatusXcd;
            break;
        }
    return st;
}

}  // namespace mla

extern "C" {

int mla_build_metadata(void* stream, int B, const int32_t* ctx_len, const int32_t* q_len,
                       const int32_t* cu_pages, const int32_t* page_ids, int page_size,
                       int max_pages, int num_pool_pages, int split_pages, int target_blocks,
                       int max_work, int max_rows, int placement, int32_t* cu_seqlens_q,
                       int32_t* cu_seqlens_k, int32_t* page_table, int32_t* slot_mapping,
                       int32_t* num_splits, int32_t* cu_splits, int32_t* work_session,
                       int32_t* work_split, int32_t* work_desc, int32_t* work_pages,
                       int32_t* info) {
    if (!scalars_ok(B, page_size, max_pages, num_pool_pages, split_pages, target_blocks,
                    max_work, max_rows) ||
        (placement != 0 && placement != 1))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_build_metadata: invalid scalar argument");
    int n_xcd = 0;
    if (placement) {
        if (B > kPlaceMaxSessions)
            return fail(MLA_ERR_UNSUPPORTED, "mla_build_metadata: XCD placement takes at most " +
                                                 std::to_string(kPlaceMaxSessions) + " sessions");
        n_xcd = mla_xcd_placement_supported();
        if (n_xcd < 1)
            return fail(MLA_ERR_UNSUPPORTED,
                        "mla_build_metadata: XCD placement unavailable on this device (" +
                            g_last_error + ")");
    }
    return build_metadata("mla_build_metadata", stream, B, ctx_len, q_len, cu_pages, page_ids,
                          page_size, max_pages, num_pool_pages, split_pages, target_blocks,
                          max_work, max_rows, n_xcd, cu_seqlens_q, cu_seqlens_k, page_table,
                          slot_mapping, num_splits, cu_splits, work_session, work_split,
                          work_desc, work_pages, info);
}

int mla_build_metadata_placed(void* stream, int B, const int32_t* ctx_len, const int32_t* q_len,
                              const int32_t* cu_pages, const int32_t* page_ids, int page_size,
                              int max_pages, int num_pool_pages, int split_pages,
                              int target_blocks, int max_work, int max_rows, int n_xcds,
                              int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int32_t* page_table,
                              int32_t* slot_mapping, int32_t* num_splits, int32_t* cu_splits,
                              int32_t* work_session, int32_t* work_split, int32_t* work_desc,
                              int32_t* work_pages, int32_t* info) {
    if (!scalars_ok(B, page_size, max_pages, num_pool_pages, split_pages, target_blocks,
                    max_work, max_rows) ||
        n_xcds < 1 || n_xcds > kPlaceMaxXcds)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "mla_build_metadata_placed: invalid scalar argument (n_xcds in 1.." +
                        std::to_string(kPlaceMaxXcds) + ")");
    if (B > kPlaceMaxSessions)
        return fail(MLA_ERR_UNSUPPORTED, "mla_build_metadata_placed: XCD placement takes at most " +
                                             std::to_string(kPlaceMaxSessions) + " sessions");
    return build_metadata("mla_build_metadata_placed", stream, B, ctx_len, q_len, cu_pages,
                          page_ids, page_size, max_pages, num_pool_pages, split_pages,
                          target_blocks, max_work, max_rows, n_xcds, cu_seqlens_q, cu_seqlens_k,
                          page_table, slot_mapping, num_splits, cu_splits, work_session,
                          work_split, work_desc, work_pages, info);
}

int mla_xcd_placement_supported(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        fail(MLA_ERR_GPU, "mla_xcd_placement_supported: no current device");
        return 0;
    }
    std::lock_guard<std::mutex> lk(g_place_mu);
    if (!g_place_known[dev]) {
        g_place_reason[dev] = probe_xcd_placement();
        g_place_known[dev] = 1 + (g_place_reason[dev].empty() ? xcd_count() : 0);
    }
    if (g_place_known[dev] == 1) {
        fail(MLA_ERR_UNSUPPORTED, g_place_reason[dev]);
        return 0;
    }
    return g_place_known[dev] - 1;
}

int mla_testing_fail_decode_status(int count) {
    if (count < 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_testing_fail_decode_status: count < 0");
    g_forced_failures.store(count);
    return MLA_OK;
}

int mla_read_metadata_info(void* stream, const int32_t* info, int32_t* host_info) {
    if (!info || !host_info)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_read_metadata_info: null buffer");
    auto s = static_cast<hipStream_t>(stream);
    int st = gpu_status(hipMemcpyAsync(host_info, info, kInfoInts * sizeof(int32_t),
                                       hipMemcpyDeviceToHost, s),
                        "mla_read_metadata_info");
    if (st)
        return st;
    st = gpu_status(hipStreamSynchronize(s), "mla_read_metadata_info");
    if (st)
        return st;
    if (host_info[0] < 0)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "invalid ragged batch: session " + std::to_string(host_info[1]) +
                        " has a bad length, page list or page id, or a capacity was exceeded");
    return MLA_OK;
}

int mla_append_latent(void* stream, int T, int kv_rank, int rope_dim, int page_size, int dtype,
                      const float* ckv, const float* krope, const int32_t* slot_mapping,
                      int num_pool_pages, void* pages) {
    if (T < 0 || kv_rank < 1 || rope_dim < 0 || page_size < 1 || num_pool_pages < 0 ||
        (dtype != MLA_DTYPE_F16 && dtype != MLA_DTYPE_BF16))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_append_latent: invalid argument");
    if (T > 0 && (!ckv || (rope_dim > 0 && !krope) || !slot_mapping || !pages))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_append_latent: null buffer");
    AppendArgs a{T, kv_rank, rope_dim, page_size, num_pool_pages, ckv, krope, slot_mapping,
                 static_cast<uint16_t*>(pages)};
    return gpu_status(launch_append(a, dtype, static_cast<hipStream_t>(stream)),
                      "mla_append_latent");
}


size_t mla_decode_workspace_bytes(int max_work, int max_sessions, int n_heads, int kv_rank) {
    if (max_work <= 0 || max_sessions < 0 || n_heads <= 0 || kv_rank <= 0)
        return 0;
    return decode_workspace_size(max_work, n_heads, kv_rank);
}

int mla_decode_status(void* stream, void* workspace, size_t workspace_bytes, int clear,
                      int32_t* status) {
    if (!status)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_decode_status: invalid argument");
    if (!workspace && workspace_bytes == 0)  // the no-allocation array of this device
        if (int st = noalloc_scratch(&workspace, &workspace_bytes))
            return st;
    if (!workspace || workspace_bytes < kMergeCounterBytes)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_decode_status: invalid argument");
    auto s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    int32_t head[kStatusOffset / sizeof(int32_t) + 1];
    hipError_t e = hipMemcpyAsync(head, ws, sizeof(head), hipMemcpyDeviceToHost, s);
    // A failed check can leave counts in the merge counters: clearing resets both.
    if (e == hipSuccess && clear)
        e = hipMemsetAsync(ws, 0, kMergeCounterBytes, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (int st = gpu_status(e, "mla_decode_status"))
        return st;
    *status = decode_head_status(head);
    return MLA_OK;
}

}  // extern "C"

namespace {

// Validates the decode-attention arguments and fills `a`; MLA_OK or an error status.
int decode_args(const char* fn, int B, int n_heads, int kv_rank, int rope_dim, int page_size,
                int dtype, float scale, const int32_t* cu_seqlens_q, const int32_t* page_table,
                int max_pages, int num_pool_pages, const void* pages, const void* q_latent,
                const void* q_rope, const int32_t* num_splits, const int32_t* cu_splits,
                const int32_t* work_desc, const int32_t* work_pages, const int32_t* info,
                int max_work, float* out, float* lse, void* workspace, size_t workspace_bytes,
                DecodeArgs& a) {
    if (B < 0 || n_heads < 1 || kv_rank < 1 || kv_rank > 1024 || rope_dim < 0 || rope_dim > 1024 ||
        page_size < 1 || max_pages < 0 || num_pool_pages < 0 || max_work < 0 ||
        max_work > kMaxWork || (dtype != MLA_DTYPE_F16 && dtype != MLA_DTYPE_BF16) ||
        !(scale > 0.0f))
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": invalid argument");
    if (B == 0 || max_work == 0)
        return MLA_OK;
    if (!cu_seqlens_q || !page_table || !pages || !q_latent || (rope_dim > 0 && !q_rope) ||
        !num_splits || !cu_splits || !work_desc || !work_pages || !info || !out)
        return fail(MLA_ERR_INVALID_ARGUMENT, std::string(fn) + ": null buffer");
    const size_t need = mla_decode_workspace_bytes(max_work, B, n_heads, kv_rank);
    if (!workspace || workspace_bytes < need)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": workspace needs " + std::to_string(need) + " bytes");
    a = DecodeArgs{};
    a.B = B;
    a.H = n_heads;
    a.kv_rank = kv_rank;
    a.rope_dim = rope_dim;
    a.page_size = page_size;
    a.max_pages = max_pages;
    a.num_pool_pages = num_pool_pages;
    a.max_work = max_work;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.cu_q = cu_seqlens_q;
    a.page_table = page_table;
    a.num_splits = num_splits;
    a.cu_splits = cu_splits;
    a.work_desc = work_desc;
    a.work_pages = work_pages;
    a.info = info;
    a.pages = static_cast<const uint16_t*>(pages);
    a.q_latent = static_cast<const uint16_t*>(q_latent);
    a.q_rope = static_cast<const uint16_t*>(q_rope);
    a.out = out;
    a.lse = lse;
    decode_workspace_layout(workspace, max_work, n_heads, kv_rank, a);
    return MLA_OK;
}

// The MFMA kernel issues 16-byte loads of q and of cache rows and 16-byte stores.
bool use_generic(const DecodeArgs& a, const void* workspace, int flags) {
    const bool aligned =
        ((reinterpret_cast<uintptr_t>(a.pages) | reinterpret_cast<uintptr_t>(a.q_latent) |
          reinterpret_cast<uintptr_t>(a.q_rope) | reinterpret_cast<uintptr_t>(a.out) |
          reinterpret_cast<uintptr_t>(workspace)) &
         15) == 0;
    return (flags & MLA_DECODE_FORCE_GENERIC) || !aligned;
}

}  // namespace

namespace mla {

// MLA_DECODE_FUSED_MERGE needs placed metadata, which holds at most kPlaceMaxSessions
// sessions on a device that passed the placement probe; the kernel then checks that the
// metadata was placed for this device's XCD count (a.xcd_n).
int fused_checks(DecodeArgs& a, int flags, const char* fn) {
    if (!(flags & MLA_DECODE_FUSED_MERGE))
        return MLA_OK;
    if (a.B > kPlaceMaxSessions)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": MLA_DECODE_FUSED_MERGE takes at most " +
                        std::to_string(kPlaceMaxSessions) + " sessions (placed metadata)");
    if (!a.fused_merge)
        return MLA_OK;  // a kernel that leaves the merge to merge_kernel: any metadata works
    a.xcd_n = mla_xcd_placement_supported();
    if (a.xcd_n < 1)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": MLA_DECODE_FUSED_MERGE needs XCD placement, which this "
                                      "device does not support (" + g_last_error + ")");
    return MLA_OK;
}

}  // namespace mla

extern "C" {

#define MLA_DECODE_PARAMS                                                                       \
    void *stream, int B, int n_heads, int kv_rank, int rope_dim, int page_size, int dtype,       \
        float scale, const int32_t *cu_seqlens_q, const int32_t *page_table, int max_pages,      \
        int num_pool_pages, const void *pages, const void *q_latent, const void *q_rope,         \
        const int32_t *num_splits, const int32_t *cu_splits, const int32_t *work_desc,           \
        const int32_t *work_pages, const int32_t *info, int max_work, float *out, float *lse,    \
        void *workspace, size_t workspace_bytes, int flags
#define MLA_DECODE_ARGS(fn)                                                                     \
    fn, B, n_heads, kv_rank, rope_dim, page_size, dtype, scale, cu_seqlens_q, page_table,        \
        max_pages, num_pool_pages, pages, q_latent, q_rope, num_splits, cu_splits, work_desc,    \
        work_pages, info, max_work, out, lse, workspace, workspace_bytes

int mla_decode_attention(MLA_DECODE_PARAMS) {
    DecodeArgs a;
    if (int st = decode_args(MLA_DECODE_ARGS("mla_decode_attention"), a))
        return st;
    if (B == 0 || max_work == 0)
        return MLA_OK;
    const auto s = static_cast<hipStream_t>(stream);
    const bool generic = use_generic(a, workspace, flags);
    a.fused_merge = (flags & MLA_DECODE_FUSED_MERGE) && decode_fuses_merge(a, generic);
    if (int st = fused_checks(a, flags, "mla_decode_attention"))
        return st;
    if (int st = gpu_status(launch_decode_partials(a, dtype, generic, s), "mla_decode_attention"))
        return st;
    if (a.fused_merge)
        return MLA_OK;
    return gpu_status(launch_merge(a, s), "mla_decode_attention");
}

int mla_decode_partials(MLA_DECODE_PARAMS) {
    DecodeArgs a;
    if (int st = decode_args(MLA_DECODE_ARGS("mla_decode_partials"), a))
        return st;
    if (B == 0 || max_work == 0)
        return MLA_OK;
    const bool generic = use_generic(a, workspace, flags);
    a.fused_merge = (flags & MLA_DECODE_FUSED_MERGE) && decode_fuses_merge(a, generic);
    if (int st = fused_checks(a, flags, "mla_decode_partials"))
        return st;
    return gpu_status(launch_decode_partials(a, dtype, generic, static_cast<hipStream_t>(stream)),
                      "mla_decode_partials");
}

int mla_decode_merge(void* stream, int B, int n_heads, int kv_rank, const int32_t* cu_seqlens_q,
                     const int32_t* num_splits, const int32_t* cu_splits, const int32_t* info,
                     int max_work, float* out, float* lse, const void* workspace,
                     size_t workspace_bytes) {
    if (B < 0 || n_heads < 1 || kv_rank < 1 || kv_rank > 1024 || max_work < 0 ||
        max_work > kMaxWork)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_decode_merge: invalid argument");
    if (B == 0 || max_work == 0)
        return MLA_OK;
    if (!cu_seqlens_q || !num_splits || !cu_splits || !info || !out)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_decode_merge: null buffer");
    const size_t need = mla_decode_workspace_bytes(max_work, B, n_heads, kv_rank);
    if (!workspace || workspace_bytes < need)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "mla_decode_merge: workspace needs " + std::to_string(need) + " bytes");
    DecodeArgs a{};
    a.B = B;
    a.H = n_heads;
    a.kv_rank = kv_rank;
    a.max_work = max_work;
    a.cu_q = cu_seqlens_q;
    a.num_splits = num_splits;
    a.cu_splits = cu_splits;
    a.info = info;
    a.out = out;
    a.lse = lse;
    decode_workspace_layout(const_cast<void*>(workspace), max_work, n_heads, kv_rank, a);
    return gpu_status(launch_merge(a, static_cast<hipStream_t>(stream)), "mla_decode_merge");
}

int mla_prefill_attention(void* stream, int B, int n_heads, int kv_rank, int rope_dim,
                          int page_size, int dtype, float scale, const int32_t* cu_seqlens_q,
                          const int32_t* cu_seqlens_k, const int32_t* page_table, int max_pages,
                          int num_pool_pages, const void* pages, const void* q_latent,
                          const void* q_rope, const int32_t* info, int max_q_len, float* out,
                          float* lse, int flags) {
    if (B < 0 || B > 65535 || n_heads < 1 || n_heads > 65535 || kv_rank < 1 || kv_rank > 1024 ||
        rope_dim < 0 || rope_dim > 1024 || page_size < 1 || max_pages < 0 ||
        num_pool_pages < 0 || max_q_len < 0 ||
        (dtype != MLA_DTYPE_F16 && dtype != MLA_DTYPE_BF16) || !(scale > 0.0f))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_prefill_attention: invalid argument");
    if (B == 0 || max_q_len < 2)
        return MLA_OK;
    if (!cu_seqlens_q || !cu_seqlens_k || !page_table || !pages || !q_latent ||
        (rope_dim > 0 && !q_rope) || !info || !out)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_prefill_attention: null buffer");
    PrefillArgs a{};
    a.B = B;
    a.H = n_heads;
    a.kv_rank = kv_rank;
    a.rope_dim = rope_dim;
    a.page_size = page_size;
    a.max_pages = max_pages;
    a.num_pool_pages = num_pool_pages;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.cu_q = cu_seqlens_q;
    a.cu_k = cu_seqlens_k;
    a.page_table = page_table;
    a.info = info;
    a.pages = static_cast<const uint16_t*>(pages);
    a.q_latent = static_cast<const uint16_t*>(q_latent);
    a.q_rope = static_cast<const uint16_t*>(q_rope);
    a.out = out;
    a.lse = lse;
    // The MFMA kernel issues 16-byte loads of q and cache chunks and 16-byte stores.
    const bool aligned =
        ((reinterpret_cast<uintptr_t>(pages) | reinterpret_cast<uintptr_t>(q_latent) |
          reinterpret_cast<uintptr_t>(q_rope) | reinterpret_cast<uintptr_t>(out)) &
         15) == 0;
    return gpu_status(launch_prefill(a, max_q_len, dtype,
                                     (flags & MLA_DECODE_FORCE_GENERIC) || !aligned,
                                     static_cast<hipStream_t>(stream)),
                      "mla_prefill_attention");
}

}  // extern "C"
