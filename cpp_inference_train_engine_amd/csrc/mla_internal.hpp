// Kernel argument blocks and launchers shared between the .hip translation
// units and the C ABI (capi.hip).  Host-visible, no device code.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include <cstddef>
#include <cstdint>

namespace mla {

// Work descriptor of one split-K work item (kWorkDescInts int32):
//   {session, first query row, k_len, page_begin, page_end, num_splits of the
//    session, partial slot of the item, q_len}; session -1 = no work.  The partial slot
//    is cu_splits[session] + the item's split index: a session's partials are
//    contiguous whatever slot of the work list the item itself occupies.
// work_pages holds the ids of the item's first kWorkPages pages (-1 past the end).
constexpr int kWorkDescInts = 8;  // MLA_WORK_DESC_INTS
constexpr int kWorkPages = 8;     // MLA_WORK_PAGES
constexpr int kMaxWork = 65535;   // MLA_MAX_WORK
// info[kInfoInts] of a build: {W, split, total_q, total_k, n (the XCD count the work list
// is placed for, 0 = session order), 0, 0, 0}, or {-1, first bad session, 0, ...}.
constexpr int kInfoInts = 8;      // MLA_INFO_INTS
constexpr int kInfoPlacement = 4;

struct MetadataArgs {
    int B;
    const int32_t *ctx_len, *q_len, *cu_pages, *page_ids;
    int page_size, max_pages, num_pool_pages, split_pages, target_blocks, max_work, max_rows;
    int32_t *cu_seqlens_q, *cu_seqlens_k, *page_table, *slot_mapping, *num_splits, *cu_splits,
        *work_session, *work_split, *work_desc, *work_pages, *info;
    // XCD placement of the work list: the number of XCDs n (0 = work items in session
    // order).  With n > 0 every session's items sit in consecutive slots x + n k of one
    // XCD (the workgroups w of a launch with one residue w % n share an XCD), dealt to the XCDs by
    // pages read, largest first, in rounds of n (see place_sessions); info[4] records n.
    // B <= kPlaceMaxSessions, n <= kPlaceMaxXcds.
    int placement;
};
constexpr int kPlaceMaxSessions = 256;  // MLA_PLACE_MAX_SESSIONS
constexpr int kPlaceMaxXcds = 8;

struct AppendArgs {
    int T, kv_rank, rope_dim, page_size, num_pool_pages;
    const float *ckv, *krope;
    const int32_t* slot_mapping;
    uint16_t* pages;
};

// Absorbed decode attention.  Partials live in the workspace:
//   part_o [max_work][H][kv_rank] fp32 (unnormalised), part_ml [max_work][H][2]
//   (running max in log2 units, running denominator).
struct DecodeArgs {
    int B, H, kv_rank, rope_dim, page_size, max_pages, num_pool_pages, max_work;
    float scale_log2;  // softmax scale * log2(e)
    const int32_t *cu_q, *page_table, *num_splits, *cu_splits, *work_desc, *work_pages, *info;
    const uint16_t *pages, *q_latent, *q_rope;
    float *out, *lse, *part_o, *part_ml;
    // Fused merge (decode_page_kernel only): the metadata was built XCD-placed, and the
    // last item of a split session to finish combines the session's partials itself.
    // merge_count[B] (in the workspace, zero between launches) counts finished items.
    int fused_merge;
    int32_t* merge_count;
    // What the fused kernel checks: the metadata must record placement for this device's
    // xcd_n XCDs (info[4]); otherwise it raises kStatusUnplaced in *status and does not merge.
    int xcd_n;
    int32_t* status;
};
// Bits of the decode status (MLA_DECODE_STATUS_*).  kStatusXcd is not raised by a kernel:
// the host derives it from merge counters left nonzero after a call (see
// decode_head_status).
constexpr int kStatusXcd = 1;       // a split session's items did not all meet in one L2
constexpr int kStatusUnplaced = 2;  // fused flag over metadata not placed for this device

// Chunked-prefill attention (sessions with q_len > 1, causal within the chunk).
struct PrefillArgs {
    int B, H, kv_rank, rope_dim, page_size, max_pages, num_pool_pages;
    float scale_log2;  // softmax scale * log2(e)
    const int32_t *cu_q, *cu_k, *page_table, *info;
    const uint16_t *pages, *q_latent, *q_rope;
    float *out, *lse;
};

hipError_t launch_build_metadata(const MetadataArgs& a, hipStream_t stream);
// Workspace of decode attention: a head block of fixed size first -- the fused merge's
// per-session counters (fused calls have placed metadata, B <= kPlaceMaxSessions), then
// the status word on a line of its own -- so that both keep their place whatever max_work
// and B a later call on the same buffer has; then the split partials, 256-byte aligned:
// part_o [max_work][H][kv_rank] and part_ml, whose (m, l) pairs of one slot take [H][2]
// floats padded to whole 128-byte lines (part_ml_stride floats per slot), so that no
// cache line holds two slots' pairs.
constexpr size_t kStatusOffset = kPlaceMaxSessions * sizeof(int32_t);  // MLA_DECODE_STATUS_OFFSET
constexpr size_t kMergeCounterBytes = kStatusOffset + 256;
__host__ __device__ inline int part_ml_stride(int n_heads) { return (2 * n_heads + 31) & ~31; }
inline size_t decode_partial_bytes(int max_work, int n_heads, int kv_rank) {
    const size_t b = (size_t)max_work *
                     ((size_t)n_heads * kv_rank + part_ml_stride(n_heads)) * sizeof(float);
    return (b + 255) & ~(size_t)255;
}
inline size_t decode_workspace_size(int max_work, int n_heads, int kv_rank) {
    return kMergeCounterBytes + decode_partial_bytes(max_work, n_heads, kv_rank);
}
inline void decode_workspace_layout(void* ws, int max_work, int n_heads, int kv_rank,
                                    DecodeArgs& a) {
    a.merge_count = static_cast<int32_t*>(ws);
    a.status = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + kStatusOffset);
    a.part_o = reinterpret_cast<float*>(static_cast<char*>(ws) + kMergeCounterBytes);
    a.part_ml = a.part_o + (size_t)max_work * n_heads * kv_rank;
}
// XCDs of the current device (0 if unknown), and whether its dispatch keeps the
// workgroups w of a launch with one residue w % n on one XCD (empty string) or why not.
int xcd_count();
std::string probe_xcd_placement();
// The decode status of a workspace head copied to the host (kMergeCounterBytes / 4
// words): the status word, plus kStatusXcd when a merge counter was left nonzero (capi.hip).
int32_t decode_head_status(const int32_t* head);
hipError_t launch_append(const AppendArgs& a, int dtype, hipStream_t stream);
// Decode kernel only (MFMA page kernel, or the generic one when force_generic or the
// shape is outside it): final rows of one-item sessions, partials of the others.
hipError_t launch_decode_partials(const DecodeArgs& a, int dtype, bool force_generic,
                                  hipStream_t stream);
// Log-sum-exp merge of the partials into the rows of split sessions.
hipError_t launch_merge(const DecodeArgs& a, hipStream_t stream);
bool decode_mfma_supported(int H, int kv_rank, int rope_dim, int page_size);
// Only the MFMA page kernel merges inside its launch; the others leave partials.
inline bool decode_fuses_merge(const DecodeArgs& a, bool generic) {
    return !generic && decode_mfma_supported(a.H, a.kv_rank, a.rope_dim, a.page_size);
}
// The DeepSeek-like shape (16 < H <= 128, kv_rank 512, rope 64, 64-token pages).
bool decode_wide_supported(int H, int kv_rank, int rope_dim, int page_size);
hipError_t launch_decode_wide(const DecodeArgs& a, int dtype, hipStream_t stream);
// Prefill attention for the sessions with q_len > 1 (max_q_len >= their q_len).
hipError_t launch_prefill(const PrefillArgs& a, int max_q_len, int dtype, bool force_generic,
                          hipStream_t stream);
bool prefill_mfma_supported(int H, int kv_rank, int rope_dim, int page_size);

}  // namespace mla
