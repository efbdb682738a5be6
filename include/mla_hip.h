/*
 * mla_hip.h -- C ABI of the MI355X (gfx950) MLA cached-decode backend.
 *
 * This is the drop-in boundary for the reference engine's inference backend
 * (Astrowebdeving/cpp_inference_train_engine).  The reference's backend plugin
 * interface is the C++ class `mini_mla::Execution`
 * (include/mini_mla/execution.hpp:28-62) with the factory `make_execution`
 * (execution.hpp:63-66, src/infer/inference.cpp:314-329) dispatching to
 * `make_mps_execution` (execution.hpp:67-68, src/backends/mps_backend.mm:1943-1977).
 * The C++20 host API in cpp_inference_train_engine_amd/host (libmla_host.so:
 * Execution / HipExecution, Tokenizer, InferenceEngine, Server) implements those
 * interfaces over these functions; other hosts bind them with ctypes / FFI.
 *
 * Conventions
 *  - Every function returns an int status: MLA_OK or MLA_ERR_* (the reference
 *    ErrorCode values of include/mini_mla/result.hpp:12-19, plus one, and
 *    MLA_ERR_UNAVAILABLE of the scheduler).  The message of the last failure on
 *    the calling thread is mla_last_error().
 *  - Pointers named d_* / documented "device" are device (HBM) pointers;
 *    `stream` is a hipStream_t (NULL = the default stream).  Work is
 *    stream-ordered and asynchronous unless stated.
 *  - Output buffers are owned by the caller.  No call is thread-safe against
 *    another call on the same objects; distinct streams/objects may be used
 *    from different threads (the reference's fork-per-thread rule,
 *    docs/architecture.md:37).
 *  - 16-bit element dtype codes: MLA_DTYPE_F16 (0), MLA_DTYPE_BF16 (1).
 *
 * Paged latent cache layout (one pool per layer): page p is one contiguous
 * record of page_size * (kv_rank + rope_dim) 16-bit words: the latent section
 * (page_size * kv_rank words) then the rope-key section (page_size * rope_dim).
 * When page_size % 16 == 0, kv_rank % 32 == 0 and rope_dim % 8 == 0 (every
 * production shape) the record is tiled in MFMA-operand order so that a wave's
 * 16-byte-per-lane load reads 1 KB contiguously: with t = slot/16, n = slot%16,
 *     latent (slot, r) -> ((t*(kv_rank/32) + r/32)*4 + (r%32)/8)*128 + n*8 + r%8
 *     rope (slot, c)   -> page_size*kv_rank + (t*(rope_dim/8) + c/8)*128 + n*8 + c%8
 * otherwise it is row-major (latent slot*kv_rank + r, rope
 * page_size*kv_rank + slot*rope_dim + c).  mla_append_latent writes this format.
 * Token position t of session b lives in page page_table[b][t / page_size],
 * slot t % page_size.  The cache holds the kv_norm-ed latent and the RoPE-ed
 * key exactly as the reference's CpuDecoder cache does
 * (src/infer/inference.cpp:91-103), rounded once to 16 bits.
 */
#ifndef MLA_HIP_H
#define MLA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLA_OK 0
#define MLA_ERR_INVALID_ARGUMENT 1 /* ErrorCode::invalid_argument */
#define MLA_ERR_IO 2               /* ErrorCode::io_error */
#define MLA_ERR_UNSUPPORTED 3      /* ErrorCode::unsupported */
#define MLA_ERR_OUT_OF_MEMORY 4    /* ErrorCode::out_of_memory */
#define MLA_ERR_GPU 5              /* ErrorCode::gpu_error */
#define MLA_ERR_NUMERICAL 6        /* ErrorCode::numerical_error */

#define MLA_DTYPE_F16 0
#define MLA_DTYPE_BF16 1

/* Decode-attention flags. */
#define MLA_DECODE_FORCE_GENERIC 1 /* use the portable VALU kernel even when the MFMA one fits */
#define MLA_DECODE_FUSED_MERGE 2   /* metadata built with placement = 1: merge inside the launch */
/* mla_model_step / mla_model_forward: no read-ahead of the decode attention's pages into L2
 * during each layer's projection kernel (the results are the same bit for bit; the
 * read-ahead only changes timing). */
#define MLA_STEP_NO_READ_AHEAD 4

/* Message of the last failed call on this thread ("" if none). */
const char* mla_last_error(void);
/* ABI version of this library: 2.  Version 1 had info[4], no placement argument of
 * mla_build_metadata, no `flags` of mla_model_step / mla_model_forward, and a decode
 * workspace without the head block (counters and status word) described at
 * mla_decode_attention; a caller built against version 1 must not bind version 2. */
int mla_abi_version(void);

/* ------------------------------------------------------------------ (a)
 * Ragged-batch metadata, built on the GPU in one launch.  No reference
 * function: the reference keeps one contiguous cache per session
 * (src/infer/inference.cpp:15-18).  Nearest precedent: the Gemma engine's
 * per-row lengths/cursors/write slots (src/infer/gemma.cpp:383-427).
 *
 * Inputs (device): ctx_len[B] tokens already cached per session, q_len[B]
 * tokens appended this step, cu_pages[B+1] + page_ids[] the per-session
 * physical page lists.  Scalars: page_size, max_pages (columns of the padded
 * table), num_pool_pages (valid page ids are [0, num_pool_pages)),
 * split_pages (>0 fixed pages per work item; 0 = auto, ceil(total pages of
 * sessions with q_len>0 / target_blocks)), max_work (<= MLA_MAX_WORK) and
 * max_rows capacities, placement (0: work items in session order; 1: XCD
 * placement, below).
 * Outputs (device): cu_seqlens_q[B+1], cu_seqlens_k[B+1],
 * page_table[B * max_pages] (-1 padded), slot_mapping[max_rows] (flat slot
 * page*page_size+offset of every appended token), num_splits[B],
 * cu_splits[B+1], work_session[max_work], work_split[max_work] (the
 * block-to-session map), work_desc[max_work * MLA_WORK_DESC_INTS] (per work
 * item: session, first query row, k_len, page_begin, page_end, num_splits of
 * the session, partial slot = cu_splits[session] + split index, q_len; session
 * -1 marks every empty slot, and all items of a failed build),
 * work_pages[max_work * MLA_WORK_PAGES] (ids of each item's first pages, -1
 * past its end) and info[MLA_INFO_INTS]:
 *     ok:    {W (work items), split_pages used, total_q, total_k,
 *             n (XCDs the work list is placed for, 0 = session order), 0, 0, 0}
 *     error: {-1, first offending session, 0, 0, 0, 0, 0, 0}
 * A session is invalid when q_len<0, ctx_len<0, it lists more than
 * max_pages pages or fewer than ceil((ctx+q)/page_size), a page id is out of
 * range, a running total exceeds INT32_MAX, or the work/row capacity is
 * exceeded.  Errors are reported through info (read it with
 * mla_read_metadata_info); every consumer kernel treats info[0] < 0 as an
 * empty batch.
 *
 * XCD placement (placement = 1; no reference counterpart): the work list is laid
 * out so that all items of a session run on one XCD of the GPU, whose dispatch
 * puts the workgroups w of a launch with one residue w % n on one XCD (n XCDs; checked
 * once per device by mla_xcd_placement_supported).  Sessions ranked by pages read, largest first
 * (ties: lower session), are dealt to the XCDs in rounds of n: rank r to XCD r % n
 * in even rounds and n - 1 - r % n in odd ones, so no XCD's pages exceed another's
 * by more than the largest session's.  Item sp of session b goes to slot
 * x_b + n * (k_b + sp), where k_b counts the items of XCD x_b's sessions of earlier
 * rounds; slots no item takes are empty
 * (session -1).  Needs B <= MLA_PLACE_MAX_SESSIONS and max_work >= n times the
 * largest item count of one XCD (info error {-1, B, 0, 0} otherwise);
 * MLA_ERR_UNSUPPORTED when the device fails the check.  Decode attention over
 * placed metadata may then merge the split partials inside its launch
 * (MLA_DECODE_FUSED_MERGE). */
#define MLA_PLACE_MAX_SESSIONS 256
#define MLA_INFO_INTS 8
#define MLA_WORK_DESC_INTS 8
#define MLA_WORK_PAGES 8
#define MLA_MAX_WORK 65535
int mla_build_metadata(void* stream, int B, const int32_t* ctx_len, const int32_t* q_len,
                       const int32_t* cu_pages, const int32_t* page_ids, int page_size,
                       int max_pages, int num_pool_pages, int split_pages, int target_blocks,
                       int max_work, int max_rows, int placement, int32_t* cu_seqlens_q,
                       int32_t* cu_seqlens_k, int32_t* page_table, int32_t* slot_mapping,
                       int32_t* num_splits, int32_t* cu_splits, int32_t* work_session,
                       int32_t* work_split, int32_t* work_desc, int32_t* work_pages,
                       int32_t* info);

/* mla_build_metadata with the work list placed for an explicit count of n_xcds XCDs
 * (1..8) instead of the current device's, and without the device probe: for tests of
 * the layout and for hosts that prepare work for another device.  Decode attention with
 * MLA_DECODE_FUSED_MERGE refuses to merge over metadata placed for another count than the
 * device's (see mla_decode_status).  No reference counterpart. */
int mla_build_metadata_placed(void* stream, int B, const int32_t* ctx_len, const int32_t* q_len,
                              const int32_t* cu_pages, const int32_t* page_ids, int page_size,
                              int max_pages, int num_pool_pages, int split_pages,
                              int target_blocks, int max_work, int max_rows, int n_xcds,
                              int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int32_t* page_table,
                              int32_t* slot_mapping, int32_t* num_splits, int32_t* cu_splits,
                              int32_t* work_session, int32_t* work_split, int32_t* work_desc,
                              int32_t* work_pages, int32_t* info);

/* Synchronises `stream`, copies info[MLA_INFO_INTS] to host_info and returns
 * MLA_ERR_INVALID_ARGUMENT (naming the session) if the build failed. */
int mla_read_metadata_info(void* stream, const int32_t* info, int32_t* host_info);

/* The XCD count n >= 1 of the current device if its dispatch keeps the workgroups w of a
 * launch with one residue w % n on one XCD, the n residues on n XCDs (the premise of XCD
 * placement; which XCD takes residue 0 may differ between hardware queues), else 0 with
 * the reason in mla_last_error().  The first call per device runs a probe kernel and
 * synchronises: call it before any stream capture that builds placed metadata. */
int mla_xcd_placement_supported(void);

/* ------------------------------------------------------------------ (b)
 * Paged latent append; refines the reference's contiguous append
 * `latent_[l][pos,:] = c_kv; rope_[l][pos,:] = k_rope`
 * (src/infer/inference.cpp:100-103; MPS scatter mps_backend.mm:542-555).
 * Row t of ckv [T x kv_rank] and krope [T x rope_dim] (device fp32) is rounded
 * (RNE, as to_half in src/core/io.cpp:152-158) and written to flat slot
 * slot_mapping[t] of the pool `pages`.  Slots must lie inside the pool
 * (num_pool_pages pages); out-of-range slots are skipped. */
int mla_append_latent(void* stream, int T, int kv_rank, int rope_dim, int page_size, int dtype,
                      const float* ckv, const float* krope, const int32_t* slot_mapping,
                      int num_pool_pages, void* pages);

/* ------------------------------------------------------------------ (c)
 * Absorbed MLA decode attention over the paged cache: the per-head loop of
 * CpuDecoder::decode (src/infer/inference.cpp:116-153) and the MPS graph
 * (mps_backend.mm:556-572), for every session with q_len == 1 in the batch:
 *     s_i = (q_latent[h] . c_i + q_rope[h] . k_i) * scale,  i in [0, k_len)
 *     out[h] = sum_i softmax(s)_i c_i           (fp32 accumulation)
 *     lse[h] = ln(sum_i exp(s_i))
 * q_latent [rows x H x kv_rank], q_rope [rows x H x rope_dim]: 16-bit of
 * `dtype` (the MPS graph keeps q_latent in the storage dtype,
 * mps_backend.mm:561).  out [rows x H x kv_rank] fp32, lse [rows x H] fp32
 * (may be NULL).  Rows of sessions with q_len != 1 are not written.
 * Work is split over the metadata's work items (split-K over pages); the
 * split partials of a session are merged with a log-sum-exp combine by a
 * second launch on the same stream (the pair is also exposed separately:
 * mla_decode_partials and mla_decode_merge, below).  With MLA_DECODE_FUSED_MERGE
 * and XCD-placed metadata (mla_build_metadata placement = 1) the MFMA page
 * kernel merges instead: the last item of a split session to finish combines
 * the session's partials through its XCD's L2, and the call is one launch.  The flag
 * needs B <= MLA_PLACE_MAX_SESSIONS and a device that passes
 * mla_xcd_placement_supported (MLA_ERR_INVALID_ARGUMENT otherwise).  Its premises are
 * checked, and a failed check never passes silently (mla_decode_status reports it):
 *   - metadata not placed for this device's XCD count (info[4]) is not merged: the kernel
 *     sets the rows of split sessions to NaN, leaves their partials for mla_decode_merge
 *     and raises MLA_DECODE_STATUS_UNPLACED in the workspace's status word;
 *   - items of one session that ran on several XCDs (a dispatch that broke the premise
 *     mla_xcd_placement_supported checked) cannot all count in one L2, so no item merges
 *     the session and its merge counter stays nonzero after the call: reported as
 *     MLA_DECODE_STATUS_XCD.  Rerun the call without the flag after clearing the
 *     workspace head (mla_decode_status with clear = 1).
 * `workspace` (device) must hold mla_decode_workspace_bytes(max_work, B, H, kv_rank)
 * bytes: a head block of MLA_DECODE_WORKSPACE_HEAD bytes (MLA_PLACE_MAX_SESSIONS int32
 * counters of the fused merge, then the status word at byte MLA_DECODE_STATUS_OFFSET;
 * zero the head before the workspace's first call; every call whose checks pass leaves
 * the counters zero), then the partials.  Calls that share a
 * workspace must be ordered on one stream.  The production kernel runs one wave per page of a work item,
 * so metadata built with split_pages == MLA_DECODE_SPLIT_PAGES keeps a whole
 * item in flight. */
#define MLA_DECODE_SPLIT_PAGES 4
#define MLA_DECODE_WORKSPACE_HEAD 1280
#define MLA_DECODE_STATUS_OFFSET 1024
#define MLA_DECODE_STATUS_XCD 1      /* a split session's items did not meet in one L2 */
#define MLA_DECODE_STATUS_UNPLACED 2 /* fused flag over metadata not placed for this device */
size_t mla_decode_workspace_bytes(int max_work, int max_sessions, int n_heads, int kv_rank);
/* Synchronises `stream` and returns in *status the decode status of `workspace` since it
 * was last cleared (0: every fused merge's premises held): the MLA_DECODE_STATUS_UNPLACED
 * bit the kernels raised, and MLA_DECODE_STATUS_XCD when a merge counter is nonzero.
 * clear = 1 also zeroes the workspace head (status and merge counters), stream-ordered.
 * workspace = NULL with workspace_bytes = 0 reads the current device's array of
 * mla_decode_attention_noalloc.  Not for use under stream capture.  No reference
 * counterpart; the reference turns backend failures into gpu_error
 * (mps_backend.mm:1050-1062). */
int mla_decode_status(void* stream, void* workspace, size_t workspace_bytes, int clear,
                      int32_t* status);
/* Test hook for the callers' recovery paths (the engine's rerun of a step): the next
 * `count` reads of a decode status -- mla_decode_status and the engine's check after each
 * placed step -- report MLA_DECODE_STATUS_XCD besides what the device left.  0 disarms. */
int mla_testing_fail_decode_status(int count);
/* The metadata arguments (cu_seqlens_q, page_table, num_splits, cu_splits,
 * work_desc, work_pages, info, max_work) are the outputs of one
 * mla_build_metadata call for this batch. */
int mla_decode_attention(void* stream, int B, int n_heads, int kv_rank, int rope_dim,
                         int page_size, int dtype, float scale, const int32_t* cu_seqlens_q,
                         const int32_t* page_table, int max_pages, int num_pool_pages,
                         const void* pages, const void* q_latent, const void* q_rope,
                         const int32_t* num_splits, const int32_t* cu_splits,
                         const int32_t* work_desc, const int32_t* work_pages, const int32_t* info,
                         int max_work, float* out, float* lse, void* workspace,
                         size_t workspace_bytes, int flags);

/* The two launches of mla_decode_attention, for callers that fold the merge into
 * their own next kernel or run it later on the stream.  mla_decode_partials
 * (same arguments) writes the final rows of sessions with one work item and
 * leaves the other sessions' partials in `workspace`; mla_decode_merge then
 * combines those partials into their rows of `out` (and `lse`).  Both must see
 * the same metadata and workspace, in this order on one stream.  With
 * MLA_DECODE_FUSED_MERGE, mla_decode_partials also writes the rows of split
 * sessions (when the MFMA page kernel runs; the partials stay in `workspace`, so a
 * following mla_decode_merge rewrites the same rows). */
int mla_decode_partials(void* stream, int B, int n_heads, int kv_rank, int rope_dim,
                        int page_size, int dtype, float scale, const int32_t* cu_seqlens_q,
                        const int32_t* page_table, int max_pages, int num_pool_pages,
                        const void* pages, const void* q_latent, const void* q_rope,
                        const int32_t* num_splits, const int32_t* cu_splits,
                        const int32_t* work_desc, const int32_t* work_pages, const int32_t* info,
                        int max_work, float* out, float* lse, void* workspace,
                        size_t workspace_bytes, int flags);
int mla_decode_merge(void* stream, int B, int n_heads, int kv_rank, const int32_t* cu_seqlens_q,
                     const int32_t* num_splits, const int32_t* cu_splits, const int32_t* info,
                     int max_work, float* out, float* lse, const void* workspace,
                     size_t workspace_bytes);

/* mla_decode_attention without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  The split partials go to a file-scope device array of
 * MLA_NOALLOC_SCRATCH_MIB MiB that each GPU the library runs on holds until the process
 * ends; the call allocates nothing.  Arguments, kernels and results are those of
 * mla_decode_attention.  MLA_ERR_INVALID_ARGUMENT when the partials would exceed the array
 * (mla_decode_workspace_bytes(max_work, B, n_heads, kv_rank) > mla_noalloc_scratch_bytes(),
 * e.g. above ~4,000 work items at H = 8, kv_rank = 128), or when `stream` belongs to a
 * device other than the calling thread's current one.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, other threads) race and must
 * be ordered by the caller. */
#define MLA_NOALLOC_SCRATCH_MIB 16
size_t mla_noalloc_scratch_bytes(void);
int mla_decode_attention_noalloc(void* stream, int B, int n_heads, int kv_rank, int rope_dim,
                                 int page_size, int dtype, float scale,
                                 const int32_t* cu_seqlens_q, const int32_t* page_table,
                                 int max_pages, int num_pool_pages, const void* pages,
                                 const void* q_latent, const void* q_rope,
                                 const int32_t* num_splits, const int32_t* cu_splits,
                                 const int32_t* work_desc, const int32_t* work_pages,
                                 const int32_t* info, int max_work, float* out, float* lse,
                                 int flags);

/* ------------------------------------------------------------------ (c)
 * Absorbed MLA chunked-prefill attention over the paged cache, for every session
 * with q_len > 1 in the batch.  Session b appended q_len tokens at positions
 * ctx .. ctx+q_len-1 (ctx = k_len - q_len, k_len = cu_seqlens_k[b+1] -
 * cu_seqlens_k[b]); its query row i attends causally to keys [0, ctx + i]:
 *     s_j = (q_latent[i,h] . c_j + q_rope[i,h] . k_j) * scale,  j <= ctx + i
 *     out[i,h] = sum_j softmax(s)_j c_j,   lse[i,h] = ln(sum_j exp(s_j))
 * i.e. the causal attention of the reference's full forward (src/model/ops.cpp:
 * 109-142, via Model::forward, src/model/model.cpp:76-155, which is what
 * CpuDecoder::prefill runs, src/infer/inference.cpp:47-68) in the absorbed form
 * of inference.cpp:116-153, restricted to rows ctx.. of the sequence: the
 * reference has no chunked prefill onto an existing context; causality
 * (tests/test_model.cpp:65-77) makes those rows equal.  The chunk's own latent
 * rows must already be appended (mla_append_latent with the metadata's
 * slot_mapping).  Arguments as for mla_decode_attention, plus cu_seqlens_k from
 * the same mla_build_metadata call and max_q_len >= every session's q_len (rows
 * of a longer session past max_q_len are not written).  Rows of sessions with
 * q_len <= 1 are not written (mla_decode_attention covers them).  flags:
 * MLA_DECODE_FORCE_GENERIC selects the portable VALU kernel.  No workspace. */
int mla_prefill_attention(void* stream, int B, int n_heads, int kv_rank, int rope_dim,
                          int page_size, int dtype, float scale, const int32_t* cu_seqlens_q,
                          const int32_t* cu_seqlens_k, const int32_t* page_table, int max_pages,
                          int num_pool_pages, const void* pages, const void* q_latent,
                          const void* q_rope, const int32_t* info, int max_q_len, float* out,
                          float* lse, int flags);

/* ------------------------------------------------------------------ model
 * The batched decode step around the attention: everything of
 * CpuDecoder::decode (src/infer/inference.cpp:76-173) for B sessions at once,
 * one new token each, on fp16 weights with fp32 accumulation.  The drop-in
 * counterpart of MpsExecution::decode / GraphBuilder::decode
 * (src/backends/mps_backend.mm:496-583,940-977), batched. */

/* The fields of mini_mla::ModelConfig (include/mini_mla/model_config.hpp:5-19). */
typedef struct {
    int vocab_size, max_sequence_length, n_layers, d_model, n_heads;
    int head_dim_nope, head_dim_rope, head_dim_value;
    int q_lora_rank, kv_lora_rank, d_ff;
    float norm_epsilon, rope_theta;
} mla_model_config;

/* ModelConfig::validate (src/model/config.cpp:20-48): MLA_OK or
 * MLA_ERR_INVALID_ARGUMENT with the reference's message. */
int mla_config_validate(const mla_model_config* config);
/* ModelConfig::parameter_count (src/model/config.cpp:7-19). */
size_t mla_config_parameter_count(const mla_model_config* config);

/* Uploads a model: `params` (host fp32) holds every parameter in the reference
 * registry order (include/mini_mla/model.hpp:15-30, src/model/model.cpp:40-63:
 * token_embedding, final_norm, then per layer attn_norm, w_dq, q_norm, w_uq,
 * w_dkv, kv_norm, w_uk, w_uv, w_o, ffn_norm, w_gate, w_up, w_down; row-major
 * [in x out]).  Weights are rounded to fp16 on the device (the MPS backend's
 * fp16 storage, mps_backend.mm:623-635); W_uv.W_o is combined per head first,
 * in fp32 (CpuDecoder::prepare_projections, inference.cpp:28-46).  The model
 * owns device activations for up to max_batch rows; page_size is the cache's.
 * The handle is used from one thread / stream at a time. */
int mla_model_create(const mla_model_config* config, const float* params, int max_batch,
                     int page_size, void** model);
int mla_model_destroy(void* model);
/* Model::mark_weights_changed (include/mini_mla/model.hpp) for an uploaded model: the
 * weights are replaced in place by `params` (same configuration, registry order; rounded
 * to fp16 and W_uv.W_o recombined, as at creation -- CpuDecoder::prepare_projections
 * recomputes per revision, inference.cpp:28-46).  Waits for the device first; not
 * stream-ordered, so no step may run concurrently.  *revision (may be NULL) receives the
 * new revision count (0 at creation).  On a failed copy the weights are undefined until
 * an update succeeds. */
int mla_model_update_weights(void* model, const float* params, uint64_t* revision);

/* One decode step for B sessions (B <= max_batch): tokens[b] (device int32, in
 * [0, vocab)) at position positions[b] (device int32: the tokens already cached,
 * in [0, max_sequence_length); the caller rejects others, as inference.cpp:71-75
 * does, and the kernels clamp them so no access leaves its buffer).
 * The metadata arguments come from one mla_build_metadata call with q_len = 1
 * and ctx_len = positions; pages is a HOST array of n_layers device page pools
 * (fp16, the mla_append_latent format); the step appends each token's latent
 * and key to them before attending (inference.cpp:100-103).  workspace is a
 * decode workspace (mla_decode_workspace_bytes).  Outputs: logits [B x vocab]
 * fp32 (device; NULL = the model's own buffer, see mla_model_logits) and
 * next_tokens[B] (device int32): the greedy token of sample_token with
 * temperature 0 and no penalty (inference.cpp:345-380: lowest index among the
 * maxima of the ids not banned, see mla_model_set_banned), -1 when a logit is not
 * finite (numerical_error), -2 when every id is banned.  flags: MLA_DECODE_FUSED_MERGE
 * when the metadata was built XCD-placed (the decode attention of each layer is then
 * one launch, see mla_decode_attention: check mla_decode_status on `workspace` after
 * the step, and rerun it without the flag if a bit is set -- the step's appends are
 * idempotent), else 0; optionally with MLA_STEP_NO_READ_AHEAD (no L2 read-ahead of the
 * attention's pages, same results). */
int mla_model_step(void* model, void* stream, int B, const int32_t* tokens,
                   const int32_t* positions, const int32_t* cu_seqlens_q,
                   const int32_t* page_table, int max_pages, int num_pool_pages,
                   const int32_t* slot_mapping, const int32_t* num_splits,
                   const int32_t* cu_splits, const int32_t* work_desc, const int32_t* work_pages,
                   const int32_t* info, int max_work, void* const* pages, void* workspace,
                   size_t workspace_bytes, float* logits, int32_t* next_tokens, int flags);
/* One forward of `rows` new tokens of B sessions in one batch (continuous batching with
 * chunked prefill): session b appends q_len = cu_seqlens_q[b+1] - cu_seqlens_q[b] >= 1
 * tokens (rows in session order; rows <= max_batch), token r at positions[r].  Per
 * layer: the projections and the paged append of every row, decode attention for the
 * q_len == 1 sessions (mla_decode_attention) and causal chunked-prefill attention for
 * the others (mla_prefill_attention), the FFN.  Then the final norm, tied logits and
 * greedy token of each session's LAST row, as the reference's prefill returns the
 * logits of the last prompt position (src/infer/inference.cpp:64-66): logits
 * [B x vocab], next_tokens [B].  max_q_len is the largest q_len (1 when rows == B).
 * The metadata arguments come from one mla_build_metadata call (ctx_len = tokens
 * already cached, q_len as above).  A prompt of n tokens prefilled in chunks through
 * successive calls gives the same rows as one call (causality, tests/test_model.cpp:
 * 65-77).  flags as for mla_model_step. */
int mla_model_forward(void* model, void* stream, int rows, const int32_t* tokens,
                      const int32_t* positions, int B, int max_q_len,
                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                      const int32_t* page_table, int max_pages, int num_pool_pages,
                      const int32_t* slot_mapping, const int32_t* num_splits,
                      const int32_t* cu_splits, const int32_t* work_desc,
                      const int32_t* work_pages, const int32_t* info, int max_work,
                      void* const* pages, void* workspace, size_t workspace_bytes, float* logits,
                      int32_t* next_tokens, int flags);
/* Token ids the greedy next token of later steps skips: sample_token's `banned`
 * (inference.cpp:345-380), which InferenceEngine::load fills with the special tokens
 * other than <|eos|> and the ids with no bytes (inference.cpp:441-447; see
 * mla_tokenizer_banned).  Ids >= vocab are ignored; n == 0 bans nothing.  A row whose
 * every id is banned gets next token -2 ("All tokens are banned"); a non-finite logit
 * still gives -1 first.  Not stream-ordered: call it between steps. */
int mla_model_set_banned(void* model, const uint16_t* ids, size_t n);
/* The model's own logits buffer [max_batch x vocab] (device). */
const float* mla_model_logits(void* model);

/* ------------------------------------------------------------------ sessions
 * The reference's per-session inference contract -- Execution::prefill, decode and
 * fork_inference (include/mini_mla/execution.hpp:34-37,56-58), implemented by
 * CpuDecoder (src/infer/inference.cpp:47-174) and MpsExecution
 * (src/backends/mps_backend.mm:872-977) -- for many sessions that share one uploaded
 * model and one paged latent cache, plus a batched step over them (continuous
 * batching with chunked prefill, modelled on the Gemma engine's session API
 * prefill_batch / decode(sessions, tokens) / release, include/mini_mla/gemma.hpp:16-20).
 * The engine owns its HIP stream, device buffers and pinned staging; logits are
 * returned in caller-owned HOST buffers (the reference returns a host span,
 * inference.cpp:67).  Calls on one engine are serialised by an internal mutex, so
 * sessions may be driven from different threads (the reference's fork-per-thread
 * use, tests/inference_sessions.hpp:191-217); concurrent sessions are served best
 * through mla_engine_step.  The weights can be replaced (mla_engine_update_weights): a
 * session whose cache predates the replacement is refused, as the reference's decode is
 * after mark_weights_changed (inference.cpp:71-75; mps_backend.mm:943-944), until it is
 * prefilled again. */

/* An engine for up to max_sessions sessions: model upload as mla_model_create,
 * num_pages pages of page_size tokens per layer (fp16, the mla_append_latent format),
 * at most max_rows new tokens per step (longer prompts are prefilled in chunks). */
int mla_engine_create(const mla_model_config* config, const float* params, int max_sessions,
                      int max_rows, int num_pages, int page_size, void** engine);
int mla_engine_destroy(void* engine);
/* info[8] = {active sessions, free pages, pages, page_size, max_rows, max_sessions,
 *            steps run, page-pool bytes}. */
int mla_engine_info(void* engine, int64_t* info);
/* The model configuration the engine was created with. */
int mla_engine_config(void* engine, mla_model_config* config);

/* A new, empty session sharing the engine's weights: Execution::fork_inference
 * (inference.cpp:182-188; mps_backend.mm:670-676 shares weights and programs, the
 * cache is private).  MLA_ERR_OUT_OF_MEMORY when every slot is in use. */
int mla_session_create(void* engine, int* session);
/* A new session holding `source`'s cached tokens: it shares source's pages (reference
 * counts) until either session appends into a shared page, which is then copied. */
int mla_session_fork(void* engine, int source, int* session);
/* Frees the session and its pages. */
int mla_session_release(void* engine, int session);
/* Tokens cached by the session (the reference's position_). */
int mla_session_length(void* engine, int session, int* length);
/* CpuDecoder::prefill (inference.cpp:47-68): restarts the session at position 0 and
 * runs the n prompt tokens (n in [1, max_sequence_length], else
 * MLA_ERR_INVALID_ARGUMENT "Prompt exceeds context or is empty"); logits (host
 * [vocab], may be NULL) receives the last position's logits. */
int mla_session_prefill(void* engine, int session, const uint16_t* ids, int n, float* logits);
/* CpuDecoder::decode (inference.cpp:69-174): appends `token` at the session's position
 * and returns the new logits.  MLA_ERR_INVALID_ARGUMENT unless 1 <= position <
 * max_sequence_length and token < vocab (inference.cpp:71-75); MLA_ERR_NUMERICAL when
 * a logit is not finite (inference.cpp:170-172; the token is appended). */
int mla_session_decode(void* engine, int session, uint16_t token, float* logits);
/* One batched step: sessions[i] (distinct) appends counts[i] >= 1 tokens taken in
 * order from `tokens` (a count > 1 is a chunked prefill on top of the session's
 * cached context; an empty session may start this way).  logits (host [n x vocab],
 * may be NULL) and next_tokens (host [n], may be NULL: the greedy token of
 * sample_token, inference.cpp:345-380, skipping the ids of mla_engine_set_banned) are
 * those of each session's last new token.  On an error no session advances, except
 * MLA_ERR_NUMERICAL (a non-finite logit) and "All tokens are banned", reported after
 * the step as the reference reports them after appending (inference.cpp:170-172). */
int mla_engine_step(void* engine, int n, const int* sessions, const int* counts,
                    const uint16_t* tokens, float* logits, int32_t* next_tokens);
/* mla_model_set_banned for the engine's model: the ids next_tokens of mla_engine_step
 * skip (MLA_ERR_INVALID_ARGUMENT "All tokens are banned" when none is left). */
int mla_engine_set_banned(void* engine, const uint16_t* ids, size_t n);
/* New weights for the engine's model (mla_model_update_weights) after the engine's stream
 * has drained.  From then on every session holding cached tokens is stale: its decode and
 * its rows in mla_engine_step fail with MLA_ERR_INVALID_ARGUMENT "Decode requires
 * current-weight prefill, available context, and a valid token" (CpuDecoder::decode,
 * inference.cpp:71-75; tests/test_training.cpp:111-122) until mla_session_prefill
 * restarts it.  Empty sessions and new prompts are unaffected. */
int mla_engine_update_weights(void* engine, const float* params);
/* Execution::stats (include/mini_mla/execution.hpp:25-27,33), engine-wide counters since
 * creation: stats[6] = {model forwards submitted (graph_submissions), host waits on the
 * engine's stream (host_waits), kernels launched (metal_kernel_submissions), copies
 * issued, weight revision, steps rerun through the two-launch decode because a fused
 * merge's check failed (after the first such step the engine stops placing work)}. */
int mla_engine_stats(void* engine, uint64_t* stats);
/* Execution::forward(ids, batch, sequence) (execution.hpp:38-39) for inference: the
 * logits of EVERY position of `batch` independent sequences of `sequence` tokens (ids
 * row-major [batch x sequence]), as Model::forward returns them (src/model/model.cpp:
 * 76-155): logits (host) [batch*sequence x vocab].  Runs through temporary sessions of
 * the engine (whole sequences batched up to max_rows rows per step, longer ones in
 * causal chunks), which are released afterwards; needs their cache pages and free session
 * slots (else MLA_ERR_OUT_OF_MEMORY).  MLA_ERR_INVALID_ARGUMENT for an empty batch, a
 * sequence beyond max_sequence_length or a token past the vocabulary; MLA_ERR_NUMERICAL
 * when a logit is not finite. */
int mla_engine_forward(void* engine, int batch, int sequence, const uint16_t* ids,
                       float* logits);

/* ------------------------------------------------------------ model exports
 * The reference's inference-side weight load, load_checkpoint(path, training =
 * false) (src/train/checkpoint.cpp:186-324; format: docs/file_formats.md,
 * "Checkpoint directory"): a mini-mla-model export or mini-mla-checkpoint
 * directory is checked in the reference's order with its codes and messages --
 * COMPLETE against the manifest's SHA-256 (MLA_ERR_IO), format and version
 * (MLA_ERR_UNSUPPORTED), config.json (ModelConfig::from_json, config.cpp:74-107)
 * against model_config_sha256 and parameter_count (MLA_ERR_INVALID_ARGUMENT
 * "Checkpoint model configuration mismatch"), tokenizer.json (Tokenizer::load's
 * checks, tokenizer.cpp:70-127) against tokenizer_sha256 and the vocabulary,
 * every listed file's SHA-256, then each tensor entry's file, uniqueness,
 * contiguous extent, CRC-32, name, role, shape and dtype (f32 or f16), and finite
 * values (all MLA_ERR_IO with the reference's message).  Training state in a
 * checkpoint (optimizer.bin) is checked and skipped. */

/* ModelConfig::load of <dir>/config.json, so a caller can size the parameters. */
int mla_export_read_config(const char* dir, mla_model_config* config);
/* The checks above; on success *config is the export's architecture and, when params
 * is not NULL, params[params_count] (params_count = mla_config_parameter_count)
 * receives every parameter as fp32 in registry order (f16 tensors widened exactly). */
int mla_export_read(const char* dir, mla_model_config* config, float* params,
                    size_t params_count);
/* ModelConfig::hash (config.cpp:71-73): SHA-256 of the architecture's canonical JSON,
 * 64 hex digits and a terminating NUL into hex_out[65]. */
int mla_config_hash(const mla_model_config* config, char* hex_out);
/* mla_export_read, then mla_model_create / mla_engine_create with the export's weights;
 * *config receives the architecture. */
int mla_model_load(const char* dir, int max_batch, int page_size, mla_model_config* config,
                   void** model);
int mla_engine_load(const char* dir, int max_sessions, int max_rows, int num_pages,
                    int page_size, mla_model_config* config, void** engine);

/* ---------------------------------------------------------------- tokenizer
 * The reference's byte-level BPE tokenizer (src/infer/tokenizer.cpp; format:
 * docs/file_formats.md, "Tokenizer"), host code.  Generation prompts are
 * <|bos|> + encode(text) (inference.cpp:461-468). */

/* Tokenizer::load (tokenizer.cpp:70-127) with its checks, codes and messages. */
int mla_tokenizer_load(const char* path, void** tokenizer);
int mla_tokenizer_destroy(void* tokenizer);
/* Vocabulary size and the SHA-256 of the file bytes (hex, into sha256_hex[65]). */
int mla_tokenizer_info(void* tokenizer, int* vocab_size, char* sha256_hex);
/* Tokenizer::special: the id of "<|bos|>", "<|eos|>", ... */
int mla_tokenizer_special(void* tokenizer, const char* name, uint16_t* id);
/* Tokenizer::encode (tokenizer.cpp:128-205): ranked merges applied lowest id first,
 * leftmost first on ties; with allow_special, special-token spellings become their ids.
 * *n_ids receives the count; ids == NULL only queries it, and a capacity below the
 * count is MLA_ERR_INVALID_ARGUMENT. */
int mla_tokenizer_encode(void* tokenizer, const char* text, size_t len, int allow_special,
                         uint16_t* ids, size_t capacity, size_t* n_ids);
/* Tokenizer::decode (tokenizer.cpp:206-215): the tokens' bytes, optionally without the
 * special tokens; an id past the vocabulary or without bytes is
 * MLA_ERR_INVALID_ARGUMENT "Unknown token ID".  Sizing as for encode. */
int mla_tokenizer_decode(void* tokenizer, const uint16_t* ids, size_t n, int skip_special,
                         char* text, size_t capacity, size_t* len);

/* --------------------------------------------------------------- generation
 * Token selection and the generation loop of InferenceEngine (src/infer/inference.cpp:
 * 330-579), host code: GenerationConfig, sample_token, the banned ids of
 * InferenceEngine::load and generate_tokens' loop (stop rules, streaming, cancel). */

/* GenerationConfig (include/mini_mla/inference.hpp:27-34).  Stop strings are stop[i]
 * of stop_len[i] bytes; stop token sequences are stop_tokens_len[i] ids each, one after
 * the other in stop_tokens. */
typedef struct mla_generation_config {
    int max_new_tokens;       /* [0, 65535]; default 128 */
    int top_k;                /* 0 = all ids; default 0 */
    float temperature;        /* 0 = greedy; default 0.8 */
    float top_p;              /* (0, 1]; default 0.95 */
    float repetition_penalty; /* > 0; default 1 */
    uint64_t seed;            /* sampling stream (SplitMix64); default 42 */
    int n_stop;
    const char* const* stop;
    const size_t* stop_len;
    int n_stop_tokens;
    const int* stop_tokens_len;
    const uint16_t* stop_tokens;
} mla_generation_config;
/* The reference's defaults, no stop lists. */
void mla_generation_config_init(mla_generation_config* config);
/* GenerationConfig::validate (inference.cpp:330-344) with its messages. */
int mla_generation_config_validate(const mla_generation_config* config);
/* sample_token (inference.cpp:345-412): greedy (temperature 0: lowest id among the
 * maxima, repetition penalty on the history's ids) or seeded sampling (penalty, bans,
 * top_k, top_p, temperature; *rng_state is the Rng state, advanced by the draw).
 * MLA_ERR_NUMERICAL "Invalid sampler logits" on a non-finite logit or vocab outside
 * [1, 65535]; MLA_ERR_INVALID_ARGUMENT "All tokens are banned". */
int mla_sample_token(const float* logits, size_t vocab, const uint16_t* history,
                     size_t n_history, const mla_generation_config* config, uint64_t* rng_state,
                     const uint16_t* banned, size_t n_banned, uint16_t* token);
/* The ids InferenceEngine::load bans from sampling (inference.cpp:441-447): the special
 * tokens other than <|eos|> and the ids with no bytes.  Sizing as for encode. */
int mla_tokenizer_banned(void* tokenizer, uint16_t* ids, size_t capacity, size_t* n);

/* Streamed text (UTF-8, cleaned); len 0 asks whether to go on.  Return 0 to cancel. */
typedef int (*mla_text_callback)(void* user, const char* text, size_t len);
/* generate_tokens (inference.cpp:469-579) as a state machine: create() checks the
 * config, prompt + max_new_tokens <= max_sequence_length and the stop tokens, with the
 * tokenizer's banned ids.  The caller prefills the prompt and passes the last
 * position's logits to step(), which sets *next_token to the token to decode and pass
 * back next, or -1 when the generation has finished (then result() holds the text,
 * tokens and finish reason "stop", "length" or "cancelled"; finish_reason[16]). */
int mla_generation_create(void* tokenizer, const mla_generation_config* config,
                          const uint16_t* prompt, size_t n, int max_sequence_length,
                          mla_text_callback callback, void* user, void** generation);
int mla_generation_step(void* generation, const float* logits, size_t vocab,
                        int32_t* next_token);
int mla_generation_finished(void* generation);
int mla_generation_result(void* generation, char* text, size_t text_capacity, size_t* text_len,
                          uint16_t* tokens, size_t tokens_capacity, size_t* n_tokens,
                          char* finish_reason);
int mla_generation_destroy(void* generation);

/* ---------------------------------------------------------------- scheduler
 * Continuous batching for a server: the reference's mini_mla_serve gives each of its
 * `workers` threads a private forked session and runs one request at a time on each
 * (src/serve/server.cpp:195-198, 254-266).  Here one stepping thread serves every
 * request through mla_engine_step: each step carries one decode row per running
 * request and prompt chunks of newly admitted ones, up to the engine's max_rows.  Kept
 * from the reference: the bounded queue (MLA_ERR_UNAVAILABLE "Request queue is full",
 * its 429), the per-request deadline counted from submission (not yet started:
 * "Request queue deadline exceeded", its 503; running: finish reason "cancelled", its
 * 408), cancellation, the request limits and the /metrics counters and text
 * (server.cpp:221-227, 272-300, 320-337).  A request is admitted when a session slot
 * and enough cache pages for prompt + max_new_tokens are free, so a running request
 * never runs out of pages.  The HTTP layer itself stays with the caller. */
#define MLA_ERR_UNAVAILABLE 7 /* no ErrorCode counterpart: queue full or deadline passed */

/* ServerConfig's limits (include/mini_mla/server.hpp:5-10). */
typedef struct mla_scheduler_config {
    int max_context;             /* <= the model's max_sequence_length; default 2048 */
    int max_new_tokens;          /* per request (also the default); default 128 */
    int max_queue;               /* requests waiting to start; default 16 */
    int request_timeout_seconds; /* from submission to the end; default 60 */
} mla_scheduler_config;
typedef struct mla_request_status {
    int done;                  /* 1: finished; this poll retired the request */
    int error;                 /* MLA_OK, or the code that ended the request */
    char error_message[240];
    char finish_reason[16];    /* "stop", "length" or "cancelled" */
    uint64_t prompt_tokens, completion_tokens;
    double queue_seconds, prefill_seconds, decode_seconds, first_token_seconds;
} mla_request_status;
typedef struct mla_scheduler_metrics {
    uint64_t requests, completed, rejected, errors, generated_tokens;
    double queue_seconds, prefill_seconds, decode_seconds, first_token_seconds;
    uint64_t queue_depth, running, steps;
} mla_scheduler_metrics;

void mla_scheduler_config_init(mla_scheduler_config* config);
/* Starts the stepping thread.  The engine's banned ids become the tokenizer's
 * (mla_engine_set_banned).  Engine and tokenizer must outlive the scheduler. */
int mla_scheduler_create(void* engine, void* tokenizer, const mla_scheduler_config* config,
                         void** scheduler);
/* Cancels what is queued or running and joins the stepping thread; idempotent.  Polls
 * waiting on other threads wake up; later polls still hand out the (cancelled) results,
 * later submits fail with MLA_ERR_UNAVAILABLE "Scheduler is stopping". */
int mla_scheduler_stop(void* scheduler);
/* mla_scheduler_stop, then waits until every call already inside the scheduler on other
 * threads has returned, then frees it.  Calls that START after destroy are the caller's
 * error (the handle is gone): a host shares the handle with a reference count or a lock,
 * as the Python binding does. */
int mla_scheduler_destroy(void* scheduler);
/* Queues a generation of prompt (token ids, <|bos|> included).  config NULL or
 * max_new_tokens < 0: the server default min(max_new_tokens, max_context - n)
 * (server.cpp:300-304).  Checks in the reference's order: queue full
 * (MLA_ERR_UNAVAILABLE, counted as rejected), generation settings, the request limits
 * ("Request exceeds context or token limit"), empty prompt, stop tokens.  stream != 0
 * hands out text as it is produced; otherwise the whole text comes at the end. */
int mla_scheduler_submit(void* scheduler, const uint16_t* prompt, size_t n,
                         const mla_generation_config* config, int stream, uint64_t* request);
/* Ends the request at its next token ("cancelled"); a queued one never starts. */
int mla_scheduler_cancel(void* scheduler, uint64_t request);
/* Waits up to timeout_ms for new text or the end, moves up to text_capacity bytes of
 * the text not yet handed out into text (*text_len), and fills status.  Once done and
 * all text is out, tokens (capacity >= completion_tokens, may be NULL) receives the
 * generated ids, status->done is 1 and the request is forgotten. */
int mla_scheduler_poll(void* scheduler, uint64_t request, int timeout_ms, char* text,
                       size_t text_capacity, size_t* text_len, uint16_t* tokens,
                       size_t tokens_capacity, mla_request_status* status);
int mla_scheduler_metrics_get(void* scheduler, mla_scheduler_metrics* metrics);
/* The /metrics page of server.cpp:272-289 (Prometheus text); sizing as for encode. */
int mla_scheduler_metrics_text(void* scheduler, char* text, size_t capacity, size_t* len);

#ifdef __cplusplus
}
#endif
#endif
