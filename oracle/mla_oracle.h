/*
 * mla_oracle.h -- CPU restatement of the reference's MLA decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product (libmla_hip.so).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  Nothing in the product links it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference checkout Astrowebdeving/cpp_inference_train_engine).  The
 * arithmetic is plain fp32 C, single thread, sequential sums: the "portable
 * CBLAS" substitution for Apple Accelerate (cblas_sgemm / cblas_sgemv in
 * src/model/ops.cpp:15-17 and src/infer/inference.cpp:38-43,122-152) is the
 * bundled naive loops below.  Only summation order differs from Accelerate.
 *
 * Pinning (see tests/test_oracle_*.py):
 *   rng            -> oracle/_ref build of include/mini_mla/rng.hpp (known answers)
 *   config/count   -> tests/test_model.cpp:21-28 known answers (35,763,840 / 26,704)
 *   forward        -> docs/verification/attention-sync/oracle fixture logits
 *   decode         -> decode == forward invariant (tests/test_training.cpp:52-76),
 *                     absorbed == non-absorbed, brute force fp64 on tiny inputs
 *   fp16 / bf16    -> exhaustive comparison with numpy RNE casts
 *   metadata       -> independent pure-Python builder + invariants
 */
#ifndef MLA_ORACLE_H
#define MLA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int vocab_size, max_sequence_length, n_layers, d_model, n_heads;
    int head_dim_nope, head_dim_rope, head_dim_value;
    int q_lora_rank, kv_lora_rank, d_ff;
    float norm_epsilon, rope_theta;
} orc_config;

/* ---- Rng: include/mini_mla/rng.hpp:7-38 ---- */
uint64_t orc_rng_next(uint64_t* state);
float orc_rng_uniform(uint64_t* state);
uint64_t orc_rng_bounded(uint64_t* state, uint64_t bound);
float orc_rng_normal(uint64_t* state);
void orc_rng_fill_normal(uint64_t* state, float* out, size_t n);
void orc_rng_fill_bounded(uint64_t* state, uint64_t bound, int32_t* out, size_t n);

/* ---- fp16 / bf16 rounding: src/core/io.cpp:152-158 (to_half = RNE cast) ---- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_round_f16(const float* in, uint16_t* out, size_t n);
void orc_round_bf16(const float* in, uint16_t* out, size_t n);

/* ---- ModelConfig: src/model/config.cpp:7-48 ---- */
size_t orc_parameter_count(const orc_config* c);
int orc_validate(const orc_config* c); /* 0 ok, 1 invalid_argument */
/* Parameter registry (include/mini_mla/model.hpp:15-30, src/model/model.cpp:40-63):
 * writes rows/cols of the 2 + 13*L tensors; returns the count. */
int orc_parameter_shapes(const orc_config* c, int* rows, int* cols);
/* Model::create init (src/model/model.cpp:20-75) into one flat fp32 array. */
int orc_model_init(const orc_config* c, uint64_t seed, float* params);

/* ---- Model::forward (src/model/model.cpp:76-155), batch 1 ----
 * logits [T x V]; ckv/krope optional [L x T x kv_rank] / [L x T x rope]. */
int orc_forward(const orc_config* c, const float* params, const uint16_t* tokens, int T,
                float* logits, float* ckv, float* krope);

/* ---- CpuDecoder::prepare_projections (src/infer/inference.cpp:28-46) ----
 * out [L x (H*kv_rank) x d_model]. */
void orc_output_projection(const orc_config* c, const float* params, float* out);

/* ---- CpuDecoder::decode (src/infer/inference.cpp:69-174) over a contiguous
 * fp32 cache latent [L x max_seq x kv_rank], rope [L x max_seq x rope].
 * `position` is the number of tokens already cached.  If round_cache != 0 the
 * appended latent/key are rounded through fp16 (mirrors fp16 storage).
 * absorbed selects the absorbed or the reconstructed-K/V attention
 * (inference.cpp:104-153).  Returns 0 ok, 1 invalid_argument, 5 numerical_error. */
int orc_decode(const orc_config* c, const float* params, const float* out_proj, float* latent,
               float* rope, int position, uint16_t token, int absorbed, int round_cache,
               float* logits);

/* Threads used by orc_attention_paged (default 1; sessions run in parallel). */
void orc_set_threads(int n);
/* A 64-bit-index CBLAS sgemm / sgemv (both, or both NULL) for the products of
 * orc_forward / orc_decode, in place of the plain loops: the portable CBLAS standing in
 * for Accelerate when the CPU baseline is timed.  Not thread-safe against running
 * calls; set it before starting any. */
void orc_set_blas(void* sgemm, void* sgemv);

/* ---- Absorbed MLA attention over a paged cache (inference.cpp:116-153, fp32).
 * Page record layout (one per page, per layer): latent section
 * (page_size x kv_rank) then rope section (page_size x rope_dim), 16-bit
 * elements (dtype 0 = fp16, 1 = bf16); tiled in MFMA-operand order when
 * page_size % 16 == 0, kv_rank % 32 == 0 and rope_dim % 8 == 0, else row-major
 * (the format of include/mla_hip.h).
 * Queries are ragged: session b owns rows cu_q[b]..cu_q[b+1]; row i of session b
 * sits at absolute position k_len[b] - q_len[b] + i and attends causally to
 * positions [0, that position].  q_latent [rows x H x kv_rank], q_rope
 * [rows x H x rope] fp32.  out [rows x H x kv_rank] fp32, lse [rows x H]
 * (natural log of the softmax denominator plus the max, may be NULL). */
int orc_attention_paged(int B, int H, int kv_rank, int rope_dim, int page_size, int dtype,
                        const int32_t* cu_q, const int32_t* k_len, const int32_t* page_table,
                        int max_pages, const uint16_t* pages, const float* q_latent,
                        const float* q_rope, float scale, float* out, float* lse);

/* ---- Ragged batch metadata (new; no reference function).  Integer, bit-exact.
 * Inputs: ctx_len[B] tokens already cached, q_len[B] new tokens, cu_pages[B+1]
 * and page_ids[] (per-session physical page lists), page_size, max_pages
 * (columns of the padded table), num_pool_pages, split_pages (>0 fixed, 0 auto
 * with target_blocks).
 * Outputs (caller-sized): cu_seqlens_q[B+1], cu_seqlens_k[B+1],
 * page_table[B x max_pages] (-1 padded), slot_mapping[total_q],
 * num_splits[B], cu_splits[B+1], work_session[W], work_split[W],
 * work_desc[max_work x 8] = {session, first query row, k_len, page_begin,
 * page_end, num_splits, partial slot cu_splits[session] + split, q_len} (session -1
 * for every empty slot and for every item of a failed build), work_pages[max_work x 8] =
 * first 8 page ids of each item (-1 past its end), info[8] =
 * {W, split_pages, total_q, total_k, placement_xcds, 0, 0, 0} or
 * {-1, first offending session, 0, ...}.
 * placement_xcds = n > 0 lays the work list out over n XCDs (each session's items
 * in slots x, x + n, ..; {-1, B, 0, ...} when max_work cannot hold it); 0 keeps
 * session order (item w = cu_splits[session] + split).
 * Returns 0, or 1 (invalid argument). */
int orc_build_metadata(int B, const int32_t* ctx_len, const int32_t* q_len,
                       const int32_t* cu_pages, const int32_t* page_ids, int page_size,
                       int max_pages, int num_pool_pages, int split_pages, int target_blocks,
                       int max_work, int max_rows, int placement_xcds, int32_t* cu_seqlens_q,
                       int32_t* cu_seqlens_k, int32_t* page_table, int32_t* slot_mapping,
                       int32_t* num_splits, int32_t* cu_splits, int32_t* work_session,
                       int32_t* work_split, int32_t* work_desc, int32_t* work_pages,
                       int32_t* info);

/* ---- Paged append (refines inference.cpp:100-103): row t of ckv/krope (fp32)
 * is rounded to 16-bit and written to slot slot_mapping[t] of the pool. */
void orc_append_paged(int T, int kv_rank, int rope_dim, int page_size, int dtype,
                      const float* ckv, const float* krope, const int32_t* slot_mapping,
                      uint16_t* pages);

/* ---- sample_token greedy branch (src/infer/inference.cpp:345-380) ----
 * Returns token id, or -1 when every id is banned. */
int orc_greedy(const float* logits, int n, const uint16_t* history, int n_history,
               float repetition_penalty, const uint16_t* banned, int n_banned);

#ifdef __cplusplus
}
#endif
#endif
