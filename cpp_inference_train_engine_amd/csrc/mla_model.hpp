// Device layout and launchers of the batched decode step (model.hip, model_capi.hip).
//
// Weight tiling.  A projection y = x.W with W [K x N] (the reference's [in x out],
// ops.cpp:8-18) is stored as fp16 in MFMA B-operand order: K padded to a multiple of
// 32, N to a multiple of 16 (padding is zero), and element (k, col) at
//     ((nt * KT + kt) * 4 + g) * 128 + n * 8 + e
// with nt = col/16, n = col%16, kt = k/32, g = (k%32)/8, e = k%8, KT = Kpad/32.  The
// 64 lanes of a wave loading tile (nt, kt) read 1 KB contiguously (lane l: 16 bytes at
// (nt*KT + kt)*512 + 8l).
#pragma once

#include <hip/hip_runtime.h>

#include "mla_hip.h"

#include <cstddef>
#include <cstdint>

namespace mla {

struct ModelDims {
    int vocab, d_model, H, nope, rope, dv, q_rank, kv_rank, d_ff, n_layers;
    int qk;                    // nope + rope
    float eps, theta;
    int page_size;
    int max_seq;   // max_sequence_length: RoPE table rows
    // padded sizes (K dimensions to 32, N dimensions to 16; see above)
    int d_pad;      // d_model -> 32
    int q_pad;      // q_rank -> 32 (N of w_dq, K of w_uq)
    int kvw_pad;    // kv_rank + rope -> 16 (N of w_dkv)
    int qk_pad;     // qk -> 16 (per-head N of w_uq)
    int nope_pad;   // nope -> 32 (K of the absorption)
    int kv_pad;     // kv_rank -> 16 (N of the absorption)
    int ctx_pad;    // H * kv_rank -> 32 (K of the output projection)
    int ff_pad;     // d_ff -> 32 (N of gate/up, K of down)
    int vocab_pad;  // vocab -> 16 (N of the tied logits)
};

struct LayerWeights {
    const float *attn_norm, *q_norm, *kv_norm, *ffn_norm;
    const uint16_t* w_dq_dkv;   // [d x (q_pad + kvw_pad)] tiled: q columns, then kv columns
    const uint16_t* w_uq;       // [q_rank x H*qk_pad] tiled, head h at columns h*qk_pad..
    const uint16_t* w_uk;       // H blocks [nope x kv_rank] tiled (W_uk_h^T)
    const uint16_t* w_out;      // [H*kv_rank x d] tiled: combined W_uv.W_o
    const uint16_t* w_gate_up;  // [d x 2*ff_pad] tiled, gate/up tiles interleaved
    const uint16_t* w_down;     // [d_ff x d] tiled
};

struct StepArgs {
    ModelDims dims;
    int B, m_pad;              // rows, rows padded to 64
    const int32_t* tokens;     // [B]
    const int32_t* positions;  // [B] position of each new token (= cached tokens)
    const int32_t* slot_mapping;
    int num_pool_pages;
    const uint16_t* embed;     // token_embedding [V x d] tiled as the logits W (K=d, N=V)
    const float* final_norm;
    const float2* rope_tab;    // [max_seq x rope/2] (cos, sin) of pos * theta^(-j/rope)
    float2* rope_rows;         // [m_pad x rope/2] the table rows of this step's positions
    // activations (rows padded to m_pad)
    float *x, *res, *ctx;       // [m_pad x d_pad], [m_pad x d_pad], [m_pad x H*kv_rank]
    uint16_t *xw, *resw;        // fp16 x o (next norm weight), res o ffn_norm [m_pad x d_pad]
    uint16_t *u;                // [m_pad x ff_pad] fp16
    uint16_t *q_latent, *q_rope;  // [B x H x kv_rank], [B x H x rope] in the cache dtype
    float* logits;              // [B x vocab]
    float* arg_v;               // [B x parts] greedy partials
    int32_t* arg_c;
    const uint32_t* ban;        // bitmap of token ids the greedy token skips, or null
    int32_t* next_tokens;       // [B]
    // Per-row sums of squares of each 16-column tile of an activation, written by its
    // producer and summed (in tile order) into 1/rms by the RMSNorm-ing consumer.
    float* ss_x;    // [m_pad x d_pad/16] of x (embed, g6) -> attn_norm (qkv), final_norm (g7)
    float* ss_res;  // [m_pad x d_pad/16] of res (g4) -> ffn_norm (g5)
};

// The decode attention's pages, read ahead into L2 by extra workgroups of the qkv launch
// that precedes it on the stream (page_prefetch, model.hip).  max_work = 0: none.
struct PagePrefetch {
    const int32_t *work_desc, *work_pages;  // the attention's work list
    int max_work;   // work items (the attention's grid), 0 = no read-ahead
    int pages;      // leading pages of each work item read ahead, <= kWorkPages
    int page_size;  // tokens per page
    int record;     // 16-bit words per page record
};

int g7_parts(const ModelDims& m);
size_t qkv_lds_bytes(const ModelDims& m);
hipError_t model_kernel_attributes(const ModelDims& m);
// first_norm: attn_norm of layer 0
hipError_t launch_embed(const StepArgs& s, const float* first_norm, hipStream_t st);
hipError_t launch_layer_pre(const StepArgs& s, const LayerWeights& w, uint16_t* pool,
                            const PagePrefetch& pf, hipStream_t st);  // qkv_kernel (which appends to `pool`)
// next_norm: attn_norm of the next layer, or final_norm after the last one; next: the
// next layer's weights (their qkv blocks are prefetched into L2), or null
hipError_t launch_layer_post(const StepArgs& s, const LayerWeights& w, const float* next_norm,
                             const LayerWeights* next, hipStream_t st);
hipError_t launch_logits(const StepArgs& s, hipStream_t st);
// Row b < B of (xw_out, ss_out) = row cu_q[b+1]-1 of (s.xw, s.ss_x) for the B sessions
// of cu_q; rows [B, round_up(B, 64)) are zeroed.  s describes the forward's rows.
hipError_t launch_gather_last(const StepArgs& s, int B, const int32_t* cu_q, uint16_t* xw_out,
                              float* ss_out, hipStream_t st);

// Device metadata of one mla_build_metadata call.
struct MetaPtrs {
    const int32_t *cu_seqlens_q, *cu_seqlens_k, *page_table, *slot_mapping, *num_splits,
        *cu_splits, *work_desc, *work_pages, *info;
    int max_pages, num_pool_pages, max_work;
    int flags = 0;  // MLA_DECODE_FUSED_MERGE when the metadata was built XCD-placed
};
struct Model;  // model_capi.hip
// One forward of `rows` new tokens belonging to B sessions (row order = session order,
// q_len = cu_q[b+1] - cu_q[b] >= 1, max_q_len the largest): per layer the projections,
// the paged append, decode attention for q_len == 1 sessions and chunked-prefill
// attention for the others, the FFN; then logits and the greedy token of each
// session's LAST row into logits [B x vocab] / next_tokens [B].  When every session
// has q_len == 1 (rows == B) the rows are the sessions.  all_rows: logits and greedy
// token of EVERY row instead (logits [rows x vocab], next_tokens [rows]), as a full
// forward returns them.  Returns an MLA status.
int model_forward(Model* M, hipStream_t st, int rows, const int32_t* tokens,
                  const int32_t* positions, int B, int max_q_len, const MetaPtrs& md,
                  void* const* pages, void* workspace, size_t workspace_bytes, float* logits,
                  int32_t* next_tokens, bool all_rows = false);
int model_max_rows(const Model* M);
// Kernels model_forward has launched since the model was created.
uint64_t model_launches(const Model* M);
const mla_model_config& model_config(const Model* M);

}  // namespace mla
