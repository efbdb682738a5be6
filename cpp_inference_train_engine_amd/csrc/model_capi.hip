// C ABI of the batched decode step (include/mla_hip.h, "model" section): model
// config validation, weight upload (fp16, tiled; see mla_model.hpp) and the step
// driver that chains the model kernels (model.hip) with the paged decode attention
// (decode.hip).
#include "mla_capi_util.hpp"
#include "mla_hip.h"
#include "mla_internal.hpp"
#include "mla_model.hpp"

#include <cmath>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace mla {
namespace {

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Leading pages of each decode work item that qkv_kernel reads ahead into L2 (page_prefetch).
// Config 3 (570 items of 4 pages): 1 page took the step from 0.3854 to 0.3816 ms; 2 and 3
// pages (20 and 30 MB) outlast qkv_kernel (14.8 and 20 us) and slowed the step.
constexpr int kReadAheadPages = 1;

// ModelConfig::validate (src/model/config.cpp:20-48) and parameter_count (:7-19).
size_t parameter_count(const mla_model_config& c) {
    const size_t d = c.d_model, h = c.n_heads, q = c.q_lora_rank, kv = c.kv_lora_rank;
    const size_t qk = (size_t)c.head_dim_nope + c.head_dim_rope;
    const size_t kvw = kv + c.head_dim_rope;
    return (size_t)c.vocab_size * d + d +
           (size_t)c.n_layers * (d * q + q * h * qk + d * kvw +
                                 kv * h * ((size_t)c.head_dim_nope + c.head_dim_value) +
                                 h * (size_t)c.head_dim_value * d + 3 * d * (size_t)c.d_ff +
                                 2 * d + q + kv);
}

int validate(const mla_model_config* c) {
    if (!c)
        return fail(MLA_ERR_INVALID_ARGUMENT, "model config: null");
    const std::pair<const char*, int> fields[] = {
        {"vocab_size", c->vocab_size},       {"max_sequence_length", c->max_sequence_length},
        {"n_layers", c->n_layers},           {"d_model", c->d_model},
        {"n_heads", c->n_heads},             {"head_dim_nope", c->head_dim_nope},
        {"head_dim_rope", c->head_dim_rope}, {"head_dim_value", c->head_dim_value},
        {"q_lora_rank", c->q_lora_rank},     {"kv_lora_rank", c->kv_lora_rank},
        {"d_ff", c->d_ff}};
    for (const auto& [name, v] : fields)
        if (v < 1 || v > 65535)
            return fail(MLA_ERR_INVALID_ARGUMENT, std::string(name) + " must be in [1, 65535]");
    if (c->vocab_size > 65535 || c->n_layers > 128 || c->n_heads > 256 ||
        c->d_model % c->n_heads || c->head_dim_rope % 2)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "Invalid vocabulary/layer/head count, d_model divisibility, or odd RoPE "
                    "dimension");
    if (!std::isfinite(c->norm_epsilon) || c->norm_epsilon <= 0 || !std::isfinite(c->rope_theta) ||
        c->rope_theta <= 1)
        return fail(MLA_ERR_INVALID_ARGUMENT, "Invalid normalization epsilon or RoPE theta");
    if (parameter_count(*c) > 1000000000ULL)
        return fail(MLA_ERR_INVALID_ARGUMENT, "Configuration exceeds one billion parameters");
    return MLA_OK;
}

uint16_t to_f16(float x) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x)); }

// Packs W [K x N] (element (k, col) from `at`) into the tiled fp16 layout.
template <typename F>
std::vector<uint16_t> pack(int K, int N, int Kpad, int Npad, F at) {
    const int KT = Kpad / 32, NT = Npad / 16;
    std::vector<uint16_t> out((size_t)NT * KT * 512, 0);
    for (int nt = 0; nt < NT; ++nt)
        for (int kt = 0; kt < KT; ++kt) {
            uint16_t* t = out.data() + ((size_t)nt * KT + kt) * 512;
            for (int g = 0; g < 4; ++g)
                for (int n = 0; n < 16; ++n)
                    for (int e = 0; e < 8; ++e) {
                        const int k = kt * 32 + g * 8 + e, col = nt * 16 + n;
                        if (k < K && col < N)
                            t[(g * 16 + n) * 8 + e] = to_f16(at(k, col));
                    }
        }
    return out;
}

// Offsets of the reference parameter registry (include/mini_mla/model.hpp:15-30,
// src/model/model.cpp:40-63): token_embedding, final_norm, then per layer attn_norm,
// w_dq, q_norm, w_uq, w_dkv, kv_norm, w_uk, w_uv, w_o, ffn_norm, w_gate, w_up, w_down.
enum { P_ATTN_NORM, P_W_DQ, P_Q_NORM, P_W_UQ, P_W_DKV, P_KV_NORM, P_W_UK, P_W_UV, P_W_O,
       P_FFN_NORM, P_W_GATE, P_W_UP, P_W_DOWN, P_COUNT };

struct Registry {
    const float* embed;
    const float* final_norm;
    std::vector<const float*> layer;  // [L * P_COUNT]
};

Registry view(const mla_model_config& c, const float* p) {
    const size_t d = c.d_model, q = c.q_lora_rank, kv = c.kv_lora_rank, H = c.n_heads;
    const size_t qk = (size_t)c.head_dim_nope + c.head_dim_rope, kvw = kv + c.head_dim_rope;
    const size_t sizes[P_COUNT] = {d,      d * q,  q,      q * H * qk, d * kvw,
                                   kv,     kv * H * c.head_dim_nope,    kv * H * c.head_dim_value,
                                   H * c.head_dim_value * d,           d,
                                   d * c.d_ff, d * c.d_ff, (size_t)c.d_ff * d};
    Registry r;
    r.embed = p;
    p += (size_t)c.vocab_size * d;
    r.final_norm = p;
    p += d;
    for (int l = 0; l < c.n_layers; ++l)
        for (int k = 0; k < P_COUNT; ++k) {
            r.layer.push_back(p);
            p += sizes[k];
        }
    return r;
}

}  // namespace

struct Model {
    mla_model_config cfg;
    ModelDims dims;
    int max_batch, m_pad_max, parts;
    std::vector<void*> allocations;
    std::vector<LayerWeights> layers;
    const uint16_t* embed = nullptr;
    const float* final_norm = nullptr;
    const float* rope_tab = nullptr;
    float *x, *res, *ctx, *logits, *arg_v;
    float *ss_x, *ss_res;
    float2* rope_rows;
    uint16_t *xw, *resw, *u, *q_latent, *q_rope;
    int32_t* arg_c;
    uint32_t* ban_bits = nullptr;  // [ceil(vocab/32)] banned token ids, allocated on first use
    bool banning = false;          // some id is banned: the greedy token skips them
    uint64_t revision = 0;         // weight uploads after the first (mla_model_update_weights)
    uint64_t launches = 0;         // kernels launched by model_forward
    // Every weight buffer in upload order, so an update rewrites them in place.
    std::vector<std::pair<void*, size_t>> weight_slots;
    size_t slot_cursor = 0;
    bool updating = false;

    ~Model() {
        for (void* p : allocations)
            (void)hipFree(p);
    }
    template <typename T>
    hipError_t alloc(T*& out, size_t count) {
        void* p = nullptr;
        const hipError_t e = hipMalloc(&p, count * sizeof(T) + 16);
        if (e != hipSuccess)
            return e;
        allocations.push_back(p);
        out = static_cast<T*>(p);
        return hipMemset(p, 0, count * sizeof(T) + 16);
    }
    // First upload: a new buffer.  During an update: the buffer this upload filled at
    // creation (same order, same size).
    template <typename T>
    hipError_t upload(const T*& out, const std::vector<T>& host) {
        const size_t bytes = host.size() * sizeof(T);
        T* p = nullptr;
        if (updating) {
            if (slot_cursor >= weight_slots.size() || weight_slots[slot_cursor].second != bytes)
                return hipErrorInvalidValue;
            p = static_cast<T*>(weight_slots[slot_cursor++].first);
        } else {
            const hipError_t e = alloc(p, host.size());
            if (e != hipSuccess)
                return e;
            weight_slots.emplace_back(p, bytes);
        }
        out = p;
        return hipMemcpy(p, host.data(), bytes, hipMemcpyHostToDevice);
    }
};

namespace {

ModelDims make_dims(const mla_model_config& c, int page_size) {
    ModelDims m{};
    m.vocab = c.vocab_size;
    m.d_model = c.d_model;
    m.H = c.n_heads;
    m.nope = c.head_dim_nope;
    m.rope = c.head_dim_rope;
    m.dv = c.head_dim_value;
    m.q_rank = c.q_lora_rank;
    m.kv_rank = c.kv_lora_rank;
    m.d_ff = c.d_ff;
    m.n_layers = c.n_layers;
    m.qk = c.head_dim_nope + c.head_dim_rope;
    m.eps = c.norm_epsilon;
    m.theta = c.rope_theta;
    m.page_size = page_size;
    m.max_seq = c.max_sequence_length;
    m.d_pad = round_up(c.d_model, 32);
    m.q_pad = round_up(c.q_lora_rank, 32);
    m.kvw_pad = round_up(c.kv_lora_rank + c.head_dim_rope, 16);
    m.qk_pad = round_up(m.qk, 16);
    m.nope_pad = round_up(c.head_dim_nope, 32);
    m.kv_pad = round_up(c.kv_lora_rank, 16);
    m.ctx_pad = round_up(c.n_heads * c.kv_lora_rank, 32);
    m.ff_pad = round_up(c.d_ff, 32);
    m.vocab_pad = round_up(c.vocab_size, 16);
    return m;
}

// Packs and uploads every weight of `params` (registry order) in one fixed order: at
// creation into new buffers, during mla_model_update_weights into the same buffers.
hipError_t upload_weights(Model* M, const float* params) {
    const mla_model_config& c = M->cfg;
    const ModelDims& m = M->dims;
    const Registry R = view(c, params);
    const int d = c.d_model, q = c.q_lora_rank, H = c.n_heads, nope = c.head_dim_nope;
    const int qk = m.qk, kv = c.kv_lora_rank, kvw = kv + c.head_dim_rope, dv = c.head_dim_value;
    const int ff = c.d_ff;
    // Tied embedding as the logits weight: K = d_model, N = vocab.
    hipError_t e = M->upload(M->embed, pack(d, c.vocab_size, m.d_pad, m.vocab_pad,
                                 [&](int k, int col) { return R.embed[(size_t)col * d + k]; }));
    if (e == hipSuccess)
        e = M->upload(M->final_norm, std::vector<float>(R.final_norm, R.final_norm + d));
    if (e == hipSuccess) {  // RoPE angles exactly as ops.cpp:88-108 forms them, per position
        const int half = c.head_dim_rope / 2;
        std::vector<float> tab((size_t)c.max_sequence_length * half * 2);
        for (int pos = 0; pos < c.max_sequence_length; ++pos)
            for (int j = 0; j < c.head_dim_rope; j += 2) {
                const float angle =
                    (float)pos * powf(c.rope_theta, -(float)j / (float)c.head_dim_rope);
                tab[((size_t)pos * half + j / 2) * 2] = cosf(angle);
                tab[((size_t)pos * half + j / 2) * 2 + 1] = sinf(angle);
            }
        e = M->upload(M->rope_tab, tab);
    }
    std::vector<float> proj((size_t)H * kv * d);
    std::vector<LayerWeights> layers;
    for (int l = 0; l < c.n_layers && e == hipSuccess; ++l) {
        const float* const* P = R.layer.data() + (size_t)l * P_COUNT;
        LayerWeights w{};
        e = M->upload(w.attn_norm, std::vector<float>(P[P_ATTN_NORM], P[P_ATTN_NORM] + d));
        if (e == hipSuccess)
            e = M->upload(w.q_norm, std::vector<float>(P[P_Q_NORM], P[P_Q_NORM] + q));
        if (e == hipSuccess)
            e = M->upload(w.kv_norm, std::vector<float>(P[P_KV_NORM], P[P_KV_NORM] + kv));
        if (e == hipSuccess)
            e = M->upload(w.ffn_norm, std::vector<float>(P[P_FFN_NORM], P[P_FFN_NORM] + d));
        if (e == hipSuccess)  // [w_dq | w_dkv]: q columns padded to q_pad, then the kv columns
            e = M->upload(w.w_dq_dkv,
                          pack(d, m.q_pad + kvw, m.d_pad, m.q_pad + m.kvw_pad, [&](int k, int col) {
                              if (col < q)
                                  return P[P_W_DQ][(size_t)k * q + col];
                              if (col < m.q_pad)
                                  return 0.0f;
                              return P[P_W_DKV][(size_t)k * kvw + (col - m.q_pad)];
                          }));
        if (e == hipSuccess)  // w_uq: head h at columns h*qk_pad ..
            e = M->upload(w.w_uq, pack(q, H * m.qk_pad, m.q_pad, H * m.qk_pad, [&](int k, int col) {
                              const int h = col / m.qk_pad, cc = col % m.qk_pad;
                              return cc < qk ? P[P_W_UQ][(size_t)k * H * qk + h * qk + cc] : 0.0f;
                          }));
        if (e == hipSuccess) {  // W_uk_h^T per head: (k = nope index, col = latent index)
            std::vector<uint16_t> all;
            for (int h = 0; h < H; ++h) {
                auto blk = pack(nope, kv, m.nope_pad, m.kv_pad, [&](int k, int col) {
                    return P[P_W_UK][(size_t)col * H * nope + h * nope + k];
                });
                all.insert(all.end(), blk.begin(), blk.end());
            }
            e = M->upload(w.w_uk, all);
        }
        if (e == hipSuccess) {  // combined W_uv.W_o (CpuDecoder::prepare_projections, inference.cpp:28-46)
            for (int h = 0; h < H; ++h)
                for (int r = 0; r < kv; ++r) {
                    float* row = proj.data() + ((size_t)h * kv + r) * d;
                    std::memset(row, 0, (size_t)d * sizeof(float));
                    for (int t = 0; t < dv; ++t) {
                        const float a = P[P_W_UV][(size_t)r * H * dv + h * dv + t];
                        const float* b = P[P_W_O] + (size_t)(h * dv + t) * d;
                        for (int j = 0; j < d; ++j)
                            row[j] += a * b[j];
                    }
                }
            e = M->upload(w.w_out, pack(H * kv, d, m.ctx_pad, m.d_pad, [&](int k, int col) {
                              return proj[(size_t)k * d + col];
                          }));
        }
        if (e == hipSuccess)  // gate/up tiles interleaved: tile 2j gate, 2j+1 up, columns 16j..
            e = M->upload(w.w_gate_up, pack(d, 2 * m.ff_pad, m.d_pad, 2 * m.ff_pad, [&](int k, int col) {
                              const int t = col / 16, fcol = (t / 2) * 16 + col % 16;
                              if (fcol >= ff)
                                  return 0.0f;
                              return (t % 2 ? P[P_W_UP] : P[P_W_GATE])[(size_t)k * ff + fcol];
                          }));
        if (e == hipSuccess)
            e = M->upload(w.w_down, pack(ff, d, m.ff_pad, m.d_pad, [&](int k, int col) {
                              return P[P_W_DOWN][(size_t)k * d + col];
                          }));
        layers.push_back(w);
    }
    if (e == hipSuccess)
        M->layers = std::move(layers);
    return e;
}

}  // namespace

int model_max_rows(const Model* M) { return M->max_batch; }
uint64_t model_launches(const Model* M) { return M->launches; }
const mla_model_config& model_config(const Model* M) { return M->cfg; }

int model_forward(Model* M, hipStream_t st, int rows, const int32_t* tokens,
                  const int32_t* positions, int B, int max_q_len, const MetaPtrs& md,
                  void* const* pages, void* workspace, size_t workspace_bytes, float* logits,
                  int32_t* next_tokens, bool all_rows) {
    if (!M || rows < 0 || rows > M->max_batch || B < 0 || B > rows || max_q_len < 1 ||
        max_q_len > rows + (rows == 0) || md.max_work < 0 || md.max_work > kMaxWork ||
        md.max_pages < 0 || md.num_pool_pages < 0 || (rows == B) != (max_q_len == 1))
        return fail(MLA_ERR_INVALID_ARGUMENT, "model forward: invalid argument");
    if (rows == 0)
        return MLA_OK;
    if (!tokens || !positions || !md.cu_seqlens_q || !md.page_table || !md.slot_mapping ||
        !md.num_splits || !md.cu_splits || !md.work_desc || !md.work_pages || !md.info ||
        !pages || !next_tokens || (max_q_len > 1 && !md.cu_seqlens_k))
        return fail(MLA_ERR_INVALID_ARGUMENT, "model forward: null buffer");
    for (int l = 0; l < M->cfg.n_layers; ++l)
        if (!pages[l])
            return fail(MLA_ERR_INVALID_ARGUMENT, "model forward: null page pool");
    const ModelDims& m = M->dims;
    const size_t need = mla_decode_workspace_bytes(md.max_work, B, m.H, m.kv_rank);
    if (!workspace || workspace_bytes < need)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "model forward: workspace needs " + std::to_string(need) + " bytes");
    StepArgs s{};
    s.dims = m;
    s.B = rows;
    s.m_pad = round_up(rows, 64);
    s.tokens = tokens;
    s.positions = positions;
    s.slot_mapping = md.slot_mapping;
    s.num_pool_pages = md.num_pool_pages;
    s.embed = M->embed;
    s.final_norm = M->final_norm;
    s.rope_tab = reinterpret_cast<const float2*>(M->rope_tab);
    s.x = M->x;
    s.res = M->res;
    s.xw = M->xw;
    s.resw = M->resw;
    s.rope_rows = M->rope_rows;
    s.ctx = M->ctx;
    s.u = M->u;
    s.q_latent = M->q_latent;
    s.q_rope = M->q_rope;
    s.logits = logits ? logits : M->logits;
    s.arg_v = M->arg_v;
    s.arg_c = M->arg_c;
    s.ban = M->banning ? M->ban_bits : nullptr;
    s.next_tokens = next_tokens;
    s.ss_x = M->ss_x;
    s.ss_res = M->ss_res;
    DecodeArgs a{};
    a.B = B;
    a.H = m.H;
    a.kv_rank = m.kv_rank;
    a.rope_dim = m.rope;
    a.page_size = m.page_size;
    a.max_pages = md.max_pages;
    a.num_pool_pages = md.num_pool_pages;
    a.max_work = md.max_work;
    a.scale_log2 = 1.4426950408889634f / std::sqrt((float)m.qk);  // inference.cpp:133
    a.cu_q = md.cu_seqlens_q;
    a.page_table = md.page_table;
    a.num_splits = md.num_splits;
    a.cu_splits = md.cu_splits;
    a.work_desc = md.work_desc;
    a.work_pages = md.work_pages;
    a.info = md.info;
    a.q_latent = M->q_latent;
    a.q_rope = M->q_rope;
    a.out = M->ctx;
    a.lse = nullptr;
    decode_workspace_layout(workspace, md.max_work, m.H, m.kv_rank, a);
    PrefillArgs pa{};
    pa.B = B;
    pa.H = m.H;
    pa.kv_rank = m.kv_rank;
    pa.rope_dim = m.rope;
    pa.page_size = m.page_size;
    pa.max_pages = md.max_pages;
    pa.num_pool_pages = md.num_pool_pages;
    pa.scale_log2 = a.scale_log2;
    pa.cu_q = md.cu_seqlens_q;
    pa.cu_k = md.cu_seqlens_k;
    pa.page_table = md.page_table;
    pa.info = md.info;
    pa.q_latent = M->q_latent;
    pa.q_rope = M->q_rope;
    pa.out = M->ctx;
    pa.lse = nullptr;
    const bool generic = (reinterpret_cast<uintptr_t>(workspace) & 15) != 0;
    a.fused_merge = (md.flags & MLA_DECODE_FUSED_MERGE) && decode_fuses_merge(a, generic);
    if (int bad = fused_checks(a, md.flags, "model forward"))
        return bad;
    // decode (+ the split merge unless the decode launch merges itself)
    const int attn_launches = md.max_work > 0 && B > 0 ? 2 - a.fused_merge : 0;
    // The MFMA page kernel's leading pages are read ahead into L2 during qkv_kernel.
    PagePrefetch pf{};
    if (attn_launches > 0 && !generic && !(md.flags & MLA_STEP_NO_READ_AHEAD) &&
        decode_mfma_supported(a.H, a.kv_rank, a.rope_dim, a.page_size)) {
        pf.work_desc = md.work_desc;
        pf.work_pages = md.work_pages;
        pf.max_work = md.max_work;
        pf.pages = kReadAheadPages;
        pf.page_size = m.page_size;
        pf.record = m.page_size * (m.kv_rank + m.rope);
    }
    hipError_t e = launch_embed(s, M->layers[0].attn_norm, st);
    uint64_t launched = 1;
    for (int l = 0; l < m.n_layers && e == hipSuccess; ++l) {
        const float* next_norm = l + 1 < m.n_layers ? M->layers[l + 1].attn_norm : M->final_norm;
        uint16_t* pool = static_cast<uint16_t*>(pages[l]);
        e = launch_layer_pre(s, M->layers[l], pool, pf, st);
        if (e != hipSuccess)
            break;
        a.pages = pool;
        pa.pages = pool;
        // decode attention for the q_len == 1 sessions (its work items of longer sessions
        // exit at once), then chunked-prefill attention for the others
        e = launch_decode_partials(a, MLA_DTYPE_F16, generic, st);
        if (e == hipSuccess && !a.fused_merge)
            e = launch_merge(a, st);
        if (e == hipSuccess && max_q_len > 1)
            e = launch_prefill(pa, max_q_len, MLA_DTYPE_F16, false, st);
        if (e == hipSuccess)
            e = launch_layer_post(s, M->layers[l], next_norm,
                                  l + 1 < m.n_layers ? &M->layers[l + 1] : nullptr, st);
        launched += 1 + attn_launches + (max_q_len > 1) + 3;
    }
    if (e == hipSuccess && rows != B && !all_rows) {  // logits of each session's last row only
        StepArgs t = s;
        t.B = B;
        t.m_pad = round_up(B, 64);
        t.xw = M->resw;  // free after the last layer's FFN
        t.ss_x = M->ss_res;
        e = launch_gather_last(s, B, md.cu_seqlens_q, t.xw, t.ss_x, st);  // from s.xw, s.ss_x
        if (e == hipSuccess)
            e = launch_logits(t, st);
        launched += 3;
    } else if (e == hipSuccess) {  // every row's logits (rows == B, or all_rows)
        e = launch_logits(s, st);
        launched += 2;
    }
    M->launches += launched;
    return gpu_status(e, "model forward");
}

}  // namespace mla

using namespace mla;

extern "C" {

int mla_config_validate(const mla_model_config* config) { return validate(config); }

size_t mla_config_parameter_count(const mla_model_config* config) {
    return config ? parameter_count(*config) : 0;
}

int mla_model_create(const mla_model_config* config, const float* params, int max_batch,
                     int page_size, void** model_out) {
    if (!model_out)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_create: null output");
    *model_out = nullptr;
    if (int st = validate(config))
        return st;
    if (!params || max_batch < 1 || max_batch > 65536 || page_size < 1)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_create: invalid argument");
    const mla_model_config& c = *config;
    const ModelDims m = make_dims(c, page_size);
    // Shapes the step kernels cover: a head's q within one workgroup (<= 4 tiles) and its
    // absorption within 4 waves x 2 tiles, at most 8 k-steps per split-K wave (d_model,
    // q_lora_rank: 4 with their on-the-fly norms), fp32 rows read 8 columns at a time.
    if (m.qk_pad / 16 > 4 || m.kv_pad / 16 > 8 || (c.n_heads * c.kv_lora_rank) % 8 ||
        c.d_model % 8 || c.q_lora_rank % 8 || m.d_pad > 1024 || m.q_pad > 256 ||
        m.nope_pad > 128 || m.ctx_pad / 32 > 64 || m.ff_pad / 32 > 64)
        return fail(MLA_ERR_UNSUPPORTED,
                    "mla_model_create: shape outside the step kernels (head_dim_nope + "
                    "head_dim_rope <= 64, kv_lora_rank <= 128, head_dim_nope <= 128, "
                    "q_lora_rank <= 256 and d_model <= 1024, both multiples of 8, "
                    "n_heads*kv_lora_rank <= 2048 and a multiple of 8, d_ff <= 2048)");
    auto* M = new (std::nothrow) Model();
    if (!M)
        return fail(MLA_ERR_OUT_OF_MEMORY, "mla_model_create: host allocation");
    M->cfg = c;
    M->dims = m;
    M->max_batch = max_batch;
    M->m_pad_max = round_up(max_batch, 64);
    M->parts = g7_parts(m);
    if (qkv_lds_bytes(m) > 150 * 1024) {  // the gfx950 workgroup LDS is 160 KB
        delete M;
        return fail(MLA_ERR_UNSUPPORTED, "mla_model_create: projection tiles exceed the LDS");
    }
    hipError_t e = model_kernel_attributes(m);
    auto bail = [&](hipError_t err) {
        delete M;
        return gpu_status(err, "mla_model_create");
    };
    if (e != hipSuccess)
        return bail(e);
    e = upload_weights(M, params);
    const size_t rows = M->m_pad_max;
    const int H = c.n_heads, kv = c.kv_lora_rank;
    if (e == hipSuccess) e = M->alloc(M->x, rows * m.d_pad);
    if (e == hipSuccess) e = M->alloc(M->res, rows * m.d_pad);
    if (e == hipSuccess) e = M->alloc(M->xw, rows * m.d_pad);
    if (e == hipSuccess) e = M->alloc(M->resw, rows * m.d_pad);
    if (e == hipSuccess) e = M->alloc(M->rope_rows, rows * (size_t)(c.head_dim_rope / 2));
    if (e == hipSuccess) e = M->alloc(M->ctx, rows * (size_t)H * kv);
    if (e == hipSuccess) e = M->alloc(M->u, rows * m.ff_pad);
    if (e == hipSuccess) e = M->alloc(M->q_latent, (size_t)max_batch * H * kv);
    if (e == hipSuccess) e = M->alloc(M->q_rope, (size_t)max_batch * H * c.head_dim_rope);
    if (e == hipSuccess) e = M->alloc(M->logits, (size_t)max_batch * c.vocab_size);
    if (e == hipSuccess) e = M->alloc(M->arg_v, (size_t)max_batch * M->parts);
    if (e == hipSuccess) e = M->alloc(M->arg_c, (size_t)max_batch * M->parts);
    if (e == hipSuccess) e = M->alloc(M->ss_x, rows * (m.d_pad / 16));
    if (e == hipSuccess) e = M->alloc(M->ss_res, rows * (m.d_pad / 16));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess)
        return bail(e);
    *model_out = M;
    return MLA_OK;
}

int mla_model_destroy(void* model) {
    delete static_cast<Model*>(model);
    return MLA_OK;
}

int mla_model_update_weights(void* model, const float* params, uint64_t* revision) {
    Model* M = static_cast<Model*>(model);
    if (!M || !params)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_update_weights: null argument");
    // Device work that may still read the weights finishes first; the copies below are
    // synchronous.
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) {
        M->updating = true;
        M->slot_cursor = 0;
        e = upload_weights(M, params);
        M->updating = false;
    }
    if (e == hipSuccess && M->slot_cursor != M->weight_slots.size())
        e = hipErrorInvalidValue;
    if (e != hipSuccess)
        return gpu_status(e, "mla_model_update_weights");
    ++M->revision;
    if (revision)
        *revision = M->revision;
    return MLA_OK;
}

int mla_model_step(void* model, void* stream, int B, const int32_t* tokens,
                   const int32_t* positions, const int32_t* cu_seqlens_q,
                   const int32_t* page_table, int max_pages, int num_pool_pages,
                   const int32_t* slot_mapping, const int32_t* num_splits,
                   const int32_t* cu_splits, const int32_t* work_desc, const int32_t* work_pages,
                   const int32_t* info, int max_work, void* const* pages, void* workspace,
                   size_t workspace_bytes, float* logits, int32_t* next_tokens, int flags) {
    // Every session appends one token: rows are sessions and no prefill attention runs,
    // so cu_seqlens_k is not read.
    const MetaPtrs md{cu_seqlens_q, nullptr,   page_table, slot_mapping,
                      num_splits,   cu_splits, work_desc,  work_pages,
                      info,         max_pages, num_pool_pages, max_work,
                      flags};
    return model_forward(static_cast<Model*>(model), static_cast<hipStream_t>(stream), B, tokens,
                         positions, B, 1, md, pages, workspace, workspace_bytes, logits,
                         next_tokens);
}

int mla_model_forward(void* model, void* stream, int rows, const int32_t* tokens,
                      const int32_t* positions, int B, int max_q_len,
                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                      const int32_t* page_table, int max_pages, int num_pool_pages,
                      const int32_t* slot_mapping, const int32_t* num_splits,
                      const int32_t* cu_splits, const int32_t* work_desc,
                      const int32_t* work_pages, const int32_t* info, int max_work,
                      void* const* pages, void* workspace, size_t workspace_bytes, float* logits,
                      int32_t* next_tokens, int flags) {
    if (!cu_seqlens_k && max_q_len > 1)
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_forward: null cu_seqlens_k");
    const MetaPtrs md{cu_seqlens_q, cu_seqlens_k, page_table,     slot_mapping,
                      num_splits,   cu_splits,    work_desc,      work_pages,
                      info,         max_pages,    num_pool_pages, max_work,
                      flags};
    return model_forward(static_cast<Model*>(model), static_cast<hipStream_t>(stream), rows,
                         tokens, positions, B, max_q_len, md, pages, workspace, workspace_bytes,
                         logits, next_tokens);
}

int mla_model_set_banned(void* model, const uint16_t* ids, size_t n) {
    Model* M = static_cast<Model*>(model);
    if (!M || (!ids && n))
        return fail(MLA_ERR_INVALID_ARGUMENT, "mla_model_set_banned: null argument");
    const int vocab = M->cfg.vocab_size;
    std::vector<uint32_t> bits((size_t)(vocab + 31) / 32, 0u);
    bool any = false;
    for (size_t k = 0; k < n; ++k)
        if (ids[k] < vocab) {  // ids outside the vocabulary are ignored (inference.cpp:357-359)
            bits[ids[k] >> 5] |= 1u << (ids[k] & 31);
            any = true;
        }
    hipError_t e = hipSuccess;
    if (!M->ban_bits)
        e = M->alloc(M->ban_bits, bits.size());
    if (e == hipSuccess)
        e = hipMemcpy(M->ban_bits, bits.data(), bits.size() * sizeof(uint32_t),
                      hipMemcpyHostToDevice);
    if (e != hipSuccess)
        return gpu_status(e, "mla_model_set_banned");
    M->banning = any;
    return MLA_OK;
}

const float* mla_model_logits(void* model) {
    return model ? static_cast<Model*>(model)->logits : nullptr;
}

}  // extern "C"
