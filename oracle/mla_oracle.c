/*
 * mla_oracle.c -- fp32 CPU restatement of the reference MLA decode path.
 * TEST INFRASTRUCTURE ONLY (the parity checker; never part of the product).
 * See mla_oracle.h for the pinning of each function.
 */
#include "mla_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Rng: include/mini_mla/rng.hpp:9-32 (SplitMix64 + Box-Muller in float)     */
/* ------------------------------------------------------------------------ */
uint64_t orc_rng_next(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
float orc_rng_uniform(uint64_t* state) { /* rng.hpp:16-18 */
    return ((float)(orc_rng_next(state) >> 40) + 0.5F) / 16777216.0F;
}
uint64_t orc_rng_bounded(uint64_t* state, uint64_t bound) { /* rng.hpp:19-28 */
    if (bound == 0)
        return 0;
    const uint64_t threshold = (0ULL - bound) % bound;
    for (;;) {
        uint64_t r = orc_rng_next(state);
        if (r >= threshold)
            return r % bound;
    }
}
float orc_rng_normal(uint64_t* state) { /* rng.hpp:29-32; left operand's uniform drawn first */
    const float u1 = orc_rng_uniform(state);
    const float a = sqrtf(-2.0F * logf(u1));
    const float u2 = orc_rng_uniform(state);
    const float b = cosf(2.0F * 3.14159265358979323846F * u2);
    return a * b;
}
void orc_rng_fill_normal(uint64_t* state, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = orc_rng_normal(state);
}
void orc_rng_fill_bounded(uint64_t* state, uint64_t bound, int32_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = (int32_t)orc_rng_bounded(state, bound);
}

/* ------------------------------------------------------------------------ */
/* 16-bit floats.  to_half is static_cast<_Float16> (src/core/io.cpp:152-158),*/
/* i.e. IEEE round-to-nearest-even; bf16 likewise keeps the upper 16 bits    */
/* with RNE.  Written from the IEEE-754 definitions.                          */
/* ------------------------------------------------------------------------ */
uint16_t orc_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000U);
    const uint32_t a = u & 0x7fffffffU;
    if (a > 0x7f800000U) /* NaN: keep it quiet */
        return (uint16_t)(sign | 0x7e00U | ((a >> 13) & 0x3ffU));
    if (a >= 0x477ff000U) /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00U);
    if (a >= 0x38800000U) { /* normal half: |x| >= 2^-14 */
        uint32_t half = (a - 0x38000000U) >> 13;
        const uint32_t rem = a & 0x1fffU;
        if (rem > 0x1000U || (rem == 0x1000U && (half & 1U)))
            ++half;
        return (uint16_t)(sign | half);
    }
    const uint32_t e = a >> 23;
    if (e < 102) /* below 2^-25 (ties at 2^-25 go to zero below) */
        return sign;
    const uint32_t mant = (a & 0x7fffffU) | 0x800000U;
    const uint32_t shift = 126 - e; /* 14..24 */
    uint32_t half = mant >> shift;
    const uint32_t rem = mant & ((1U << shift) - 1U), mid = 1U << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1U)))
        ++half;
    return (uint16_t)(sign | half);
}
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000U) << 16;
    uint32_t e = (h >> 10) & 0x1fU, m = h & 0x3ffU, u;
    if (e == 0x1f)
        u = sign | 0x7f800000U | (m << 13);
    else if (e != 0)
        u = sign | ((e + 112U) << 23) | (m << 13);
    else if (m == 0)
        u = sign;
    else { /* subnormal: normalise */
        e = 113;
        while (!(m & 0x400U)) {
            m <<= 1;
            --e;
        }
        u = sign | (e << 23) | ((m & 0x3ffU) << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}
uint16_t orc_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffU) > 0x7f800000U)
        return (uint16_t)((u >> 16) | 0x40U);
    u += 0x7fffU + ((u >> 16) & 1U);
    return (uint16_t)(u >> 16);
}
float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
void orc_round_f16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = orc_f32_to_f16(in[i]);
}
void orc_round_bf16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = orc_f32_to_bf16(in[i]);
}
static float load16(const uint16_t* p, int dtype) {
    return dtype ? orc_bf16_to_f32(*p) : orc_f16_to_f32(*p);
}
static uint16_t store16(float x, int dtype) {
    return dtype ? orc_f32_to_bf16(x) : orc_f32_to_f16(x);
}

/* ------------------------------------------------------------------------ */
/* ModelConfig: src/model/config.cpp:7-48                                    */
/* ------------------------------------------------------------------------ */
static int qk_dim(const orc_config* c) { return c->head_dim_nope + c->head_dim_rope; }
static int kv_width(const orc_config* c) { return c->kv_lora_rank + c->head_dim_rope; }
static int attn_width(const orc_config* c) { return c->n_heads * c->head_dim_value; }

size_t orc_parameter_count(const orc_config* c) { /* config.cpp:7-19 */
    const size_t d = (size_t)c->d_model, h = (size_t)c->n_heads, q = (size_t)c->q_lora_rank,
                 kv = (size_t)c->kv_lora_rank;
    return (size_t)c->vocab_size * d + d +
           (size_t)c->n_layers *
               (d * q + q * h * (size_t)qk_dim(c) + d * (size_t)kv_width(c) +
                kv * h * (size_t)(c->head_dim_nope + c->head_dim_value) +
                h * (size_t)c->head_dim_value * d + 3 * d * (size_t)c->d_ff + 2 * d + q + kv);
}
int orc_validate(const orc_config* c) { /* config.cpp:20-48 */
    const int v[11] = {c->vocab_size,    c->max_sequence_length, c->n_layers,     c->d_model,
                       c->n_heads,       c->head_dim_nope,       c->head_dim_rope, c->head_dim_value,
                       c->q_lora_rank,   c->kv_lora_rank,        c->d_ff};
    for (int i = 0; i < 11; ++i)
        if (v[i] < 1 || v[i] > 65535)
            return 1;
    if (c->vocab_size > 65535 || c->n_layers > 128 || c->n_heads > 256 ||
        c->d_model % c->n_heads || c->head_dim_rope % 2)
        return 1;
    if (!isfinite(c->norm_epsilon) || c->norm_epsilon <= 0 || !isfinite(c->rope_theta) ||
        c->rope_theta <= 1)
        return 1;
    if (orc_parameter_count(c) > 1000000000ULL)
        return 1;
    return 0;
}

enum { P_ATTN_NORM, P_W_DQ, P_Q_NORM, P_W_UQ, P_W_DKV, P_KV_NORM, P_W_UK, P_W_UV, P_W_O,
       P_FFN_NORM, P_W_GATE, P_W_UP, P_W_DOWN, P_COUNT };

int orc_parameter_shapes(const orc_config* c, int* rows, int* cols) { /* model.cpp:40-63 */
    int n = 0;
#define ADD(r, k)                                                                                  \
    do {                                                                                           \
        rows[n] = (r);                                                                             \
        cols[n] = (k);                                                                             \
        ++n;                                                                                       \
    } while (0)
    ADD(c->vocab_size, c->d_model);
    ADD(1, c->d_model);
    for (int l = 0; l < c->n_layers; ++l) {
        ADD(1, c->d_model);
        ADD(c->d_model, c->q_lora_rank);
        ADD(1, c->q_lora_rank);
        ADD(c->q_lora_rank, c->n_heads * qk_dim(c));
        ADD(c->d_model, kv_width(c));
        ADD(1, c->kv_lora_rank);
        ADD(c->kv_lora_rank, c->n_heads * c->head_dim_nope);
        ADD(c->kv_lora_rank, attn_width(c));
        ADD(attn_width(c), c->d_model);
        ADD(1, c->d_model);
        ADD(c->d_model, c->d_ff);
        ADD(c->d_model, c->d_ff);
        ADD(c->d_ff, c->d_model);
    }
#undef ADD
    return n;
}

typedef struct {
    const float* p[2 + 128 * P_COUNT];
} param_view;

static void view_params(const orc_config* c, const float* params, param_view* v) {
    int rows[2 + 128 * P_COUNT], cols[2 + 128 * P_COUNT];
    int n = orc_parameter_shapes(c, rows, cols);
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        v->p[i] = params + off;
        off += (size_t)rows[i] * (size_t)cols[i];
    }
}
static const float* W(const param_view* v, int l, int which) {
    return v->p[2 + l * P_COUNT + which];
}

int orc_model_init(const orc_config* c, uint64_t seed, float* params) { /* model.cpp:20-75 */
    if (orc_validate(c))
        return 1;
    int rows[2 + 128 * P_COUNT], cols[2 + 128 * P_COUNT];
    const int n = orc_parameter_shapes(c, rows, cols);
    uint64_t state = seed;
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        const int layer_slot = i < 2 ? -1 : (i - 2) % P_COUNT;
        const int is_norm = i == 1 || layer_slot == P_ATTN_NORM || layer_slot == P_Q_NORM ||
                            layer_slot == P_KV_NORM || layer_slot == P_FFN_NORM;
        const int residual = layer_slot == P_W_O || layer_slot == P_W_DOWN;
        const float scale = residual ? 0.02F / sqrtf((float)(2 * c->n_layers)) : 0.02F;
        const size_t count = (size_t)rows[i] * (size_t)cols[i];
        for (size_t k = 0; k < count; ++k)
            params[off + k] = is_norm ? 1.0F : orc_rng_normal(&state) * scale;
        off += count;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* ops (src/model/ops.cpp)                                                   */
/* ------------------------------------------------------------------------ */
/* Optional CBLAS for the CPU-baseline timing.  The reference's products are Accelerate
   cblas_sgemm / cblas_sgemv calls (ops.cpp:15-17,119-122,138-140; inference.cpp:38-43,
   107-113,122-132,146-152).  Accelerate does not exist on Linux, so orc_set_blas can hand
   in a portable CBLAS with 64-bit indices (the OpenBLAS numpy ships); with none set, the
   plain loops below run.  The parity tests use the loops; a BLAS only reorders sums. */
typedef void (*orc_sgemm_fn)(int, int, int, int64_t, int64_t, int64_t, float, const float*,
                             int64_t, const float*, int64_t, float, float*, int64_t);
typedef void (*orc_sgemv_fn)(int, int, int64_t, int64_t, float, const float*, int64_t,
                             const float*, int64_t, float, float*, int64_t);
static orc_sgemm_fn g_sgemm = NULL;
static orc_sgemv_fn g_sgemv = NULL;
enum { CB_ROW_MAJOR = 101, CB_NO_TRANS = 111, CB_TRANS = 112 }; /* CBLAS enum values */

void orc_set_blas(void* sgemm, void* sgemv) {
    g_sgemm = (orc_sgemm_fn)sgemm;
    g_sgemv = (orc_sgemv_fn)sgemv;
}

/* out[m x n] = a[m x k] . b[k x n]   (ops.cpp:8-18; sequential k sums) */
static void matmul(const float* a, const float* b, float* out, int m, int k, int n) {
    if (g_sgemv && g_sgemm) {
        if (m == 1)
            g_sgemv(CB_ROW_MAJOR, CB_TRANS, k, n, 1.0F, b, n, a, 1, 0.0F, out, 1);
        else
            g_sgemm(CB_ROW_MAJOR, CB_NO_TRANS, CB_NO_TRANS, m, n, k, 1.0F, a, k, b, n, 0.0F, out,
                    n);
        return;
    }
    for (int i = 0; i < m; ++i) {
        float* o = out + (size_t)i * n;
        for (int j = 0; j < n; ++j)
            o[j] = 0.0F;
        for (int t = 0; t < k; ++t) {
            const float x = a[(size_t)i * k + t];
            const float* br = b + (size_t)t * n;
            for (int j = 0; j < n; ++j)
                o[j] += x * br[j];
        }
    }
}
/* out[m x n] = a[m x k] . b[n x k]^T  (tied logits, ops.cpp matmul with tb) */
static void matmul_bt(const float* a, const float* b, float* out, int m, int k, int n) {
    if (g_sgemv && g_sgemm) {
        if (m == 1)
            g_sgemv(CB_ROW_MAJOR, CB_NO_TRANS, n, k, 1.0F, b, k, a, 1, 0.0F, out, 1);
        else
            g_sgemm(CB_ROW_MAJOR, CB_NO_TRANS, CB_TRANS, m, n, k, 1.0F, a, k, b, k, 0.0F, out, n);
        return;
    }
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
            float s = 0.0F;
            for (int t = 0; t < k; ++t)
                s += a[(size_t)i * k + t] * b[(size_t)j * k + t];
            out[(size_t)i * n + j] = s;
        }
}
static void rmsnorm(const float* x, const float* w, float* out, int rows, int cols, float eps) {
    for (int i = 0; i < rows; ++i) { /* ops.cpp:33-45 */
        float sum = 0.0F;
        for (int j = 0; j < cols; ++j)
            sum += x[(size_t)i * cols + j] * x[(size_t)i * cols + j];
        const float inv = 1.0F / sqrtf(sum / (float)cols + eps);
        for (int j = 0; j < cols; ++j)
            out[(size_t)i * cols + j] = x[(size_t)i * cols + j] * inv * w[j];
    }
}
static float sigmoid(float x) { /* ops.cpp:65-70 */
    if (x >= 0)
        return 1.0F / (1.0F + expf(-x));
    const float e = expf(x);
    return e / (1.0F + e);
}
/* Adjacent-pair RoPE of columns [begin, begin+rope) of every head (ops.cpp:88-108).
 * Row r of x sits at position r + offset. */
static void rope(float* x, int rows, int heads, int width, int begin, int rope_width, float theta,
                 int offset) {
    for (int t = 0; t < rows; ++t)
        for (int j = 0; j < rope_width; j += 2) {
            const float angle =
                (float)(t + offset) * powf(theta, -(float)j / (float)rope_width);
            const float cs = cosf(angle), sn = sinf(angle);
            for (int h = 0; h < heads; ++h) {
                float* p = x + (size_t)t * heads * width + h * width + begin + j;
                const float a = p[0], v = p[1];
                p[0] = a * cs - v * sn;
                p[1] = a * sn + v * cs;
            }
        }
}

/* ------------------------------------------------------------------------ */
/* Model::forward, batch 1 (src/model/model.cpp:76-155)                      */
/* ------------------------------------------------------------------------ */
int orc_forward(const orc_config* c, const float* params, const uint16_t* tokens, int T,
                float* logits, float* ckv_out, float* krope_out) {
    if (T < 1 || T > c->max_sequence_length)
        return 1;
    for (int i = 0; i < T; ++i)
        if (tokens[i] >= c->vocab_size)
            return 1;
    param_view v;
    view_params(c, params, &v);
    const int d = c->d_model, H = c->n_heads, qk = qk_dim(c), kv = c->kv_lora_rank,
              rp = c->head_dim_rope, nope = c->head_dim_nope, dv = c->head_dim_value,
              ff = c->d_ff, q = c->q_lora_rank, kw = kv_width(c);
    const size_t Tz = (size_t)T;
    float* x = malloc(Tz * d * 4);
    float* h = malloc(Tz * d * 4);
    float* raw_cq = malloc(Tz * q * 4);
    float* cq = malloc(Tz * q * 4);
    float* qm = malloc(Tz * H * qk * 4);
    float* kvp = malloc(Tz * kw * 4);
    float* raw_ckv = malloc(Tz * kv * 4);
    float* ckv = malloc(Tz * kv * 4);
    float* kr = malloc(Tz * rp * 4);
    float* knope = malloc(Tz * H * nope * 4);
    float* vv = malloc(Tz * H * dv * 4);
    float* k = malloc(Tz * H * qk * 4);
    float* prob = malloc(Tz * 4);
    float* att = malloc(Tz * H * dv * 4);
    float* res = malloc(Tz * d * 4);
    float* h2 = malloc(Tz * d * 4);
    float* gate = malloc(Tz * ff * 4);
    float* up = malloc(Tz * ff * 4);
    float* out = malloc(Tz * d * 4);
    const float* emb = v.p[0];
    for (int i = 0; i < T; ++i)
        memcpy(x + (size_t)i * d, emb + (size_t)tokens[i] * d, (size_t)d * 4);
    const float scale = 1.0F / sqrtf((float)qk);
    for (int l = 0; l < c->n_layers; ++l) {
        rmsnorm(x, W(&v, l, P_ATTN_NORM), h, T, d, c->norm_epsilon);
        matmul(h, W(&v, l, P_W_DQ), raw_cq, T, d, q);
        rmsnorm(raw_cq, W(&v, l, P_Q_NORM), cq, T, q, c->norm_epsilon);
        matmul(cq, W(&v, l, P_W_UQ), qm, T, q, H * qk);
        rope(qm, T, H, qk, nope, rp, c->rope_theta, 0);
        matmul(h, W(&v, l, P_W_DKV), kvp, T, d, kw);
        for (int i = 0; i < T; ++i) {
            memcpy(raw_ckv + (size_t)i * kv, kvp + (size_t)i * kw, (size_t)kv * 4);
            memcpy(kr + (size_t)i * rp, kvp + (size_t)i * kw + kv, (size_t)rp * 4);
        }
        rmsnorm(raw_ckv, W(&v, l, P_KV_NORM), ckv, T, kv, c->norm_epsilon);
        rope(kr, T, 1, rp, 0, rp, c->rope_theta, 0);
        if (ckv_out)
            memcpy(ckv_out + (size_t)l * Tz * kv, ckv, Tz * kv * 4);
        if (krope_out)
            memcpy(krope_out + (size_t)l * Tz * rp, kr, Tz * rp * 4);
        matmul(ckv, W(&v, l, P_W_UK), knope, T, kv, H * nope);
        matmul(ckv, W(&v, l, P_W_UV), vv, T, kv, H * dv);
        for (int i = 0; i < T; ++i)
            for (int hh = 0; hh < H; ++hh) {
                for (int j = 0; j < nope; ++j)
                    k[(size_t)i * H * qk + hh * qk + j] = knope[(size_t)i * H * nope + hh * nope + j];
                for (int j = 0; j < rp; ++j)
                    k[(size_t)i * H * qk + hh * qk + nope + j] = kr[(size_t)i * rp + j];
            }
        /* causal attention, ops.cpp:109-142 */
        for (int hh = 0; hh < H; ++hh)
            for (int i = 0; i < T; ++i) {
                const float* qi = qm + (size_t)i * H * qk + hh * qk;
                float mx = 0;
                for (int j = 0; j <= i; ++j) {
                    const float* kj = k + (size_t)j * H * qk + hh * qk;
                    float s = 0;
                    for (int t = 0; t < qk; ++t)
                        s += qi[t] * kj[t];
                    prob[j] = scale * s;
                    if (j == 0 || prob[j] > mx)
                        mx = prob[j];
                }
                float sum = 0;
                for (int j = 0; j <= i; ++j) {
                    prob[j] = expf(prob[j] - mx);
                    sum += prob[j];
                }
                for (int j = 0; j <= i; ++j)
                    prob[j] /= sum;
                float* o = att + (size_t)i * H * dv + hh * dv;
                for (int t = 0; t < dv; ++t)
                    o[t] = 0;
                for (int j = 0; j <= i; ++j) {
                    const float* vj = vv + (size_t)j * H * dv + hh * dv;
                    for (int t = 0; t < dv; ++t)
                        o[t] += prob[j] * vj[t];
                }
            }
        matmul(att, W(&v, l, P_W_O), res, T, H * dv, d);
        for (size_t i = 0; i < Tz * d; ++i)
            res[i] += x[i];
        rmsnorm(res, W(&v, l, P_FFN_NORM), h2, T, d, c->norm_epsilon);
        matmul(h2, W(&v, l, P_W_GATE), gate, T, d, ff);
        matmul(h2, W(&v, l, P_W_UP), up, T, d, ff);
        for (size_t i = 0; i < Tz * ff; ++i)
            gate[i] = gate[i] * sigmoid(gate[i]) * up[i];
        matmul(gate, W(&v, l, P_W_DOWN), out, T, ff, d);
        for (size_t i = 0; i < Tz * d; ++i)
            x[i] = out[i] + res[i];
    }
    rmsnorm(x, v.p[1], h, T, d, c->norm_epsilon);
    matmul_bt(h, emb, logits, T, d, c->vocab_size);
    int bad = 0;
    for (size_t i = 0; i < Tz * c->vocab_size; ++i)
        if (!isfinite(logits[i]))
            bad = 5;
    free(x), free(h), free(raw_cq), free(cq), free(qm), free(kvp), free(raw_ckv), free(ckv);
    free(kr), free(knope), free(vv), free(k), free(prob), free(att), free(res), free(h2);
    free(gate), free(up), free(out);
    return bad;
}

/* ------------------------------------------------------------------------ */
/* CpuDecoder (src/infer/inference.cpp:28-174)                               */
/* ------------------------------------------------------------------------ */
void orc_output_projection(const orc_config* c, const float* params, float* out) {
    param_view v; /* inference.cpp:28-46 */
    view_params(c, params, &v);
    const int kv = c->kv_lora_rank, d = c->d_model, dv = c->head_dim_value, aw = attn_width(c);
    for (int l = 0; l < c->n_layers; ++l) {
        const float* uv = W(&v, l, P_W_UV);
        const float* wo = W(&v, l, P_W_O);
        float* o = out + (size_t)l * c->n_heads * kv * d;
        for (int h = 0; h < c->n_heads; ++h)
            for (int r = 0; r < kv; ++r) {
                float* row = o + ((size_t)h * kv + r) * d;
                for (int j = 0; j < d; ++j)
                    row[j] = 0;
                for (int t = 0; t < dv; ++t) {
                    const float a = uv[(size_t)r * aw + h * dv + t];
                    const float* b = wo + (size_t)(h * dv + t) * d;
                    for (int j = 0; j < d; ++j)
                        row[j] += a * b[j];
                }
            }
    }
}

int orc_decode(const orc_config* c, const float* params, const float* out_proj, float* latent,
               float* rope_cache, int position, uint16_t token, int absorbed, int round_cache,
               float* logits) {
    if (position < 1 || position >= c->max_sequence_length || token >= c->vocab_size)
        return 1; /* inference.cpp:71-75 */
    param_view v;
    view_params(c, params, &v);
    const int d = c->d_model, H = c->n_heads, qk = qk_dim(c), kv = c->kv_lora_rank,
              rp = c->head_dim_rope, nope = c->head_dim_nope, dv = c->head_dim_value,
              ff = c->d_ff, q = c->q_lora_rank, kw = kv_width(c), S = c->max_sequence_length;
    const int len = position + 1;
    float* hidden = malloc((size_t)d * 4);
    float* h = malloc((size_t)d * 4);
    float* raw_cq = malloc((size_t)q * 4);
    float* cq = malloc((size_t)q * 4);
    float* qv = malloc((size_t)H * qk * 4);
    float* kvp = malloc((size_t)kw * 4);
    float* ckv = malloc((size_t)kv * 4);
    float* kr = malloc((size_t)rp * 4);
    float* lq = malloc((size_t)kv * 4);
    float* lctx = malloc((size_t)H * kv * 4);
    float* scores = malloc((size_t)len * 4);
    float* rk = absorbed ? NULL : malloc((size_t)len * H * nope * 4);
    float* rv = absorbed ? NULL : malloc((size_t)len * H * dv * 4);
    float* att = malloc((size_t)H * dv * 4);
    float* res = malloc((size_t)d * 4);
    float* h2 = malloc((size_t)d * 4);
    float* gate = malloc((size_t)ff * 4);
    float* up = malloc((size_t)ff * 4);
    memcpy(hidden, v.p[0] + (size_t)token * d, (size_t)d * 4);
    const float scale = 1.0F / sqrtf((float)qk);
    for (int l = 0; l < c->n_layers; ++l) {
        float* cache = latent + (size_t)l * S * kv;
        float* kc = rope_cache + (size_t)l * S * rp;
        rmsnorm(hidden, W(&v, l, P_ATTN_NORM), h, 1, d, c->norm_epsilon);
        matmul(h, W(&v, l, P_W_DQ), raw_cq, 1, d, q);
        rmsnorm(raw_cq, W(&v, l, P_Q_NORM), cq, 1, q, c->norm_epsilon);
        matmul(cq, W(&v, l, P_W_UQ), qv, 1, q, H * qk);
        rope(qv, 1, H, qk, nope, rp, c->rope_theta, position);
        matmul(h, W(&v, l, P_W_DKV), kvp, 1, d, kw);
        rmsnorm(kvp, W(&v, l, P_KV_NORM), ckv, 1, kv, c->norm_epsilon);
        memcpy(kr, kvp + kv, (size_t)rp * 4);
        rope(kr, 1, 1, rp, 0, rp, c->rope_theta, position);
        for (int j = 0; j < kv; ++j) /* append, inference.cpp:100-103 */
            cache[(size_t)position * kv + j] =
                round_cache ? orc_f16_to_f32(orc_f32_to_f16(ckv[j])) : ckv[j];
        for (int j = 0; j < rp; ++j)
            kc[(size_t)position * rp + j] =
                round_cache ? orc_f16_to_f32(orc_f32_to_f16(kr[j])) : kr[j];
        if (!absorbed) { /* inference.cpp:104-114 */
            matmul(cache, W(&v, l, P_W_UK), rk, len, kv, H * nope);
            matmul(cache, W(&v, l, P_W_UV), rv, len, kv, H * dv);
        }
        const float* uk = W(&v, l, P_W_UK);
        for (int hh = 0; hh < H; ++hh) { /* inference.cpp:116-153 */
            const float* qh = qv + hh * qk;
            if (absorbed && g_sgemv) { /* the same products as CBLAS gemv calls */
                g_sgemv(CB_ROW_MAJOR, CB_NO_TRANS, kv, nope, 1.0F, uk + hh * nope, H * nope, qh, 1,
                        0.0F, lq, 1);
                g_sgemv(CB_ROW_MAJOR, CB_NO_TRANS, len, kv, 1.0F, cache, kv, lq, 1, 0.0F, scores, 1);
                g_sgemv(CB_ROW_MAJOR, CB_NO_TRANS, len, rp, 1.0F, kc, rp, qh + nope, 1, 1.0F, scores,
                        1);
            } else if (absorbed) {
                for (int r = 0; r < kv; ++r) {
                    float s = 0;
                    for (int n = 0; n < nope; ++n)
                        s += uk[(size_t)r * H * nope + hh * nope + n] * qh[n];
                    lq[r] = s;
                }
                for (int i = 0; i < len; ++i) {
                    float s = 0;
                    for (int r = 0; r < kv; ++r)
                        s += cache[(size_t)i * kv + r] * lq[r];
                    scores[i] = s;
                }
            } else
                for (int i = 0; i < len; ++i) {
                    float s = 0;
                    for (int n = 0; n < nope; ++n)
                        s += rk[(size_t)i * H * nope + hh * nope + n] * qh[n];
                    scores[i] = s;
                }
            if (!(absorbed && g_sgemv))
                for (int i = 0; i < len; ++i) {
                    float s = 0;
                    for (int j = 0; j < rp; ++j)
                        s += kc[(size_t)i * rp + j] * qh[nope + j];
                    scores[i] = s + scores[i];
                }
            float mx = scores[0] * scale;
            for (int i = 0; i < len; ++i) {
                scores[i] *= scale;
                mx = fmaxf(mx, scores[i]);
            }
            float sum = 0;
            for (int i = 0; i < len; ++i) {
                scores[i] = expf(scores[i] - mx);
                sum += scores[i];
            }
            for (int i = 0; i < len; ++i)
                scores[i] /= sum;
            if (absorbed && g_sgemv)
                g_sgemv(CB_ROW_MAJOR, CB_TRANS, len, kv, 1.0F, cache, kv, scores, 1, 0.0F,
                        lctx + hh * kv, 1);
            else if (absorbed)
                for (int r = 0; r < kv; ++r) {
                    float s = 0;
                    for (int i = 0; i < len; ++i)
                        s += cache[(size_t)i * kv + r] * scores[i];
                    lctx[hh * kv + r] = s;
                }
            else
                for (int t = 0; t < dv; ++t) {
                    float s = 0;
                    for (int i = 0; i < len; ++i)
                        s += rv[(size_t)i * H * dv + hh * dv + t] * scores[i];
                    att[hh * dv + t] = s;
                }
        }
        if (absorbed) /* inference.cpp:154-156 */
            matmul(lctx, out_proj + (size_t)l * H * kv * d, res, 1, H * kv, d);
        else
            matmul(att, W(&v, l, P_W_O), res, 1, H * dv, d);
        for (int j = 0; j < d; ++j)
            res[j] += hidden[j];
        rmsnorm(res, W(&v, l, P_FFN_NORM), h2, 1, d, c->norm_epsilon);
        matmul(h2, W(&v, l, P_W_GATE), gate, 1, d, ff);
        matmul(h2, W(&v, l, P_W_UP), up, 1, d, ff);
        for (int j = 0; j < ff; ++j)
            gate[j] = gate[j] * sigmoid(gate[j]) * up[j];
        matmul(gate, W(&v, l, P_W_DOWN), hidden, 1, ff, d);
        for (int j = 0; j < d; ++j)
            hidden[j] += res[j];
    }
    rmsnorm(hidden, v.p[1], h, 1, d, c->norm_epsilon);
    matmul_bt(h, v.p[0], logits, 1, d, c->vocab_size);
    int status = 0;
    for (int j = 0; j < c->vocab_size; ++j)
        if (!isfinite(logits[j]))
            status = 5;
    free(hidden), free(h), free(raw_cq), free(cq), free(qv), free(kvp), free(ckv), free(kr);
    free(lq), free(lctx), free(scores), free(rk), free(rv), free(att), free(res), free(h2);
    free(gate), free(up);
    return status;
}

/* ------------------------------------------------------------------------ */
/* Page record layout (the format the GPU kernels read and write).  Tiled    */
/* when page_size % 16 == 0, kv_rank % 32 == 0 and rope_dim % 8 == 0:        */
/* 16-token tiles t, 32-column K-steps j, 8-column groups g, token n in the   */
/* tile, column e in the group; otherwise plain row-major.                   */
/* ------------------------------------------------------------------------ */
static int tiled_layout(int page_size, int kv_rank, int rope_dim) {
    return page_size % 16 == 0 && kv_rank % 32 == 0 && rope_dim % 8 == 0;
}
static size_t lat_index(int tiled, int slot, int r, int kv_rank) {
    if (!tiled)
        return (size_t)slot * kv_rank + r;
    const size_t tile = (size_t)(slot / 16), n = (size_t)(slot % 16);
    const size_t j = (size_t)(r / 32), g = (size_t)((r % 32) / 8), e = (size_t)(r % 8);
    return ((tile * (size_t)(kv_rank / 32) + j) * 4 + g) * 128 + n * 8 + e;
}
static size_t rope_index(int tiled, int slot, int c, int page_size, int kv_rank, int rope_dim) {
    const size_t base = (size_t)page_size * kv_rank;
    if (!tiled)
        return base + (size_t)slot * rope_dim + c;
    const size_t tile = (size_t)(slot / 16), n = (size_t)(slot % 16);
    return base + (tile * (size_t)(rope_dim / 8) + (size_t)(c / 8)) * 128 + n * 8 + (size_t)(c % 8);
}

/* ------------------------------------------------------------------------ */
/* Absorbed attention over a paged 16-bit cache (inference.cpp:116-153)      */
/* ------------------------------------------------------------------------ */
static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }

/* One session of orc_attention_paged; cbuf/rbuf/scores hold k_len rows. */
static void attend_session(int b, int H, int kv_rank, int rope_dim, int page_size, int dtype,
                           int tiled, size_t rec, const int32_t* cu_q, const int32_t* k_len,
                           const int32_t* page_table, int max_pages, const uint16_t* pages,
                           const float* q_latent, const float* q_rope, float scale, float* out,
                           float* lse, float* scores, float* cbuf, float* rbuf) {
    const int nq = cu_q[b + 1] - cu_q[b];
    const int kl = k_len[b];
    for (int t = 0; t < kl; ++t) {
        const int page = page_table[(size_t)b * max_pages + t / page_size];
        const uint16_t* base = pages + (size_t)page * rec;
        const int slot = t % page_size;
        for (int r = 0; r < kv_rank; ++r)
            cbuf[(size_t)t * kv_rank + r] = load16(base + lat_index(tiled, slot, r, kv_rank), dtype);
        for (int j = 0; j < rope_dim; ++j)
            rbuf[(size_t)t * rope_dim + j] =
                load16(base + rope_index(tiled, slot, j, page_size, kv_rank, rope_dim), dtype);
    }
    for (int i = 0; i < nq; ++i) {
        const int row = cu_q[b] + i;
        const int len = kl - nq + i + 1;
        for (int h = 0; h < H; ++h) {
            const float* lq = q_latent + ((size_t)row * H + h) * kv_rank;
            const float* qr = q_rope + ((size_t)row * H + h) * rope_dim;
            for (int t = 0; t < len; ++t) {
                float s = 0, sr = 0;
                for (int r = 0; r < kv_rank; ++r)
                    s += cbuf[(size_t)t * kv_rank + r] * lq[r];
                for (int j = 0; j < rope_dim; ++j)
                    sr += rbuf[(size_t)t * rope_dim + j] * qr[j];
                scores[t] = sr + s;
            }
            float mx = scores[0] * scale;
            for (int t = 0; t < len; ++t) {
                scores[t] *= scale;
                mx = fmaxf(mx, scores[t]);
            }
            float sum = 0;
            for (int t = 0; t < len; ++t) {
                scores[t] = expf(scores[t] - mx);
                sum += scores[t];
            }
            for (int t = 0; t < len; ++t)
                scores[t] /= sum;
            float* o = out + ((size_t)row * H + h) * kv_rank;
            for (int r = 0; r < kv_rank; ++r) {
                float s = 0;
                for (int t = 0; t < len; ++t)
                    s += cbuf[(size_t)t * kv_rank + r] * scores[t];
                o[r] = s;
            }
            if (lse)
                lse[(size_t)row * H + h] = mx + logf(sum);
        }
    }
}

int orc_attention_paged(int B, int H, int kv_rank, int rope_dim, int page_size, int dtype,
                        const int32_t* cu_q, const int32_t* k_len, const int32_t* page_table,
                        int max_pages, const uint16_t* pages, const float* q_latent,
                        const float* q_rope, float scale, float* out, float* lse) {
    const size_t rec = (size_t)page_size * (size_t)(kv_rank + rope_dim);
    const int tiled = tiled_layout(page_size, kv_rank, rope_dim);
    int max_len = 1;
    for (int b = 0; b < B; ++b) {
        const int nq = cu_q[b + 1] - cu_q[b];
        if (nq <= 0)
            continue;
        if (k_len[b] < nq || (k_len[b] + page_size - 1) / page_size > max_pages)
            return 1;
        if (k_len[b] > max_len)
            max_len = k_len[b];
    }
    /* Sessions are independent (the reference decodes one session per fork and
       thread, src/infer/inference.cpp:238); the thread count does not change any
       result bit. */
#pragma omp parallel num_threads(g_threads)
    {
        float* scores = malloc((size_t)max_len * 4);
        float* cbuf = malloc((size_t)max_len * (size_t)kv_rank * 4);
        float* rbuf = malloc((size_t)max_len * (size_t)(rope_dim > 0 ? rope_dim : 1) * 4);
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < B; ++b)
            if (cu_q[b + 1] - cu_q[b] > 0)
                attend_session(b, H, kv_rank, rope_dim, page_size, dtype, tiled, rec, cu_q, k_len,
                               page_table, max_pages, pages, q_latent, q_rope, scale, out, lse,
                               scores, cbuf, rbuf);
        free(scores), free(cbuf), free(rbuf);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Ragged batch metadata (new)                                               */
/* ------------------------------------------------------------------------ */
static int metadata_error(int max_work, int32_t* work_desc, int32_t* info, int session) {
    for (int w = 0; w < max_work; ++w)
        work_desc[(size_t)w * 8] = -1;
    for (int k = 0; k < 8; ++k)
        info[k] = 0;
    info[0] = -1;
    info[1] = session;
    return 1;
}

int orc_build_metadata(int B, const int32_t* ctx_len, const int32_t* q_len,
                       const int32_t* cu_pages, const int32_t* page_ids, int page_size,
                       int max_pages, int num_pool_pages, int split_pages, int target_blocks,
                       int max_work, int max_rows, int placement_xcds, int32_t* cu_seqlens_q,
                       int32_t* cu_seqlens_k, int32_t* page_table, int32_t* slot_mapping,
                       int32_t* num_splits, int32_t* cu_splits, int32_t* work_session,
                       int32_t* work_split, int32_t* work_desc, int32_t* work_pages,
                       int32_t* info) {
    if (B < 0 || page_size < 1 || max_pages < 0 || split_pages < 0 || target_blocks < 1 ||
        placement_xcds < 0)
        return metadata_error(max_work, work_desc, info, -1);
    long long total_q = 0, total_k = 0, total_pages = 0;
    cu_seqlens_q[0] = 0;
    cu_seqlens_k[0] = 0;
    for (int b = 0; b < B; ++b) {
        const long long q = q_len[b], ctx = ctx_len[b];
        const long long npages = (long long)cu_pages[b + 1] - cu_pages[b];
        const long long kl = ctx + q;
        const long long need = (kl + page_size - 1) / page_size;
        int bad = q < 0 || ctx < 0 || npages < 0 || npages > max_pages || need > npages;
        for (long long j = 0; !bad && j < npages; ++j) {
            const int32_t pid = page_ids[cu_pages[b] + j];
            bad = pid < 0 || pid >= num_pool_pages;
        }
        total_q += q;
        total_k += kl;
        if (bad || total_q > INT_MAX || total_k > INT_MAX || total_q > max_rows)
            return metadata_error(max_work, work_desc, info, b);
        cu_seqlens_q[b + 1] = (int32_t)total_q;
        cu_seqlens_k[b + 1] = (int32_t)total_k;
        if (q > 0)
            total_pages += need;
        for (int j = 0; j < max_pages; ++j)
            page_table[(size_t)b * max_pages + j] = j < npages ? page_ids[cu_pages[b] + j] : -1;
    }
    long long split = split_pages;
    if (split == 0) {
        split = (total_pages + target_blocks - 1) / target_blocks;
        if (split < 1)
            split = 1;
    }
    cu_splits[0] = 0;
    long long w = 0;
    for (int b = 0; b < B; ++b) {
        const long long kl = (long long)ctx_len[b] + q_len[b];
        const long long need = (kl + page_size - 1) / page_size;
        const long long ns = q_len[b] > 0 ? (need + split - 1) / split : 0;
        num_splits[b] = (int32_t)ns;
        w += ns;
        if (w > max_work)
            return metadata_error(max_work, work_desc, info, b);
        cu_splits[b + 1] = (int32_t)w;
    }
    /* XCD placement (no reference counterpart; the GPU builder's layout, restated):
     * sessions ranked by pages read (q_len > 0), largest first, ties to the lower
     * session; rank r goes to XCD r % n in even rounds (r / n) and n - 1 - r % n in odd
     * ones; item s of session b in slot xcd[b] + n * (first[b] + s), first[b] = items
     * of the XCD's sessions of earlier rounds. */
    const int n = placement_xcds;
    int *xcd = NULL, *first = NULL;
    long long slots = w;
    if (n > 0) {
        xcd = (int*)calloc((size_t)B + 1, sizeof(int));
        first = (int*)calloc((size_t)B + 1, sizeof(int));
        int* order = (int*)calloc((size_t)B + 1, sizeof(int));
        long long* pages = (long long*)calloc((size_t)B + 1, sizeof(long long));
        long long* count = (long long*)calloc((size_t)n, sizeof(long long));
        for (int b = 0; b < B; ++b) {
            const long long kl = (long long)ctx_len[b] + q_len[b];
            pages[b] = q_len[b] > 0 ? (kl + page_size - 1) / page_size : 0;
            order[b] = b;
        }
        for (int i = 1; i < B; ++i)  /* insertion sort: pages desc, session asc */
            for (int j = i; j > 0 && pages[order[j - 1]] < pages[order[j]]; --j) {
                const int t = order[j];
                order[j] = order[j - 1];
                order[j - 1] = t;
            }
        for (int r = 0; r < B; ++r) {
            const int b = order[r];
            const int x = (r / n) % 2 == 0 ? r % n : n - 1 - r % n;
            xcd[b] = x;
            first[b] = (int)count[x];
            count[x] += num_splits[b];
        }
        long long most = 0;
        for (int i = 0; i < n; ++i)
            most = count[i] > most ? count[i] : most;
        slots = most * n;
        free(order), free(pages), free(count);
        if (slots > max_work) {
            free(xcd), free(first);
            return metadata_error(max_work, work_desc, info, B);
        }
    }
    for (long long x = 0; x < max_work; ++x)
        work_desc[(size_t)x * 8] = -1;
    for (int b = 0; b < B; ++b) {
        const int kl = ctx_len[b] + q_len[b];
        const int need = (kl + page_size - 1) / page_size;
        for (int s = 0; s < num_splits[b]; ++s) {
            const int w = n > 0 ? xcd[b] + n * (first[b] + s) : cu_splits[b] + s;
            const int p0 = (int)(s * split), p1 = p0 + split < need ? (int)(p0 + split) : need;
            int32_t* d = work_desc + (size_t)w * 8;
            work_session[w] = b;
            work_split[w] = s;
            d[0] = b;
            d[1] = cu_seqlens_q[b];
            d[2] = kl;
            d[3] = p0;
            d[4] = p1;
            d[5] = num_splits[b];
            d[6] = cu_splits[b] + s;
            d[7] = q_len[b];
            for (int j = 0; j < 8; ++j)
                work_pages[(size_t)w * 8 + j] = p0 + j < p1 ? page_ids[cu_pages[b] + p0 + j] : -1;
        }
        for (int i = 0; i < q_len[b]; ++i) {
            const int pos = ctx_len[b] + i;
            slot_mapping[cu_seqlens_q[b] + i] =
                page_table[(size_t)b * max_pages + pos / page_size] * page_size + pos % page_size;
        }
    }
    free(xcd), free(first);
    info[0] = (int32_t)w;
    info[1] = (int32_t)split;
    info[2] = (int32_t)total_q;
    info[3] = (int32_t)total_k;
    info[4] = n; /* the XCD count the work list is placed for (0: session order) */
    info[5] = info[6] = info[7] = 0;
    return 0;
}

void orc_append_paged(int T, int kv_rank, int rope_dim, int page_size, int dtype,
                      const float* ckv, const float* krope, const int32_t* slot_mapping,
                      uint16_t* pages) {
    const size_t rec = (size_t)page_size * (size_t)(kv_rank + rope_dim);
    const int tiled = tiled_layout(page_size, kv_rank, rope_dim);
    for (int t = 0; t < T; ++t) {
        const int page = slot_mapping[t] / page_size, slot = slot_mapping[t] % page_size;
        uint16_t* base = pages + (size_t)page * rec;
        for (int r = 0; r < kv_rank; ++r)
            base[lat_index(tiled, slot, r, kv_rank)] = store16(ckv[(size_t)t * kv_rank + r], dtype);
        for (int j = 0; j < rope_dim; ++j)
            base[rope_index(tiled, slot, j, page_size, kv_rank, rope_dim)] =
                store16(krope[(size_t)t * rope_dim + j], dtype);
    }
}

/* ------------------------------------------------------------------------ */
/* sample_token greedy branch (src/infer/inference.cpp:345-380)              */
/* ------------------------------------------------------------------------ */
int orc_greedy(const float* logits, int n, const uint16_t* history, int n_history,
               float repetition_penalty, const uint16_t* banned, int n_banned) {
    if (n < 1 || n > 65535)
        return -2;
    for (int i = 0; i < n; ++i)
        if (!isfinite(logits[i]))
            return -2;
    char* excluded = calloc((size_t)n, 1);
    char* repeated = calloc((size_t)n, 1);
    for (int i = 0; i < n_banned; ++i)
        if (banned[i] < n)
            excluded[banned[i]] = 1;
    if (repetition_penalty != 1.0F)
        for (int i = 0; i < n_history; ++i)
            if (history[i] < n)
                repeated[history[i]] = 1;
    int best = n;
    float maximum = -INFINITY;
    for (int i = 0; i < n; ++i) {
        if (excluded[i])
            continue;
        float score = logits[i];
        if (repeated[i])
            score = score > 0 ? score / repetition_penalty : score * repetition_penalty;
        if (best == n || score > maximum) {
            best = i;
            maximum = score;
        }
    }
    free(excluded);
    free(repeated);
    return best == n ? -1 : best;
}
