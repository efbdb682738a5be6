// Batched MLA decode step on gfx950: everything of CpuDecoder::decode around the
// attention (src/infer/inference.cpp:76-173) for B sessions at once, one new token
// each.
//
// Per layer, in launch order (y = x.W for every projection, as in ops.cpp:8-18):
//   g1_kernel   RMSNorm(x, attn_norm) -> [w_dq | w_dkv]; the q part is stored for g23,
//               the kv part is kv_norm-ed (latent) / RoPE-d (key), rounded to the cache
//               dtype and appended to the paged cache (inference.cpp:84-103)
//   g23_kernel  per head: q_norm -> w_uq -> RoPE of the rope columns (q_rope, stored in
//               the cache dtype) -> absorption q_latent = W_uk_h^T q_nope
//               (inference.cpp:85-90,121-124; the MPS graph keeps q_latent in the
//               storage dtype, mps_backend.mm:561)
//   (decode attention partials + merge: decode.hip)
//   g4_kernel   latent_ctx [H*kv_rank] . out_proj + x  (inference.cpp:154-156; out_proj
//               is the combined W_uv.W_o of prepare_projections, inference.cpp:28-46)
//   g5_kernel   RMSNorm(ffn_norm) -> [w_gate | w_up] -> SwiGLU  (inference.cpp:157-161)
//   g6_kernel   . w_down + residual  (inference.cpp:162-165)
// Per step: embed_kernel (token rows), g7_kernel (final RMSNorm, tied logits
// h.E^T, inference.cpp:166-168, with a per-workgroup greedy partial) and
// argmax_kernel (sample_token's greedy rule, inference.cpp:345-380).
//
// Every projection is a skinny GEMM (M = the batch rows, 64 per chunk) on
// v_mfma_f32_16x16x32_f16: activations are rounded to fp16 as A operands, weights are
// fp16 in the TILED layout below (each wave's B-operand load reads 1 KB contiguously),
// accumulation is fp32, norms / RoPE / SwiGLU / residuals run in fp32.
#include "mla_common.hpp"
#include "mla_internal.hpp"
#include "mla_model.hpp"

#include <cmath>

namespace mla {
namespace {

using V8 = half8;

__device__ __forceinline__ floatx4 mma(V8 a, V8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---- A operands: lane (g, n) supplies A[16mt + n][32kt + 8g .. +7] ----------------
struct ALds16 {  // fp16 rows in LDS
    const _Float16* p;
    int ld;
    __device__ V8 operator()(int m, int k) const { return *reinterpret_cast<const V8*>(p + m * ld + k); }
};
struct AGlb16 {  // fp16 rows in global memory
    const uint16_t* p;
    int ld;
    __device__ V8 operator()(int m, int k) const {
        return *reinterpret_cast<const V8*>(p + (long long)m * ld + k);
    }
};
struct AGlb32 {  // fp32 rows in global memory (K columns, K % 8 == 0), rounded to fp16
    const float* p;
    int ld, K;
    __device__ V8 operator()(int m, int k) const {
        if (k >= K)
            return V8{};
        const floatx4* q = reinterpret_cast<const floatx4*>(p + (long long)m * ld + k);
        const floatx4 a = q[0], b = q[1];
        return V8{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
                  (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
    }
};

// Weight (B operand) registers of one wave: k-steps [kt0, kt0+KW) of tiles
// [nt0, nt0+NT), fetched at kernel start, before the activations are ready, so every
// GEMM pays one weight round trip.  W is tiled (see mla_model.hpp): tile (nt, kt) is
// 512 contiguous fp16 words; tiles past `ntv` or k-steps past KT stay zero.
template <int NT, int KW>
struct BPre {
    V8 b[KW][NT];
    __device__ __forceinline__ void load(const uint16_t* w, int nt0, int ntv, int KT, int kt0,
                                         int lane) {
#pragma unroll
        for (int kk = 0; kk < KW; ++kk)
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                b[kk][j] = V8{};
                if (kt0 + kk < KT && j < ntv)
                    b[kk][j] = *reinterpret_cast<const V8*>(
                        w + ((long long)(nt0 + j) * KT + kt0 + kk) * 512 + lane * 8);
            }
    }
    // acc[mt][j] += A[16mt.., 32kt..] . W[32kt.., 16(nt0+j)..] over the fetched k-steps.
    template <typename A>
    __device__ __forceinline__ void mma_all(floatx4 (&acc)[4][NT], const A& a, int KT, int kt0,
                                            int lane) const {
        const int g = lane >> 4, n = lane & 15;
#pragma unroll
        for (int kk = 0; kk < KW; ++kk) {
            if (kt0 + kk >= KT)
                break;
            V8 av[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                av[mt] = a(16 * mt + n, 32 * (kt0 + kk) + 8 * g);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[mt][j] = mma(av[mt], b[kk][j], acc[mt][j]);
        }
    }
};

// Split-K reduction over the W waves of a workgroup through LDS (`part` holds at least
// W*4*NT*64 floatx4); then epi(mt, j, v) for every (M-tile, N-tile) pair, pairs dealt
// round-robin to the waves.  v is lane (g, n)'s C[16mt + 4g + i][16(nt0+j) + n].
template <int NT, int W, typename Epi>
__device__ __forceinline__ void splitk_reduce(floatx4 (&acc)[4][NT], floatx4* part, Epi epi) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < NT; ++j)
            part[((wave * 4 + mt) * NT + j) * 64 + lane] = acc[mt][j];
    __syncthreads();
    for (int p = wave; p < 4 * NT; p += W) {
        const int mt = p / NT, j = p % NT;
        floatx4 v = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < W; ++w)
            v += part[((w * 4 + mt) * NT + j) * 64 + lane];
        epi(mt, j, v);
    }
}

template <int NT>
__device__ __forceinline__ void zero(floatx4 (&acc)[4][NT]) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < NT; ++j)
            acc[mt][j] = floatx4{0, 0, 0, 0};
}

// RMSNorm of 64 fp32 rows of width K (ops.cpp:33-45: inv = 1/sqrt(mean(x^2) + eps),
// fp32 sums) times the norm weight, rounded to fp16 into LDS rows of pitch ld (the
// padding columns [K, Kpad) are zero).  One wave per 16 rows, RB rows at a time with
// every load of the batch in flight (lane l holds columns l, l+64, ...; CPL >= Kpad/64
// columns per lane; RB*CPL <= 64 registers), so a prologue costs a few global round
// trips, not two per row.
template <int CPL, int RB = 64 / CPL < 8 ? 64 / CPL : 8>
__device__ __forceinline__ void rmsnorm_rows_to_lds_t(const float* x, int ldx, int K, int Kpad, const float* wn,
                                      float eps, _Float16* lds, int ld) {
    constexpr int kRowBatch = RB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float w[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        w[j] = c < K ? wn[c] : 0.0f;
    }
#pragma unroll 1
    for (int r0 = wave * 16; r0 < wave * 16 + 16; r0 += kRowBatch) {
        float v[kRowBatch][CPL];
#pragma unroll
        for (int rr = 0; rr < kRowBatch; ++rr)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                v[rr][j] = c < K ? x[(long long)(r0 + rr) * ldx + c] : 0.0f;
            }
#pragma unroll
        for (int rr = 0; rr < kRowBatch; ++rr) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                ss += v[rr][j] * v[rr][j];
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                if (c < Kpad)
                    lds[(r0 + rr) * ld + c] = (_Float16)(v[rr][j] * inv * w[j]);
            }
        }
    }
}

__device__ __forceinline__ void rmsnorm_rows_to_lds(const float* x, int ldx, int K, int Kpad,
                                                    const float* wn, float eps, _Float16* lds,
                                                    int ld) {
    if (Kpad <= 256)
        rmsnorm_rows_to_lds_t<4>(x, ldx, K, Kpad, wn, eps, lds, ld);
    else if (Kpad <= 512)
        rmsnorm_rows_to_lds_t<8>(x, ldx, K, Kpad, wn, eps, lds, ld);
    else
        rmsnorm_rows_to_lds_t<16>(x, ldx, K, Kpad, wn, eps, lds, ld);
}

// Adjacent-pair RoPE (ops.cpp:88-108) of the value v in column col_in_span of the
// rotated span, for a lane whose partner column is lane ^ 1 (the MFMA output layout
// puts adjacent columns in adjacent lanes).  cos/sin of pos * theta^(-j/rope) come
// from the model's table (computed on the host with the reference's float formula).
// Positions past the table (the caller rejects them, as inference.cpp:71-75 does) are
// clamped so the lookup stays in bounds.
__device__ __forceinline__ float rope_lane(float v, int col_in_span, int rope, int pos,
                                           int max_seq, const float2* tab) {
    const float other = __shfl_xor(v, 1, 64);
    pos = min(max(pos, 0), max_seq - 1);
    const float2 cs = tab[(long long)pos * (rope / 2) + (col_in_span >> 1)];
    return (col_in_span & 1) ? other * cs.y + v * cs.x : v * cs.x - other * cs.y;
}

// ------------------------------------------------------------------ embed ----
// x[b] = E[token[b]] (fp32), rows [B, Mpad) zeroed.  E is read from its tiled
// logits layout (K = d_model, N = vocab).
__global__ __launch_bounds__(256) void embed_kernel(StepArgs s) {
    const int b = blockIdx.x;
    const ModelDims& m = s.dims;
    float* x = s.x + (long long)b * m.d_pad;
    if (b >= s.B) {
        for (int c = threadIdx.x; c < m.d_pad; c += 256)
            x[c] = 0.0f;
        return;
    }
    int tok = s.tokens[b];
    tok = tok < 0 || tok >= m.vocab ? 0 : tok;  // the caller validates tokens
    const int KT = m.d_pad / 32;
    for (int c = threadIdx.x; c < m.d_pad; c += 256) {
        float v = 0.0f;
        if (c < m.d_model) {
            const long long w = ((long long)(tok >> 4) * KT + (c >> 5)) * 512 +
                                (((c & 31) >> 3) * 16 + (tok & 15)) * 8 + (c & 7);
            v = (float)__builtin_bit_cast(_Float16, s.embed[w]);
        }
        x[c] = v;
    }
}

constexpr int kLdsPad = 8;

// --------------------------------------------------------------------- g1 ----
// RMSNorm(x, attn_norm) . [w_dq | w_dkv] -> cq (q columns) and kvraw (kv columns), fp32.
// One workgroup per 16-column tile; its 4 waves split K.
template <int KW>
__global__ __launch_bounds__(256) void g1_kernel(StepArgs s, LayerWeights L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const ModelDims& m = s.dims;
    const int mc = blockIdx.y, nt = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32;
    BPre<1, KW> bw;
    bw.load(L.w_dq_dkv, nt, 1, KT, wave * KW, lane);
    const int lda = m.d_pad + kLdsPad;
    _Float16* a_s = reinterpret_cast<_Float16*>(smem);
    rmsnorm_rows_to_lds(s.x + (long long)mc * 64 * m.d_pad, m.d_pad, m.d_model, m.d_pad, L.attn_norm,
                        m.eps, a_s, lda);
    __syncthreads();
    floatx4 acc[4][1];
    zero(acc);
    bw.mma_all(acc, ALds16{a_s, lda}, KT, wave * KW, lane);
    __syncthreads();  // the A tile is dead: its LDS holds the split-K partials
    splitk_reduce<1, 4>(acc, reinterpret_cast<floatx4*>(smem), [&](int mt, int, floatx4 v) {
        const int col = nt * 16 + n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long r = (long long)mc * 64 + 16 * mt + 4 * g + i;
            if (col < m.q_pad)
                s.cq[r * m.q_pad + col] = v[i];
            else
                s.kvraw[r * m.kvw_pad + (col - m.q_pad)] = v[i];
        }
    });
}

// -------------------------------------------------------------------- g23 ----
// Workgroups h < H: per head, q_norm of the q rows (prologue, fp32 -> fp16 LDS),
// q_h = cq . w_uq[:, head columns] (one tile per wave) with RoPE on the rope columns
// (q_rope, stored in the cache dtype), then q_latent_h = q_h[:, :nope] . W_uk_h^T.
// Workgroup H: kv_norm of the latent, RoPE of the key, rounding to the cache dtype
// and the paged append of every row (inference.cpp:94-103).
template <int KWQ, int KWU>
__global__ __launch_bounds__(256) void g23_kernel(StepArgs s, LayerWeights L, uint16_t* pool) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const ModelDims& m = s.dims;
    const int h = blockIdx.x, mc = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    if (h == m.H) {  // ---- kv append ----
        const bool tiled = page_tiled(m.page_size, m.kv_rank, m.rope);
        const int width = m.kv_rank + m.rope;
        const int r0 = wave * 16;
        float v[16][4];  // this wave's 16 rows, columns lane + 64 j (width <= 256)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = lane + 64 * j;
                v[rr][j] = c < width ? s.kvraw[((long long)mc * 64 + r0 + rr) * m.kvw_pad + c] : 0.0f;
            }
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const int row = mc * 64 + r0 + rr;
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ss += lane + 64 * j < m.kv_rank ? v[rr][j] * v[rr][j] : 0.0f;
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)m.kv_rank + m.eps);
            const int pos = row < s.B ? s.positions[row] : 0;
            const int slot = row < s.B ? s.slot_mapping[row] : -1;
            const int page = slot / m.page_size, off = slot % m.page_size;
            const bool ok = row < s.B && slot >= 0 && page < s.num_pool_pages;
            uint16_t* base = pool + (long long)(ok ? page : 0) * m.page_size * width;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = lane + 64 * j;
                const bool key = c >= m.kv_rank && c < width;
                // key pairs (c, c+1) sit in adjacent lanes: the shuffle runs on every lane
                const float rv = rope_lane(v[rr][j], key ? c - m.kv_rank : 0, m.rope, pos, m.max_seq,
                                           s.rope_tab);
                if (!ok || c >= width)
                    continue;
                if (c < m.kv_rank)
                    base[latent_word(tiled, off, c, m.page_size, m.kv_rank)] =
                        F16::from_float(v[rr][j] * inv * L.kv_norm[c]);
                else
                    base[rope_word(tiled, off, c - m.kv_rank, m.page_size, m.kv_rank, m.rope)] =
                        F16::from_float(rv);
            }
        }
        return;
    }
    // ---- one head ----
    const int qk_tiles = m.qk_pad / 16, KTQ = m.q_pad / 32;
    const int kv_tiles = m.kv_pad / 16, KTU = m.nope_pad / 32;
    const uint16_t* wuk = L.w_uk + (long long)h * kv_tiles * KTU * 512;
    BPre<1, KWQ> bq;  // this wave's q tile, whole K
    bq.load(L.w_uq, h * qk_tiles + wave, wave < qk_tiles ? 1 : 0, KTQ, 0, lane);
    BPre<2, KWU> bu;  // this wave's two latent tiles of the absorption, whole K
    bu.load(wuk, 2 * wave, min(2, kv_tiles - 2 * wave), KTU, 0, lane);
    const int lda = m.q_pad + kLdsPad;
    _Float16* a_s = reinterpret_cast<_Float16*>(smem);
    rmsnorm_rows_to_lds(s.cq + (long long)mc * 64 * m.q_pad, m.q_pad, m.q_rank, m.q_pad, L.q_norm,
                        m.eps, a_s, lda);
    const int ldq = m.nope_pad + kLdsPad;  // q_h (nope columns) for the absorption
    _Float16* q_s = a_s + 64 * lda;
    for (int i = threadIdx.x; i < 64 * ldq; i += 256)
        q_s[i] = (_Float16)0.0f;
    __syncthreads();
    if (wave < qk_tiles) {
        floatx4 acc[4][1];
        zero(acc);
        bq.mma_all(acc, ALds16{a_s, lda}, KTQ, 0, lane);
        const int c = wave * 16 + n;  // column inside the head's q
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * mt + 4 * g + i, row = mc * 64 + r;
                float v = acc[mt][0][i];
                const bool rope_col = c >= m.nope && c < m.qk;
                const int cs = rope_col ? c - m.nope : 0;
                const float rv = rope_lane(v, cs, m.rope, row < s.B ? s.positions[row] : 0,
                                           m.max_seq, s.rope_tab);  // every lane joins the pair shuffle
                if (rope_col)
                    v = rv;
                if (c < m.nope)
                    q_s[r * ldq + c] = (_Float16)v;
                else if (rope_col && row < s.B)
                    s.q_rope[((long long)row * m.H + h) * m.rope + (c - m.nope)] =
                        F16::from_float(v);
            }
    }
    __syncthreads();
    if (2 * wave < kv_tiles) {
        floatx4 acc[4][2];
        zero(acc);
        bu.mma_all(acc, ALds16{q_s, ldq}, KTU, 0, lane);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = (2 * wave + j) * 16 + n;
            if (c < m.kv_rank)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = mc * 64 + 16 * mt + 4 * g + i;
                        if (row < s.B)
                            s.q_latent[((long long)row * m.H + h) * m.kv_rank + c] =
                                F16::from_float(acc[mt][j][i]);
                    }
        }
    }
}

// ----------------------------------------------------------- g4 and g6 ----
// out = A . W + residual for one 16-column tile per workgroup; 8 waves split K.
constexpr int kSplitWaves = 8;

template <int KW, typename A>
__device__ __forceinline__ void splitk_residual(const A& a, const uint16_t* w, int KT, int N,
                                                const float* residual, float* out, int ld, int mc,
                                                int B) {
    __shared__ __attribute__((aligned(16))) floatx4 part[kSplitWaves * 4 * 64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int nt = blockIdx.x;
    BPre<1, KW> bw;
    bw.load(w, nt, 1, KT, wave * KW, lane);
    floatx4 acc[4][1];
    zero(acc);
    bw.mma_all(acc, a, KT, wave * KW, lane);
    splitk_reduce<1, kSplitWaves>(acc, part, [&](int mt, int, floatx4 v) {
        const int col = nt * 16 + n;
        if (col >= N)
            return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mc * 64 + 16 * mt + 4 * g + i;
            if (row < B)
                out[(long long)row * ld + col] = v[i] + residual[(long long)row * ld + col];
        }
    });
}

template <int KW>
__global__ __launch_bounds__(64 * kSplitWaves) void g4_kernel(StepArgs s, LayerWeights L) {
    const ModelDims& m = s.dims;
    const int mc = blockIdx.y, ctx_w = m.H * m.kv_rank;  // attention rows are H*kv_rank wide
    splitk_residual<KW>(AGlb32{s.ctx + (long long)mc * 64 * ctx_w, ctx_w, ctx_w}, L.w_out,
                        m.ctx_pad / 32, m.d_model, s.x, s.res, m.d_pad, mc, s.B);
}

template <int KW>
__global__ __launch_bounds__(64 * kSplitWaves) void g6_kernel(StepArgs s, LayerWeights L) {
    const ModelDims& m = s.dims;
    const int mc = blockIdx.y;
    splitk_residual<KW>(AGlb16{s.u + (long long)mc * 64 * m.ff_pad, m.ff_pad}, L.w_down,
                        m.ff_pad / 32, m.d_model, s.res, s.x, m.d_pad, mc, s.B);
}

// --------------------------------------------------------------------- g5 ----
// RMSNorm(res, ffn_norm) prologue; w_gate_up interleaves 16-column tiles of gate and
// up (tile 2j = gate columns 16j.., tile 2j+1 = up columns 16j..).  One workgroup per
// pair, 4 waves split K, and SwiGLU (ops.cpp:65-77: gate * sigmoid(gate) * up) is
// formed after the reduction.
__device__ __forceinline__ float silu_stable(float x) {
    if (x >= 0.0f)
        return x * (1.0f / (1.0f + expf(-x)));
    const float e = expf(x);
    return x * (e / (1.0f + e));
}

template <int KW>
__global__ __launch_bounds__(256) void g5_kernel(StepArgs s, LayerWeights L) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const ModelDims& m = s.dims;
    const int mc = blockIdx.y, p = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32;
    BPre<2, KW> bw;
    bw.load(L.w_gate_up, 2 * p, 2, KT, wave * KW, lane);
    const int lda = m.d_pad + kLdsPad;
    _Float16* a_s = reinterpret_cast<_Float16*>(smem);
    rmsnorm_rows_to_lds(s.res + (long long)mc * 64 * m.d_pad, m.d_pad, m.d_model, m.d_pad,
                        L.ffn_norm, m.eps, a_s, lda);
    __syncthreads();
    floatx4 acc[4][2];
    zero(acc);
    bw.mma_all(acc, ALds16{a_s, lda}, KT, wave * KW, lane);
    __syncthreads();
    floatx4* part = reinterpret_cast<floatx4*>(smem);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            part[((wave * 4 + mt) * 2 + j) * 64 + lane] = acc[mt][j];
    __syncthreads();
    const int mt = wave, col = p * 16 + n;  // wave v finishes M-tile v (gate and up)
    floatx4 gt = {0, 0, 0, 0}, up = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        gt += part[((w * 4 + mt) * 2 + 0) * 64 + lane];
        up += part[((w * 4 + mt) * 2 + 1) * 64 + lane];
    }
    if (col < m.d_ff)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mc * 64 + 16 * mt + 4 * g + i;
            if (row < s.B)
                s.u[(long long)row * m.ff_pad + col] = F16::from_float(silu_stable(gt[i]) * up[i]);
        }
}

// --------------------------------------------------------------------- g7 ----
// Final RMSNorm + tied logits h . E^T, kG7Tiles tiles per workgroup (4 waves split K);
// each workgroup also leaves, per row, the greedy winner of its columns (strict >, so
// the lowest index wins ties) and whether all of them were finite.
constexpr int kG7Tiles = 4;
constexpr int kG7Cols = kG7Tiles * 16;  // columns per workgroup

template <int KW>
__global__ __launch_bounds__(256) void g7_kernel(StepArgs s) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const ModelDims& m = s.dims;
    const int mc = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32, n_tiles = m.vocab_pad / 16, nt0 = blockIdx.x * kG7Tiles;
    BPre<kG7Tiles, KW> bw;
    bw.load(s.embed, nt0, min(kG7Tiles, n_tiles - nt0), KT, wave * KW, lane);
    const int lda = m.d_pad + kLdsPad;
    _Float16* a_s = reinterpret_cast<_Float16*>(smem);
    rmsnorm_rows_to_lds(s.x + (long long)mc * 64 * m.d_pad, m.d_pad, m.d_model, m.d_pad,
                        s.final_norm, m.eps, a_s, lda);
    __syncthreads();
    floatx4 acc[4][kG7Tiles];
    zero(acc);
    bw.mma_all(acc, ALds16{a_s, lda}, KT, wave * KW, lane);
    __syncthreads();
    __shared__ float best_v[kG7Tiles][64];
    __shared__ int best_c[kG7Tiles][64], all_finite[kG7Tiles][64];
    // wave v reduces tile j = v for every M-tile (4 waves, 4 tiles)
    splitk_reduce<kG7Tiles, 4>(acc, reinterpret_cast<floatx4*>(smem), [&](int mt, int j, floatx4 v) {
        const int col = (nt0 + j) * 16 + n;
        const bool valid = nt0 + j < n_tiles && col < m.vocab;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 16 * mt + 4 * g + i, row = mc * 64 + r;
            if (valid && row < s.B)
                s.logits[(long long)row * m.vocab + col] = v[i];
            float bv = valid ? v[i] : -INFINITY;
            int bc = valid ? col : 0x7fffffff, fin = !valid || isfinite(v[i]) ? 1 : 0;
            // the 16 lanes of a row hold 16 columns: larger value, then lower column
            for (int off = 8; off > 0; off >>= 1) {
                const float ov = __shfl_xor(bv, off, 16);
                const int oc = __shfl_xor(bc, off, 16);
                fin &= __shfl_xor(fin, off, 16);
                if (oc != 0x7fffffff && (bc == 0x7fffffff || ov > bv || (ov == bv && oc < bc))) {
                    bv = ov;
                    bc = oc;
                }
            }
            if (n == 0) {
                best_v[j][r] = bv;
                best_c[j][r] = bc;
                all_finite[j][r] = fin;
            }
        }
    });
    __syncthreads();
    if (threadIdx.x < 64) {
        const int r = threadIdx.x, row = mc * 64 + r;
        float bv = -INFINITY;
        int bc = 0x7fffffff, fin = 1;
        for (int j = 0; j < kG7Tiles; ++j) {  // tiles in increasing column order
            fin &= all_finite[j][r];
            const int oc = best_c[j][r];
            if (oc != 0x7fffffff && (bc == 0x7fffffff || best_v[j][r] > bv)) {
                bv = best_v[j][r];
                bc = oc;
            }
        }
        if (row < s.B) {
            const long long idx = (long long)row * gridDim.x + blockIdx.x;
            s.arg_v[idx] = bv;
            s.arg_c[idx] = fin ? bc : -1;
        }
    }
}

// Greedy token per row (inference.cpp:363-373 with no penalty or bans): the lowest
// column among the maxima; -1 when a logit is not finite (numerical_error).
__global__ __launch_bounds__(64) void argmax_kernel(StepArgs s, int parts) {
    const int row = blockIdx.x;
    float bv = -INFINITY;
    int bc = 0x7fffffff, bad = 0;
    for (int p = threadIdx.x; p < parts; p += 64) {  // parts cover increasing columns
        const float v = s.arg_v[(long long)row * parts + p];
        const int c = s.arg_c[(long long)row * parts + p];
        if (c < 0)
            bad = 1;
        else if (c != 0x7fffffff && (bc == 0x7fffffff || v > bv)) {
            bv = v;
            bc = c;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oc = __shfl_xor(bc, off, 64);
        bad |= __shfl_xor(bad, off, 64);
        if (oc != 0x7fffffff && (bc == 0x7fffffff || ov > bv || (ov == bv && oc < bc))) {
            bv = ov;
            bc = oc;
        }
    }
    if (threadIdx.x == 0)
        s.next_tokens[row] = bad || bc == 0x7fffffff ? -1 : bc;
}

}  // namespace

// ------------------------------------------------------------------ launches ----
namespace {
// k-steps per wave rounded up to a compiled variant
int kw_variant(int ksteps) { return ksteps <= 1 ? 1 : ksteps <= 2 ? 2 : ksteps <= 4 ? 4 : 8; }

template <template <int> class K>
struct Dummy;
}  // namespace

size_t g1_lds_bytes(const ModelDims& m) {
    const size_t a = 64 * (size_t)(m.d_pad + kLdsPad) * 2;
    const size_t part = 4 * 4 * 64 * 16;  // split-K partials alias the A tile
    return a > part ? a : part;
}
size_t g23_lds_bytes(const ModelDims& m) {
    return 64 * (size_t)(m.q_pad + kLdsPad) * 2 + 64 * (size_t)(m.nope_pad + kLdsPad) * 2;
}
size_t dpad_lds_bytes(const ModelDims& m) {
    const size_t a = 64 * (size_t)(m.d_pad + kLdsPad) * 2;
    const size_t part = 4 * 4 * kG7Tiles * 64 * 16;  // g7 (g5: 4*4*2*64*16)
    return a > part ? a : part;
}

int g7_parts(const ModelDims& m) { return (m.vocab_pad / 16 + kG7Tiles - 1) / kG7Tiles; }

#define MLA_KW_DISPATCH(kw, KERNEL, ...)                                                        \
    switch (kw) {                                                                                \
    case 1: hipLaunchKernelGGL(KERNEL<1>, __VA_ARGS__); break;                                   \
    case 2: hipLaunchKernelGGL(KERNEL<2>, __VA_ARGS__); break;                                   \
    case 4: hipLaunchKernelGGL(KERNEL<4>, __VA_ARGS__); break;                                   \
    default: hipLaunchKernelGGL(KERNEL<8>, __VA_ARGS__); break;                                  \
    }

// Kernels whose dynamic LDS can exceed 64 KB.
hipError_t model_kernel_attributes() {
    const int bytes = 160 * 1024 - 16 * 1024;
    const void* ks[] = {
        reinterpret_cast<const void*>(&g1_kernel<1>), reinterpret_cast<const void*>(&g1_kernel<2>),
        reinterpret_cast<const void*>(&g1_kernel<4>), reinterpret_cast<const void*>(&g1_kernel<8>),
        reinterpret_cast<const void*>(&g5_kernel<1>), reinterpret_cast<const void*>(&g5_kernel<2>),
        reinterpret_cast<const void*>(&g5_kernel<4>), reinterpret_cast<const void*>(&g5_kernel<8>),
        reinterpret_cast<const void*>(&g7_kernel<1>), reinterpret_cast<const void*>(&g7_kernel<2>),
        reinterpret_cast<const void*>(&g7_kernel<4>), reinterpret_cast<const void*>(&g7_kernel<8>)};
    for (const void* k : ks) {
        const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

hipError_t launch_embed(const StepArgs& s, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3(s.m_pad), dim3(256), 0, st, s);
    return hipGetLastError();
}

hipError_t launch_layer_pre(const StepArgs& s, const LayerWeights& w, uint16_t* pool,
                            hipStream_t st) {
    const ModelDims& m = s.dims;
    const int chunks = s.m_pad / 64;
    const int g1_tiles = (m.q_pad + m.kvw_pad) / 16;
    MLA_KW_DISPATCH(kw_variant((m.d_pad / 32 + 3) / 4), g1_kernel, dim3(g1_tiles, chunks),
                    dim3(256), g1_lds_bytes(m), st, s, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    const int kwq = kw_variant(m.q_pad / 32), kwu = kw_variant(m.nope_pad / 32);
    const dim3 grid(m.H + 1, chunks);
    const size_t lds = g23_lds_bytes(m);
    if (kwq <= 4 && kwu <= 2)
        hipLaunchKernelGGL((g23_kernel<4, 2>), grid, dim3(256), lds, st, s, w, pool);
    else if (kwq <= 8 && kwu <= 2)
        hipLaunchKernelGGL((g23_kernel<8, 2>), grid, dim3(256), lds, st, s, w, pool);
    else
        hipLaunchKernelGGL((g23_kernel<8, 4>), grid, dim3(256), lds, st, s, w, pool);
    return hipGetLastError();
}

hipError_t launch_layer_post(const StepArgs& s, const LayerWeights& w, hipStream_t st) {
    const ModelDims& m = s.dims;
    const int chunks = s.m_pad / 64;
    const int d_tiles = m.d_pad / 16;
    MLA_KW_DISPATCH(kw_variant((m.ctx_pad / 32 + kSplitWaves - 1) / kSplitWaves), g4_kernel,
                    dim3(d_tiles, chunks), dim3(64 * kSplitWaves), 0, st, s, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    MLA_KW_DISPATCH(kw_variant((m.d_pad / 32 + 3) / 4), g5_kernel, dim3(m.ff_pad / 16, chunks),
                    dim3(256), dpad_lds_bytes(m), st, s, w);
    e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    MLA_KW_DISPATCH(kw_variant((m.ff_pad / 32 + kSplitWaves - 1) / kSplitWaves), g6_kernel,
                    dim3(d_tiles, chunks), dim3(64 * kSplitWaves), 0, st, s, w);
    return hipGetLastError();
}

hipError_t launch_logits(const StepArgs& s, hipStream_t st) {
    const ModelDims& m = s.dims;
    const int parts = g7_parts(m);
    MLA_KW_DISPATCH(kw_variant((m.d_pad / 32 + 3) / 4), g7_kernel, dim3(parts, s.m_pad / 64),
                    dim3(256), dpad_lds_bytes(m), st, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    if (s.B > 0)
        hipLaunchKernelGGL(argmax_kernel, dim3(s.B), dim3(64), 0, st, s, parts);
    return hipGetLastError();
}

}  // namespace mla
