// Batched MLA decode step on gfx950: everything of CpuDecoder::decode around the
// attention (src/infer/inference.cpp:76-173) for B sessions at once, one new token
// each.
//
// Per layer, in launch order (y = x.W for every projection, as in ops.cpp:8-18):
//   g1_kernel   RMSNorm(x, attn_norm) . [w_dq | w_dkv] -> q part (cq) and kv part (kvraw)
//   g23_kernel  per head: q_norm -> w_uq -> RoPE of the rope columns (q_rope, stored in
//               the cache dtype) -> absorption q_latent = W_uk_h^T q_nope
//               (inference.cpp:85-90,121-124; the MPS graph keeps q_latent in the
//               storage dtype, mps_backend.mm:561); four more workgroups kv_norm the
//               latent, RoPE the key, round both and append them to the paged cache
//               (inference.cpp:91-103)
//   (decode attention partials + merge: decode.hip)
//   g4_kernel   latent_ctx [H*kv_rank] . out_proj + x  (inference.cpp:154-156; out_proj
//               is the combined W_uv.W_o of prepare_projections, inference.cpp:28-46)
//   g5_kernel   RMSNorm(ffn_norm) -> [w_gate | w_up] -> SwiGLU  (inference.cpp:157-161)
//   g6_kernel   . w_down + residual  (inference.cpp:162-165)
// Per step: embed_kernel (token rows, RoPE rows), g7_kernel (final RMSNorm, tied logits
// h.E^T, inference.cpp:166-168, with a per-workgroup greedy partial) and argmax_kernel
// (sample_token's greedy rule, inference.cpp:345-380).
//
// Every projection is a skinny GEMM on v_mfma_f32_16x16x32_f16 (fp16 operands, fp32
// accumulation).  A workgroup owns 16 rows (64 for the logits) and one to four 16-column
// output tiles; its 8 waves split K.  Each wave fetches its weight tiles (fp16, TILED:
// each wave load reads 1 KB contiguously) and its slice of the activation rows into
// registers at kernel start, so a GEMM pays about one memory round trip, and the
// partial sums meet in LDS.  Small row blocks keep the bytes each CU must pull low:
// the load phase, not the arithmetic, is what these kernels wait on.
//
// RMSNorm (ops.cpp:33-45) is RMSNorm(x)_k = x_k * inv * w_k with inv = 1/rms(x) per row,
// so RMSNorm(x).W = inv * ((x o w).W): the kernel that writes an activation x also
// writes (x o w) in fp16 for the consumer's A operand (w = the norm weight of the next
// consumer) and, per row and 16-column tile, the sum of squares of x; the consumer adds
// those partials (in a fixed order) into inv and scales its output rows by it.
#include "mla_common.hpp"
#include "mla_internal.hpp"
#include "mla_model.hpp"

#include <cmath>

namespace mla {
namespace {

using V8 = half8;
constexpr int kWaves = 8;  // waves per GEMM workgroup
constexpr int kLdsPad = 8;

__device__ __forceinline__ floatx4 mma(V8 a, V8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ V8 to_half8(floatx4 a, floatx4 b) {
    return V8{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
              (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
}

// Sum over the 16 lanes of an MFMA output row group (lanes with equal g hold the same
// rows, one column each).
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int off = 8; off > 0; off >>= 1)
        v += __shfl_xor(v, off, 16);
    return v;
}

template <int MT, int NT>
__device__ __forceinline__ void zero(floatx4 (&acc)[MT][NT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < NT; ++j)
            acc[mt][j] = floatx4{0, 0, 0, 0};
}

// ---- operand prefetch ----------------------------------------------------------
// A wave's k-steps are kt0, kt0 + ks, kt0 + 2ks, ... (KW of them; kt0 = the wave's
// K group and ks = the number of K groups, so uneven K spreads evenly); k-steps past KT
// load zeros and add nothing.
//
// Weight (B operand) registers of one wave: its k-steps of tiles [nt0, nt0+NT); tiles
// past `ntv` stay zero.  Tile (nt, kt) of a tiled W (mla_model.hpp) is 512 contiguous
// fp16 words; lane l reads 16 bytes at 8l.
template <int NT, int KW>
struct BPre {
    V8 b[KW][NT];
    __device__ __forceinline__ void load(const uint16_t* w, int nt0, int ntv, int KT, int kt0,
                                         int ks, int lane) {
#pragma unroll
        for (int kk = 0; kk < KW; ++kk)
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int kt = kt0 + kk * ks;
                b[kk][j] = V8{};
                if (kt < KT && j < ntv)
                    b[kk][j] = *reinterpret_cast<const V8*>(
                        w + ((long long)(nt0 + j) * KT + kt) * 512 + lane * 8);
            }
    }
};

// Activation (A operand) registers: lane (g, n) needs rows 16mt + n (mt < MT) and
// columns 32kt + 8g .. +7 of each of its k-steps.
template <int KW, int MT>
struct APre16 {  // fp16 rows, zero-padded to KT*32 columns
    V8 x[KW][MT];
    __device__ __forceinline__ void load(const uint16_t* X, int ld, int KT, int kt0, int ks,
                                         int lane) {
        const int g = lane >> 4, n = lane & 15;
#pragma unroll
        for (int kk = 0; kk < KW; ++kk)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int kt = kt0 + kk * ks;
                x[kk][mt] = V8{};
                if (kt < KT)
                    x[kk][mt] = *reinterpret_cast<const V8*>(X + (long long)(16 * mt + n) * ld +
                                                             32 * kt + 8 * g);
            }
    }
};
template <int KW, int MT>
struct AHalf32 {  // fp32 rows (K % 8 == 0; columns past K read as zero), rounded to fp16
    V8 x[KW][MT];
    __device__ __forceinline__ void load(const float* X, int ld, int K, int KT, int kt0, int ks,
                                         int lane) {
        const int g = lane >> 4, n = lane & 15;
#pragma unroll
        for (int kk = 0; kk < KW; ++kk) {
            const int kt = kt0 + kk * ks;
            const int k = 32 * kt + 8 * g;
            const bool ok = kt < KT && k < K;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                x[kk][mt] = V8{};
                if (ok) {
                    const floatx4* p =
                        reinterpret_cast<const floatx4*>(X + (long long)(16 * mt + n) * ld + k);
                    x[kk][mt] = to_half8(p[0], p[1]);
                }
            }
        }
    }
};

template <int MT, int NT, int KW, typename AOp>
__device__ __forceinline__ void mma_steps(floatx4 (&acc)[MT][NT], const BPre<NT, KW>& b,
                                          AOp aop) {
#pragma unroll
    for (int kk = 0; kk < KW; ++kk)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const V8 a = aop(kk, mt);
#pragma unroll
            for (int j = 0; j < NT; ++j)
                acc[mt][j] = mma(a, b.b[kk][j], acc[mt][j]);
        }
}

// 1/rms of `rows` rows (ops.cpp:33-45: inv = 1/sqrt(mean(x^2) + eps)) from the
// producer's per-tile partial sums of squares (n_tiles <= 64): four threads a row each
// load every fourth tile at once (one round trip), then combine in a fixed order.
// Threads [0, 4*rows) take part; rows is 16 or 64, so they fill whole waves.  Visible
// to the workgroup after its next barrier.
__device__ __forceinline__ void inv_rms_to_lds(const float* ss, int n_tiles, int K, float eps,
                                               int row0, float* inv_s, int rows) {
    const int t = threadIdx.x;
    if (t < 4 * rows) {
        const float* p = ss + (long long)(row0 + (t >> 2)) * n_tiles;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int tile = (t & 3) + 4 * i;
            v[i] = tile < n_tiles ? p[tile] : 0.0f;
        }
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            sum += v[i];
        sum += __shfl_xor(sum, 1, 4);
        sum += __shfl_xor(sum, 2, 4);
        if ((t & 3) == 0)
            inv_s[t >> 2] = 1.0f / sqrtf(sum / (float)K + eps);
    }
}

// Split-K reduction through LDS `part` (kWaves*MT*NTW*64 floatx4).  Wave w computed K
// group w % KG of tiles [(w / KG) * NTW, +NTW); after the barrier wave mt < MT sums all
// K groups of M-tile mt into v[t] for the workgroup's NT = NTW * kWaves / KG tiles
// (lane (g, n): C[16mt + 4g + i][16t + n]); other waves get false.
template <int MT, int NTW, int KG>
__device__ __forceinline__ bool splitk_reduce(floatx4 (&acc)[MT][NTW], floatx4* part, int& mt,
                                              floatx4 (&v)[NTW * (kWaves / KG)]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < NTW; ++j)
            part[((wave * MT + m) * NTW + j) * 64 + lane] = acc[m][j];
    __syncthreads();
    if (wave >= MT)
        return false;
    mt = wave;
#pragma unroll
    for (int ng = 0; ng < kWaves / KG; ++ng)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            floatx4 sum = {0, 0, 0, 0};
#pragma unroll
            for (int kg = 0; kg < KG; ++kg)
                sum += part[(((ng * KG + kg) * MT + mt) * NTW + j) * 64 + lane];
            v[ng * NTW + j] = sum;
        }
    return true;
}

// Per-row sum of squares of this lane group's 16 columns (y holds rows 4g+i of one
// column; columns that do not count add 0), written by lane n == 0 to
// ss[row * n_tiles + tile] for rows < B.
__device__ __forceinline__ void write_ss(floatx4 y, bool col_counts, float* ss, int n_tiles,
                                         int tile, int row0, int B) {
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float q = sum16(col_counts ? y[i] * y[i] : 0.0f);
        const int row = row0 + 4 * g + i;
        if (n == 0 && row < B)
            ss[(long long)row * n_tiles + tile] = q;
    }
}

__device__ __forceinline__ float2 rope_table(const StepArgs& s, int pos, int j2) {
    const ModelDims& m = s.dims;
    pos = min(max(pos, 0), m.max_seq - 1);  // the caller rejects others (inference.cpp:71-75)
    return s.rope_tab[(long long)pos * (m.rope / 2) + j2];
}

// ------------------------------------------------------------------ embed ----
// x[b] = E[token[b]] (fp32), xw[b] = x o attn_norm of layer 0 (fp16), the per-tile sums
// of squares of x, and the (cos, sin) row of b's position for every layer's RoPE; rows
// [B, m_pad) are zeroed.  E is read from its tiled logits layout (K = d_model, N = vocab).
__global__ __launch_bounds__(256) void embed_kernel(StepArgs s, const float* norm0) {
    const int b = blockIdx.x;
    const ModelDims& m = s.dims;
    const int d_tiles = m.d_pad / 16, KT = m.d_pad / 32, half = m.rope / 2;
    int tok = b < s.B ? s.tokens[b] : 0;
    tok = tok < 0 || tok >= m.vocab ? 0 : tok;  // the caller validates tokens
    if ((int)threadIdx.x < half)
        s.rope_rows[(long long)b * half + threadIdx.x] =
            b < s.B ? rope_table(s, s.positions[b], threadIdx.x) : float2{1.0f, 0.0f};
    for (int c0 = 0; c0 < m.d_pad; c0 += 256) {
        const int c = c0 + threadIdx.x;
        float v = 0.0f, w = 0.0f;
        if (b < s.B && c < m.d_model) {
            const long long e = ((long long)(tok >> 4) * KT + (c >> 5)) * 512 +
                                (((c & 31) >> 3) * 16 + (tok & 15)) * 8 + (c & 7);
            v = (float)__builtin_bit_cast(_Float16, s.embed[e]);
            w = norm0[c];
        }
        if (c < m.d_pad) {
            s.x[(long long)b * m.d_pad + c] = v;
            s.xw[(long long)b * m.d_pad + c] = F16::from_float(v * w);
        }
        const float q = sum16(v * v);
        if ((threadIdx.x & 15) == 0 && c < m.d_pad)
            s.ss_x[(long long)b * d_tiles + c / 16] = q;
    }
}

// --------------------------------------------------------------------- g1 ----
// RMSNorm(x, attn_norm) . [w_dq | w_dkv] for 16 rows and one 16-column tile: q columns
// to cqw = cq o q_norm (fp16, with cq's sums of squares for q_norm's inv), kv columns
// to kvraw (fp32, with the sums of squares of the latent columns for kv_norm).
template <int KW>
__global__ __launch_bounds__(64 * kWaves) void g1_kernel(StepArgs s, LayerWeights L) {
    constexpr int MT = 1, KG = kWaves;
    __shared__ __attribute__((aligned(16))) floatx4 part[kWaves * MT * 64];
    __shared__ float inv_s[16 * MT];
    const ModelDims& m = s.dims;
    const int nt = blockIdx.x, row0 = blockIdx.y * 16 * MT;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32, col = nt * 16 + n;
    inv_rms_to_lds(s.ss_x, m.d_pad / 16, m.d_model, m.eps, row0, inv_s, 16 * MT);
    BPre<1, KW> bw;
    bw.load(L.w_dq_dkv, nt, 1, KT, wave, KG, lane);
    APre16<KW, MT> a;
    a.load(s.xw + (long long)row0 * m.d_pad, m.d_pad, KT, wave, KG, lane);
    const float qn = col < m.q_rank ? L.q_norm[col] : 0.0f;
    floatx4 acc[MT][1];
    zero(acc);
    mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
    int mt;
    floatx4 v[1];
    if (!splitk_reduce<MT, 1, KG>(acc, part, mt, v))
        return;
    const int q_tiles = m.q_pad / 16, r0 = row0 + 16 * mt;
    floatx4 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long r = r0 + 4 * g + i;
        y[i] = v[0][i] * inv_s[16 * mt + 4 * g + i];
        if (col < m.q_pad)
            s.cqw[r * m.q_pad + col] = F16::from_float(y[i] * qn);
        else
            s.kvraw[r * m.kvw_pad + (col - m.q_pad)] = y[i];
    }
    if (nt < q_tiles)
        write_ss(y, true, s.ss_q, q_tiles, nt, r0, s.B);
    else if ((nt - q_tiles) * 16 < m.kv_rank)
        write_ss(y, col - m.q_pad < m.kv_rank, s.ss_kv, m.kv_pad / 16, nt - q_tiles, r0, s.B);
}

// -------------------------------------------------------------------- g23 ----
// Workgroups h < H (4 waves, 64 rows): q_h = q_norm(cq) . w_uq[:, head columns], the
// waves splitting K over all of the head's tiles; RoPE of the rope columns (pairs read
// from LDS); q_rope stored in the cache dtype; q_latent_h = q_h[:, :nope] . W_uk_h^T.
// Workgroups H ..: kv_norm of the latent, RoPE of the key, rounding, append.
constexpr int kQTiles = 4;                        // q tiles of a head (qk <= 64)
constexpr int kRopeItems = 64 * 32 / 256;         // RoPE pairs a thread (rope <= 64)
constexpr int kKvWGs = 4, kKvRows = 64 / kKvWGs;  // kv-append workgroups per 64 rows
constexpr int kKvItems = (kKvRows * (128 + 32) + 255) / 256;  // kv_rank <= 128, rope <= 64

template <int KWQ, int KWU>
__global__ __launch_bounds__(256) void g23_kernel(StepArgs s, LayerWeights L, uint16_t* pool) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const ModelDims& m = s.dims;
    const int h = blockIdx.x, mc = blockIdx.y, row0 = mc * 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int half = m.rope / 2;
    __shared__ float inv_s[64];
    if (h >= m.H) {  // ---- kv append: kKvRows rows per workgroup, elementwise ----
        const int r0 = row0 + (h - m.H) * kKvRows;
        inv_rms_to_lds(s.ss_kv, m.kv_pad / 16, m.kv_rank, m.eps, r0, inv_s, kKvRows);
        const bool tiled = page_tiled(m.page_size, m.kv_rank, m.rope);
        const int width = m.kv_rank + m.rope;
        const int per_row = m.kv_rank + half;  // latent columns, then rope pairs
        // every load in flight first (per_row <= 160: kKvItems items a thread), then the
        // rounded stores
        float va[kKvItems], vb[kKvItems], wn[kKvItems];
        float2 cs[kKvItems];
        int slot[kKvItems];
#pragma unroll
        for (int i = 0; i < kKvItems; ++i) {
            const int e = threadIdx.x + 256 * i, r = e / per_row, c = e % per_row;
            const int row = r0 + r;
            va[i] = vb[i] = wn[i] = 0.0f;
            cs[i] = float2{1.0f, 0.0f};
            slot[i] = -1;
            if (r < kKvRows && row < s.B) {
                slot[i] = s.slot_mapping[row];
                const float* kr = s.kvraw + (long long)row * m.kvw_pad;
                if (c < m.kv_rank) {
                    va[i] = kr[c];
                    wn[i] = L.kv_norm[c];
                } else {
                    const int j2 = c - m.kv_rank;
                    va[i] = kr[m.kv_rank + 2 * j2];
                    vb[i] = kr[m.kv_rank + 2 * j2 + 1];
                    cs[i] = s.rope_rows[(long long)row * half + j2];
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kKvItems; ++i) {
            const int e = threadIdx.x + 256 * i, r = e / per_row, c = e % per_row;
            const int page = slot[i] / m.page_size, off = slot[i] % m.page_size;
            if (slot[i] < 0 || page >= s.num_pool_pages)
                continue;
            uint16_t* base = pool + (long long)page * m.page_size * width;
            if (c < m.kv_rank) {
                base[latent_word(tiled, off, c, m.page_size, m.kv_rank)] =
                    F16::from_float(va[i] * inv_s[r] * wn[i]);
            } else {
                const int jp = 2 * (c - m.kv_rank);
                base[rope_word(tiled, off, jp, m.page_size, m.kv_rank, m.rope)] =
                    F16::from_float(va[i] * cs[i].x - vb[i] * cs[i].y);
                base[rope_word(tiled, off, jp + 1, m.page_size, m.kv_rank, m.rope)] =
                    F16::from_float(va[i] * cs[i].y + vb[i] * cs[i].x);
            }
        }
        return;
    }
    // ---- one head: q_h over the head's tiles, 4 waves splitting K ----
    const int qk_tiles = m.qk_pad / 16, KTQ = m.q_pad / 32;
    const int kv_tiles = m.kv_pad / 16, KTU = m.nope_pad / 32;
    inv_rms_to_lds(s.ss_q, m.q_pad / 16, m.q_rank, m.eps, row0, inv_s, 64);
    BPre<kQTiles, KWQ> bq;
    bq.load(L.w_uq, h * qk_tiles, qk_tiles, KTQ, wave, 4, lane);
    BPre<2, KWU> bu;  // this wave's two latent tiles of the absorption, whole K
    bu.load(L.w_uk + (long long)h * kv_tiles * KTU * 512, 2 * wave, min(2, kv_tiles - 2 * wave),
            KTU, 0, 1, lane);
    APre16<KWQ, 4> a;
    a.load(s.cqw + (long long)row0 * m.q_pad, m.q_pad, KTQ, wave, 4, lane);
    float2 cs[kRopeItems];  // RoPE rows of this thread's pairs
#pragma unroll
    for (int i = 0; i < kRopeItems; ++i) {
        const int e = threadIdx.x + 256 * i, r = e / max(half, 1);
        cs[i] = e < 64 * half ? s.rope_rows[(long long)(row0 + r) * half + e % half]
                              : float2{1.0f, 0.0f};
    }
    floatx4 acc[4][kQTiles];
    zero(acc);
    mma_steps(acc, bq, [&](int kk, int mt) { return a.x[kk][mt]; });
    // reduce the 4 waves' partials: wave w finishes M-tile w, all of the head's tiles
    floatx4* part = reinterpret_cast<floatx4*>(smem);  // [4 waves][4 mt][kQTiles][64]
    float* qf = reinterpret_cast<float*>(smem);         // then q_h fp32 [64][qk_pad + 4]
    const int ldf = m.qk_pad + 4;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < kQTiles; ++j)
            part[((wave * 4 + mt) * kQTiles + j) * 64 + lane] = acc[mt][j];
    __syncthreads();
    floatx4 q[kQTiles];
#pragma unroll
    for (int j = 0; j < kQTiles; ++j) {
        q[j] = floatx4{0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < 4; ++w)
            q[j] += part[((w * 4 + wave) * kQTiles + j) * 64 + lane];
    }
    __syncthreads();  // partials consumed: the LDS now holds q_h in fp32
#pragma unroll
    for (int j = 0; j < kQTiles; ++j)
        if (j < qk_tiles)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * wave + 4 * g + i;
                qf[r * ldf + 16 * j + n] = q[j][i] * inv_s[r];
            }
    __syncthreads();
    // RoPE + q_rope; q_nope to the fp16 A tile of the absorption
    const int ldq = m.nope_pad + kLdsPad;
    _Float16* q_s = reinterpret_cast<_Float16*>(smem + 64 * ldf * sizeof(float));
    for (int e = threadIdx.x; e < 64 * m.nope_pad; e += 256) {
        const int r = e / m.nope_pad, c = e % m.nope_pad;
        q_s[r * ldq + c] = (_Float16)(c < m.nope ? qf[r * ldf + c] : 0.0f);
    }
#pragma unroll
    for (int i = 0; i < kRopeItems; ++i) {
        const int e = threadIdx.x + 256 * i, r = e / max(half, 1), jp = 2 * (e % max(half, 1));
        const int row = row0 + r;
        if (e < 64 * half && row < s.B) {
            const float a0 = qf[r * ldf + m.nope + jp], a1 = qf[r * ldf + m.nope + jp + 1];
            uint16_t* qr = s.q_rope + ((long long)row * m.H + h) * m.rope;
            qr[jp] = F16::from_float(a0 * cs[i].x - a1 * cs[i].y);
            qr[jp + 1] = F16::from_float(a0 * cs[i].y + a1 * cs[i].x);
        }
    }
    __syncthreads();
    // q_latent_h = q_h[:, :nope] . W_uk_h^T  (K = nope_pad, N = kv_pad; two tiles a wave)
    if (2 * wave < kv_tiles) {
        floatx4 acc2[4][2];
        zero(acc2);
        mma_steps(acc2, bu, [&](int kk, int mt) {  // k-steps past nope_pad: zeros, not LDS
            return kk < KTU ? *reinterpret_cast<const V8*>(q_s + (16 * mt + n) * ldq + 32 * kk +
                                                           8 * g)
                            : V8{};
        });
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = (2 * wave + j) * 16 + n;
            if (c < m.kv_rank)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = row0 + 16 * mt + 4 * g + i;
                        if (row < s.B)
                            s.q_latent[((long long)row * m.H + h) * m.kv_rank + c] =
                                F16::from_float(acc2[mt][j][i]);
                    }
        }
    }
}

// ----------------------------------------------------------- g4 and g6 ----
// y = A . W + residual for 16 rows and one 16-column tile (8 waves split K): y to `out`
// (fp32), y o wnorm to `outw` (fp16, the next consumer's normalised A operand), and
// y's per-tile sums of squares.  The residual and norm columns are fetched with the
// operands.
template <int KW, typename ALoad>
__device__ __forceinline__ void splitk_residual(ALoad&& aload, const uint16_t* w, int KT, int N,
                                                const float* residual, const float* wnorm,
                                                float* out, uint16_t* outw, float* ss,
                                                int n_tiles, int ld, int row0, int B) {
    __shared__ __attribute__((aligned(16))) floatx4 part[kWaves * 64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int nt = blockIdx.x, col = nt * 16 + n;
    BPre<1, KW> bw;
    bw.load(w, nt, 1, KT, wave, kWaves, lane);
    floatx4 res = {0, 0, 0, 0};
    float wn = 0.0f;
    if (wave == 0 && col < N) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            res[i] = residual[(long long)(row0 + 4 * g + i) * ld + col];
        wn = wnorm[col];
    }
    floatx4 acc[1][1];
    zero(acc);
    aload(acc, bw, wave, lane);
    int mt;
    floatx4 v[1];
    if (!splitk_reduce<1, 1, kWaves>(acc, part, mt, v))
        return;
    floatx4 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long row = row0 + 4 * g + i;
        y[i] = col < N ? v[0][i] + res[i] : 0.0f;
        if (row < B && col < N) {
            out[row * ld + col] = y[i];
            outw[row * ld + col] = F16::from_float(y[i] * wn);
        }
    }
    write_ss(y, col < N, ss, n_tiles, nt, row0, B);
}

template <int KW>
__global__ __launch_bounds__(64 * kWaves) void g4_kernel(StepArgs s, LayerWeights L) {
    const ModelDims& m = s.dims;
    const int row0 = blockIdx.y * 16, ctx_w = m.H * m.kv_rank;  // attention rows: H*kv_rank
    const int KT = m.ctx_pad / 32;
    splitk_residual<KW>(
        [&](floatx4(&acc)[1][1], const BPre<1, KW>& bw, int kt0, int lane) {
            AHalf32<KW, 1> a;
            a.load(s.ctx + (long long)row0 * ctx_w, ctx_w, ctx_w, KT, kt0, kWaves, lane);
            mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
        },
        L.w_out, KT, m.d_model, s.x, L.ffn_norm, s.res, s.resw, s.ss_res, m.d_pad / 16, m.d_pad,
        row0, s.B);
}

// next_norm: the norm weight of x's next consumer (attn_norm of the next layer, or
// final_norm after the last layer).
template <int KW>
__global__ __launch_bounds__(64 * kWaves) void g6_kernel(StepArgs s, LayerWeights L,
                                                         const float* next_norm) {
    const ModelDims& m = s.dims;
    const int row0 = blockIdx.y * 16, KT = m.ff_pad / 32;
    splitk_residual<KW>(
        [&](floatx4(&acc)[1][1], const BPre<1, KW>& bw, int kt0, int lane) {
            APre16<KW, 1> a;
            a.load(s.u + (long long)row0 * m.ff_pad, m.ff_pad, KT, kt0, kWaves, lane);
            mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
        },
        L.w_down, KT, m.d_model, s.res, next_norm, s.x, s.xw, s.ss_x, m.d_pad / 16, m.d_pad,
        row0, s.B);
}

// --------------------------------------------------------------------- g5 ----
// RMSNorm(res, ffn_norm) . [w_gate | w_up] for 16 rows: w_gate_up interleaves 16-column
// tiles of gate and up (tile 2j = gate columns 16j.., tile 2j+1 = up columns 16j..); one
// pair per workgroup, 8 waves split K, then SwiGLU (ops.cpp:65-77: gate*sigmoid(gate)*up).
__device__ __forceinline__ float silu_stable(float x) {
    if (x >= 0.0f)
        return x * (1.0f / (1.0f + expf(-x)));
    const float e = expf(x);
    return x * (e / (1.0f + e));
}

template <int KW>
__global__ __launch_bounds__(64 * kWaves) void g5_kernel(StepArgs s, LayerWeights L) {
    __shared__ __attribute__((aligned(16))) floatx4 part[kWaves * 2 * 64];
    __shared__ float inv_s[16];
    const ModelDims& m = s.dims;
    const int row0 = blockIdx.y * 16, p = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32;
    inv_rms_to_lds(s.ss_res, m.d_pad / 16, m.d_model, m.eps, row0, inv_s, 16);
    BPre<2, KW> bw;
    bw.load(L.w_gate_up, 2 * p, 2, KT, wave, kWaves, lane);
    APre16<KW, 1> a;
    a.load(s.resw + (long long)row0 * m.d_pad, m.d_pad, KT, wave, kWaves, lane);
    floatx4 acc[1][2];
    zero(acc);
    mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
    int mt;
    floatx4 v[2];
    if (!splitk_reduce<1, 2, kWaves>(acc, part, mt, v))
        return;
    const int col = p * 16 + n;
    if (col < m.d_ff)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + 4 * g + i;
            const float inv = inv_s[4 * g + i];
            if (row < s.B)
                s.u[(long long)row * m.ff_pad + col] =
                    F16::from_float(silu_stable(v[0][i] * inv) * (v[1][i] * inv));
        }
}

// --------------------------------------------------------------------- g7 ----
// Final RMSNorm + tied logits h . E^T for 64 rows and four 16-column tiles per
// workgroup (the waves split K four ways and the tiles two ways); each workgroup also
// leaves, per row, the greedy winner of its 64 columns (strict >, so the lowest index
// wins ties) and whether all of them were finite.
constexpr int kG7Tiles = 4, kG7KG = 4;

template <int KW>
__global__ __launch_bounds__(64 * kWaves) void g7_kernel(StepArgs s) {
    constexpr int NTW = kG7Tiles / (kWaves / kG7KG);
    __shared__ __attribute__((aligned(16))) floatx4 part[kWaves * 4 * NTW * 64];
    __shared__ float inv_s[64];
    const ModelDims& m = s.dims;
    const int row0 = blockIdx.y * 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32, kg = wave % kG7KG, ng = wave / kG7KG;
    const int n_tiles = m.vocab_pad / 16, nt0 = blockIdx.x * kG7Tiles;
    inv_rms_to_lds(s.ss_x, m.d_pad / 16, m.d_model, m.eps, row0, inv_s, 64);
    BPre<NTW, KW> bw;
    bw.load(s.embed, nt0 + ng * NTW, min(NTW, n_tiles - nt0 - ng * NTW), KT, kg, kG7KG, lane);
    APre16<KW, 4> a;
    a.load(s.xw + (long long)row0 * m.d_pad, m.d_pad, KT, kg, kG7KG, lane);
    floatx4 acc[4][NTW];
    zero(acc);
    mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
    int mt;
    floatx4 v[kG7Tiles];
    if (!splitk_reduce<4, NTW, kG7KG>(acc, part, mt, v))
        return;
    float bv[4], fin[4];
    int bc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        bv[i] = -INFINITY;
        bc[i] = 0x7fffffff;
        fin[i] = 1.0f;
    }
#pragma unroll
    for (int j = 0; j < kG7Tiles; ++j) {  // tiles in increasing column order
        const int col = (nt0 + j) * 16 + n;
        const bool valid = nt0 + j < n_tiles && col < m.vocab;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + 16 * mt + 4 * g + i;
            const float y = v[j][i] * inv_s[16 * mt + 4 * g + i];
            if (valid && row < s.B)
                s.logits[(long long)row * m.vocab + col] = y;
            if (valid && !isfinite(y))
                fin[i] = 0.0f;
            if (valid && (bc[i] == 0x7fffffff || y > bv[i])) {  // strict >: lowest column
                bv[i] = y;
                bc[i] = col;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // the 16 lanes of a row hold 16 columns each: larger value, then lower column
        for (int off = 8; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv[i], off, 16);
            const int oc = __shfl_xor(bc[i], off, 16);
            fin[i] = fminf(fin[i], __shfl_xor(fin[i], off, 16));
            if (oc != 0x7fffffff &&
                (bc[i] == 0x7fffffff || ov > bv[i] || (ov == bv[i] && oc < bc[i]))) {
                bv[i] = ov;
                bc[i] = oc;
            }
        }
        const int row = row0 + 16 * mt + 4 * g + i;
        if (n == 0 && row < s.B) {
            const long long idx = (long long)row * gridDim.x + blockIdx.x;
            s.arg_v[idx] = bv[i];
            s.arg_c[idx] = fin[i] > 0.0f ? bc[i] : -1;
        }
    }
}

// Last row of each session (cu_q[b+1] - 1) to row b of the logits operands: the
// normalised activation xw (fp16) and its per-tile sums of squares.  The reference
// returns the logits of a prefill's last position only (inference.cpp:64-66).  Rows
// [B, m_pad) are zeroed.
__global__ __launch_bounds__(256) void gather_last_kernel(StepArgs s, int B, const int32_t* cu_q,
                                                          uint16_t* xw_out, float* ss_out) {
    const ModelDims& m = s.dims;
    const int b = blockIdx.x, d_tiles = m.d_pad / 16;
    const int src = b < B ? cu_q[b + 1] - 1 : -1;
    for (int c = threadIdx.x; c < m.d_pad; c += 256)
        xw_out[(long long)b * m.d_pad + c] = src >= 0 ? s.xw[(long long)src * m.d_pad + c] : 0;
    for (int c = threadIdx.x; c < d_tiles; c += 256)
        ss_out[(long long)b * d_tiles + c] = src >= 0 ? s.ss_x[(long long)src * d_tiles + c] : 0.0f;
}

// Greedy token per row (inference.cpp:363-373 with no penalty or bans): the lowest
// column among the maxima; -1 when a logit is not finite (numerical_error).  256
// threads load up to four partials each at once (parts <= 1024).
constexpr int kArgItems = 4;

__global__ __launch_bounds__(256) void argmax_kernel(StepArgs s, int parts) {
    __shared__ float sv[4];
    __shared__ int sc[4], sbad[4];
    const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float pv[kArgItems];
    int pc[kArgItems];
#pragma unroll
    for (int i = 0; i < kArgItems; ++i) {
        const int p = threadIdx.x + 256 * i;
        pv[i] = -INFINITY;
        pc[i] = 0x7fffffff;
        if (p < parts) {
            pv[i] = s.arg_v[(long long)row * parts + p];
            pc[i] = s.arg_c[(long long)row * parts + p];
        }
    }
    float bv = -INFINITY;
    int bc = 0x7fffffff, bad = 0;
#pragma unroll
    for (int i = 0; i < kArgItems; ++i) {  // increasing columns
        if (pc[i] < 0)
            bad = 1;
        else if (pc[i] != 0x7fffffff && (bc == 0x7fffffff || pv[i] > bv)) {
            bv = pv[i];
            bc = pc[i];
        }
    }
    auto better = [](float ov, int oc, float v, int c) {
        return oc != 0x7fffffff && (c == 0x7fffffff || ov > v || (ov == v && oc < c));
    };
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oc = __shfl_xor(bc, off, 64);
        bad |= __shfl_xor(bad, off, 64);
        if (better(ov, oc, bv, bc)) {
            bv = ov;
            bc = oc;
        }
    }
    if (lane == 0) {
        sv[wave] = bv;
        sc[wave] = bc;
        sbad[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            bad |= sbad[w];
            if (better(sv[w], sc[w], bv, bc)) {
                bv = sv[w];
                bc = sc[w];
            }
        }
        s.next_tokens[row] = bad || bc == 0x7fffffff ? -1 : bc;
    }
}

// k-steps per wave, rounded up to a compiled variant
int kw_variant(int ksteps) {
    return ksteps <= 1 ? 1 : ksteps <= 2 ? 2 : ksteps <= 3 ? 3 : ksteps <= 4 ? 4 : ksteps <= 6 ? 6 : 8;
}
int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace

// ------------------------------------------------------------------ launches ----
size_t g23_lds_bytes(const ModelDims& m) {
    const size_t part = 4 * 4 * kQTiles * 64 * sizeof(floatx4);
    const size_t q = 64 * (size_t)(m.qk_pad + 4) * 4 + 64 * (size_t)(m.nope_pad + kLdsPad) * 2;
    return part > q ? part : q;
}

int g7_parts(const ModelDims& m) { return ceil_div(m.vocab_pad / 16, kG7Tiles); }

#define MLA_KW_DISPATCH(kw, KERNEL, ...)                                                        \
    switch (kw) {                                                                                \
    case 1: hipLaunchKernelGGL(KERNEL<1>, __VA_ARGS__); break;                                   \
    case 2: hipLaunchKernelGGL(KERNEL<2>, __VA_ARGS__); break;                                   \
    case 3: hipLaunchKernelGGL(KERNEL<3>, __VA_ARGS__); break;                                   \
    case 4: hipLaunchKernelGGL(KERNEL<4>, __VA_ARGS__); break;                                   \
    case 6: hipLaunchKernelGGL(KERNEL<6>, __VA_ARGS__); break;                                   \
    default: hipLaunchKernelGGL(KERNEL<8>, __VA_ARGS__); break;                                  \
    }
// K = d_model <= 1024 over 8 K groups: at most 4 k-steps a wave
#define MLA_KW4_DISPATCH(kw, KERNEL, ...)                                                       \
    switch (kw) {                                                                                \
    case 1: hipLaunchKernelGGL(KERNEL<1>, __VA_ARGS__); break;                                   \
    case 2: hipLaunchKernelGGL(KERNEL<2>, __VA_ARGS__); break;                                   \
    case 3: hipLaunchKernelGGL(KERNEL<3>, __VA_ARGS__); break;                                   \
    default: hipLaunchKernelGGL(KERNEL<4>, __VA_ARGS__); break;                                  \
    }

// Kernels whose dynamic LDS can exceed 64 KB.
hipError_t model_kernel_attributes() {
    const int bytes = 160 * 1024 - 32 * 1024;
    const void* ks[] = {reinterpret_cast<const void*>(&g23_kernel<2, 2>),
                        reinterpret_cast<const void*>(&g23_kernel<2, 4>)};
    for (const void* k : ks) {
        const hipError_t e =
            hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

hipError_t launch_embed(const StepArgs& s, const float* first_norm, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3(s.m_pad), dim3(256), 0, st, s, first_norm);
    return hipGetLastError();
}

hipError_t launch_layer_pre(const StepArgs& s, const LayerWeights& w, uint16_t* pool,
                            hipStream_t st) {
    const ModelDims& m = s.dims;
    MLA_KW4_DISPATCH(kw_variant(ceil_div(m.d_pad / 32, kWaves)), g1_kernel,
                     dim3((m.q_pad + m.kvw_pad) / 16, ceil_div(s.B, 16)), dim3(64 * kWaves), 0,
                     st, s, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    // q_pad <= 256: at most 2 k-steps of w_uq per wave; nope_pad <= 128: 4 of w_uk
    const dim3 grid(m.H + kKvWGs, ceil_div(s.B, 64));
    const size_t lds = g23_lds_bytes(m);
    if (m.nope_pad / 32 <= 2)
        hipLaunchKernelGGL((g23_kernel<2, 2>), grid, dim3(256), lds, st, s, w, pool);
    else
        hipLaunchKernelGGL((g23_kernel<2, 4>), grid, dim3(256), lds, st, s, w, pool);
    return hipGetLastError();
}

hipError_t launch_layer_post(const StepArgs& s, const LayerWeights& w, const float* next_norm,
                             hipStream_t st) {
    const ModelDims& m = s.dims;
    const int chunks = ceil_div(s.B, 16), d_tiles = m.d_pad / 16;
    MLA_KW_DISPATCH(kw_variant(ceil_div(m.ctx_pad / 32, kWaves)), g4_kernel,
                    dim3(d_tiles, chunks), dim3(64 * kWaves), 0, st, s, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    MLA_KW4_DISPATCH(kw_variant(ceil_div(m.d_pad / 32, kWaves)), g5_kernel,
                     dim3(m.ff_pad / 16, chunks), dim3(64 * kWaves), 0, st, s, w);
    e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    MLA_KW_DISPATCH(kw_variant(ceil_div(m.ff_pad / 32, kWaves)), g6_kernel,
                    dim3(d_tiles, chunks), dim3(64 * kWaves), 0, st, s, w, next_norm);
    return hipGetLastError();
}

hipError_t launch_gather_last(const StepArgs& s, int B, const int32_t* cu_q, uint16_t* xw_out,
                              float* ss_out, hipStream_t st) {
    hipLaunchKernelGGL(gather_last_kernel, dim3((B + 63) / 64 * 64), dim3(256), 0, st, s, B, cu_q,
                       xw_out, ss_out);
    return hipGetLastError();
}

hipError_t launch_logits(const StepArgs& s, hipStream_t st) {
    const ModelDims& m = s.dims;
    const int parts = g7_parts(m);
    MLA_KW_DISPATCH(kw_variant(ceil_div(m.d_pad / 32, kG7KG)), g7_kernel,
                    dim3(parts, ceil_div(s.B, 64)), dim3(64 * kWaves), 0, st, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    if (s.B > 0)
        hipLaunchKernelGGL(argmax_kernel, dim3(s.B), dim3(256), 0, st, s, parts);
    return hipGetLastError();
}

}  // namespace mla
