// Batched MLA decode step on gfx950: everything of CpuDecoder::decode around the
// attention (src/infer/inference.cpp:76-173) for B sessions at once, one new token
// each.
//
// Per layer, in launch order (y = x.W for every projection, as in ops.cpp:8-18):
//   qkv_kernel  per 16 rows: RMSNorm(x, attn_norm) . [w_dq | w_dkv], then per head q_norm
//               -> w_uq -> RoPE of the rope columns (q_rope, stored in the cache dtype)
//               -> absorption q_latent = W_uk_h^T q_nope (inference.cpp:85-90,121-124;
//               the MPS graph keeps q_latent in the storage dtype, mps_backend.mm:561);
//               one more workgroup kv_norms the latent, RoPEs the key, rounds both and
//               appends them to the paged cache (inference.cpp:91-103)
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

__device__ __forceinline__ floatx4 mma(V8 a, V8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ V8 to_half8(floatx4 a, floatx4 b) {
    return V8{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
              (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
}

// ---- L2 prefetch for the next kernel on the stream -------------------------------------
// Workgroups b of a launch (x-fastest linear id) with one residue b % 8 run on one XCD:
// the dispatcher deals workgroups to the 8 XCDs in turn, starting on an XCD that depends
// on the hardware queue (constant for the queue, so the same residue lands on the same
// XCD in consecutive kernels of one stream).  Each XCD has its own L2, which keeps its lines across
// kernel boundaries, while the attention's page stream evicts every layer's weights from
// it.  So the kernel that runs before a weight-latency-bound one touches, from each XCD,
// the 1 KB weight blocks that the next kernel's workgroups on that XCD will read; the next
// kernel's grid is padded to a multiple of 8 columns, so that each of its column tiles runs
// on one fixed XCD.  The loads go straight to a scratch block of LDS (global_load_lds: no
// VGPR is written behind the compiler's back), issued by the split-K waves that have handed
// their partial sums over and have nothing left to do: issued any earlier, the compiler's
// waits for the kernel's own operands would wait for them too (vmcnt retires in order),
// which measured slower than no prefetch.  A different placement only costs the prefetch
// its effect, never a result.
constexpr int kXcds = 8;

__device__ __forceinline__ int block_xcd() {
    return (int)((blockIdx.y * gridDim.x + blockIdx.x) % kXcds);
}

// Blocks [0, n) of this XCD's list (block k at addr(k)), spread over waves
// [first, blockDim/64) of all of this launch's workgroups on the XCD.
template <typename F>
__device__ __forceinline__ void l2_prefetch(int n, F&& addr, uint16_t* scratch, int first) {
    const int lin = blockIdx.y * gridDim.x + blockIdx.x, total = gridDim.x * gridDim.y;
    const int x = lin % kXcds, wgs = (total - x + kXcds - 1) / kXcds;
    const int nw = (blockDim.x >> 6) - first, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) - first;
    for (int k = (lin / kXcds) * nw + wave; k < n; k += wgs * nw)
        copy_block_to_lds(addr(k), lane * 16, scratch);
}

// ---- the decode attention's pages, read ahead during qkv_kernel ----------------------
// qkv_kernel occupies a few dozen CUs for several microseconds, and the attention that
// follows it on the stream starts its 40 MB page stream only when qkv ends.  The attention
// runs work item w with residue w % 8 (decode_page_kernel: one workgroup per item), so the
// qkv launch gets one more block of 8 columns, and its workgroups of residue x copy the
// leading pf.pages pages of the items x, x + 8, ... into LDS scratch: the lines land in
// that XCD's L2, where the attention's page loads then hit.  The page that a decode
// session's new token is appended to in this same launch (index (k_len - 1) / page_size)
// is skipped: a copy taken before the append lands would be stale.  Items of prefill
// sessions (q_len > 1), whose chunk is appended here too, are skipped whole.  Each wave
// reads the descriptors of its items once (one vector load round), then issues the
// copies of each valid page, 1 KB per instruction; nothing waits for them.
__device__ void page_prefetch(const PagePrefetch& pf, const uint16_t* pool, int npool,
                              uint16_t* scratch, int x, int gw, int nw) {
    const int lane = threadIdx.x & 63;
    const int items = x < pf.max_work ? (pf.max_work - 1 - x) / kXcds + 1 : 0;
    const int pairs = items * pf.pages, bytes = pf.record * 2;
    const uint32_t lds = lds_u32(scratch + (threadIdx.x >> 6) * 512);
    for (int r0 = gw; r0 < pairs; r0 += 64 * nw) {
        const int p = r0 + nw * lane;  // this lane's (item, page) pair of the round
        bool ok = false;
        int page = 0;
        if (p < pairs) {
            const int t = p / pf.pages, j = p % pf.pages, w = x + kXcds * t;
            const int32_t* d = pf.work_desc + (long long)w * kWorkDescInts;
            const int sess = d[0], kl = d[2], first = d[3], end = d[4], q_len = d[7];
            page = pf.work_pages[(long long)w * kWorkPages + j];
            ok = sess >= 0 && q_len == 1 && first + j < end &&
                 first + j != (kl - 1) / pf.page_size && (unsigned)page < (unsigned)npool;
        }
        // The ids are read here, once: a wait for them inside the loop below would also
        // wait for the copies already issued (vmcnt retires in order).
        asm volatile("" ::"v"(page));
        for (uint64_t m = __ballot(ok); m; m &= m - 1) {
            const int pg = __builtin_amdgcn_readlane(page, __builtin_ctzll(m));
            const uint16_t* base = pool + (long long)pg * pf.record;
            for (int b = 0; b * 1024 < bytes; ++b)
                if (b * 1024 + lane * 16 < bytes)
                    copy_block_to_lds_at(base + b * 512, lane * 16, lds);
        }
    }
}

// Sums over aligned groups of G = 4, 8 or 16 lanes of a 16-lane row, left in every lane
// of the group, on DPP lane moves (VALU) instead of LDS permutes: the two quad swaps give
// every lane its quad's sum, then the half-row mirror pairs the quads of each half and the
// row mirror the halves (each pairs lanes that hold equal partial sums, so every lane ends
// with the same bits).  Every lane of the row must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 4 || G == 8 || G == 16, "group of 4, 8 or 16 lanes");
    v += dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
    if constexpr (G >= 8)
        v += dpp_mov<0x141>(v);  // row_half_mirror
    if constexpr (G >= 16)
        v += dpp_mov<0x140>(v);  // row_mirror
    return v;
}
// Sum over the 16 lanes of an MFMA output row group (lanes with equal g hold the same
// rows, one column each).
__device__ __forceinline__ float sum16(float v) { return group_sum<16>(v); }

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
// producer's per-tile partial sums of squares (n_tiles <= 64): TPR threads a row each
// load every TPR-th tile, then combine in a fixed order.  Threads [0, TPR*rows) take
// part (whole waves).  issue() goes before the kernel's operand loads and finish()
// after its MFMAs, so the sums travel with the operands instead of delaying them by a
// round trip; inv_s is visible after the next barrier.
template <int TPR>
struct RmsPrefetch {
    static_assert(TPR >= 4 && TPR <= 16 && (TPR & (TPR - 1)) == 0, "threads per row");
    static constexpr int kPer = 64 / TPR;
    float v[kPer];
    __device__ __forceinline__ void issue(const float* ss, int n_tiles, int row0, int rows) {
        const int t = threadIdx.x;
        const bool mine = t < TPR * rows;
        const float* p = ss + (long long)(row0 + (mine ? t / TPR : 0)) * n_tiles;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int tile = t % TPR + TPR * i;
            v[i] = mine && tile < n_tiles ? p[tile] : 0.0f;
        }
    }
    __device__ __forceinline__ void finish(int K, float eps, float* inv_s, int rows) {
        const int t = threadIdx.x;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            sum += v[i];
        sum = group_sum<TPR>(sum);
        if (t < TPR * rows && t % TPR == 0)
            inv_s[t / TPR] = 1.0f / sqrtf(sum / (float)K + eps);
    }
};

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

// -------------------------------------------------------------------- qkv ----
// Everything between the residual stream x and the attention, for 16 rows per
// workgroup (inference.cpp:85-103): workgroup h < H computes head h's queries,
// workgroup H the cache append.  Both start with the same split-K GEMM
//     y = RMSNorm(x, attn_norm) . [w_dq | w_dkv]        (their column ranges)
// (8 waves, wave w taking k-steps w, w+8, ..; the partial tiles meet in LDS), so no
// other workgroup's output is waited for: each head workgroup recomputes the whole cq
// row it needs for q_norm (w_dq is L2-resident, read once per workgroup).  Then
//   head h:  q_norm(cq) -> . w_uq[:, head h] -> RoPE of the rope columns (q_rope in the
//            cache dtype) -> q_latent = q_nope . W_uk_h^T (the MPS graph keeps q_latent
//            in the storage dtype, mps_backend.mm:561)
//   kv:      kv_norm of the latent columns, RoPE of the key, rounding, paged append
// The norms are RMSNorm(v)_c = v_c * inv * w_c with one inv per row, and everything after
// them is linear, so the split-K reduction writes v o w straight away, with the rows'
// sums of squares per 16-column tile, and inv is applied later: to the w_uq products
// (head) or at the append (kv).  No pass over the rows waits for a row norm.
constexpr int kQkvWaves = 8;
constexpr int kQkvRows = 16;
constexpr int kQkvMaxTiles = 16;  // q_pad <= 256, kvw_pad <= 192: at most 16 column tiles
constexpr int kQkvPad = 8;        // fp16 pad of the LDS A-operand rows
// fp32 pad of the LDS y rows: with a pitch of 36 mod 64 words, the split-K reduction's
// writes (rows 4g + i of lane group g) fall 16 banks apart per group, conflict-free.
constexpr int kQkvYPad = 36;

// LDS layout of qkv_kernel (bytes), from the model dims.
struct QkvLds {
    int part, y, ya, qf, qn, total;
};
__host__ __device__ inline QkvLds qkv_lds(const ModelDims& m) {
    const int nt = max(m.q_pad, m.kvw_pad) / 16;
    const int ncol = max(m.q_pad, m.kvw_pad);
    // The split-K partials are dead once they are summed, so qf / qn reuse them; a head
    // workgroup writes ya where the append workgroup keeps y (neither needs the other).
    QkvLds l;
    l.part = 0;                                             // [8 waves][nt][64] floatx4
    l.qf = 0;                                               // [16][qk_pad + 4] fp32
    l.qn = l.qf + kQkvRows * (m.qk_pad + 4) * 4;            // [16][nope_pad + pad] fp16
    const int end = l.qn + kQkvRows * (m.nope_pad + kQkvPad) * 2;
    l.y = max(kQkvWaves * nt * 64 * 16, end);               // [16][ncol + kQkvYPad] fp32
    l.ya = l.y;                                             // [16][q_pad + pad] fp16
    l.total = l.y + kQkvRows * (ncol + kQkvYPad) * 4;
    return l;
}

// KC: chunks of two k-steps per wave (KT <= 16 * KC); NT >= the workgroup's column tiles.
template <int KC, int NT>
__global__ __launch_bounds__(64 * kQkvWaves) void qkv_kernel(StepArgs s, LayerWeights L,
                                                             uint16_t* pool, PagePrefetch pf) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const ModelDims& m = s.dims;
    const QkvLds lay = qkv_lds(m);
    floatx4* part = reinterpret_cast<floatx4*>(smem + lay.part);
    float* y = reinterpret_cast<float*>(smem + lay.y);
    _Float16* ya = reinterpret_cast<_Float16*>(smem + lay.ya);
    float* qf = reinterpret_cast<float*>(smem + lay.qf);
    _Float16* qn = reinterpret_cast<_Float16*>(smem + lay.qn);
    __shared__ float inv_x[kQkvRows];

    const int h = blockIdx.x, row0 = blockIdx.y * kQkvRows;
    if (h > m.H) {  // the heads' columns are padded to a multiple of 8 (head h: residue h % 8)
        if (h >= (m.H + kXcds) / kXcds * kXcds)  // the read-ahead block past them
            page_prefetch(pf, pool, s.num_pool_pages, reinterpret_cast<uint16_t*>(smem),
                          block_xcd(), blockIdx.y * kQkvWaves + (threadIdx.x >> 6),
                          gridDim.y * kQkvWaves);
        return;
    }
    const bool kv = h == m.H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32, q_tiles = m.q_pad / 16;
    const int nt0 = kv ? q_tiles : 0, ntv = kv ? m.kvw_pad / 16 : q_tiles;
    const int ncol = 16 * ntv, ldy = max(m.q_pad, m.kvw_pad) + kQkvYPad;
    __shared__ int32_t slot_s[kQkvRows];
    RmsPrefetch<16> rms;
    rms.issue(s.ss_x, m.d_pad / 16, row0, kQkvRows);
    // Side inputs of the later phases travel with the GEMM operands: the norm weight of
    // the two columns this thread reduces (16 * (wave + 8k) + n: 1 for the key's RoPE
    // columns, 0 past q_rank), the RoPE rotation of its first RoPE element, and (kv
    // workgroup) the rows' cache slots.
    const int ncols = kv ? m.kv_rank : m.q_rank;
    const float* nwp = kv ? L.kv_norm : L.q_norm;
    float nw[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int c = 16 * (wave + kQkvWaves * k) + n;
        nw[k] = c < ncols ? nwp[c] : kv ? 1.0f : 0.0f;
    }
    const int rhalf = m.rope / 2;
    float2 rcs = {0.0f, 0.0f};
    if (tid < kQkvRows * rhalf && row0 + tid / rhalf < s.B)
        rcs = s.rope_rows[(long long)(row0 + tid / rhalf) * rhalf + tid % rhalf];
    int32_t slot_pf = -1;
    if (kv && tid < kQkvRows && row0 + tid < s.B)
        slot_pf = s.slot_mapping[row0 + tid];

    // ---- GEMM 1: every operand of this wave in flight at once, chunk by chunk ----
    floatx4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
        acc[j] = floatx4{0, 0, 0, 0};
    const uint16_t* xw = s.xw + (long long)(row0 + n) * m.d_pad;
    // head workgroups also prefetch their w_uq / W_uk tiles (used after the reduction)
    const int qk_tiles = m.qk_pad / 16, KTQ = m.q_pad / 32;
    const int kv_tiles = m.kv_pad / 16, KTU = m.nope_pad / 32;
    V8 bq[8], bu[4];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        V8 a[2], b[2][NT];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int kt = wave + kQkvWaves * (2 * c + kk);
            a[kk] = kt < KT ? *reinterpret_cast<const V8*>(xw + 32 * kt + 8 * g) : V8{};
#pragma unroll
            for (int j = 0; j < NT; ++j)
                b[kk][j] = kt < KT && j < ntv
                               ? *reinterpret_cast<const V8*>(
                                     L.w_dq_dkv + ((long long)(nt0 + j) * KT + kt) * 512 + lane * 8)
                               : V8{};
        }
        if (c == 0 && !kv) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
                bq[k] = wave < qk_tiles && k < KTQ
                            ? *reinterpret_cast<const V8*>(
                                  L.w_uq + ((long long)(h * qk_tiles + wave) * KTQ + k) * 512 +
                                  lane * 8)
                            : V8{};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                bu[k] = wave < kv_tiles && k < KTU
                            ? *reinterpret_cast<const V8*>(
                                  L.w_uk + (long long)h * kv_tiles * KTU * 512 +
                                  ((long long)wave * KTU + k) * 512 + lane * 8)
                            : V8{};
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int j = 0; j < NT; ++j)
                acc[j] = mma(a[kk], b[kk][j], acc[j]);
    }
    rms.finish(m.d_model, m.eps, inv_x, kQkvRows);
    if (kv && tid < kQkvRows)
        slot_s[tid] = slot_pf;
#pragma unroll
    for (int j = 0; j < NT; ++j)
        if (j < ntv)
            part[(wave * ntv + j) * 64 + lane] = acc[j];
    __shared__ float ss_part[kQkvRows][kQkvMaxTiles];  // row sums of squares per column tile
    __shared__ float inv_n[kQkvRows];                  // q_norm / kv_norm factor per row
    __syncthreads();
    // v[r][c] = inv_x[r] * sum over the waves (rows 4g+i, column 16j+n of lane group e);
    // head: ya = v o q_norm weight (fp16 A operand); kv: y = v o kv_norm weight (1 for the
    // key's RoPE columns).  ss_part[r][j] = sum of v^2 over tile j's norm columns.
    for (int e = tid, k = 0; e < ntv * 64; e += 64 * kQkvWaves, ++k) {
        const int j = e >> 6, l = e & 63, col = 16 * j + (l & 15);
        floatx4 v = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < kQkvWaves; ++w)
            v += part[(w * ntv + j) * 64 + l];
        const float wc = k == 0 ? nw[0] : nw[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * (l >> 4) + i;
            const float yv = v[i] * inv_x[r];
            if (kv)
                y[r * ldy + col] = yv * wc;
            else
                ya[r * (m.q_pad + kQkvPad) + col] = (_Float16)(yv * wc);
            const float sq = sum16(col < ncols ? yv * yv : 0.0f);
            if ((l & 15) == 0)
                ss_part[r][j] = sq;
        }
    }
    __syncthreads();
    // inv of each row (ops.cpp:37-44: 1/sqrt(mean(v^2) + eps)) by the last wave's first
    // lanes, visible after the next barrier
    if (wave == kQkvWaves - 1 && lane < kQkvRows) {
        float ss = 0.0f;
        for (int j = 0; j * 16 < ncols; ++j)
            ss += ss_part[lane][j];
        inv_n[lane] = 1.0f / sqrtf(ss / (float)ncols + m.eps);
    }

    if (kv) {  // ---- RoPE of the key (in place), then rounding and the paged append ----
        {
            for (int e = tid; e < kQkvRows * rhalf; e += 64 * kQkvWaves) {
                const int rr = e / rhalf, jp = 2 * (e % rhalf);
                const float2 cs =
                    e == tid ? rcs : s.rope_rows[(long long)(row0 + rr) * rhalf + e % rhalf];
                float* yk = y + rr * ldy + m.kv_rank + jp;
                const float a0 = yk[0], a1 = yk[1];
                yk[0] = a0 * cs.x - a1 * cs.y;
                yk[1] = a0 * cs.y + a1 * cs.x;
            }
        }
        __syncthreads();
        const bool tiled = page_tiled(m.page_size, m.kv_rank, m.rope);
        const int width = m.kv_rank + m.rope;
        for (int e = tid; e < kQkvRows * width; e += 64 * kQkvWaves) {
            const int r = e / width, c = e % width, row = row0 + r;
            if (row >= s.B)
                continue;
            const int slot = slot_s[r];
            const int page = slot / m.page_size, off = slot % m.page_size;
            if (slot < 0 || page >= s.num_pool_pages)
                continue;
            uint16_t* base = pool + (long long)page * m.page_size * width;
            const uint16_t v = F16::from_float(c < m.kv_rank ? y[r * ldy + c] * inv_n[r]
                                                             : y[r * ldy + c]);
            if (c < m.kv_rank)
                base[latent_word(tiled, off, c, m.page_size, m.kv_rank)] = v;
            else
                base[rope_word(tiled, off, c - m.kv_rank, m.page_size, m.kv_rank, m.rope)] = v;
        }
        return;
    }
    (void)ncol;

    // ---- q_h = (cq o q_norm weight) . w_uq[:, head h], times the row's inv below: wave
    // w < qk_tiles owns column tile w ----
    if (wave < qk_tiles) {
        floatx4 q = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k < KTQ)
                q = mma(*reinterpret_cast<const V8*>(ya + n * (m.q_pad + kQkvPad) + 32 * k + 8 * g),
                        bq[k], q);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            qf[(4 * g + i) * (m.qk_pad + 4) + 16 * wave + n] = q[i];
    }
    __syncthreads();
    {   // RoPE of the rope columns (pairs adjacent, ops.cpp:88-108) -> q_rope; q_nope -> fp16
        const int half = rhalf, ldq = m.nope_pad + kQkvPad;
        for (int e = tid; e < kQkvRows * half; e += 64 * kQkvWaves) {
            const int r = e / half, j2 = e % half, jp = 2 * j2, row = row0 + r;
            if (row >= s.B)
                continue;
            const float2 cs = e == tid ? rcs : s.rope_rows[(long long)row * half + j2];
            const float a0 = qf[r * (m.qk_pad + 4) + m.nope + jp] * inv_n[r];
            const float a1 = qf[r * (m.qk_pad + 4) + m.nope + jp + 1] * inv_n[r];
            uint16_t* qr = s.q_rope + ((long long)row * m.H + h) * m.rope;
            qr[jp] = F16::from_float(a0 * cs.x - a1 * cs.y);
            qr[jp + 1] = F16::from_float(a0 * cs.y + a1 * cs.x);
        }
        for (int e = tid; e < kQkvRows * m.nope_pad; e += 64 * kQkvWaves) {
            const int r = e / m.nope_pad, c = e % m.nope_pad;
            qn[r * ldq + c] = (_Float16)(c < m.nope ? qf[r * (m.qk_pad + 4) + c] * inv_n[r] : 0.0f);
        }
    }
    __syncthreads();
    // ---- q_latent_h = q_nope . W_uk_h^T: wave w < kv_tiles owns latent tile w ----
    if (wave < kv_tiles) {
        const int ldq = m.nope_pad + kQkvPad;
        floatx4 ql = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (k < KTU)
                ql = mma(*reinterpret_cast<const V8*>(qn + n * ldq + 32 * k + 8 * g), bu[k], ql);
        const int c = 16 * wave + n;
        if (c < m.kv_rank)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + 4 * g + i;
                if (row < s.B)
                    s.q_latent[((long long)row * m.H + h) * m.kv_rank + c] = F16::from_float(ql[i]);
            }
    }
}

// ----------------------------------------------------------- g4 and g6 ----
// y = A . W + residual for 16 rows and one 16-column tile (8 waves split K): y to `out`
// (fp32), y o wnorm to `outw` (fp16, the next consumer's normalised A operand), and
// y's per-tile sums of squares.  The residual and norm columns are fetched with the
// operands.
template <int KW, typename ALoad, typename Pf>
__device__ __forceinline__ void splitk_residual(ALoad&& aload, const uint16_t* w, int KT, int N,
                                                const float* residual, const float* wnorm,
                                                float* out, uint16_t* outw, float* ss,
                                                int n_tiles, int ld, int row0, int B,
                                                Pf&& prefetch) {
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
    if (!splitk_reduce<1, 1, kWaves>(acc, part, mt, v)) {
        prefetch();  // waves 1.. have nothing left to do but this
        return;
    }
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
    __shared__ __attribute__((aligned(16))) uint16_t pf_scratch[512];
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
        row0, s.B, [&]() {
            // g5 (next on the stream) runs column pair p with residue p % 8: its two tiles of
            // every k-step are 2 * KT5 contiguous blocks
            const int x = block_xcd(), np = m.ff_pad / 16, KT5 = m.d_pad / 32, per = 2 * KT5;
            const int pairs = x < np ? (np - x + kXcds - 1) / kXcds : 0;
            l2_prefetch(pairs * per, [&](int k) {
                const int p = x + kXcds * (k / per);
                return L.w_gate_up + ((long long)2 * p * KT5 + k % per) * 512;
            }, pf_scratch, 1);
        });
}

// next_norm: the norm weight of x's next consumer (attn_norm of the next layer, or
// final_norm after the last layer).  next: the next layer's weights (qkv_kernel runs
// next on the stream), or null after the last layer.
template <int KW>
__global__ __launch_bounds__(64 * kWaves) void g6_kernel(StepArgs s, LayerWeights L,
                                                         const float* next_norm,
                                                         const uint16_t* next_dq_dkv,
                                                         const uint16_t* next_uq,
                                                         const uint16_t* next_uk) {
    __shared__ __attribute__((aligned(16))) uint16_t pf_scratch[512];
    const ModelDims& m = s.dims;
    const int row0 = blockIdx.y * 16, KT = m.ff_pad / 32;
    splitk_residual<KW>(
        [&](floatx4(&acc)[1][1], const BPre<1, KW>& bw, int kt0, int lane) {
            APre16<KW, 1> a;
            a.load(s.u + (long long)row0 * m.ff_pad, m.ff_pad, KT, kt0, kWaves, lane);
            mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
        },
        L.w_down, KT, m.d_model, s.res, next_norm, s.x, s.xw, s.ss_x, m.d_pad / 16, m.d_pad,
        row0, s.B, [&]() {
            if (!next_dq_dkv)
                return;
            // qkv_kernel runs head h with residue h % 8 and the append workgroup (h = H) with H % 8:
            // head workgroups read the w_dq tiles, the append one the w_dkv tiles, and head h
            // its w_uq and W_uk blocks (contiguous per head)
            const int x = block_xcd(), KTq = m.d_pad / 32, q_tiles = m.q_pad / 16;
            const int n_dq = x < m.H ? q_tiles * KTq : 0;
            const int n_dkv = m.H % kXcds == x ? (m.kvw_pad / 16) * KTq : 0;
            const int n_uq = (m.qk_pad / 16) * (m.q_pad / 32), n_uk = (m.kv_pad / 16) * (m.nope_pad / 32);
            const int heads = x < m.H ? (m.H - x + kXcds - 1) / kXcds : 0;
            l2_prefetch(n_dq + n_dkv + heads * (n_uq + n_uk), [&](int k) {
                if (k < n_dq)
                    return next_dq_dkv + (long long)k * 512;
                k -= n_dq;
                if (k < n_dkv)
                    return next_dq_dkv + ((long long)q_tiles * KTq + k) * 512;
                k -= n_dkv;
                const int h = x + kXcds * (k / (n_uq + n_uk));
                k %= n_uq + n_uk;
                return k < n_uq ? next_uq + ((long long)h * n_uq + k) * 512
                                : next_uk + ((long long)h * n_uk + k - n_uq) * 512;
            }, pf_scratch, 1);
        });
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
    if (p >= m.ff_pad / 16)
        return;  // the grid's columns are padded to a multiple of 8 (one XCD per pair)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int KT = m.d_pad / 32;
    RmsPrefetch<16> rms;
    rms.issue(s.ss_res, m.d_pad / 16, row0, 16);
    BPre<2, KW> bw;
    bw.load(L.w_gate_up, 2 * p, 2, KT, wave, kWaves, lane);
    APre16<KW, 1> a;
    a.load(s.resw + (long long)row0 * m.d_pad, m.d_pad, KT, wave, kWaves, lane);
    floatx4 acc[1][2];
    zero(acc);
    mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
    rms.finish(m.d_model, m.eps, inv_s, 16);
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
// workgroup (the waves split K eight ways: measured 11.7 us at config 3 against 13.1 us
// for four ways times two tile groups, whose waves each loaded twice the activation
// rows); each workgroup also leaves, per row, the greedy winner of its 64 columns
// (strict >, so the lowest index wins ties; banned ids never win) and whether all of
// them were finite (banned or not: sample_token checks every logit,
// inference.cpp:352-353).
constexpr int kG7Tiles = 4, kG7KG = 8;

// Greedy key of a logit: larger value first, then lower column.  The value's bits are
// mapped to an order-preserving unsigned (after -0 -> +0, which compares equal to it),
// the column to its complement; 0 marks "no candidate" (every real key is larger).
__device__ __forceinline__ uint64_t greedy_key(float y, int col) {
    const uint32_t b = __float_as_uint(y + 0.0f);
    const uint32_t ord = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint32_t)~(uint32_t)col;
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_shr64(uint64_t v) {  // lanes without a source get 0
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, true);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}
// Running maximum along each row of 16 lanes: lane 15 of the row ends with the row's max.
__device__ __forceinline__ uint64_t row_max16(uint64_t v) {
    uint64_t t = dpp_shr64<0x111>(v);
    v = t > v ? t : v;
    t = dpp_shr64<0x112>(v);
    v = t > v ? t : v;
    t = dpp_shr64<0x114>(v);
    v = t > v ? t : v;
    t = dpp_shr64<0x118>(v);
    return t > v ? t : v;
}

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
    RmsPrefetch<8> rms;
    rms.issue(s.ss_x, m.d_pad / 16, row0, 64);
    BPre<NTW, KW> bw;
    bw.load(s.embed, nt0 + ng * NTW, min(NTW, n_tiles - nt0 - ng * NTW), KT, kg, kG7KG, lane);
    APre16<KW, 4> a;
    a.load(s.xw + (long long)row0 * m.d_pad, m.d_pad, KT, kg, kG7KG, lane);
    floatx4 acc[4][NTW];
    zero(acc);
    mma_steps(acc, bw, [&](int kk, int mt) { return a.x[kk][mt]; });
    rms.finish(m.d_model, m.eps, inv_s, 64);
    int mt;
    floatx4 v[kG7Tiles];
    if (!splitk_reduce<4, NTW, kG7KG>(acc, part, mt, v))
        return;
    uint64_t best[4] = {0, 0, 0, 0};
    uint64_t nonfinite[4] = {0, 0, 0, 0};  // 1 when some logit of the row is not finite
#pragma unroll
    for (int j = 0; j < kG7Tiles; ++j) {
        const int col = (nt0 + j) * 16 + n;
        const bool valid = nt0 + j < n_tiles && col < m.vocab;
        const bool open = valid && !(s.ban && ((s.ban[col >> 5] >> (col & 31)) & 1u));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + 16 * mt + 4 * g + i;
            const float y = v[j][i] * inv_s[16 * mt + 4 * g + i];
            if (valid && row < s.B)
                s.logits[(long long)row * m.vocab + col] = y;
            if (valid && !isfinite(y))
                nonfinite[i] = 1;
            const uint64_t k = open ? greedy_key(y, col) : 0;
            best[i] = k > best[i] ? k : best[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // the 16 lanes of a row hold 16 columns each; lane 15 gathers the row's winner
        const uint64_t k = row_max16(best[i]);
        const uint64_t bad = row_max16(nonfinite[i]);
        const int row = row0 + 16 * mt + 4 * g + i;
        if (n == 15 && row < s.B) {
            const long long idx = (long long)row * gridDim.x + blockIdx.x;
            const uint32_t ord = (uint32_t)(k >> 32);
            const uint32_t b = ord & 0x80000000u ? ord ^ 0x80000000u : ~ord;
            s.arg_v[idx] = k ? __uint_as_float(b) : -INFINITY;
            s.arg_c[idx] = bad ? -1 : k ? (int)~(uint32_t)k : 0x7fffffff;
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

// Greedy token per row (inference.cpp:354-380 with no repetition penalty): the lowest
// column among the maxima of the ids not banned; -1 when a logit is not finite
// (numerical_error, checked first as the reference does), -2 when every id is banned
// ("All tokens are banned").  256
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
        s.next_tokens[row] = bad ? -1 : bc == 0x7fffffff ? -2 : bc;
    }
}

// k-steps per wave, rounded up to a compiled variant
int kw_variant(int ksteps) {
    return ksteps <= 1 ? 1 : ksteps <= 2 ? 2 : ksteps <= 3 ? 3 : ksteps <= 4 ? 4 : ksteps <= 6 ? 6 : 8;
}
int ceil_div(int a, int b) { return (a + b - 1) / b; }
int round_up_to(int a, int b) { return ceil_div(a, b) * b; }

}  // namespace

// ------------------------------------------------------------------ launches ----
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

size_t qkv_lds_bytes(const ModelDims& m) { return (size_t)qkv_lds(m).total; }

// Kernels whose dynamic LDS can exceed 64 KB: allow what this model's shape needs.
hipError_t model_kernel_attributes(const ModelDims& m) {
    const int bytes = (int)qkv_lds_bytes(m);
    const void* ks[] = {
        reinterpret_cast<const void*>(&qkv_kernel<1, 4>), reinterpret_cast<const void*>(&qkv_kernel<1, 8>),
        reinterpret_cast<const void*>(&qkv_kernel<1, 12>), reinterpret_cast<const void*>(&qkv_kernel<1, 16>),
        reinterpret_cast<const void*>(&qkv_kernel<2, 4>), reinterpret_cast<const void*>(&qkv_kernel<2, 8>),
        reinterpret_cast<const void*>(&qkv_kernel<2, 12>), reinterpret_cast<const void*>(&qkv_kernel<2, 16>)};
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
                            const PagePrefetch& pf, hipStream_t st) {
    const ModelDims& m = s.dims;
    const size_t lds = qkv_lds_bytes(m);
    // heads padded to 8 columns (see l2_prefetch), then 8 read-ahead columns (page_prefetch,
    // 1 KB of the LDS per wave)
    const bool ahead = pf.max_work > 0 && pf.pages > 0 && lds >= kQkvWaves * 1024;
    const dim3 grid(round_up_to(m.H + 1, kXcds) + (ahead ? kXcds : 0), ceil_div(s.B, kQkvRows));
    const int nt = max(m.q_pad, m.kvw_pad) / 16;  // <= 16 (mla_model_create checks)
    const int tiles = nt <= 4 ? 4 : nt <= 8 ? 8 : nt <= 12 ? 12 : 16;
    // d_pad <= 512: one chunk of two k-steps per wave; <= 1024: two
    const int kc = m.d_pad / 32 <= 2 * kQkvWaves ? 1 : 2;
#define MLA_QKV(KC, NT)                                                                         \
    hipLaunchKernelGGL((qkv_kernel<KC, NT>), grid, dim3(64 * kQkvWaves), lds, st, s, w, pool, pf)
    if (kc == 1) {
        if (tiles == 4) MLA_QKV(1, 4); else if (tiles == 8) MLA_QKV(1, 8);
        else if (tiles == 12) MLA_QKV(1, 12); else MLA_QKV(1, 16);
    } else {
        if (tiles == 4) MLA_QKV(2, 4); else if (tiles == 8) MLA_QKV(2, 8);
        else if (tiles == 12) MLA_QKV(2, 12); else MLA_QKV(2, 16);
    }
#undef MLA_QKV
    return hipGetLastError();
}

hipError_t launch_layer_post(const StepArgs& s, const LayerWeights& w, const float* next_norm,
                             const LayerWeights* next, hipStream_t st) {
    const ModelDims& m = s.dims;
    const int chunks = ceil_div(s.B, 16), d_tiles = m.d_pad / 16;
    MLA_KW_DISPATCH(kw_variant(ceil_div(m.ctx_pad / 32, kWaves)), g4_kernel,
                    dim3(d_tiles, chunks), dim3(64 * kWaves), 0, st, s, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    MLA_KW4_DISPATCH(kw_variant(ceil_div(m.d_pad / 32, kWaves)), g5_kernel,
                     dim3(round_up_to(m.ff_pad / 16, kXcds), chunks), dim3(64 * kWaves), 0, st, s,
                     w);  // columns padded: see l2_prefetch
    e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    MLA_KW_DISPATCH(kw_variant(ceil_div(m.ff_pad / 32, kWaves)), g6_kernel,
                    dim3(d_tiles, chunks), dim3(64 * kWaves), 0, st, s, w, next_norm,
                    next ? next->w_dq_dkv : nullptr, next ? next->w_uq : nullptr,
                    next ? next->w_uk : nullptr);
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
