// (c) Absorbed MLA chunked-prefill attention over the paged latent cache, gfx950.
//
// A session with q_len > 1 appends q_len tokens at positions ctx .. ctx+q_len-1
// (ctx = k_len - q_len tokens were cached before) and each of them attends causally:
// query i sees keys [0, ctx + i].  Per query row i and head h
//     s_j   = (q_latent[i,h] . c_j + q_rope[i,h] . k_j) * scale,   j <= ctx + i
//     out   = sum_j softmax(s)_j c_j,      lse = ln sum_j exp(s_j)
// which is the reference's causal attention (src/model/ops.cpp:109-142) over the
// prefix plus chunk, in the absorbed form of CpuDecoder (src/infer/inference.cpp:
// 116-153): W_uk is folded into q_latent and W_uv is applied after the attention,
// so the keys and values are the shared latent rows.  The reference's prefill always
// restarts at position 0 (inference.cpp:47-68); a chunk on top of an existing
// context equals that full forward's rows ctx.. (causality, tests/test_model.cpp:65-77).
//
// prefill_page_kernel -- the production kernel (H <= 16, kv_rank 128, rope 16,
//   64-token tiled pages).  Every head of a query shares the latent, so the kernel
//   flattens (query, head) into q-rows r = i*H + h: a workgroup of 4 waves (two
//   q-groups x two halves of each page's tokens) owns 32 consecutive q-rows of one
//   session (4 queries at H = 8), a q-group QT = 1 16-row tile.
//   The session's pages stream through a double-buffered LDS copy (the tiled record
//   as stored); per page and q-tile
//     S^T = K . Q^T     v_mfma_f32_16x16x32: the page's token tiles, read from LDS
//                       as loaded (one 1 KB block per wave read), are the A operand;
//                       Q^T (latent k-steps + the rope step) is the B operand held in
//                       registers for the whole kernel
//     causal mask, online softmax in the log2 domain
//     O^T += C^T . P^T  the S^T accumulators already are P^T's B operand; C^T comes
//                       straight from the tiled LDS record through the gfx950
//                       transpose read ds_read_b64_tr_b16 (lane j of a 16-lane group
//                       points at 4 latent values of one token; lane 4a+b receives
//                       value b of lanes a, a+4, a+8, a+12), shared by the wave's
//                       q-tiles
//   This work is MFMA-bound (512 queries x 8 heads over a 2k context is ~6k flop per
//   cached byte).
// prefill_generic_kernel -- any H / kv_rank / rope / page size / layout: one
//   256-thread block per (query row, head), VALU fp32.
#include "mla_common.hpp"
#include "mla_internal.hpp"

#include <cmath>

namespace mla {
namespace {

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s4 __attribute__((address_space(3)))*)((__attribute__((address_space(3))) char*)p));
    return __builtin_bit_cast(u32x2, v);
}

constexpr float kPfNoMax = -1.0e30f;  // running-max floor: below every real score
constexpr float kPfRescale = 8.0f;    // log2 headroom before the running max is raised
constexpr int kPfQG = 2;        // q-groups per workgroup (QT 16-row tiles each)
constexpr int kPfKH = 2;        // token halves: the two waves of a q-group split each page
constexpr int kPfWaves = kPfQG * kPfKH;
constexpr int kPfMaxIds = 2048;  // page ids staged in LDS: sessions up to 2048 pages

template <typename T, int KV, int RP, int PS, int QT>
__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(2, 8)))
void prefill_page_kernel(PrefillArgs a) {
    static_assert(KV % 32 == 0 && RP % 8 == 0 && RP <= 32 && PS == 64, "tile shape");
    constexpr int KS = KV / 32;               // latent k-steps of the score MFMAs
    constexpr int RT = KV / 16;               // 16-row (latent) tiles of O^T
    constexpr int REC = PS * (KV + RP);       // words of a page record
    constexpr int CHUNKS = REC / 8;           // 16-byte chunks of a record
    constexpr int THREADS = 64 * kPfWaves;
    constexpr int CPT = (CHUNKS + THREADS - 1) / THREADS;  // chunks per thread and page
    constexpr int WG_ROWS = kPfQG * QT * 16;
    using V8 = typename T::vec8;
    __shared__ __attribute__((aligned(16))) uint16_t buf0[REC];
    __shared__ __attribute__((aligned(16))) uint16_t buf1[REC];
    __shared__ int32_t pids[kPfMaxIds];

    const int b = blockIdx.y;
    if (a.info[0] <= 0)
        return;  // failed metadata build (or an empty batch)
    const int q0 = a.cu_q[b], q_len = a.cu_q[b + 1] - q0;
    const int k_len = a.cu_k[b + 1] - a.cu_k[b];
    const int H = a.H;
    const int n_rows = q_len * H;
    // Heavier workgroups (later queries see more keys) first.
    const int rb = (gridDim.x - 1 - blockIdx.x) * WG_ROWS;
    if (q_len < 2 || rb >= n_rows)
        return;
    const int ctx = k_len - q_len;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = tid >> 6, qg = wave >> 1, kh = wave & 1;
    // keys [0, k_hi) are visible to some q-row of this workgroup
    const int last_q = min(n_rows - 1, rb + WG_ROWS - 1) / H;
    const int k_hi = ctx + last_q + 1;
    const int n_pages = (k_hi + PS - 1) / PS;
    const int32_t* ptab = a.page_table + (long long)b * a.max_pages;

    // ---- page staging: 16-byte chunks through registers, slots at or past k_len zeroed.
    // One register set holds page p+1 while page p is consumed from LDS (a second set
    // holding p+2 as well measured no faster and cost 20 VGPRs).
    // Raw buffer loads over the page record: a chunk that must read as zero (slot at or
    // past k_len, an invalid page id, or p >= n_pages) gets an offset outside the record,
    // which the hardware returns as zero.  Every load is issued unconditionally, so no
    // register merges (and no early waits) appear between the loads and their use.
    auto load_page = [&](u32x4 (&st)[CPT], int page_id, int p) {
        const int page = __builtin_amdgcn_readfirstlane(page_id);  // uniform: scalar rsrc
        const bool ok = (unsigned)page < (unsigned)a.num_pool_pages && p < n_pages;
        const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(a.pages + (long long)(ok ? page : 0) * REC), 0, REC * 2,
            0x00020000);
        const int valid = ok ? k_len - p * PS : 0;  // slots of the page that hold keys
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + k * THREADS;
            bool live = c < CHUNKS && valid > 0;
            if (valid < PS) {  // the session's last page (or nothing to load)
                // slot of chunk c: latent chunks run (t, j, g, n), rope chunks (t, ch, n)
                const int slot = c < PS * KV / 8 ? (c / (16 * 4 * KS)) * 16 + (c & 15)
                                                 : ((c - PS * KV / 8) / (16 * (RP / 8))) * 16 +
                                                       (c & 15);
                live = live && slot < valid;
            }
            st[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rsrc, live ? c * 16 : 0x40000000, 0, 0));
        }
    };
    auto store_page = [&](const u32x4 (&st)[CPT], uint16_t* dst) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + k * THREADS;
            if (c < CHUNKS)
                *reinterpret_cast<u32x4*>(dst + c * 8) = st[k];
        }
    };
    // Prologue, in issue order: the page ids (staged in LDS, so issuing a later page
    // never waits on memory), the Q operands, then the first two pages.
    const int id0 = ptab[0];
    constexpr int IDS_PT = kPfMaxIds / THREADS;
    int ids[IDS_PT];
#pragma unroll
    for (int k = 0; k < IDS_PT; ++k) {
        const int i = tid + k * THREADS;
        ids[k] = i < n_pages ? ptab[i] : 0;
    }
    const int wr0 = rb + qg * QT * 16;  // first session q-row of the wave
    V8 qv[QT][KS + 1];
    int lim[QT];  // lane's q-row n sees keys [0, lim]; -1 = no such row
    const bool rope_lane = 8 * g < RP;
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        const int r = wr0 + q * 16 + n;
        const bool valid = r < n_rows;
        lim[q] = valid ? ctx + r / H : -1;
        const long long fr = (long long)q0 * H + r;  // flat (row, head) index
#pragma unroll
        for (int j = 0; j < KS; ++j)
            qv[q][j] = valid ? *reinterpret_cast<const V8*>(a.q_latent + fr * KV + 32 * j + 8 * g)
                             : V8{};
        qv[q][KS] = valid && rope_lane
                        ? *reinterpret_cast<const V8*>(a.q_rope + fr * RP + 8 * g)
                        : V8{};
    }
    u32x4 st0[CPT];
    load_page(st0, id0, 0);
#pragma unroll
    for (int k = 0; k < IDS_PT; ++k)
        pids[tid + k * THREADS] = ids[k];
    store_page(st0, buf0);
    __syncthreads();
    const int rope_off = (16 * (rope_lane ? g : g % (RP / 8)) + n) * 8;
    // transpose-read address of lane (g, j=n) inside a token tile: token 4g + n/4,
    // latent 4*(n%4) + (row-tile offset)
    const int tr_lane = (((n & 3) >> 1) * 128) + (4 * g + (n >> 2)) * 8 + 4 * (n & 1);

    // The lowest causal limit of the wave's rows (-1 when some row is past the chunk).
    const int lim_min = wr0 + QT * 16 <= n_rows ? ctx + wr0 / H : -1;
    float m_run[QT], l_run[QT];
    floatx4 acc[QT][RT];
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        m_run[q] = kPfNoMax;
        l_run[q] = 0.0f;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            acc[q][rt] = floatx4{0, 0, 0, 0};
    }

    // Scores, mask, online softmax and PV of this wave's token half of page p.
    auto compute = [&](const uint16_t* pg, int p) {
        const int tok0 = p * PS + 32 * kh;
        floatx4 sc[2][QT];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 2 * kh + tt;
#pragma unroll
            for (int q = 0; q < QT; ++q)
                sc[tt][q] = floatx4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const V8 ka = *reinterpret_cast<const V8*>(pg + (t * KS + j) * 512 + lane * 8);
#pragma unroll
                for (int q = 0; q < QT; ++q)
                    sc[tt][q] = T::mma32(ka, qv[q][j], sc[tt][q]);
            }
            const V8 kr =
                *reinterpret_cast<const V8*>(pg + PS * KV + t * (RP / 8) * 128 + rope_off);
#pragma unroll
            for (int q = 0; q < QT; ++q)
                sc[tt][q] = T::mma32(kr, qv[q][KS], sc[tt][q]);
        }
        V8 pb[QT], pl[QT];  // P^T operands (pl: the low part, bf16 only)
        // Every row of the wave sees all 32 tokens of this half unless it holds the
        // causal edge (or rows past the chunk): only then are tokens masked.
        const bool full = tok0 + 31 <= lim_min;
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            float mp = -INFINITY;  // this lane's max, raw score units (the scale is > 0)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (!full && tok0 + 16 * tt + 4 * g + i > lim[q])
                        sc[tt][q][i] = -INFINITY;
                    mp = fmaxf(mp, sc[tt][q][i]);
                }
            // log2 units; m_run starts at a finite floor, so exp2 never sees inf - inf.
            // The reference max m_run is raised only when a score exceeds it by more than
            // kPfRescale; below that the probabilities are exp2(x - m_run) <= 2^kPfRescale,
            // exact in fp32 and fp16, and the final normalisation divides by the same-based
            // sum.  Each lane checks its own scores, so the row max (a cross-lane
            // reduction) is formed only on the rare pages that raise the reference.
            if (__builtin_amdgcn_ballot_w64(mp * a.scale_log2 > m_run[q] + kPfRescale)) {
                mp = rows_max(mp);
                const float m_new = fmaxf(m_run[q], mp * a.scale_log2);
                const float alpha = exp2_fast(m_run[q] - m_new);
                l_run[q] *= alpha;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    acc[q][rt] *= alpha;
                m_run[q] = m_new;
            }
            const float m_ref = m_run[q];
            float psum = 0.0f;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = exp2_fast(fmaf(sc[tt][q][i], a.scale_log2, -m_ref));
                    psum += e;
                    const auto hi = static_cast<typename T::scalar>(e);
                    pb[q][4 * tt + i] = hi;
                    if constexpr (T::split_p)
                        pl[q][4 * tt + i] =
                            static_cast<typename T::scalar>(e - static_cast<float>(hi));
                }
            l_run[q] += psum;  // per lane; summed over the 4 lane groups at the end
        }
        // O^T += C^T . P^T over the 32 tokens of this half (one K-step)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int blk = ((rt >> 1) * 4 + 2 * (rt & 1)) * 128;  // latent rows 16rt..
            const u32x2 lo = lds_read_tr16(pg + (2 * kh) * KS * 512 + blk + tr_lane);
            const u32x2 hi = lds_read_tr16(pg + (2 * kh + 1) * KS * 512 + blk + tr_lane);
            const V8 ca = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                acc[q][rt] = T::mma32(ca, pb[q], acc[q][rt]);
                if constexpr (T::split_p)
                    acc[q][rt] = T::mma32(ca, pl[q], acc[q][rt]);
            }
        }
    };
    // Page p lives in buf[p % 2]; its successor waits in the registers st0.  One step:
    // load page p+1 into the registers, consume page p, store page p+1 into the other
    // buffer (its last readers finished before the previous barrier), barrier.  Steps
    // are unrolled in pairs so every buffer is named statically.
    auto step = [&](const uint16_t* cur, uint16_t* nx, int p) {
        load_page(st0, pids[min(p + 1, n_pages - 1)], p + 1);
        compute(cur, p);
        if (p + 1 < n_pages)
            store_page(st0, nx);
        __syncthreads();
    };
    for (int p = 0; p < n_pages; p += 2) {
        step(buf0, buf1, p);
        if (p + 1 >= n_pages)
            break;
        step(buf1, buf0, p + 1);
    }

    // ---- the two token halves of each q-group meet in LDS; normalise and store ----
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        l_run[q] = rows_sum(l_run[q]);
    }
    __syncthreads();  // every wave is done with the page buffers
    static_assert((QT * RT * 256 + QT * 128) * 4 <= REC * 2, "exchange fits a page buffer");
    float* xo = reinterpret_cast<float*>(qg == 0 ? buf0 : buf1);
    if (kh == 1) {
#pragma unroll
        for (int q = 0; q < QT; ++q) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                *reinterpret_cast<floatx4*>(xo + ((q * RT + rt) * 64 + lane) * 4) = acc[q][rt];
            if (g == 0) {
                xo[QT * RT * 256 + q * 128 + n] = m_run[q];
                xo[QT * RT * 256 + q * 128 + 64 + n] = l_run[q];
            }
        }
    }
    __syncthreads();
    if (kh == 1)
        return;
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        const float m1 = xo[QT * RT * 256 + q * 128 + n];
        const float l1 = xo[QT * RT * 256 + q * 128 + 64 + n];
        const float M = fmaxf(m_run[q], m1);
        const float f0 = exp2_fast(m_run[q] - M), f1 = exp2_fast(m1 - M);
        const float l = l_run[q] * f0 + l1 * f1;
        const int r = wr0 + q * 16 + n;
        if (r >= n_rows)
            continue;
        const long long fr = (long long)q0 * H + r;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const floatx4 o1 =
                *reinterpret_cast<const floatx4*>(xo + ((q * RT + rt) * 64 + lane) * 4);
            *reinterpret_cast<floatx4*>(a.out + fr * KV + 16 * rt + 4 * g) =
                (acc[q][rt] * f0 + o1 * f1) * inv;
        }
        if (a.lse && g == 0)
            a.lse[fr] = (M + __log2f(l)) * kLn2;
    }
}

// ------------------------------------------------------------- generic ----
constexpr int kPgThreads = 256;
constexpr int kPgChunk = 1024;  // keys scored per LDS pass
constexpr int kPgMaxAcc = 4;    // kv_rank <= 4 * 256

__device__ float pg_block_reduce(float v, float* red, bool is_max) {
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kPgThreads / 64; ++i)
        r = is_max ? fmaxf(r, red[i]) : r + red[i];
    __syncthreads();
    return r;
}

// Block (i, b, h): query i of session b, head h.
template <typename T>
__global__ __launch_bounds__(kPgThreads) void prefill_generic_kernel(PrefillArgs a) {
    extern __shared__ float smem[];
    const int KV = a.kv_rank, RP = a.rope_dim, PS = a.page_size;
    float* qs = smem;              // KV + RP
    float* sc = smem + KV + RP;    // kPgChunk
    float* red = sc + kPgChunk;    // 4
    const int i = blockIdx.x, b = blockIdx.y, h = blockIdx.z, tid = threadIdx.x;
    if (a.info[0] <= 0)
        return;
    const int q0 = a.cu_q[b], q_len = a.cu_q[b + 1] - q0;
    const int k_len = a.cu_k[b + 1] - a.cu_k[b];
    if (q_len < 2 || i >= q_len)
        return;
    const int len = k_len - q_len + i + 1;  // keys [0, ctx + i]
    const long long fr = ((long long)q0 + i) * a.H + h;
    const long long rec = (long long)PS * (KV + RP);
    const bool tiled = page_tiled(PS, KV, RP);
    const int32_t* ptab = a.page_table + (long long)b * a.max_pages;
    for (int e = tid; e < KV + RP; e += kPgThreads)
        qs[e] = e < KV ? T::to_float(a.q_latent[fr * KV + e])
                       : T::to_float(a.q_rope[fr * RP + e - KV]);
    __syncthreads();
    float m_run = -INFINITY, l_run = 0.0f, acc[kPgMaxAcc] = {0, 0, 0, 0};
    for (int c0 = 0; c0 < len; c0 += kPgChunk) {
        const int cn = min(kPgChunk, len - c0);
        float lmax = -INFINITY;
        for (int t = tid; t < cn; t += kPgThreads) {
            const int tok = c0 + t;
            const int page = ptab[tok / PS];
            float x = -INFINITY;
            if ((unsigned)page < (unsigned)a.num_pool_pages) {
                const uint16_t* base = a.pages + page * rec;
                const int slot = tok % PS;
                float d = 0.0f, dr = 0.0f;
                for (int r = 0; r < KV; ++r)
                    d += T::to_float(base[latent_word(tiled, slot, r, PS, KV)]) * qs[r];
                for (int j = 0; j < RP; ++j)
                    dr += T::to_float(base[rope_word(tiled, slot, j, PS, KV, RP)]) * qs[KV + j];
                x = (dr + d) * a.scale_log2;
            }
            sc[t] = x;
            lmax = fmaxf(lmax, x);
        }
        const float cmax = pg_block_reduce(lmax, red, true);
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m_run - m_new);
        float lsum = 0.0f;
        for (int t = tid; t < cn; t += kPgThreads) {
            const float e = m_new == -INFINITY ? 0.0f : exp2_fast(sc[t] - m_new);
            sc[t] = e;
            lsum += e;
        }
        const float csum = pg_block_reduce(lsum, red, false);  // also orders the sc[] writes
        l_run = l_run * alpha + csum;
        m_run = m_new;
        for (int k = 0; k < kPgMaxAcc; ++k) {
            const int r = tid + k * kPgThreads;
            if (r >= KV)
                break;
            float v = acc[k] * alpha;
            for (int t = 0; t < cn; ++t) {
                const int tok = c0 + t;
                const int page = ptab[tok / PS];
                if ((unsigned)page < (unsigned)a.num_pool_pages && sc[t] != 0.0f)
                    v += sc[t] * T::to_float(a.pages[page * rec + latent_word(tiled, tok % PS, r,
                                                                             PS, KV)]);
            }
            acc[k] = v;
        }
        __syncthreads();
    }
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    for (int k = 0; k < kPgMaxAcc; ++k) {
        const int r = tid + k * kPgThreads;
        if (r < KV)
            a.out[fr * KV + r] = acc[k] * inv;
    }
    if (a.lse && tid == 0)
        a.lse[fr] = (m_run + __log2f(l_run)) * kLn2;
}

// One 16-row tile per q-group: 32 q-rows per workgroup, 138 VGPRs, three workgroups per
// CU (four, at 124 VGPRs and 1024 staged page ids, measured slower: 62.3 us).  Twice as many workgroups as two tiles would give (measured on config 4: 55.7 us
// against 62.4 us), so the dispatcher can even out the sessions' unequal key ranges.
constexpr int kPfQT = 1;

template <typename T>
hipError_t launch_prefill_page(const PrefillArgs& a, int max_q_len, hipStream_t stream) {
    constexpr int rows = kPfQG * kPfQT * 16;
    const long long gx = ((long long)max_q_len * a.H + rows - 1) / rows;
    hipLaunchKernelGGL((prefill_page_kernel<T, 128, 16, 64, kPfQT>), dim3((unsigned)gx, a.B),
                       dim3(64 * kPfWaves), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

bool prefill_mfma_supported(int H, int kv_rank, int rope_dim, int page_size) {
    return H <= 16 && page_size == 64 && kv_rank == 128 && rope_dim == 16;
}

// The MFMA kernel stages a session's page ids in LDS (at most kPfMaxIds pages).
static bool prefill_mfma_fits(const PrefillArgs& a) {
    return prefill_mfma_supported(a.H, a.kv_rank, a.rope_dim, a.page_size) &&
           a.max_pages <= kPfMaxIds;
}

hipError_t launch_prefill(const PrefillArgs& a, int max_q_len, int dtype, bool force_generic,
                          hipStream_t stream) {
    if (a.B <= 0 || max_q_len < 2)
        return hipSuccess;
    if (!force_generic && prefill_mfma_fits(a))
        return dtype == 0 ? launch_prefill_page<F16>(a, max_q_len, stream)
                          : launch_prefill_page<BF16>(a, max_q_len, stream);
    const size_t shmem = (a.kv_rank + a.rope_dim + kPgChunk + 8) * sizeof(float);
    const dim3 grid(max_q_len, a.B, a.H);
    if (dtype == 0)
        hipLaunchKernelGGL(prefill_generic_kernel<F16>, grid, dim3(kPgThreads), shmem, stream, a);
    else
        hipLaunchKernelGGL(prefill_generic_kernel<BF16>, grid, dim3(kPgThreads), shmem, stream,
                           a);
    return hipGetLastError();
}

}  // namespace mla
