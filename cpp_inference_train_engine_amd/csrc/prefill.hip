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
//   flattens (query, head) into q-rows r = i*H + h.  A workgroup of 4 waves owns 32
//   consecutive q-rows of one session (4 queries at H = 8; two 16-row tiles), and every
//   wave holds all 32: Q^T of both tiles in registers, O^T of both in accumulators.  The
//   session's key range is cut into 32-token units (half a page), and wave w streams
//   units w, w+4, w+8, ... through its own two-slot LDS ring (direct global->LDS copies
//   of the tiled record as stored, the next unit in flight while this one is consumed),
//   with its own online-softmax state; no barrier is taken until the four states meet in
//   LDS at the end.  Per unit and q-tile
//     S^T = K . Q^T     v_mfma_f32_16x16x32: the unit's token tiles, read from LDS as
//                       copied, are the A operand; Q^T (latent k-steps + the rope step)
//                       the B operand
//     causal mask (units that hold a row's causal edge only), online softmax in the
//                       log2 domain
//     O^T += C^T . P^T  the S^T accumulators already are P^T's B operand; C^T comes
//                       straight from the tiled unit through the gfx950 transpose read
//                       ds_read_b64_tr_b16 (lane j of a 16-lane group points at 4 latent
//                       values of one token; lane 4a+b receives value b of lanes a, a+4,
//                       a+8, a+12)
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
constexpr int kPfWaves = 4;           // waves per workgroup, each streaming its own units
constexpr int kPfQT = 2;              // 16-row q-tiles per workgroup (shared by its waves)
constexpr int kPfUnit = 32;           // tokens per unit (two 16-token tiles)
constexpr int kPfMaxIds = 512;        // page ids staged in LDS (later pages: page table)
// Latent token rows of odd 256-byte sub-chunks sit at slot row ^ kPfRot in LDS, which puts
// the transpose reads of a sub-chunk pair in disjoint banks (the decode_wide_kernel
// measurement: 0 conflict cycles with 12, 168.6 M per config-5 dispatch as stored).
constexpr int kPfRot = 12;

template <typename T, int KV, int RP, int PS>
__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(2, 8)))
void prefill_page_kernel(PrefillArgs a) {
    static_assert(KV % 32 == 0 && RP % 8 == 0 && RP <= 32 && PS % kPfUnit == 0, "tile shape");
    constexpr int QT = kPfQT;
    constexpr int KS = KV / 32;                // latent k-steps of the score MFMAs
    constexpr int RT = KV / 16;                // 16-row (latent) tiles of O^T
    constexpr int LAT_BLOCKS = 2 * KS;         // 1 KB latent blocks of a unit (two tiles)
    constexpr int ROPE_WORDS = 2 * 16 * RP;    // rope words of a unit
    static_assert(ROPE_WORDS == 512, "a unit's rope keys fill one 1 KB block");
    constexpr int UBLOCKS = LAT_BLOCKS + 1;    // 1 KB blocks of a unit
    constexpr int UREC = UBLOCKS * 512;        // words of a unit
    constexpr int UPP = PS / kPfUnit;          // units per page
    constexpr int WG_ROWS = QT * 16;
    using V8 = typename T::vec8;
    // Unit ring of each wave: even units of its stream in slot0, odd ones in slot1.
    __shared__ __attribute__((aligned(16))) uint16_t slot0[kPfWaves][UREC];
    __shared__ __attribute__((aligned(16))) uint16_t slot1[kPfWaves][UREC];
    __shared__ int32_t pids[kPfMaxIds];  // the session's first page ids

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
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // keys [0, k_hi) are visible to some q-row of this workgroup
    const int last_q = min(n_rows - 1, rb + WG_ROWS - 1) / H;
    const int k_hi = ctx + last_q + 1;
    const int n_units = (k_hi + kPfUnit - 1) / kPfUnit;
    const int32_t* ptab = a.page_table + (long long)b * a.max_pages;
    const long long rec = (long long)PS * (KV + RP);

    // The wave's units: wave, wave + kPfWaves, ...  Unit u is half u % UPP of page u / UPP:
    // its latent is the LAT_BLOCKS contiguous blocks from block LAT_BLOCKS * (u % UPP) of
    // the record, its rope keys the 1 KB at PS*KV + ROPE_WORDS * (u % UPP).  A unit of an
    // invalid page id is not copied (it is zeroed in LDS instead).
    const int n_pages = (n_units + UPP - 1) / UPP;
    auto page_of = [&](int u) {
        const int pg = u / UPP;
        int id;
        if (pg < kPfMaxIds)
            id = pids[pg];
        else
            id = ptab[pg];
        return __builtin_amdgcn_readfirstlane(id);
    };
    // lane l of a latent copy fetches the chunk of LDS slot l: sub-chunk l / 16, token row
    // (l % 16) ^ kPfRot in odd sub-chunks (byte offset in the 1 KB block)
    const uint32_t lat_off = 2 * ((lane >> 4) * 128 + ((lane & 15) ^ (((lane >> 4) & 1) * kPfRot)) * 8);
    auto issue_unit = [&](int u, int page, uint16_t* dst) {
        if ((unsigned)page >= (unsigned)a.num_pool_pages)
            return false;
        const uint16_t* base = a.pages + page * rec;
        const int h = u % UPP;
        const uint32_t l0 = lds_u32(dst);
        static_assert(LAT_BLOCKS % 4 == 0, "latent blocks go in fours");
#pragma unroll
        for (int k = 0; k < LAT_BLOCKS; k += 4)
            copy_4blocks_to_lds_at(base + (LAT_BLOCKS * h + k) * 512, lat_off, l0 + k * 1024);
        copy_block_to_lds_at(base + PS * KV + ROPE_WORDS * h, 16 * lane, l0 + LAT_BLOCKS * 1024);
        return true;
    };

    // ---- Q^T operands of the workgroup's q-rows (every wave holds all of them) ----
    V8 qv[QT][KS + 1];
    int lim[QT];  // lane's q-row n sees keys [0, lim]; -1 = no such row
    const bool rope_lane = 8 * g < RP;
    int u = wave;  // this wave's current unit
    int page_cur = u < n_units ? __builtin_amdgcn_readfirstlane(ptab[u / UPP]) : 0;
    if (u < n_units)
        issue_unit(u, page_cur, slot0[wave]);
    for (int i = tid; i < min(n_pages, kPfMaxIds); i += 64 * kPfWaves)
        pids[i] = ptab[i];
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        const int r = rb + q * 16 + n;
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
    // The first unit and the q operands landed (an explicit wait: the compiler does not
    // see the unit copies, and would otherwise wait for the q loads inside the loop,
    // where that wait would also hold back on the next unit's copies).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();                     // the staged page ids
    int page_nxt = u + kPfWaves < n_units ? page_of(u + kPfWaves) : 0;
    const float inv_scale = 1.0f / a.scale_log2;
    const int rope_off = (16 * (rope_lane ? g : g % (RP / 8)) + n) * 8;
    // transpose-read address of lane (g, j=n) inside a token tile: token 4g + n/4 (its row
    // permuted in odd sub-chunks), latent 4*(n%4) + (row-tile offset)
    const int tr_par = (n & 3) >> 1;
    const int tr_lane = tr_par * 128 + ((4 * g + (n >> 2)) ^ (tr_par * kPfRot)) * 8 + 4 * (n & 1);
    // score A-operand read of lane (g, n): sub-chunk g, token n
    const int s_lane = g * 128 + (n ^ ((g & 1) * kPfRot)) * 8;
    // The lowest causal limit of the workgroup's rows (-1 when some row is past the chunk).
    const int lim_min = rb + WG_ROWS <= n_rows ? ctx + rb / H : -1;

    // The row sums of P come out of the MFMA too: lsum[q] = ONES . P^T, whose A operand is
    // 1 in row 0 (lanes with n == 0) and 0 elsewhere, so lane n of lane group 0 holds the
    // sum for q-row n in element 0 (every other lane and element holds 0).  They are sums
    // of the probabilities as rounded for the P.C product, the weights the numerator uses.
    float m_run[QT], l_run[QT];
    floatx4 acc[QT][RT], lsum[QT];
    const V8 ones = n == 0 ? T::ones8() : V8{};
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        m_run[q] = kPfNoMax;
        lsum[q] = floatx4{0, 0, 0, 0};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            acc[q][rt] = floatx4{0, 0, 0, 0};
    }

    // Scores, mask, online softmax and PV of unit u (in LDS at sp).
    auto compute = [&](const uint16_t* sp, int uu) {
        const int tok0 = uu * kPfUnit;
        // the 2 x QT score tiles advance together, k-step by k-step: four independent
        // accumulation chains, so no MFMA waits on the one before it
        floatx4 sc[2][QT];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int q = 0; q < QT; ++q)
                sc[tt][q] = floatx4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j <= KS; ++j) {
            V8 ka[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
                ka[tt] = j < KS ? *reinterpret_cast<const V8*>(sp + (tt * KS + j) * 512 + s_lane)
                                : *reinterpret_cast<const V8*>(sp + LAT_BLOCKS * 512 +
                                                               tt * 16 * RP + rope_off);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int q = 0; q < QT; ++q)
                    sc[tt][q] = T::mma32(ka[tt], qv[q][j], sc[tt][q]);
        }
        // Every row of the workgroup sees all 32 tokens of this unit unless it holds the
        // causal edge (or rows past the chunk): only then are tokens masked.
        if (!(tok0 + kPfUnit - 1 <= lim_min)) {
#pragma unroll
            for (int q = 0; q < QT; ++q)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (tok0 + 16 * tt + 4 * g + i > lim[q])
                            sc[tt][q][i] = -INFINITY;
        }
        V8 pb[QT], pl[QT];  // P^T operands (pl: the low part, bf16 only)
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            // log2 units; m_run starts at a finite floor, so exp2 never sees inf - inf.
            // The reference max m_run is raised only when a score exceeds it by more than
            // kPfRescale; below that the probabilities are exp2(x - m_run) <= 2^kPfRescale,
            // exact in fp32 and fp16, and the final normalisation divides by the same-based
            // sum.  Each lane compares its own raw scores with the threshold (the scale is
            // > 0), so the row max (a cross-lane reduction) is formed only on the rare
            // units that raise the reference, and the accumulators are rescaled only when
            // a row that has accumulated something is raised.
            const float thr = (m_run[q] + kPfRescale) * inv_scale;
            bool rise = false;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    rise |= sc[tt][q][i] > thr;
            if (__builtin_amdgcn_ballot_w64(rise)) {
                float mp = fmaxf(fmaxf(fmaxf(sc[0][q][0], sc[0][q][1]), fmaxf(sc[0][q][2], sc[0][q][3])),
                                 fmaxf(fmaxf(sc[1][q][0], sc[1][q][1]), fmaxf(sc[1][q][2], sc[1][q][3])));
                mp = rows_max(mp);
                const float m_new = fmaxf(m_run[q], mp * a.scale_log2);
                const bool had = m_run[q] != kPfNoMax;  // the row has accumulated state
                if (__builtin_amdgcn_ballot_w64(had && m_new > m_run[q])) {
                    const float alpha = exp2_fast(m_run[q] - m_new);
                    lsum[q] *= alpha;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        acc[q][rt] *= alpha;
                }
                m_run[q] = m_new;
            }
            const float m_ref = m_run[q];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = exp2_fast(fmaf(sc[tt][q][i], a.scale_log2, -m_ref));
                    const auto hi = static_cast<typename T::scalar>(e);
                    pb[q][4 * tt + i] = hi;
                    if constexpr (T::split_p)
                        pl[q][4 * tt + i] =
                            static_cast<typename T::scalar>(e - static_cast<float>(hi));
                }
        }
        // O^T += C^T . P^T over the unit's 32 tokens (one K-step per 16 latent rows)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int blk = ((rt >> 1) * 4 + 2 * (rt & 1)) * 128;  // latent rows 16rt..
            const u32x2 lo = lds_read_tr16(sp + blk + tr_lane);
            const u32x2 hi = lds_read_tr16(sp + KS * 512 + blk + tr_lane);
            const V8 ca = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                acc[q][rt] = T::mma32(ca, pb[q], acc[q][rt]);
                if constexpr (T::split_p)
                    acc[q][rt] = T::mma32(ca, pl[q], acc[q][rt]);
            }
        }
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            lsum[q] = T::mma32(ones, pb[q], lsum[q]);
            if constexpr (T::split_p)
                lsum[q] = T::mma32(ones, pl[q], lsum[q]);
        }
    };
    // Tokens of unit uu at or past k_len, or the whole unit when its page id is invalid,
    // read as zero: the unit's chunks are cleared in LDS (chunk c of block k holds token
    // 16 * (k / KS) + ((c % 16) ^ kPfRot when c / 16 is odd) of a latent block, and
    // 16 * (c / 32) + c % 16 of the rope block).
    auto clear_tail = [&](uint16_t* sp, int uu, int page) {
        const int valid = (unsigned)page < (unsigned)a.num_pool_pages ? k_len - uu * kPfUnit : 0;
        if (valid >= kPfUnit)
            return;
#pragma unroll
        for (int k = 0; k < UBLOCKS; ++k) {
            const int tok = k < LAT_BLOCKS ? 16 * (k / KS) + (n ^ ((g & 1) * kPfRot))
                                           : 16 * (lane >> 5) + n;
            if (tok >= valid)
                *reinterpret_cast<u32x4*>(sp + k * 512 + lane * 8) = u32x4{0, 0, 0, 0};
        }
        wave_lds_fence();
    };

    // The wave's stream: unit u sits in slot (i & 1) for its i-th unit; the copy of the
    // next unit goes out before this one is consumed.  Only this wave touches its slots,
    // so no workgroup barrier is needed until the final merge.
    for (int i = 0; u < n_units; ++i, u += kPfWaves) {
        uint16_t* cur = (i & 1) ? slot1[wave] : slot0[wave];
        uint16_t* nxt = (i & 1) ? slot0[wave] : slot1[wave];
        const bool more = u + kPfWaves < n_units;
        const int page_after = u + 2 * kPfWaves < n_units ? page_of(u + 2 * kPfWaves) : 0;
        if (more && issue_unit(u + kPfWaves, page_nxt, nxt))
            __builtin_amdgcn_s_waitcnt(0x0F70 | UBLOCKS);  // vmcnt(UBLOCKS): the next unit's
                                                           // copies may still be in flight
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        wave_lds_fence();
        clear_tail(cur, u, page_cur);
        compute(cur, u);
        page_cur = page_nxt;
        page_nxt = page_after;
        wave_lds_fence();  // this slot's reads are done before the next copy into it
    }

    // ---- the waves' softmax states meet in LDS; normalise and store ----
#pragma unroll
    for (int q = 0; q < QT; ++q)
        l_run[q] = rows_sum(lsum[q][0]);  // lane group 0's value, to every lane of column n
    __syncthreads();  // every wave is done with its slots
    // per wave: acc [QT][RT][64 lanes] floatx4, then m and l of its 32 rows
    constexpr int XO = QT * RT * 64 * 4;
    static_assert((XO + 2 * WG_ROWS) * 4 <= UREC * 2 * 2, "a wave's state fits its two slots");
    auto xo_of = [&](int v) {
        return reinterpret_cast<float*>(v < 2 ? &slot0[2 * v][0] : &slot1[2 * (v - 2)][0]);
    };
    {
        float* xo = xo_of(wave);
#pragma unroll
        for (int q = 0; q < QT; ++q) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                *reinterpret_cast<floatx4*>(xo + ((q * RT + rt) * 64 + lane) * 4) = acc[q][rt];
            if (g == 0) {
                xo[XO + q * 16 + n] = m_run[q];
                xo[XO + WG_ROWS + q * 16 + n] = l_run[q];
            }
        }
    }
    __syncthreads();
    // thread t: q-row r = t / RT (of the workgroup's 32), latent rows 16 rt .. 16 rt + 15
    static_assert(WG_ROWS * RT == 64 * kPfWaves, "one thread per (row, latent tile)");
    const int r = tid / RT, rt = tid % RT;
    const int q = r / 16, rn = r % 16;
    float mv[kPfWaves], M = kPfNoMax;
#pragma unroll
    for (int v = 0; v < kPfWaves; ++v) {
        mv[v] = xo_of(v)[XO + r];
        M = fmaxf(M, mv[v]);
    }
    float L = 0.0f;
    floatx4 o[4] = {};
#pragma unroll
    for (int v = 0; v < kPfWaves; ++v) {
        const float* xo = xo_of(v);
        const float f = exp2_fast(mv[v] - M);
        L += xo[XO + WG_ROWS + r] * f;
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
            o[gg] += *reinterpret_cast<const floatx4*>(xo + ((q * RT + rt) * 64 + gg * 16 + rn) * 4) * f;
    }
    const int row = rb + r;
    if (row >= n_rows)
        return;
    const long long fr = (long long)q0 * H + row;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg)
        *reinterpret_cast<floatx4*>(a.out + fr * KV + 16 * rt + 4 * gg) = o[gg] * inv;
    if (a.lse && rt == 0)
        a.lse[fr] = (M + __log2f(L)) * kLn2;
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

template <typename T>
hipError_t launch_prefill_page(const PrefillArgs& a, int max_q_len, hipStream_t stream) {
    constexpr int rows = kPfQT * 16;
    const long long gx = ((long long)max_q_len * a.H + rows - 1) / rows;
    hipLaunchKernelGGL((prefill_page_kernel<T, 128, 16, 64>), dim3((unsigned)gx, a.B),
                       dim3(64 * kPfWaves), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

bool prefill_mfma_supported(int H, int kv_rank, int rope_dim, int page_size) {
    return H <= 16 && page_size == 64 && kv_rank == 128 && rope_dim == 16;
}


hipError_t launch_prefill(const PrefillArgs& a, int max_q_len, int dtype, bool force_generic,
                          hipStream_t stream) {
    if (a.B <= 0 || max_q_len < 2)
        return hipSuccess;
    if (!force_generic && prefill_mfma_supported(a.H, a.kv_rank, a.rope_dim, a.page_size))
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
