// (c) Absorbed MLA decode attention at the DeepSeek-like latent shape, gfx950:
// 128 heads, kv_rank 512, rope 64, 64-token tiled pages (bf16 or fp16).
//
// Same math as decode_page_kernel (src/infer/inference.cpp:116-153), but the shape
// turns it MFMA-heavy: per cached token 128 heads x (576 + 512) MACs against 1152
// bytes, ~242 flop per byte, close to the bf16 MFMA ridge (2.5 PFLOP/s / 8 TB/s).
//
// decode_wide_kernel -- one workgroup of WAVES waves per work item (session, page
//   range); wave v owns HT 16-head tiles (heads 16*HT*v ..), so the waves never
//   exchange softmax state.  Each wave keeps its Q^T operands (HT x 18 k-steps) in
//   registers and its O^T accumulators (kv_rank x 16*HT fp32) in AGPRs.  The item's
//   pages stream through two LDS page buffers (2 x 72 KB) filled by gfx950 direct
//   global->LDS loads (global_load_lds_dwordx4: each wave instruction copies 1 KB of
//   the tiled record, no VGPR staging), so page p+1 is in flight while page p is
//   consumed.  Per 32-token unit of a page:
//     S^T = K . Q^T      v_mfma_f32_16x16x32: token tiles read from LDS as stored
//                        (1 KB per wave read), 16 latent + 2 rope k-steps
//     online softmax     log2 domain; the accumulators are rescaled only when a
//                        head's running maximum rises
//     O^T += C^T . P^T   C^T through the transpose read ds_read_b64_tr_b16 straight
//                        from the tiled record; the S^T accumulators are P^T's B
//                        operand as they stand (bf16: hi + lo parts)
//   Slots past the session's end in its last page are zeroed in LDS before use.
#include "mla_common.hpp"
#include "mla_internal.hpp"

#include <cmath>

namespace mla {
namespace {

constexpr int kWideMaxItemPages = 512;  // page ids of an item staged in LDS
constexpr float kWideNoMax = -1.0e30f;  // running-max floor: below every real score
constexpr float kWideRescale = 8.0f;    // log2 headroom before the running max is raised
// Latent token rows of odd 256-byte sub-chunks sit at slot row ^ kWideRot in LDS.  With 12
// the transpose reads of the two sub-chunks of a pair fall in disjoint banks: measured at
// config 5, SQ_LDS_BANK_CONFLICT is 0 cycles per dispatch (168.6 M with 0, 1, 2, 3 or 8;
// 337 M with 4).
constexpr int kWideRot = 12;

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s4 __attribute__((address_space(3)))*)((__attribute__((address_space(3))) char*)p));
    return __builtin_bit_cast(u32x2, v);
}

template <typename T, int KV, int RP, int PS, int HT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void decode_wide_kernel(DecodeArgs a) {
    static_assert(KV % 32 == 0 && RP % 32 == 0 && PS % 32 == 0, "tile shape");
    constexpr int KS = KV / 32;          // latent k-steps
    constexpr int RS = RP / 32;          // rope k-steps
    constexpr int UPP = PS / 32;         // 32-token units per page
    constexpr int RT = KV / 16;          // latent row tiles of O^T
    constexpr int REC = PS * (KV + RP);  // words of a page record
    constexpr int BLOCKS = REC / 512;    // 1 KB blocks of a record
    constexpr int CHUNKS = REC / 8;      // 16-byte chunks of a record
    constexpr int LAT_BLOCKS = PS * KV / 512;  // latent 1 KB blocks (the rest is rope)
    constexpr int THREADS = 64 * WAVES;
    constexpr int kBlocksPerWave = BLOCKS / WAVES;  // page-copy blocks each wave issues
    static_assert(REC % 512 == 0 && BLOCKS % WAVES == 0, "record blocks");
    static_assert(kBlocksPerWave <= KS + RS, "a wave's copy blocks fit the first unit's k-steps");
    using V8 = typename T::vec8;
    __shared__ __attribute__((aligned(16))) uint16_t buf0[REC];
    __shared__ __attribute__((aligned(16))) uint16_t buf1[REC];
    __shared__ int32_t pids[kWideMaxItemPages];  // the item's page ids

    const int w = blockIdx.x;
    const int32_t* d = a.work_desc + (long long)w * kWorkDescInts;
    const int s = d[0];
    if (s < 0 || d[7] != 1)
        return;  // past the last item (or a failed build), or not a decode row
    const int row = d[1], kl = d[2], p_begin = d[3], p_end = d[4], ns = d[5], slot = d[6];
    const int H = a.H;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t* ptab = a.page_table + (long long)s * a.max_pages;

    // Latent blocks land in LDS with the token rows of odd 256-byte sub-chunks permuted
    // (row ^ kWideRot; lane l of the copy fetches the chunk that belongs at LDS slot l):
    // the transpose reads of two adjacent sub-chunks then hit disjoint banks.  Rope blocks
    // are copied as stored.
    const int lat_src = (lane >> 4) * 128 + ((lane & 15) ^ (((lane >> 4) & 1) * kWideRot)) * 8;
    auto page_src = [&](int page) {
        return a.pages + (long long)((unsigned)page < (unsigned)a.num_pool_pages ? page : 0) * REC;
    };
    // Block k of this wave's share of a page copy: record block wave + WAVES * k.
    const uint32_t lat_off = 2 * lat_src, rope_off_b = 16 * lane;  // lane byte offsets
    auto issue_block = [&](const uint16_t* base, uint16_t* dst, int k) {
        const int bk = wave + WAVES * k;
        copy_block_to_lds(base + bk * 512, bk < LAT_BLOCKS ? lat_off : rope_off_b,
                          dst + bk * 512);
    };
    // Page ids come from LDS (staged below) for the item's first kWideMaxItemPages pages.
    auto page_id = [&](int p) {
        const int i = p - p_begin;
        int id;
        if (i < kWideMaxItemPages)
            id = pids[i];
        else
            id = ptab[p];
        return __builtin_amdgcn_readfirstlane(id);
    };
    {  // the first page in flight while q and the ids load
        const uint16_t* base = page_src(__builtin_amdgcn_readfirstlane(ptab[p_begin]));
#pragma unroll
        for (int k = 0; k < kBlocksPerWave; ++k)
            issue_block(base, buf0, k);
    }
    for (int i = tid; i < min(p_end - p_begin, kWideMaxItemPages); i += THREADS)
        pids[i] = ptab[p_begin + i];

    // ---- Q^T operands: head 16*(HT*wave + ht) + n, dims 32j + 8g .. +7 ----
    V8 qv[HT][KS + RS];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
        const int head = 16 * (HT * wave + ht) + n;
        const bool ok = head < H;
        const long long q = (long long)row * H + head;
#pragma unroll
        for (int j = 0; j < KS; ++j)
            qv[ht][j] = ok ? *reinterpret_cast<const V8*>(a.q_latent + q * KV + 32 * j + 8 * g)
                           : V8{};
#pragma unroll
        for (int j = 0; j < RS; ++j)
            qv[ht][KS + j] =
                ok ? *reinterpret_cast<const V8*>(a.q_rope + q * RP + 32 * j + 8 * g) : V8{};
    }
    // transpose-read address of lane (g, n) in a 16-token tile: sub-chunk parity
    // (n & 3) >> 1 (odd sub-chunks: rows permuted by ^ kWideRot), token 4g + n/4, half n & 1
    const int tr_par = (n & 3) >> 1;
    const int tr_lane = tr_par * 128 + ((4 * g + (n >> 2)) ^ (tr_par * kWideRot)) * 8 + 4 * (n & 1);
    // score A-operand read of lane (g, n): sub-chunk g, token n
    const int s_lane = g * 128 + (n ^ ((g & 1) * kWideRot)) * 8;

    float m_run[HT], l_run[HT];
    floatx4 acc[RT][HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
        m_run[ht] = kWideNoMax;
        l_run[ht] = 0.0f;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            acc[rt][ht] = floatx4{0, 0, 0, 0};
    }

    // With has_next, the page after p (record `next`) is copied into `next_dst` one block
    // per k-step of the first unit's scores, so the copies go out while the wave
    // computes instead of ahead of it.
    auto compute_page = [&](const uint16_t* pg, int p, bool has_next, const uint16_t* next,
                            uint16_t* next_dst) {
        const int valid = min(PS, kl - p * PS);  // >= 1 inside [p_begin, p_end)
        if (valid < PS) {
            // the session's last page: zero the slots past its end (they may hold any bits)
            uint16_t* wpg = const_cast<uint16_t*>(pg);
            for (int c = tid; c < CHUNKS; c += THREADS) {
                const int slot =
                    c < PS * KV / 8
                        ? (c / (16 * 4 * KS)) * 16 + ((c & 15) ^ (((c >> 4) & 1) * kWideRot))
                        : ((c - PS * KV / 8) / (16 * (RP / 8))) * 16 + (c & 15);
                if (slot >= valid)
                    *reinterpret_cast<u32x4*>(wpg + c * 8) = u32x4{0, 0, 0, 0};
            }
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < UPP; ++u) {
            // S^T of the unit's two token tiles, k-step by k-step (two independent MFMA
            // chains), the next k-step's operands read while this one's MFMAs run.
            floatx4 sc[2][HT];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int ht = 0; ht < HT; ++ht)
                    sc[tt][ht] = floatx4{0, 0, 0, 0};
            auto k_operand = [&](int tt, int j) {
                const int t = 2 * u + tt;
                return j < KS ? *reinterpret_cast<const V8*>(pg + (t * KS + j) * 512 + s_lane)
                              : *reinterpret_cast<const V8*>(
                                    pg + PS * KV + (t * (RP / 8) + 4 * (j - KS)) * 128 + lane * 8);
            };
            V8 kn[2] = {k_operand(0, 0), k_operand(1, 0)};
#pragma unroll
            for (int j = 0; j < KS + RS; ++j) {
                if (u == 0 && j < kBlocksPerWave && has_next)
                    issue_block(next, next_dst, j);
                const V8 k0 = kn[0], k1 = kn[1];
                if (j + 1 < KS + RS) {
                    kn[0] = k_operand(0, j + 1);
                    kn[1] = k_operand(1, j + 1);
                }
#pragma unroll
                for (int ht = 0; ht < HT; ++ht) {
                    sc[0][ht] = T::mma32(k0, qv[ht][j], sc[0][ht]);
                    sc[1][ht] = T::mma32(k1, qv[ht][j], sc[1][ht]);
                }
            }
            V8 pb[HT], pl[HT];
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) {
                // log2 units.  The reference max m_run (from a finite floor) is raised only
                // when a score passes it by more than kWideRescale: below that the
                // probabilities are at most 2^kWideRescale (exact in fp32, and the bf16
                // hi + lo split is relative), and the partial (m, l, o) is consistent for
                // any reference.  Each lane compares its own scores, so the row max (a
                // cross-lane reduction) is formed only on the units that raise it, and the
                // accumulators are rescaled only when a head with accumulated state is.
                bool rise = false;
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int slot = 32 * u + 16 * tt + 4 * g + i;
                        const float x = slot < valid ? sc[tt][ht][i] * a.scale_log2 : -INFINITY;
                        sc[tt][ht][i] = x;
                        rise |= x > m_run[ht] + kWideRescale;
                    }
                if (__ballot(rise)) {
                    float mp = -INFINITY;
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            mp = fmaxf(mp, sc[tt][ht][i]);
                    const float m_new = fmaxf(m_run[ht], rows_max(mp));
                    const bool had = m_run[ht] != kWideNoMax;  // the head has accumulated
                    if (__ballot(had && m_new > m_run[ht])) {
                        const float alpha = exp2_fast(m_run[ht] - m_new);
                        l_run[ht] *= alpha;
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt)
                            acc[rt][ht] *= alpha;
                    }
                    m_run[ht] = m_new;
                }
                float psum = 0.0f;
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float e = exp2_fast(sc[tt][ht][i] - m_run[ht]);
                        psum += e;
                        const auto hi = static_cast<typename T::scalar>(e);
                        pb[ht][4 * tt + i] = hi;
                        if constexpr (T::split_p)
                            pl[ht][4 * tt + i] =
                                static_cast<typename T::scalar>(e - static_cast<float>(hi));
                    }
                l_run[ht] += psum;
            }
            // O^T += C^T . P^T, two latent tiles at a time: the transpose reads of the
            // next pair are issued before this pair's MFMAs, and the hi / lo MFMAs of the
            // two tiles alternate so no MFMA waits on the one just issued.
            const uint16_t* c0 = pg + (2 * u) * KS * 512 + tr_lane;
            const uint16_t* c1 = pg + (2 * u + 1) * KS * 512 + tr_lane;
            auto tile_off = [](int rt) { return ((rt >> 1) * 4 + 2 * (rt & 1)) * 128; };
            V8 ca[2], cn[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const u32x2 lo = lds_read_tr16(c0 + tile_off(k)), hi = lds_read_tr16(c1 + tile_off(k));
                cn[k] = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt += 2) {
                ca[0] = cn[0];
                ca[1] = cn[1];
                if (rt + 2 < RT) {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const u32x2 lo = lds_read_tr16(c0 + tile_off(rt + 2 + k));
                        const u32x2 hi = lds_read_tr16(c1 + tile_off(rt + 2 + k));
                        cn[k] = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                    }
                }
#pragma unroll
                for (int ht = 0; ht < HT; ++ht) {
                    acc[rt][ht] = T::mma32(ca[0], pb[ht], acc[rt][ht]);
                    acc[rt + 1][ht] = T::mma32(ca[1], pb[ht], acc[rt + 1][ht]);
                    if constexpr (T::split_p) {
                        acc[rt][ht] = T::mma32(ca[0], pl[ht], acc[rt][ht]);
                        acc[rt + 1][ht] = T::mma32(ca[1], pl[ht], acc[rt + 1][ht]);
                    }
                }
            }
        }
    };

    // Page p of the item lives in buf0 when (p - p_begin) is even, buf1 when odd.  Each
    // round: wait for this wave's copies of page p, barrier (every wave's copies landed,
    // and every wave is done with page p - 1, whose buffer the copies of page p + 1 now
    // overwrite), consume page p while issuing page p + 1.
    for (int p = p_begin; p < p_end; ++p) {
        const bool odd = (p - p_begin) & 1;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of page p landed
        __syncthreads();
        const bool has_next = p + 1 < p_end;
        const uint16_t* next = has_next ? page_src(page_id(p + 1)) : a.pages;
        compute_page(odd ? buf1 : buf0, p, has_next, next, odd ? buf0 : buf1);
    }

    // ---- this wave's heads: final rows (one-item sessions) or split partials ----
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
        float l = l_run[ht];
        l = rows_sum(l);
        const int head = 16 * (HT * wave + ht) + n;
        if (head >= H)
            continue;
        if (ns == 1) {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            float* o = a.out + ((long long)row * H + head) * KV;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                *reinterpret_cast<floatx4*>(o + 16 * rt + 4 * g) = acc[rt][ht] * inv;
            if (a.lse && g == 0)
                a.lse[(long long)row * H + head] = (m_run[ht] + __log2f(l)) * kLn2;
        } else {
            float* o = a.part_o + ((long long)slot * H + head) * KV;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                *reinterpret_cast<floatx4*>(o + 16 * rt + 4 * g) = acc[rt][ht];
            if (g == 0) {
                a.part_ml[(long long)slot * part_ml_stride(H) + 2 * head] = m_run[ht];
                a.part_ml[(long long)slot * part_ml_stride(H) + 2 * head + 1] = l;
            }
        }
    }
}

constexpr int kWideHT = 1, kWideWaves = 8;

template <typename T>
hipError_t launch_wide_t(const DecodeArgs& a, int grid, hipStream_t stream) {
    hipLaunchKernelGGL((decode_wide_kernel<T, 512, 64, 64, kWideHT, kWideWaves>), dim3(grid),
                       dim3(64 * kWideWaves), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

bool decode_wide_supported(int H, int kv_rank, int rope_dim, int page_size) {
    return H > 16 && H <= 16 * kWideHT * kWideWaves && kv_rank == 512 && rope_dim == 64 &&
           page_size == 64;
}

hipError_t launch_decode_wide(const DecodeArgs& a, int dtype, hipStream_t stream) {
    return dtype == 0 ? launch_wide_t<F16>(a, a.max_work, stream)
                      : launch_wide_t<BF16>(a, a.max_work, stream);
}

}  // namespace mla
