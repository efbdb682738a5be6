// (c) Absorbed MLA decode attention over the paged latent cache, gfx950.
//
// Math (src/infer/inference.cpp:116-153; mps_backend.mm:556-572), per session
// b with one query row and per head h:
//     s_i   = (q_latent[h] . c_i + q_rope[h] . k_i) * scale,   i < k_len
//     out_h = sum_i softmax(s)_i c_i,      lse_h = ln sum_i exp(s_i)
//
// Work decomposition: the metadata's work items (session, split) each cover
// `split` pages of one session (split-K).  Every item produces the online-
// softmax state (m, l, o) of its pages; sessions with one item write the
// final row directly, the rest are combined by merge_kernel (log-sum-exp).
//
// decode_mfma_kernel -- one workgroup of 2 waves per work item, pages of 64 tokens
//   in the tiled record layout, processed as 32-token units:
//   S^T[tok][head] = K[tok][:] . Q^T on v_mfma_f32_16x16x32 (latent K-steps, then
//   the rope key zero-padded to one 32-wide K-step): the unit's cache tile is the
//   A operand straight from HBM (each 16-byte lane load reads 1 KB contiguously)
//   and Q^T (heads padded to 16) is the B operand, read from the workgroup's LDS
//   Q tile.  The S^T output layout puts, in lane (g, n), head n and tokens
//   16t+4g+{0..3}: exactly the lane's B operand of O^T = C^T . P^T, so P never
//   leaves registers.  C^T is obtained by writing the unit's latent rows to a
//   per-wave row-major LDS tile and reading it back with the gfx950 transpose
//   load (ds_read_b64_tr_b16).  Online softmax runs in the log2 domain with a
//   lazy rescale (the shared max is only raised when a score exceeds it by 2^8).
//   Each wave keeps the next unit's loads in flight while computing the current
//   one; the two waves' states merge in LDS at the end of the item.
// decode_generic_kernel -- any H / kv_rank / rope / page size / layout: one
//   256-thread block per (work item, head), VALU fp32.
// merge_kernel -- log-sum-exp combine of the split partials, one block per
//   (session, head), launched after the decode kernel on the same stream.
#include "mla_common.hpp"
#include "mla_internal.hpp"

#include <cmath>

namespace mla {
namespace {

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- MFMA ----
// A 32-token unit = two 16-token MFMA tiles.  Lane (g, n) holds, as the A
// operands of S^T, token 16t+n of the unit: 16 latent bytes per 32-wide K-step
// and the rope key padded to 32-wide K-steps (lane groups past rope_dim hold
// zeros in both operands).  Every MFMA of the kernel is 16x16x32: the legacy
// 16x16x16 form got a destination partially overlapping its accumulator input
// from the register allocator, which corrupts results.
template <int KV, int RP>
struct UnitRegs {
    static constexpr int KS = KV / 32, RS = (RP + 31) / 32;
    u32x4 lat[2][KS];
    u32x4 rop[2][RS];
};

// Loads tokens slot0..slot0+31 of a TILED page record (see page_tiled): every
// 16-byte lane load of the wave reads one contiguous 1 KB block (or 512 B of rope).
// Only the first `valid` tokens are read; the rest are zero.
template <int KV, int RP, int PS>
__device__ __forceinline__ void load_unit(UnitRegs<KV, RP>& u, const uint16_t* base, int slot0,
                                          int valid, int g, int n) {
    constexpr int KS = UnitRegs<KV, RP>::KS, RS = UnitRegs<KV, RP>::RS;
    const int lane8 = (16 * g + n) * 8;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int tile = (slot0 >> 4) + t;
        const bool ok = 16 * t + n < valid;
#pragma unroll
        for (int j = 0; j < KS; ++j)
            u.lat[t][j] = ok ? *reinterpret_cast<const u32x4*>(base + (tile * KS + j) * 512 + lane8)
                             : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < RS; ++k)
            u.rop[t][k] = ok && 32 * k + 8 * g < RP
                              ? *reinterpret_cast<const u32x4*>(base + PS * KV +
                                                                (tile * (RP / 8) + 4 * k) * 128 +
                                                                lane8)
                              : u32x4{0, 0, 0, 0};
    }
}

// Row-major latent unit in LDS for the C^T operand: [32 tokens][kv_rank + 16]
// 16-bit words.  The pad puts consecutive rows 32 bytes apart in the banks, which
// makes the transpose reads (4 rows x 32 bytes per 16 lanes) conflict-free; the
// 16-byte row writes (8 or 16 lanes at a time, rows n = 0..15) then hit every bank
// pair twice, so each row's 16-byte chunks are swapped in pairs (chunk c stored at
// c ^ lds_swz(row)) when bit 2 and bit 3 of the row differ.  That XOR only flips the
// lane-constant part of a transpose read's column, so the reads stay conflict-free
// and keep immediate offsets.
template <int KV>
constexpr int unit_pitch() {
    return KV + 16;
}
__device__ __forceinline__ int lds_swz(int row) { return ((row >> 2) ^ (row >> 3)) & 1; }

// Q tile in LDS: row h = [latent KV | rope padded to 32*RS | 8 pad], 16 rows.
template <int KV, int RP>
constexpr int q_stride() {
    return KV + 32 * ((RP + 31) / 32) + 8;
}

// Lazy online softmax: probabilities are taken against a shared reference max that
// is only raised (with a rescale of the state) when some score exceeds it by more
// than 2^kRescaleLog2; otherwise p <= 2^8 and the state needs no rescale.
constexpr float kRescaleLog2 = 8.0f;

// gfx950 LDS transpose read: in each 16-lane group, lane j supplies an 8-byte row
// R_j; lane i = 4a+b receives {R_a[b], R_{a+4}[b], R_{a+8}[b], R_{a+12}[b]}.
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s4 __attribute__((address_space(3)))*)((__attribute__((address_space(3))) char*)p));
    return __builtin_bit_cast(u32x2, v);
}

// Scores of one unit, online-softmax update, O^T += C^T . P^T.  `valid` tokens of
// the unit count; the rest are masked.  myl is this wave's LDS unit tile.
template <typename T, int KV, int RP>
__device__ __forceinline__ void process_unit(const UnitRegs<KV, RP>& u, int valid,
                                             const uint16_t* qs, float scale_log2, float& m_run,
                                             float& l_run, floatx4* acc, uint16_t* myl, int g,
                                             int n) {
    constexpr int KS = UnitRegs<KV, RP>::KS, RS = UnitRegs<KV, RP>::RS;
    constexpr int RT = KV / 16;
    constexpr int UP = unit_pitch<KV>();
    constexpr int QS = q_stride<KV, RP>();
    using V8 = typename T::vec8;
    // S^T[16t + 4g + i][head n]; B operand Q^T read from the LDS tile (head n).
    const uint16_t* qrow = qs + n * QS + 8 * g;
    floatx4 sc[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int j = 0; j < KS + RS; ++j) {
        const V8 b = *reinterpret_cast<const V8*>(qrow + 32 * j);
#pragma unroll
        for (int t = 0; t < 2; ++t)
            sc[t] = T::mma32(__builtin_bit_cast(V8, j < KS ? u.lat[t][j] : u.rop[t][j - KS]), b,
                             sc[t]);
    }
    // Latent rows to the LDS tile: lane (g, n) stores token 16t+n, columns 32j+8g..+7 at
    // 8-column chunk g ^ swz(n) (see lds_swz).
    const int wchunk = g ^ lds_swz(n);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < KS; ++j)
            *reinterpret_cast<u32x4*>(myl + (16 * t + n) * UP + 32 * j + 8 * wchunk) = u.lat[t][j];
    float mloc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = 16 * t + 4 * g + i < valid ? sc[t][i] * scale_log2 : -INFINITY;
            sc[t][i] = x;
            mloc = fmaxf(mloc, x);
        }
    if (__ballot(mloc > m_run + kRescaleLog2)) {  // wave-uniform, rare after the first unit
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int r = 0; r < RT; ++r)
            acc[r] *= alpha;
        m_run = m_new;
    }
    float psum = 0.0f;
    V8 pb;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e = m_run == -INFINITY ? 0.0f : exp2_fast(sc[t][i] - m_run);
            psum += e;
            pb[4 * t + i] = static_cast<typename T::scalar>(e);
        }
    l_run += psum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // A = C^T: lane (g, n) needs column 16rt+n of tokens 4g..4g+3 (K-slots 0..3) and
    // 16+4g..16+4g+3 (slots 4..7); lane (g, j) of the transpose read points at row
    // 4g+j/4, columns 16rt+4(j%4).. .  B = P^T (lane: head n, the same 8 tokens).
    const uint16_t* src = myl + (4 * g + (n >> 2)) * UP + 4 * ((n & 3) ^ (2 * lds_swz(4 * g)));
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const u32x2 lo = lds_read_tr16(src + 16 * rt);
        const u32x2 hi = lds_read_tr16(src + 16 * UP + 16 * rt);
        acc[rt] = T::mma32(__builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]}), pb, acc[rt]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One workgroup of WAVES waves per work item (session, split); wave v streams the
// 32-token units of pages p_begin+v, p_begin+v+WAVES, ... keeping the next unit's
// loads in flight while it computes the current one.  The waves' softmax states
// merge in LDS; a session split over several
// workgroups leaves one partial per workgroup for merge_kernel (the next launch on
// the stream, so the partials are coherent without device-scope fences).
// Up to 256 VGPRs (2 waves/SIMD); each wave keeps one 32-token unit in flight while
// computing the other and reads Q^T from the workgroup's LDS tile.
#ifndef MLA_DECODE_WAVES_PER_EU
#define MLA_DECODE_WAVES_PER_EU 2
#endif

template <typename T, int KV, int RP, int PS, int WAVES>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(MLA_DECODE_WAVES_PER_EU, 8))) void decode_mfma_kernel(DecodeArgs a) {
    static_assert(KV % 32 == 0 && RP % 8 == 0 && PS % 32 == 0, "tile shape");
    constexpr int UPP = PS / 32;      // 32-token units per page
    constexpr int KS = KV / 32, RS = (RP + 31) / 32;
    constexpr int RT = KV / 16;       // 16-row tiles of O^T
    constexpr int TBUF = 32 * unit_pitch<KV>();  // per-wave LDS unit tile, 16-bit words
    constexpr int MSTRIDE = KV + 4;   // LDS merge pitch, floats
    constexpr int THREADS = 64 * WAVES;
    static_assert(16 * MSTRIDE * 4 <= TBUF * 2, "merge buffer aliases transpose buffer");
    using V8 = typename T::vec8;
    constexpr int QS = q_stride<KV, RP>();
    __shared__ __attribute__((aligned(16))) uint16_t lds[WAVES][TBUF];
    __shared__ __attribute__((aligned(16))) uint16_t q_s[16 * QS];
    __shared__ float sm_m[WAVES][16], sm_l[WAVES][16];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const long long rec = (long long)PS * (KV + RP);
    const bool head_ok = n < a.H;
    uint16_t* myl = lds[wave];
    float* mb = reinterpret_cast<float*>(&lds[0][0]);  // [WAVES][16][MSTRIDE] after the loop

    for (int w = blockIdx.x; w < a.max_work; w += gridDim.x) {
        // One descriptor load (plus this wave's first page id) starts the item.
        const int32_t* d = a.work_desc + (long long)w * kWorkDescInts;
        const int page0 = wave < kWorkPages ? a.work_pages[(long long)w * kWorkPages + wave] : -1;
        const int page1 =
            wave + WAVES < kWorkPages ? a.work_pages[(long long)w * kWorkPages + wave + WAVES] : -1;
        const int s = d[0];
        if (s < 0)
            break;  // items past the last one are all marked empty
        if (d[7] != 1)
            continue;  // not a decode row
        const int row = d[1], kl = d[2], p_begin = d[3], p_end = d[4], ns = d[5];

        float m_run = -INFINITY, l_run = 0.0f;
        floatx4 acc[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r)
            acc[r] = floatx4{0, 0, 0, 0};

        // This wave streams the 32-token units of pages p_begin+wave, +WAVES, ...
        // with one unit in flight while the other is computed (rolling prefetch).
        const int np = p_begin + wave < p_end ? (p_end - p_begin - wave + WAVES - 1) / WAVES : 0;
        const int nk = np * UPP;
        auto page_of = [&](int pi) -> int {
            const int rel = wave + WAVES * pi;  // page offset inside the work item
            const int id = pi == 0 ? page0
                           : pi == 1 ? page1
                           : rel < kWorkPages ? a.work_pages[(long long)w * kWorkPages + rel]
                                              : a.page_table[(long long)s * a.max_pages + p_begin + rel];
            return __builtin_amdgcn_readfirstlane(id);  // wave-uniform: scalar base address
        };
        auto issue = [&](UnitRegs<KV, RP>& u, int k) -> int {  // returns the unit's valid tokens
            const int p = p_begin + wave + WAVES * (k / UPP);
            const int page = page_of(k / UPP);
            const int slot0 = 32 * (k % UPP);
            const bool ok = (unsigned)page < (unsigned)a.num_pool_pages;
            const int valid = ok ? min(PS, kl - p * PS) - slot0 : 0;
            load_unit<KV, RP, PS>(u, a.pages + (ok ? page : 0) * rec, slot0, valid, g, n);
            return valid;
        };
        UnitRegs<KV, RP> ub0, ub1;
        int v0 = 0, v1 = 0;
        if (nk > 0)
            v0 = issue(ub0, 0);
        if (nk > 1)
            v1 = issue(ub1, 1);
        // Q tile to LDS (heads >= H and the rope padding are zero), shared by the waves;
        // fetched while the first units are in flight.
        for (int i = tid; i < 16 * (QS / 8); i += THREADS) {
            const int h = i / (QS / 8), c8 = (i % (QS / 8)) * 8;
            u32x4 v = {0, 0, 0, 0};
            if (h < a.H) {
                if (c8 < KV)
                    v = *reinterpret_cast<const u32x4*>(a.q_latent + ((long long)row * a.H + h) * KV + c8);
                else if (c8 - KV < RP)
                    v = *reinterpret_cast<const u32x4*>(a.q_rope + ((long long)row * a.H + h) * RP +
                                                        c8 - KV);
            }
            *reinterpret_cast<u32x4*>(q_s + h * QS + c8) = v;
        }
        __syncthreads();

        for (int k = 0; k < nk; k += 2) {
            if (v0 > 0)
                process_unit<T, KV, RP>(ub0, v0, q_s, a.scale_log2, m_run, l_run, acc, myl, g, n);
            if (k + 2 < nk)
                v0 = issue(ub0, k + 2);
            if (k + 1 < nk) {
                if (v1 > 0)
                    process_unit<T, KV, RP>(ub1, v1, q_s, a.scale_log2, m_run, l_run, acc, myl, g,
                                            n);
                if (k + 3 < nk)
                    v1 = issue(ub1, k + 3);
            }
        }
        l_run += __shfl_xor(l_run, 16, 64);
        l_run += __shfl_xor(l_run, 32, 64);

        // ---- merge the WAVES softmax states of this work item in LDS ----
        if (g == 0) {
            sm_m[wave][n] = m_run;
            sm_l[wave][n] = l_run;
        }
        __syncthreads();  // every wave is done with its transpose buffer
        {
            float mh = -INFINITY;
#pragma unroll
            for (int v = 0; v < WAVES; ++v)
                mh = fmaxf(mh, sm_m[v][n]);
            const float f = m_run == -INFINITY ? 0.0f : exp2_fast(m_run - mh);
            if (head_ok)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    *reinterpret_cast<floatx4*>(mb + (wave * 16 + n) * MSTRIDE + 16 * rt + 4 * g) =
                        acc[rt] * f;
        }
        __syncthreads();
        for (int e = tid; e < a.H * (KV / 4); e += THREADS) {
            const int h = e / (KV / 4), c = (e % (KV / 4)) * 4;
            float mh = -INFINITY;
#pragma unroll
            for (int v = 0; v < WAVES; ++v)
                mh = fmaxf(mh, sm_m[v][h]);
            float lh = 0.0f;
            floatx4 o = {0, 0, 0, 0};
#pragma unroll
            for (int v = 0; v < WAVES; ++v) {
                const float mv = sm_m[v][h];
                lh += mv == -INFINITY ? 0.0f : sm_l[v][h] * exp2_fast(mv - mh);
                o += *reinterpret_cast<const floatx4*>(mb + (v * 16 + h) * MSTRIDE + c);
            }
            if (ns == 1) {
                const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
                *reinterpret_cast<floatx4*>(a.out + ((long long)row * a.H + h) * KV + c) = o * inv;
                if (a.lse && c == 0)
                    a.lse[(long long)row * a.H + h] = (mh + __log2f(lh)) * kLn2;
            } else {
                *reinterpret_cast<floatx4*>(a.part_o + ((long long)w * a.H + h) * KV + c) = o;
                if (c == 0) {
                    a.part_ml[((long long)w * a.H + h) * 2] = mh;
                    a.part_ml[((long long)w * a.H + h) * 2 + 1] = lh;
                }
            }
        }
        __syncthreads();  // LDS and sm_* are reused by the next work item
    }
}

// ------------------------------------------------------------- generic ----
constexpr int kGenThreads = 256;
constexpr int kGenChunk = 1024;   // tokens scored per LDS pass
constexpr int kGenMaxAcc = 4;     // kv_rank <= 4 * 256

__device__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kGenThreads / 64; ++i)
        r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}
__device__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    float r = 0.0f;
    for (int i = 0; i < kGenThreads / 64; ++i)
        r += red[i];
    __syncthreads();
    return r;
}

template <typename T>
__global__ __launch_bounds__(kGenThreads) void decode_generic_kernel(DecodeArgs a) {
    extern __shared__ float smem[];
    float* qs = smem;                         // kv_rank + rope_dim
    float* sc = smem + a.kv_rank + a.rope_dim;  // kGenChunk
    float* red = sc + kGenChunk;              // 4
    const int tid = threadIdx.x, h = blockIdx.y;
    const int KV = a.kv_rank, RP = a.rope_dim, PS = a.page_size;
    const long long rec = (long long)PS * (KV + RP);
    const bool tiled = page_tiled(PS, KV, RP);
    for (int w = blockIdx.x; w < a.max_work; w += gridDim.x) {
        const int32_t* d = a.work_desc + (long long)w * kWorkDescInts;
        const int s = d[0];
        if (s < 0)
            break;
        if (d[7] != 1)
            continue;
        const int row = d[1], kl = d[2], p_begin = d[3], p_end = d[4], ns = d[5];
        const int t_begin = p_begin * PS, t_end = min(kl, p_end * PS);
        for (int i = tid; i < KV + RP; i += kGenThreads)
            qs[i] = i < KV ? T::to_float(a.q_latent[((long long)row * a.H + h) * KV + i])
                           : T::to_float(a.q_rope[((long long)row * a.H + h) * RP + i - KV]);
        __syncthreads();
        float m_run = -INFINITY, l_run = 0.0f, acc[kGenMaxAcc] = {0, 0, 0, 0};
        for (int c0 = t_begin; c0 < t_end; c0 += kGenChunk) {
            const int cn = min(kGenChunk, t_end - c0);
            float lmax = -INFINITY;
            for (int t = tid; t < cn; t += kGenThreads) {
                const int tok = c0 + t;
                const int page = a.page_table[(long long)s * a.max_pages + tok / PS];
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
            const float cmax = block_max(lmax, red);
            const float m_new = fmaxf(m_run, cmax);
            const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m_run - m_new);
            float lsum = 0.0f;
            for (int t = tid; t < cn; t += kGenThreads) {
                const float e = m_new == -INFINITY ? 0.0f : exp2_fast(sc[t] - m_new);
                sc[t] = e;
                lsum += e;
            }
            const float csum = block_sum(lsum, red);  // also orders the sc[] writes
            l_run = l_run * alpha + csum;
            m_run = m_new;
            for (int k = 0; k < kGenMaxAcc; ++k) {
                const int r = tid + k * kGenThreads;
                if (r >= KV)
                    break;
                float v = acc[k] * alpha;
                for (int t = 0; t < cn; ++t) {
                    const int tok = c0 + t;
                    const int page = a.page_table[(long long)s * a.max_pages + tok / PS];
                    if ((unsigned)page < (unsigned)a.num_pool_pages && sc[t] != 0.0f)
                        v += sc[t] * T::to_float(
                                         a.pages[page * rec + latent_word(tiled, tok % PS, r, PS, KV)]);
                }
                acc[k] = v;
            }
            __syncthreads();
        }
        if (ns == 1) {
            const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
            for (int k = 0; k < kGenMaxAcc; ++k) {
                const int r = tid + k * kGenThreads;
                if (r < KV)
                    a.out[((long long)row * a.H + h) * KV + r] = acc[k] * inv;
            }
            if (a.lse && tid == 0)
                a.lse[(long long)row * a.H + h] = (m_run + __log2f(l_run)) * kLn2;
        } else {
            for (int k = 0; k < kGenMaxAcc; ++k) {
                const int r = tid + k * kGenThreads;
                if (r < KV)
                    a.part_o[((long long)w * a.H + h) * KV + r] = acc[k];
            }
            if (tid == 0) {
                a.part_ml[((long long)w * a.H + h) * 2] = m_run;
                a.part_ml[((long long)w * a.H + h) * 2 + 1] = l_run;
            }
        }
        __syncthreads();
    }
}

// --------------------------------------------------------------- merge ----
// Log-sum-exp combine of a session's split partials (log2 domain).  One block per
// (session, head); every split's (max, sum) is fetched in parallel into LDS, then
// each thread sums its columns over the splits with kMergeUnroll loads in flight.
constexpr int kMergeThreads = 128;
constexpr int kMergeUnroll = 8;

__global__ __launch_bounds__(kMergeThreads) void merge_kernel(DecodeArgs a) {
    __shared__ float f_s[kMergeThreads];
    __shared__ float red[kMergeThreads / 64 * 2];
    __shared__ float m_all, l_all;
    if (a.info[0] <= 0)
        return;  // empty or invalid batch: the metadata arrays are not meaningful
    const int tid = threadIdx.x, KV = a.kv_rank;
    for (int sh = blockIdx.x; sh < a.B * a.H; sh += gridDim.x) {
        const int s = sh / a.H, h = sh % a.H;
        const int row = a.cu_q[s];
        const int ns = a.num_splits[s];
        const int w0 = a.cu_splits[s];
        if (a.cu_q[s + 1] - row != 1 || ns <= 1 || w0 < 0 || w0 + ns > a.max_work)
            continue;
        float* o_row = a.out + ((long long)row * a.H + h) * KV;
        // Global max and denominator over the splits.
        float mloc = -INFINITY;
        for (int i = tid; i < ns; i += kMergeThreads)
            mloc = fmaxf(mloc, a.part_ml[((long long)(w0 + i) * a.H + h) * 2]);
        mloc = wave_max(mloc);
        if ((tid & 63) == 0)
            red[tid >> 6] = mloc;
        __syncthreads();
        if (tid == 0) {
            float m = red[0];
            for (int v = 1; v < kMergeThreads / 64; ++v)
                m = fmaxf(m, red[v]);
            m_all = m;
        }
        __syncthreads();
        const float M = m_all;
        float lloc = 0.0f;
        for (int i = tid; i < ns; i += kMergeThreads) {
            const long long idx = (long long)(w0 + i) * a.H + h;
            const float mv = a.part_ml[idx * 2];
            lloc += mv == -INFINITY ? 0.0f : a.part_ml[idx * 2 + 1] * exp2_fast(mv - M);
        }
        lloc = wave_sum(lloc);
        if ((tid & 63) == 0)
            red[kMergeThreads / 64 + (tid >> 6)] = lloc;
        __syncthreads();
        if (tid == 0) {
            float l = 0.0f;
            for (int v = 0; v < kMergeThreads / 64; ++v)
                l += red[kMergeThreads / 64 + v];
            l_all = l;
        }
        __syncthreads();
        const float inv = l_all > 0.0f ? 1.0f / l_all : 0.0f;
        if (a.lse && tid == 0)
            a.lse[(long long)row * a.H + h] = (M + __log2f(l_all)) * kLn2;
        for (int i0 = 0; i0 < ns; i0 += kMergeThreads) {
            const int cnt = min(kMergeThreads, ns - i0);
            if (tid < cnt) {
                const float mv = a.part_ml[((long long)(w0 + i0 + tid) * a.H + h) * 2];
                f_s[tid] = mv == -INFINITY ? 0.0f : exp2_fast(mv - M) * inv;
            }
            __syncthreads();
            for (int r = tid; r < KV; r += kMergeThreads) {
                float o = i0 == 0 ? 0.0f : o_row[r];
                for (int j0 = 0; j0 < cnt; j0 += kMergeUnroll) {
                    float v[kMergeUnroll];
#pragma unroll
                    for (int j = 0; j < kMergeUnroll; ++j)
                        v[j] = j0 + j < cnt
                                   ? a.part_o[((long long)(w0 + i0 + j0 + j) * a.H + h) * KV + r]
                                   : 0.0f;
#pragma unroll
                    for (int j = 0; j < kMergeUnroll; ++j)
                        if (j0 + j < cnt)
                            o += f_s[j0 + j] * v[j];
                }
                o_row[r] = o;
            }
            __syncthreads();
        }
    }
}

#ifndef MLA_DECODE_WAVES
#define MLA_DECODE_WAVES 2
#endif
constexpr int kMfmaWaves = MLA_DECODE_WAVES;

template <typename T>
hipError_t launch_mfma(const DecodeArgs& a, int grid, hipStream_t stream) {
    if (a.kv_rank == 128 && a.rope_dim == 16 && a.page_size == 64)
        hipLaunchKernelGGL((decode_mfma_kernel<T, 128, 16, 64, kMfmaWaves>), dim3(grid),
                           dim3(64 * kMfmaWaves), 0, stream, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(int H, int kv_rank, int rope_dim, int page_size) {
    return H <= 16 && page_size == 64 && kv_rank == 128 && rope_dim == 16;
}

hipError_t launch_decode(const DecodeArgs& a, int dtype, bool force_generic, hipStream_t stream) {
    if (a.max_work <= 0 || a.B <= 0)
        return hipSuccess;
    const int grid = a.max_work;  // <= kMaxWork
    hipError_t err;
    if (!force_generic && decode_mfma_supported(a.H, a.kv_rank, a.rope_dim, a.page_size)) {
        err = dtype == 0 ? launch_mfma<F16>(a, grid, stream) : launch_mfma<BF16>(a, grid, stream);
    } else {
        const size_t shmem = (a.kv_rank + a.rope_dim + kGenChunk + 8) * sizeof(float);
        const dim3 g(grid, a.H);
        if (dtype == 0)
            hipLaunchKernelGGL(decode_generic_kernel<F16>, g, dim3(kGenThreads), shmem, stream, a);
        else
            hipLaunchKernelGGL(decode_generic_kernel<BF16>, g, dim3(kGenThreads), shmem, stream, a);
        err = hipGetLastError();
    }
    if (err != hipSuccess)
        return err;
    const long long pairs = (long long)a.B * a.H;
    const int mgrid = pairs < 65535 ? (int)pairs : 65535;
    hipLaunchKernelGGL(merge_kernel, dim3(mgrid), dim3(kMergeThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla
