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
// final row directly, the rest are combined with a log-sum-exp merge.
//
// decode_page_kernel -- the production kernel (H <= 16, kv_rank 128, rope 16,
//   64-token tiled pages): one wave per page with all of the page's loads in
//   flight at once, MFMA scores and PV.
// decode_generic_kernel -- any H / kv_rank / rope / page size / layout: one
//   256-thread block per (work item, head), VALU fp32.
// merge_kernel -- log-sum-exp combine of the split partials of either kernel, one
//   workgroup per session, launched after it on the same stream (the kernel
//   boundary makes the partials written on every XCD visible).
#include "mla_common.hpp"
#include "mla_internal.hpp"

#include <cmath>

namespace mla {
namespace {

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- MFMA ----
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

// gfx950 LDS transpose read: in each 16-lane group, lane j supplies an 8-byte row
// R_j; lane i = 4a+b receives {R_a[b], R_{a+4}[b], R_{a+8}[b], R_{a+12}[b]}.
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s4 __attribute__((address_space(3)))*)((__attribute__((address_space(3))) char*)p));
    return __builtin_bit_cast(u32x2, v);
}

// Buffer resource over `bytes` bytes from `base` (raw, stride 0): loads past it read
// as zero.  Only the query rows are read this way (at offsets 64 bytes apart): in this
// toolchain the optimizer can merge or drop buffer-intrinsic loads that share a
// resource at nearby offsets (a raw_buffer_load at +4 bytes was folded into the one at
// +0), so nothing else goes through buffer intrinsics.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// The split merge inside the decode launch (DecodeArgs::fused_merge), called by every
// item of a split session after its partial stores.  The metadata was built XCD-placed,
// so all items of the session ran on this XCD and their partials sit in its L2: each
// item waits for its own stores to be acknowledged, then bumps the session's counter
// with an atomic in that L2 (no device-scope traffic); the item that brings it to
// num_splits knows every partial has landed, takes the session's counts back out of the
// counter for the next launch and folds the partials (log-sum-exp, as merge_kernel) into
// the session's row.  The partial stores are plain ones so that the lines stay in the L2.
// No item waits on another.
// Folds the partials of head h in slots slot0 .. slot0 + N - 1 (columns c..c+3 of their o
// rows) into the running log-sum-exp state (M, L, O).  Plain loads: the lines were written
// in this launch on other CUs of this XCD, and this CU's L1 holds no copy of them (it is
// invalidated at the launch, part_o slots are whole lines, part_ml slots are padded to
// whole lines, and only this merge reads them).
template <int N, int KV>
__device__ __forceinline__ void fold_partials(const DecodeArgs& a, long long slot0, int h, int c,
                                              float& M, float& L, floatx4& O) {
    float m[N], l[N];
    floatx4 o[N];
    const int mls = part_ml_stride(a.H);
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const long long sl = slot0 + j;
        m[j] = a.part_ml[sl * mls + 2 * h];
        l[j] = a.part_ml[sl * mls + 2 * h + 1];
        o[j] = *reinterpret_cast<const floatx4*>(a.part_o + (sl * a.H + h) * KV + c);
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < N; ++j)
        Mn = fmaxf(Mn, m[j]);
    const float r = M == -INFINITY ? 0.0f : exp2_fast(M - Mn);
    L *= r;
    O *= r;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const float f = m[j] == -INFINITY ? 0.0f : exp2_fast(m[j] - Mn);
        L += l[j] * f;
        O += o[j] * f;
    }
    M = Mn;
}

// Sets `bit` of the decode status word (read by the host through mla_decode_status).
__device__ __forceinline__ void raise_status(const DecodeArgs& a, int bit) {
    __hip_atomic_fetch_or(a.status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KV, int THREADS>
__device__ __forceinline__ void fused_merge_tail(const DecodeArgs& a, int s, int row, int ns,
                                                 long long first) {
    __shared__ int s_last;
    const int tid = threadIdx.x;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are in L2
    __syncthreads();
    if (tid == 0) {
        // If the items of a session ran on several XCDs (the dispatch did not keep slots of
        // one residue mod n on one XCD), no L2 counts all of them: nobody merges and the
        // counter stays nonzero after the launch, which is what the host's status check
        // (mla_decode_status) looks for.
        const int old = __hip_atomic_fetch_add(a.merge_count + s, 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
        s_last = old == ns - 1;
        // Take the session's ns counts back out (an atomic add, not a store of 0: a count
        // that was already wrong when the launch began must survive it, so the host's check
        // still sees it, and no increment racing with the reset can be erased).
        if (old == ns - 1)
            __hip_atomic_fetch_add(a.merge_count + s, -ns, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (!s_last)
        return;
    // N partials at a time (N <= 16, fixed per instantiation so that every load is
    // unconditional and all of them are in flight together): (m, l) and o rows, folded with
    // the weights 2^(m_j - M) into the running (M, L, O).
    for (int e = tid; e < a.H * (KV / 4); e += THREADS) {
        const int h = e / (KV / 4), c = (e % (KV / 4)) * 4;
        float M = -INFINITY, L = 0.0f;
        floatx4 O = {0, 0, 0, 0};
        for (int j0 = 0; j0 < ns; j0 += 16) {
            switch (min(ns - j0, 16)) {
#define MLA_FOLD_CASE(N) \
    case N:                 \
        fold_partials<N, KV>(a, first + j0, h, c, M, L, O); \
        break;
                MLA_FOLD_CASE(1) MLA_FOLD_CASE(2) MLA_FOLD_CASE(3) MLA_FOLD_CASE(4)
                MLA_FOLD_CASE(5) MLA_FOLD_CASE(6) MLA_FOLD_CASE(7) MLA_FOLD_CASE(8)
                MLA_FOLD_CASE(9) MLA_FOLD_CASE(10) MLA_FOLD_CASE(11) MLA_FOLD_CASE(12)
                MLA_FOLD_CASE(13) MLA_FOLD_CASE(14) MLA_FOLD_CASE(15) MLA_FOLD_CASE(16)
#undef MLA_FOLD_CASE
            }
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        __builtin_nontemporal_store(
            O * inv, reinterpret_cast<floatx4*>(a.out + ((long long)row * a.H + h) * KV + c));
        if (a.lse && c == 0)
            a.lse[(long long)row * a.H + h] = (M + __log2f(L)) * kLn2;
    }
}

// The fused flag over metadata that is not placed for this device (info[4] != xcd_n): the
// session's items ran on several XCDs, so they do not merge.  Each leaves its partial (as
// the two-launch path does: mla_decode_merge completes the rows), the first item sets the
// session's rows to NaN so that no stale row passes for a result, and the call is flagged.
template <int KV, int THREADS>
__device__ __forceinline__ void unplaced_tail(const DecodeArgs& a, int row, bool first_item) {
    const int tid = threadIdx.x;
    if (tid == 0)
        raise_status(a, kStatusUnplaced);
    if (!first_item)
        return;
    const float nan = __builtin_nanf("");
    for (int e = tid; e < a.H * KV; e += THREADS)
        a.out[(long long)row * a.H * KV + e] = nan;
    if (a.lse)
        for (int h = tid; h < a.H; h += THREADS)
            a.lse[(long long)row * a.H + h] = nan;
}

// Split index of a work item from its descriptor: items cover `split` pages each, the
// session's last one (ending at its last page) possibly fewer.
__device__ __forceinline__ int item_split_index(int kl, int p_begin, int p_end, int ns, int PS) {
    const int need = (kl + PS - 1) / PS;
    return p_end == need ? ns - 1 : p_begin / (p_end - p_begin);
}

// decode_page_kernel -- one workgroup of WAVES waves per work item (session, split);
// wave v owns pages p_begin+v, p_begin+v+WAVES, ... of the item and issues ALL loads
// of a page (PS tokens, TILED record: every 16-byte lane load reads 1 KB
// contiguously) before touching any of it, so with split_pages == WAVES the whole
// item is in flight at once.
//
// Per page, with lane (g, n) = (lane/16, lane%16):
//   S^T[16t+4g+i][head n] = K . Q^T on v_mfma_f32_16x16x32 (latent K-steps, then the
//   rope key zero-padded to one 32-wide K-step).  The page tile is the A operand as
//   loaded; Q^T (heads padded to 16) is the B operand, held in registers.
//   Softmax over the page's PS tokens at once (log2 domain; the running state is
//   rescaled only when a later page raises the maximum).
//   O^T += C^T . P^T per 32-token unit: the S^T layout already is P^T's B operand;
//   C^T comes from the unit's latent rows written to a per-wave LDS tile and read
//   back with ds_read_b64_tr_b16.
// The waves' states merge in LDS.  A session with one work item writes its final
// row; otherwise each item stores its partial (m, l, o) for merge_kernel.  (Combining
// the partials inside this launch, by the session's last item to finish, needs
// device-scope partial stores and loads because the items run on different XCDs,
// whose L2s do not see each other's writes; measured on config 3 that tail costs
// 4-8 us against 2-3 us for the separate merge launch.)
template <typename T, int KV, int RP, int PS, int WAVES, int PPW, bool FUSED>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(PPW == 1 ? 3 : PPW == 2 ? 2 : 1, 8)))
void decode_page_kernel(DecodeArgs a) {
    static_assert(KV % 32 == 0 && RP % 8 == 0 && RP <= 32 && PS % 32 == 0, "tile shape");
    static_assert(WAVES * PPW <= kWorkPages, "a wave's first page ids come from work_pages");
    constexpr int KS = KV / 32;       // latent K-steps of the score MFMAs
    constexpr int TT = PS / 16;       // 16-token tiles per page
    constexpr int UPP = PS / 32;      // 32-token units per page (PV K-steps)
    constexpr int RT = KV / 16;       // 16-row tiles of O^T
    constexpr int UP = unit_pitch<KV>();
    constexpr int TBUF = 32 * UP;     // per-wave LDS unit tile, 16-bit words
    constexpr int MSTRIDE = KV + 4;   // LDS merge pitch, floats
    constexpr int THREADS = 64 * WAVES;
    static_assert(16 * MSTRIDE * 4 <= TBUF * 2, "a wave's merge rows fit its own tile");
    using V8 = typename T::vec8;
    __shared__ __attribute__((aligned(16))) uint16_t lds[WAVES][TBUF];
    __shared__ float sm_m[WAVES][16], sm_l[WAVES][16];

    const int w = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // The whole 32-byte descriptor and this wave's first page id are fetched together,
    // as scalar loads (every entry below max_work is readable; the id is only used when
    // the item is real).
    typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
    const i32x8 d = *reinterpret_cast<const i32x8*>(a.work_desc + (long long)w * kWorkDescInts);
    int pid[PPW];  // ids of this wave's first PPW pages (item pages wave, wave + WAVES, ..)
#pragma unroll
    for (int k = 0; k < PPW; ++k)
        pid[k] = a.work_pages[(long long)w * kWorkPages + wave + k * WAVES];
    // Kernel arguments used below, fetched with the descriptor (one wait, not one per use).
    const int H = a.H, npool = a.num_pool_pages;
    const uint16_t* const pool = a.pages;
    const float scale_log2 = a.scale_log2;
    // The XCD count the metadata was placed for (the fused merge's premise, checked at the end).
    const int placed_n = FUSED ? a.info[kInfoPlacement] : 0;
    asm volatile("" ::"s"(pid[0]), "s"(H), "s"(npool), "s"(pool), "s"(scale_log2), "s"(placed_n));
    const int s = d[0];
    if (s < 0 || d[7] != 1)
        return;  // past the last item (or a failed build), or not a decode row
    const int row = d[1], kl = d[2], p_begin = d[3], p_end = d[4], ns = d[5], slot = d[6];
    const long long rec = (long long)PS * (KV + RP);
    // Rope chunks: lanes with 8g >= RP read a duplicate of a valid chunk of the page
    // (in bounds, no extra traffic); their Q^T operand is zero, so they add nothing.
    const bool rope_lane = 8 * g < RP;
    const int rope_lane_off = (16 * (rope_lane ? g : g % (RP / 8)) + n) * 8;

    // Q^T operand registers: head n, columns 32j+8g..+7 (rope in step KS).  Buffer loads
    // over this row's query: padded heads (n >= H) and padded rope lanes fall outside
    // the resource and read as zero, with no select that would wait on the data.
    V8 qv[KS + 1];
    auto load_q = [&]() {
        const auto rq = buffer_rsrc(a.q_latent + (long long)row * H * KV, H * KV * 2);
        const auto rr = buffer_rsrc(a.q_rope + (long long)row * H * RP, H * RP * 2);
        const int oob = 0x40000000;
#pragma unroll
        for (int j = 0; j < KS; ++j)
            qv[j] = __builtin_bit_cast(
                V8, __builtin_amdgcn_raw_buffer_load_b128(
                        rq, n < H ? (n * KV + 32 * j + 8 * g) * 2 : oob, 0, 0));
        qv[KS] = __builtin_bit_cast(
            V8, __builtin_amdgcn_raw_buffer_load_b128(
                    rr, n < H && rope_lane ? (n * RP + 8 * g) * 2 : oob, 0, 0));
    };

    float m_run = -INFINITY, l_run = 0.0f;
    floatx4 acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
        acc[r] = floatx4{0, 0, 0, 0};
    uint16_t* myl = lds[wave];
    const int wchunk = g ^ lds_swz(n);  // swizzled 8-column chunk of this lane's LDS row writes
    const uint16_t* src = myl + (4 * g + (n >> 2)) * UP + 4 * ((n & 3) ^ (2 * lds_swz(4 * g)));

    u32x4 lats[PPW][TT][KS], rops[PPW][TT];
    // Every load of one page, issued back to back.  The cache is read once per step,
    // so the loads are non-temporal (measured: a plain read of one layer's pages takes
    // 9.2 us, a non-temporal one 8.2 us).
    auto load_page = [&](u32x4 (&lat)[TT][KS], u32x4 (&rop)[TT], int page) {
        const uint16_t* base = pool + page * rec;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int j = 0; j < KS; ++j)
                lat[t][j] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(base + (t * KS + j) * 512 + lane * 8));
            rop[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                base + PS * KV + t * (RP / 8) * 128 + rope_lane_off));
        }
    };
    // Scores, softmax update and PV of the loaded page (`valid` tokens of it count).
    auto compute_page = [&](u32x4 (&lat)[TT][KS], u32x4 (&rop)[TT], int valid) {
        // A wave whose page has landed takes issue priority over waves still waiting on
        // theirs, which shortens the tail after the last page arrives (measured: 10.95 us
        // against 11.01-11.06 us per config-3 launch).
        __builtin_amdgcn_s_setprio(2);
        if (valid < PS) {  // the session's last page: zero the slots past its end
#pragma unroll
            for (int t = 0; t < TT; ++t)
                if (16 * t + n >= valid) {
#pragma unroll
                    for (int j = 0; j < KS; ++j)
                        lat[t][j] = u32x4{0, 0, 0, 0};
                    rop[t] = u32x4{0, 0, 0, 0};
                }
        }
        floatx4 sc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            sc[t] = floatx4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < KS; ++j)
                sc[t] = T::mma32(__builtin_bit_cast(V8, lat[t][j]), qv[j], sc[t]);
            sc[t] = T::mma32(__builtin_bit_cast(V8, rop[t]), qv[KS], sc[t]);
        }
        float mp = -INFINITY;
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = sc[t][i] * scale_log2;
                if (valid < PS && 16 * t + 4 * g + i >= valid)
                    x = -INFINITY;
                sc[t][i] = x;
                mp = fmaxf(mp, x);
            }
        mp = rows_max(mp);
        if (m_run == -INFINITY) {
            m_run = mp;  // first page of this wave: nothing accumulated yet
        } else if (__ballot(mp > m_run)) {
            const float m_new = fmaxf(m_run, mp);
            const float alpha = exp2_fast(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int r = 0; r < RT; ++r)
                acc[r] *= alpha;
            m_run = m_new;
        }
        V8 pb[UPP], pl[UPP];  // P^T operands (pl: the low part, bf16 only)
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = exp2_fast(sc[t][i] - m_run);
                psum += e;
                const auto hi = static_cast<typename T::scalar>(e);
                pb[t / 2][4 * (t % 2) + i] = hi;
                if constexpr (T::split_p)
                    pl[t / 2][4 * (t % 2) + i] =
                        static_cast<typename T::scalar>(e - static_cast<float>(hi));
            }
        l_run += psum;
#pragma unroll
        for (int u = 0; u < UPP; ++u) {
            // Latent rows of tokens 32u..32u+31 to the LDS tile (row 16tt+n, swizzled chunk).
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int j = 0; j < KS; ++j)
                    *reinterpret_cast<u32x4*>(myl + (16 * tt + n) * UP + 32 * j + 8 * wchunk) =
                        lat[2 * u + tt][j];
            wave_lds_fence();
            // A = C^T: lane (g, n) gets column 16rt+n of tokens 4g..4g+3 (K-slots 0..3)
            // and 16+4g..16+4g+3 (slots 4..7), matching P^T's K order in pb[u].
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const u32x2 lo = lds_read_tr16(src + 16 * rt);
                const u32x2 hi = lds_read_tr16(src + 16 * UP + 16 * rt);
                const V8 ca = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                acc[rt] = T::mma32(ca, pb[u], acc[rt]);
                if constexpr (T::split_p)
                    acc[rt] = T::mma32(ca, pl[u], acc[rt]);
            }
            wave_lds_fence();
        }
    };

    // The query's loads go out first (vmcnt completes in order, so each score MFMA then
    // waits only for its own tile), then ALL loads of the wave's first PPW pages, page
    // by page: the first page lands early and is consumed while the later ones stream.
    // Further pages (items longer than WAVES * PPW pages) follow one at a time.
    const int p0 = p_begin + wave;
    if (p0 < p_end) {
        load_q();
        bool ok[PPW];
#pragma unroll
        for (int k = 0; k < PPW; ++k) {
            const int page = __builtin_amdgcn_readfirstlane(pid[k]);
            ok[k] = p0 + k * WAVES < p_end && (unsigned)page < (unsigned)npool;
            if (ok[k])
                load_page(lats[k], rops[k], page);
        }
#pragma unroll
        for (int k = 0; k < PPW; ++k)
            if (ok[k])
                compute_page(lats[k], rops[k], min(PS, kl - (p0 + k * WAVES) * PS));
        for (int p = p0 + PPW * WAVES; p < p_end; p += WAVES) {
            const int rel = p - p_begin;
            const int page = __builtin_amdgcn_readfirstlane(
                rel < kWorkPages ? a.work_pages[(long long)w * kWorkPages + rel]
                                 : a.page_table[(long long)s * a.max_pages + p]);
            if ((unsigned)page >= (unsigned)npool)
                continue;
            load_page(lats[0], rops[0], page);
            compute_page(lats[0], rops[0], min(PS, kl - p * PS));
        }
    }
    __builtin_amdgcn_s_setprio(0);
    l_run = rows_sum(l_run);

    // ---- merge the WAVES softmax states of this work item in LDS ----
    // Each wave parks its unscaled state in its own unit tile (its 16 x MSTRIDE floats fit
    // in the TBUF words it alone used), so one barrier suffices: no wave can overwrite a
    // tile another wave is still reading.  The combine weights wave v by 2^(m_v - max).
    float* mine = reinterpret_cast<float*>(&lds[wave][0]);  // [16][MSTRIDE]
    if (g == 0) {
        sm_m[wave][n] = m_run;
        sm_l[wave][n] = l_run;
    }
    if (n < H)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            *reinterpret_cast<floatx4*>(mine + n * MSTRIDE + 16 * rt + 4 * g) = acc[rt];
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
            const float f = mv == -INFINITY ? 0.0f : exp2_fast(mv - mh);
            lh += sm_l[v][h] * f;
            o += *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(&lds[v][0]) +
                                                   h * MSTRIDE + c) *
                 f;
        }
        // The rows are read once, by the next kernel: non-temporal stores (measured
        // 0.3 us less per config-3 launch than plain ones).
        if (ns == 1) {
            const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
            __builtin_nontemporal_store(
                o * inv, reinterpret_cast<floatx4*>(a.out + ((long long)row * a.H + h) * KV + c));
            if (a.lse && c == 0)
                a.lse[(long long)row * a.H + h] = (mh + __log2f(lh)) * kLn2;
        } else if constexpr (FUSED) {  // plain stores: the partials stay in this XCD's L2
            *reinterpret_cast<floatx4*>(a.part_o + ((long long)slot * a.H + h) * KV + c) = o;
            if (c == 0) {
                a.part_ml[(long long)slot * part_ml_stride(a.H) + 2 * h] = mh;
                a.part_ml[(long long)slot * part_ml_stride(a.H) + 2 * h + 1] = lh;
            }
        } else {
            __builtin_nontemporal_store(
                o, reinterpret_cast<floatx4*>(a.part_o + ((long long)slot * a.H + h) * KV + c));
            if (c == 0) {
                a.part_ml[(long long)slot * part_ml_stride(a.H) + 2 * h] = mh;
                a.part_ml[(long long)slot * part_ml_stride(a.H) + 2 * h + 1] = lh;
            }
        }
    }
    if constexpr (FUSED)
        if (ns > 1) {  // the session's first partial slot: this item's, less its split index
            const int sp = item_split_index(kl, p_begin, p_end, ns, PS);
            if (placed_n == a.xcd_n)
                fused_merge_tail<KV, THREADS>(a, s, row, ns, slot - sp);
            else
                unplaced_tail<KV, THREADS>(a, row, sp == 0);
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
        if (s < 0 || d[7] != 1)
            continue;  // an empty slot (the placed work list has them between items)
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
                    a.part_o[((long long)d[6] * a.H + h) * KV + r] = acc[k];
            }
            if (tid == 0) {
                a.part_ml[(long long)d[6] * part_ml_stride(a.H) + 2 * h] = m_run;
                a.part_ml[(long long)d[6] * part_ml_stride(a.H) + 2 * h + 1] = l_run;
            }
        }
        __syncthreads();
    }
}

// --------------------------------------------------------------- merge ----
// Log-sum-exp combine of a session's split partials (log2 domain).  Workgroup (s, y)
// owns kMergeElems consecutive (head, V-column) elements of session s.  Its G thread
// groups take one element per thread each and split the session's splits into G
// consecutive ranges: each thread folds its range in order into a running (max, sum, o),
// kMergeUnroll splits per round with the next round's partials in flight, and the
// groups' states are then folded in group order through LDS.  G = 4 for small batches of
// many splits per session (config 3: ~9 splits, one round per thread instead of two); G =
// 1 when the batch has many elements (config 5: 256 sessions x 16 K elements, ~3 splits
// each), where workgroups of 256 threads fit eight to a CU and the launch runs in a
// quarter of the rounds (measured at config 5: 262 us per call with G = 4).
constexpr int kMergeElems = 256;
constexpr int kMergeUnroll = 8;
constexpr long long kMergeGroupedMax = 512LL * kMergeElems;  // elements of a batch for G = 4

template <int V, int G>
__global__ __launch_bounds__(kMergeElems* G) void merge_kernel(DecodeArgs a) {
    typedef float vecV __attribute__((ext_vector_type(V)));
    __shared__ float sm_m[G][kMergeElems], sm_l[G][kMergeElems];
    __shared__ vecV sm_o[G][kMergeElems];
    const int s = blockIdx.x;
    const int built = a.info[0], row = a.cu_q[s], row_end = a.cu_q[s + 1];
    const int ns = a.num_splits[s], w0 = a.cu_splits[s];
    if (built <= 0 || row_end - row != 1 || ns <= 1 || w0 < 0 || w0 + ns > a.max_work)
        return;  // failed build, not a decode row, or nothing to combine
    const int H = a.H, KV = a.kv_rank, per_head = KV / V;
    const int grp = threadIdx.x / kMergeElems, t = threadIdx.x % kMergeElems;
    const int e = blockIdx.y * kMergeElems + t;
    const bool live = e < H * per_head;
    const int h = live ? e / per_head : 0, c = live ? (e % per_head) * V : 0;
    // this group's splits [i_lo, i_hi)
    const int i_lo = ns * grp / G, i_hi = ns * (grp + 1) / G;
    float M = -INFINITY, L = 0.0f;
    vecV O = {};
    auto load = [&](int i0, float (&mi)[kMergeUnroll], float (&li)[kMergeUnroll],
                    vecV (&oi)[kMergeUnroll]) {
#pragma unroll
        for (int k = 0; k < kMergeUnroll; ++k) {
            const long long sl = w0 + min(i0 + k, i_hi - 1), idx = sl * H + h;
            mi[k] = a.part_ml[sl * part_ml_stride(H) + 2 * h];
            li[k] = a.part_ml[sl * part_ml_stride(H) + 2 * h + 1];
            oi[k] = *reinterpret_cast<const vecV*>(a.part_o + idx * KV + c);
        }
    };
    auto fold1 = [&](float mk, float lk, vecV ok) {
        if (mk == -INFINITY)
            return;  // a split (or group) with no tokens
        const float Mn = fmaxf(M, mk);
        const float sa = M == -INFINITY ? 0.0f : exp2_fast(M - Mn);
        const float sb = exp2_fast(mk - Mn);
        L = L * sa + lk * sb;
        O = O * sa + ok * sb;
        M = Mn;
    };
    auto fold = [&](int i0, const float (&mi)[kMergeUnroll], const float (&li)[kMergeUnroll],
                    const vecV (&oi)[kMergeUnroll]) {
#pragma unroll
        for (int k = 0; k < kMergeUnroll; ++k)
            if (i0 + k < i_hi)
                fold1(mi[k], li[k], oi[k]);
    };
    if (live && i_lo < i_hi) {
        float ma[kMergeUnroll], la[kMergeUnroll], mb[kMergeUnroll], lb[kMergeUnroll];
        vecV oa[kMergeUnroll], ob[kMergeUnroll];
        load(i_lo, ma, la, oa);
        for (int i0 = i_lo; i0 < i_hi; i0 += 2 * kMergeUnroll) {
            if (i0 + kMergeUnroll < i_hi)
                load(i0 + kMergeUnroll, mb, lb, ob);
            fold(i0, ma, la, oa);
            if (i0 + kMergeUnroll >= i_hi)
                break;
            if (i0 + 2 * kMergeUnroll < i_hi)
                load(i0 + 2 * kMergeUnroll, ma, la, oa);
            fold(i0 + kMergeUnroll, mb, lb, ob);
        }
    }
    if (grp > 0) {
        sm_m[grp][t] = M;
        sm_l[grp][t] = L;
        sm_o[grp][t] = O;
    }
    __syncthreads();
    if (grp > 0 || !live)
        return;
#pragma unroll
    for (int q = 1; q < G; ++q)
        fold1(sm_m[q][t], sm_l[q][t], sm_o[q][t]);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    *reinterpret_cast<vecV*>(a.out + ((long long)row * H + h) * KV + c) = O * inv;
    if (a.lse && c == 0)
        a.lse[(long long)row * H + h] = (M + __log2f(L)) * kLn2;
}

// Waves per work item of decode_page_kernel; the metadata's split_pages should match
// (one page per wave, every load of an item in flight at once).
#ifndef MLA_DECODE_WAVES
#define MLA_DECODE_WAVES 4
#endif
#ifndef MLA_DECODE_PPW
#define MLA_DECODE_PPW 1
#endif
constexpr int kPageWaves = MLA_DECODE_WAVES;
constexpr int kPagesPerWave = MLA_DECODE_PPW;

template <typename T>
hipError_t launch_page(const DecodeArgs& a, int grid, hipStream_t stream) {
    if (a.kv_rank == 128 && a.rope_dim == 16 && a.page_size == 64 && a.fused_merge)
        hipLaunchKernelGGL((decode_page_kernel<T, 128, 16, 64, kPageWaves, kPagesPerWave, true>),
                           dim3(grid), dim3(64 * kPageWaves), 0, stream, a);
    else if (a.kv_rank == 128 && a.rope_dim == 16 && a.page_size == 64)
        hipLaunchKernelGGL((decode_page_kernel<T, 128, 16, 64, kPageWaves, kPagesPerWave, false>),
                           dim3(grid), dim3(64 * kPageWaves), 0, stream, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(int H, int kv_rank, int rope_dim, int page_size) {
    return H <= 16 && page_size == 64 && kv_rank == 128 && rope_dim == 16;
}

hipError_t launch_decode_partials(const DecodeArgs& a, int dtype, bool force_generic,
                                  hipStream_t stream) {
    if (a.max_work <= 0 || a.B <= 0)
        return hipSuccess;
    const int grid = a.max_work;  // <= kMaxWork
    if (!force_generic && decode_mfma_supported(a.H, a.kv_rank, a.rope_dim, a.page_size))
        return dtype == 0 ? launch_page<F16>(a, grid, stream) : launch_page<BF16>(a, grid, stream);
    if (!force_generic && decode_wide_supported(a.H, a.kv_rank, a.rope_dim, a.page_size))
        return launch_decode_wide(a, dtype, stream);
    const size_t shmem = (a.kv_rank + a.rope_dim + kGenChunk + 8) * sizeof(float);
    const dim3 g(grid, a.H);
    if (dtype == 0)
        hipLaunchKernelGGL(decode_generic_kernel<F16>, g, dim3(kGenThreads), shmem, stream, a);
    else
        hipLaunchKernelGGL(decode_generic_kernel<BF16>, g, dim3(kGenThreads), shmem, stream, a);
    return hipGetLastError();
}

hipError_t launch_merge(const DecodeArgs& a, hipStream_t stream) {
    if (a.max_work <= 0 || a.B <= 0)
        return hipSuccess;
    // float4 columns when the rows allow it (16-byte aligned buffers, kv_rank % 4 == 0)
    const bool vec4 = a.kv_rank % 4 == 0 &&
                      ((reinterpret_cast<uintptr_t>(a.out) | reinterpret_cast<uintptr_t>(a.part_o)) &
                       15) == 0;
    const int per_session = a.H * (a.kv_rank / (vec4 ? 4 : 1));  // elements of a row
    const dim3 grid(a.B, (per_session + kMergeElems - 1) / kMergeElems);
    const bool grouped = (long long)a.B * per_session <= kMergeGroupedMax;
    if (vec4 && grouped)
        hipLaunchKernelGGL((merge_kernel<4, 4>), grid, dim3(kMergeElems * 4), 0, stream, a);
    else if (vec4)
        hipLaunchKernelGGL((merge_kernel<4, 1>), grid, dim3(kMergeElems), 0, stream, a);
    else if (grouped)
        hipLaunchKernelGGL((merge_kernel<1, 4>), grid, dim3(kMergeElems * 4), 0, stream, a);
    else
        hipLaunchKernelGGL((merge_kernel<1, 1>), grid, dim3(kMergeElems), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla
