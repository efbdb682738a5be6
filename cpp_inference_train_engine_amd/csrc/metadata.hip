// (a) Ragged-batch metadata and (b) paged latent append, gfx950.
//
// The metadata build runs as ONE workgroup of 1024 threads: batches are at
// most a few thousand sessions, so a single-block scan beats a multi-kernel
// device-wide scan (no inter-block traffic, one launch).  All arithmetic is
// int32/int64 and bit-exact with the CPU builder in the oracle.
#include "mla_common.hpp"
#include "mla_internal.hpp"

#include <algorithm>
#include <climits>
#include <string>
#include <vector>

namespace mla {
namespace {

constexpr int kMetaThreads = 1024;
constexpr int kMetaWaves = kMetaThreads / 64;

// Inclusive block scan of three int64 values; returns the chunk totals in tot[].
__device__ void block_scan3(long long v[3], long long tot[3], long long* lds) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int k = 0; k < 3; ++k)
        for (int off = 1; off < 64; off <<= 1) {
            const long long up = __shfl_up(v[k], off, 64);
            if (lane >= off)
                v[k] += up;
        }
    if (lane == 63)
        for (int k = 0; k < 3; ++k)
            lds[k * kMetaWaves + wave] = v[k];
    __syncthreads();
    if (wave == 0) {
        for (int k = 0; k < 3; ++k) {
            long long x = lane < kMetaWaves ? lds[k * kMetaWaves + lane] : 0;
            for (int off = 1; off < kMetaWaves; off <<= 1) {
                const long long up = __shfl_up(x, off, 64);
                if (lane >= off)
                    x += up;
            }
            if (lane < kMetaWaves)
                lds[k * kMetaWaves + lane] = x;
        }
    }
    __syncthreads();
    for (int k = 0; k < 3; ++k) {
        if (wave > 0)
            v[k] += lds[k * kMetaWaves + wave - 1];
        tot[k] = lds[k * kMetaWaves + kMetaWaves - 1];
    }
    __syncthreads();
}

// Largest b in [0, n] with a[b] <= x  (a non-decreasing, a[0] <= x).
__device__ int upper_index(const int32_t* a, int n, long long x) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a[mid] <= x)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// For batches up to kMetaLdsCap sessions the per-session inputs and prefix arrays live
// in LDS, and so does the padded page table when it has at most kMetaPtCap entries, so
// the build waits on global memory twice (the session inputs, then the page ids) and
// every later lookup and binary search reads LDS.
constexpr int kMetaLdsCap = 4096;
constexpr int kMetaPtCap = 16384;
constexpr int kMetaUnroll = 16;  // page-table entries whose loads a thread issues together

__device__ void write_error(const MetadataArgs& a, int session) {
    for (int w = threadIdx.x; w < a.max_work; w += kMetaThreads)
        a.work_desc[(long long)w * kWorkDescInts] = -1;
    if (threadIdx.x < kInfoInts)
        a.info[threadIdx.x] = threadIdx.x == 0 ? -1 : threadIdx.x == 1 ? session : 0;
}

// ceil(x / d) for x >= 0 and d >= 1, in 32-bit arithmetic when both are below 2^31.
__device__ __forceinline__ long long ceil_div_nn(long long x, long long d) {
    if (x < 0x80000000LL && d < 0x80000000LL)
        return (long long)(((uint32_t)x + (uint32_t)(d - 1)) / (uint32_t)d);
    return (x + d - 1) / d;
}

// ------------------------------------------------------------ placement ----
// XCD placement of the work list (MetadataArgs::placement = n XCDs): every session's
// items go to one XCD so that a decode kernel's items of one session share an L2 (the
// fused split merge relies on it).  Sessions are ranked by pages read, largest first
// (ties: lower session first), and dealt to the XCDs in a snake: ranks 0..n-1 to XCDs
// 0..n-1, ranks n..2n-1 to XCDs n-1..0, and so on, so each XCD takes one session per
// round of n ranks and no two XCDs' pages differ by more than the largest session's.  A
// session's items then take its XCD's next slots: item sp of the session of round q on
// XCD x lands in slot x + n * (k + sp), k the items of that XCD's sessions of rounds < q.
// There are ceil(B / n) rounds (up to 256 when n = 1); wave x takes them 64 at a time,
// one lane per round, carrying the running item count from pass to pass.
__device__ long long wave_scan_incl(long long v);  // inclusive sum over the wave's lanes

struct Placement {
    int32_t weight[kPlaceMaxSessions], order[kPlaceMaxSessions], bin[kPlaceMaxSessions],
        k0[kPlaceMaxSessions], cnt[kPlaceMaxXcds];
};

// All threads call it (B <= kPlaceMaxSessions, 1 <= n <= kPlaceMaxXcds <= kMetaWaves); q(b),
// ctx(b) and cus(b) read the session inputs and the work-item prefix.  Ends with a barrier.
template <typename Q, typename C, typename S>
__device__ void place_sessions(int B, int n, int page_size, Q q, C ctx, S cus, Placement& p) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int b = tid; b < B; b += kMetaThreads)
        p.weight[b] = q(b) > 0 ? (int32_t)ceil_div_nn((long long)ctx(b) + q(b), page_size) : 0;
    __syncthreads();
    // rank by (weight desc, session asc): tps threads per session (a power of two <= 64,
    // an aligned lane group) each count every tps-th other session, then sum in the group
    int tps = 64;
    while (tps > 1 && tps * B > kMetaThreads)
        tps >>= 1;
    {
        const int b = tid / tps, part = tid % tps;
        int r = 0, wb = 0;
        if (b < B) {
            wb = p.weight[b];
            for (int c = part; c < B; c += tps) {
                const int wc = p.weight[c];
                r += wc > wb || (wc == wb && c < b);
            }
        }
        for (int off = tps >> 1; off > 0; off >>= 1)
            r += __shfl_xor(r, off, 64);
        if (b < B && part == 0)
            p.order[r] = b;
    }
    __syncthreads();
    if (wave < n) {  // wave x: lane l holds XCD x's session of round q0 + l
        const int x = wave;
        long long carry = 0;  // items of XCD x's sessions of earlier passes
        for (int q0 = 0; q0 * n < B; q0 += 64) {
            const int qr = q0 + lane;
            const int r = qr * n + ((qr & 1) ? n - 1 - x : x);
            const bool real = r < B;  // rounds past the last, or the last round's gaps
            const int b = real ? p.order[r] : 0;
            const long long items = real ? cus(b + 1) - cus(b) : 0;
            const long long incl = carry + wave_scan_incl(items);
            if (real) {
                p.bin[b] = x;
                p.k0[b] = (int32_t)(incl - items);
            }
            carry = __shfl(incl, 63, 64);
        }
        if (lane == 0)
            p.cnt[x] = (int32_t)carry;
    }
    __syncthreads();
}

// Slots of the placed work list: the largest item count of one XCD, times n.
__device__ __forceinline__ long long placed_slots(const Placement& p, int n) {
    int m = 0;
    for (int i = 0; i < n; ++i)
        m = max(m, p.cnt[i]);
    return (long long)m * n;
}

// L: the batch fits the LDS mirrors (B <= kMetaLdsCap); the compiler then reads them
// with LDS instructions rather than flat loads.
template <bool L>
__global__ __launch_bounds__(kMetaThreads) void build_metadata_kernel(MetadataArgs a) {
    constexpr int CAP = L ? kMetaLdsCap : 1, PT = L ? kMetaPtCap : 1;
    __shared__ long long lds[3 * kMetaWaves];
    __shared__ long long carry[3];
    __shared__ int err;
    __shared__ int32_t s_cup[CAP + 1], s_cuq[CAP + 1], s_cus[CAP + 1];
    __shared__ int32_t s_q[CAP], s_ctx[CAP], s_pt[PT];
    const int tid = threadIdx.x;
    constexpr bool in_lds = L;
    const long long entries = (long long)a.B * a.max_pages;
    const bool pt_lds = L && entries <= kMetaPtCap;
    const int32_t* __restrict__ qlen = L ? s_q : a.q_len;
    const int32_t* __restrict__ ctxl = L ? s_ctx : a.ctx_len;
    const int32_t* cup = L ? s_cup : a.cu_pages;
    const int32_t* cuq = L ? s_cuq : a.cu_seqlens_q;
    const int32_t* cus = L ? s_cus : a.cu_splits;
    if (tid == 0) {
        carry[0] = carry[1] = carry[2] = 0;
        err = INT_MAX;
        a.cu_seqlens_q[0] = 0;
        a.cu_seqlens_k[0] = 0;
        a.cu_splits[0] = 0;
        if (L) {
            s_cuq[0] = 0;
            s_cus[0] = 0;
        }
    }
    if (in_lds)
        for (int b = tid; b <= a.B; b += kMetaThreads) {
            const int32_t cp = a.cu_pages[b];
            const int32_t q = b < a.B ? a.q_len[b] : 0, c = b < a.B ? a.ctx_len[b] : 0;
            s_cup[b] = cp;
            if (b < a.B) {
                s_q[b] = q;
                s_ctx[b] = c;
            }
        }
    __syncthreads();
    // Phase 1: padded page table and page-id validation (a session listing more than
    // max_pages pages is invalid anyway and only its first max_pages ids are read), then
    // cu_seqlens_q/k, validation and the total pages of sessions with queries.
    const bool small = entries <= INT_MAX;  // 32-bit index arithmetic
    for (long long e0 = tid; e0 < entries; e0 += (long long)kMetaThreads * kMetaUnroll) {
        int32_t pid[kMetaUnroll];
        int bs[kMetaUnroll], js[kMetaUnroll];
#pragma unroll
        for (int k = 0; k < kMetaUnroll; ++k) {
            const long long e = e0 + (long long)k * kMetaThreads;
            pid[k] = -1;
            bs[k] = -1;
            js[k] = 0;
            if (e < entries) {
                if (small) {
                    bs[k] = (int)e / a.max_pages;
                    js[k] = (int)e - bs[k] * a.max_pages;
                } else {
                    bs[k] = (int)(e / a.max_pages);
                    js[k] = (int)(e % a.max_pages);
                }
                if (js[k] < cup[bs[k] + 1] - cup[bs[k]])
                    pid[k] = a.page_ids[cup[bs[k]] + js[k]];
                else
                    bs[k] = -2;  // padding entry
            }
        }
        int bad_b = INT_MAX;
#pragma unroll
        for (int k = 0; k < kMetaUnroll; ++k) {
            const long long e = e0 + (long long)k * kMetaThreads;
            if (bs[k] == -1)
                continue;  // past the table
            if (bs[k] >= 0 && (pid[k] < 0 || pid[k] >= a.num_pool_pages))
                bad_b = min(bad_b, bs[k]);
            a.page_table[e] = pid[k];
            if (pt_lds)
                s_pt[e] = pid[k];
        }
        if (bad_b != INT_MAX)
            atomicMin(&err, bad_b);
    }
    for (int base = 0; base < a.B; base += kMetaThreads) {
        const int b = base + tid;
        long long v[3] = {0, 0, 0}, tot[3];
        int bad = 0;
        if (b < a.B) {
            const long long q = qlen[b], ctx = ctxl[b];
            const long long npages = (long long)cup[b + 1] - cup[b];
            const long long kl = ctx + q;
            const long long need = kl < 0 ? 0 : ceil_div_nn(kl, a.page_size);
            bad = q < 0 || ctx < 0 || npages < 0 || npages > a.max_pages || need > npages;
            v[0] = q;
            v[1] = kl;
            v[2] = q > 0 ? need : 0;
        }
        block_scan3(v, tot, lds);
        if (b < a.B) {
            const long long iq = v[0] + carry[0], ik = v[1] + carry[1];
            if (bad || iq > INT_MAX || ik > INT_MAX || iq > a.max_rows)
                atomicMin(&err, b);
            a.cu_seqlens_q[b + 1] = (int32_t)iq;
            a.cu_seqlens_k[b + 1] = (int32_t)ik;
            if (in_lds)
                s_cuq[b + 1] = (int32_t)iq;
        }
        __syncthreads();
        if (tid == 0)
            for (int k = 0; k < 3; ++k)
                carry[k] += tot[k];
        __syncthreads();
    }
    if (err != INT_MAX) {
        write_error(a, err);
        return;
    }
    const long long total_q = carry[0], total_k = carry[1], total_pages = carry[2];
    long long split = a.split_pages;
    if (split == 0) {
        split = (total_pages + a.target_blocks - 1) / a.target_blocks;
        if (split < 1)
            split = 1;
    }
    __syncthreads();
    if (tid == 0)
        carry[0] = 0;
    __syncthreads();
    // Phase 2: split-K work items per session.
    for (int base = 0; base < a.B; base += kMetaThreads) {
        const int b = base + tid;
        long long v[3] = {0, 0, 0}, tot[3];
        if (b < a.B && qlen[b] > 0) {
            const long long kl = (long long)ctxl[b] + qlen[b];
            v[0] = ceil_div_nn(ceil_div_nn(kl, a.page_size), split);
        }
        const long long ns = v[0];
        block_scan3(v, tot, lds);
        if (b < a.B) {
            const long long w = v[0] + carry[0];
            if (w > a.max_work)
                atomicMin(&err, b);
            a.num_splits[b] = (int32_t)ns;
            a.cu_splits[b + 1] = (int32_t)w;
            if (in_lds)
                s_cus[b + 1] = (int32_t)w;
        }
        __syncthreads();
        if (tid == 0)
            carry[0] += tot[0];
        __syncthreads();
    }
    if (err != INT_MAX) {
        write_error(a, err);
        return;
    }
    const long long W = carry[0];
    // Phase 3: block-to-session map, work descriptors, slot mapping.
    __shared__ Placement place[1];
    const int n = L ? a.placement : 0;
    if (n > 0) {
        place_sessions(a.B, n, a.page_size, [&](int b) { return qlen[b]; },
                       [&](int b) { return ctxl[b]; }, [&](int b) { return cus[b]; }, place[0]);
        if (placed_slots(place[0], n) > a.max_work) {
            write_error(a, a.B);  // max_work cannot hold the placed work list
            return;
        }
    }
    for (long long w = tid; w < a.max_work; w += kMetaThreads) {
        const bool empty = n > 0 ? w / n >= place[0].cnt[w % n] : w >= W;
        if (empty)
            a.work_desc[w * kWorkDescInts] = -1;
    }
    for (long long u = tid; u < W; u += kMetaThreads) {
        const int b = upper_index(cus, a.B, u);
        const int sp = (int)(u - cus[b]);
        const long long w = n > 0 ? place[0].bin[b] + (long long)n * (place[0].k0[b] + sp) : u;
        int32_t* d = a.work_desc + w * kWorkDescInts;
        int32_t* pg = a.work_pages + w * kWorkPages;
        const int kl = ctxl[b] + qlen[b];
        const int need = (kl + a.page_size - 1) / a.page_size;
        const int p0 = (int)(sp * split);
        const int p1 = (int)(p0 + split < need ? p0 + split : need);
        a.work_session[w] = b;
        a.work_split[w] = sp;
        d[0] = b;
        d[1] = cuq[b];
        d[2] = kl;
        d[3] = p0;
        d[4] = p1;
        d[5] = cus[b + 1] - cus[b];
        d[6] = (int32_t)u;
        d[7] = qlen[b];
#pragma unroll
        for (int j = 0; j < kWorkPages; ++j)
            pg[j] = p0 + j < p1 ? (pt_lds ? s_pt[(long long)b * a.max_pages + p0 + j]
                                          : a.page_ids[cup[b] + p0 + j])
                                : -1;
    }
    for (long long i = tid; i < total_q; i += kMetaThreads) {
        const int b = upper_index(cuq, a.B, i);
        const long long pos = (long long)ctxl[b] + (i - cuq[b]);
        const long long j = pos / a.page_size;
        const int32_t page = pt_lds ? s_pt[(long long)b * a.max_pages + j] : a.page_ids[cup[b] + j];
        a.slot_mapping[i] = (int32_t)(page * (long long)a.page_size + pos % a.page_size);
    }
    if (tid == 0) {
        a.info[0] = (int32_t)W;
        a.info[1] = (int32_t)split;
        a.info[2] = (int32_t)total_q;
        a.info[3] = (int32_t)total_k;
        a.info[kInfoPlacement] = n;
        for (int k = kInfoPlacement + 1; k < kInfoInts; ++k)
            a.info[k] = 0;
    }
}

// The build for batches whose session arrays and padded page table fit in LDS
// (B <= kMetaLdsCap, B * max_pages <= kMetaSmallPt).  All waves stage the inputs and the
// page ids in LDS (one load round trip each); wave 0 alone runs both scans, 64 sessions
// per pass with the running total carried between passes (a 6-step wave scan instead of
// a 1024-thread block scan, whose 64-bit shuffles and barriers cost microseconds); then
// all waves write every output, with no global store before the last barrier.  Outputs
// are bit-identical to build_metadata_kernel's.
constexpr int kMetaSmallPt = 8192;

// One DPP move of a 64-bit value (both halves with the same control); lanes the
// control gives no source, and rows outside row_mask, receive 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ long long dpp64(long long v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xf,
                                               true);
    return (long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Inclusive scan over the 64 lanes of a wave on DPP moves (no LDS round trips): shifts
// of 1, 2, 4, 8 lanes within each row of 16, then lane 15 of each row broadcast into
// the next row (rows 1, 3) and lane 31 into the upper half (rows 2, 3).
__device__ __forceinline__ long long wave_scan_incl(long long v) {
    v += dpp64<0x111, 0xf>(v);  // row_shr:1
    v += dpp64<0x112, 0xf>(v);  // row_shr:2
    v += dpp64<0x114, 0xf>(v);  // row_shr:4
    v += dpp64<0x118, 0xf>(v);  // row_shr:8
    v += dpp64<0x142, 0xa>(v);  // row_bcast:15
    v += dpp64<0x143, 0xc>(v);  // row_bcast:31
    return v;
}

__global__ __launch_bounds__(kMetaThreads) void build_metadata_lds_kernel(MetadataArgs a) {
    __shared__ int32_t s_cup[kMetaLdsCap + 1], s_q[kMetaLdsCap], s_ctx[kMetaLdsCap];
    __shared__ int32_t s_cuq[kMetaLdsCap + 1], s_cuk[kMetaLdsCap + 1], s_cus[kMetaLdsCap + 1];
    __shared__ int32_t s_pt[kMetaSmallPt];
    __shared__ int err;
    __shared__ long long s_tot[4];  // total_q, total_k, split, W
    const int tid = threadIdx.x, lane = tid & 63, B = a.B, mp = a.max_pages;
    const int entries = B * mp;  // <= kMetaSmallPt
    // ---- inputs to LDS ----
    for (int b = tid; b <= B; b += kMetaThreads) {
        s_cup[b] = a.cu_pages[b];
        if (b < B) {
            s_q[b] = a.q_len[b];
            s_ctx[b] = a.ctx_len[b];
        }
    }
    if (tid == 0) {
        err = INT_MAX;
        s_cuq[0] = s_cuk[0] = s_cus[0] = 0;
    }
    __syncthreads();
    // ---- padded page table in LDS; ids out of the pool name their session ----
    {
        constexpr int U = kMetaSmallPt / kMetaThreads;
        int32_t pid[U];
        int bad_b = INT_MAX;
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int e = tid + k * kMetaThreads;
            const int b = e < entries ? (int)((uint32_t)e / (uint32_t)mp) : 0;
            const int j = e - b * mp;
            const int p0 = s_cup[b], np = s_cup[b + 1] - p0;
            const bool listed = e < entries && j < np;
            pid[k] = listed ? a.page_ids[p0 + j] : -1;
            if (listed && (pid[k] < 0 || pid[k] >= a.num_pool_pages))
                bad_b = min(bad_b, b);
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int e = tid + k * kMetaThreads;
            if (e < entries)
                s_pt[e] = pid[k];
        }
        if (bad_b != INT_MAX)
            atomicMin(&err, bad_b);
    }
    __syncthreads();
    // ---- wave 0: cumulative rows / keys / pages, then work items per session ----
    if (tid < 64) {
        long long cq = 0, ck = 0, cp = 0;
        int bad = INT_MAX;
        for (int base = 0; base < B; base += 64) {
            const int b = base + lane;
            long long q = 0, kl = 0, pages = 0;
            if (b < B) {
                q = s_q[b];
                const long long ctx = s_ctx[b];
                const long long npages = (long long)s_cup[b + 1] - s_cup[b];
                kl = ctx + q;
                const long long need = kl < 0 ? 0 : ceil_div_nn(kl, a.page_size);
                if (q < 0 || ctx < 0 || npages < 0 || npages > mp || need > npages)
                    bad = min(bad, b);
                pages = q > 0 ? need : 0;
            }
            const long long iq = cq + wave_scan_incl(q), ik = ck + wave_scan_incl(kl);
            const long long ip = cp + wave_scan_incl(pages);
            if (b < B) {
                if (iq > INT_MAX || ik > INT_MAX || iq > a.max_rows)
                    bad = min(bad, b);
                s_cuq[b + 1] = (int32_t)iq;
                s_cuk[b + 1] = (int32_t)ik;
            }
            cq = __shfl(iq, 63, 64);
            ck = __shfl(ik, 63, 64);
            cp = __shfl(ip, 63, 64);
        }
        long long split = a.split_pages;
        if (split == 0) {
            split = (cp + a.target_blocks - 1) / a.target_blocks;
            if (split < 1)
                split = 1;
        }
        long long cw = 0;
        for (int base = 0; base < B; base += 64) {
            const int b = base + lane;
            long long ns = 0;
            if (b < B && s_q[b] > 0)
                ns = ceil_div_nn(ceil_div_nn((long long)s_ctx[b] + s_q[b], a.page_size), split);
            const long long iw = cw + wave_scan_incl(ns);
            if (b < B) {
                if (iw > a.max_work)
                    bad = min(bad, B + b);  // reported only when the first scan found nothing
                s_cus[b + 1] = (int32_t)iw;
            }
            cw = __shfl(iw, 63, 64);
        }
        // First offending session: the row/key/page checks outrank the work-item one.
        for (int off = 32; off > 0; off >>= 1)
            bad = min(bad, __shfl_xor(bad, off, 64));
        if (lane == 0) {
            if (bad != INT_MAX)
                atomicMin(&err, bad >= B ? bad - B + (1 << 30) : bad);
            s_tot[0] = cq;
            s_tot[1] = ck;
            s_tot[2] = split;
            s_tot[3] = cw;
        }
    }
    __syncthreads();
    if (err != INT_MAX) {
        write_error(a, err >= (1 << 30) ? err - (1 << 30) : err);
        return;
    }
    const long long total_q = s_tot[0], total_k = s_tot[1], split = s_tot[2];
    const int W = (int)s_tot[3];
    __shared__ Placement place;
    if (a.placement > 0) {
        place_sessions(B, a.placement, a.page_size, [&](int b) { return s_q[b]; },
                       [&](int b) { return s_ctx[b]; }, [&](int b) { return s_cus[b]; }, place);
        if (placed_slots(place, a.placement) > a.max_work) {
            write_error(a, B);  // max_work cannot hold the placed work list
            return;
        }
    }
    // ---- outputs: global stores only from here on ----
    for (int b = tid; b <= B; b += kMetaThreads) {
        a.cu_seqlens_q[b] = s_cuq[b];
        a.cu_seqlens_k[b] = s_cuk[b];
        a.cu_splits[b] = s_cus[b];
        if (b < B)
            a.num_splits[b] = s_cus[b + 1] - s_cus[b];
    }
    for (int e = tid; e < entries; e += kMetaThreads)
        a.page_table[e] = s_pt[e];
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    const int n = a.placement;
    for (int w = tid; w < a.max_work; w += kMetaThreads) {
        const bool empty = n > 0 ? w / n >= place.cnt[w % n] : w >= W;
        if (empty)
            a.work_desc[(long long)w * kWorkDescInts] = -1;
    }
    for (int u = tid; u < W; u += kMetaThreads) {
        const int b = upper_index(s_cus, B, u);
        const int sp = u - s_cus[b];
        const int w = n > 0 ? place.bin[b] + n * (place.k0[b] + sp) : u;
        const int q = s_q[b], kl = s_ctx[b] + q;
        const int need = (kl + a.page_size - 1) / a.page_size;
        const int p0 = (int)(sp * split);
        const int p1 = (int)(p0 + split < need ? p0 + split : need);
        a.work_session[w] = b;
        a.work_split[w] = sp;
        i32x4* d = reinterpret_cast<i32x4*>(a.work_desc + (long long)w * kWorkDescInts);
        d[0] = i32x4{b, s_cuq[b], kl, p0};
        d[1] = i32x4{p1, s_cus[b + 1] - s_cus[b], u, q};
        int32_t pg[kWorkPages];
#pragma unroll
        for (int j = 0; j < kWorkPages; ++j)
            pg[j] = p0 + j < p1 ? s_pt[b * mp + p0 + j] : -1;
        i32x4* dp = reinterpret_cast<i32x4*>(a.work_pages + (long long)w * kWorkPages);
        dp[0] = i32x4{pg[0], pg[1], pg[2], pg[3]};
        dp[1] = i32x4{pg[4], pg[5], pg[6], pg[7]};
    }
    for (int i = tid; i < (int)total_q; i += kMetaThreads) {
        const int b = upper_index(s_cuq, B, i);
        const int pos = s_ctx[b] + (i - s_cuq[b]);
        const int page = s_pt[b * mp + pos / a.page_size];
        a.slot_mapping[i] = (int32_t)(page * (long long)a.page_size + pos % a.page_size);
    }
    if (tid == 0) {
        a.info[0] = W;
        a.info[1] = (int32_t)split;
        a.info[2] = (int32_t)total_q;
        a.info[3] = (int32_t)total_k;
        a.info[kInfoPlacement] = n;
        for (int k = kInfoPlacement + 1; k < kInfoInts; ++k)
            a.info[k] = 0;
    }
}

// One thread per element of the appended rows; RNE rounding to 16 bits.
template <typename T>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    const int width = a.kv_rank + a.rope_dim;
    const long long total = (long long)a.T * width;
    const long long rec = (long long)a.page_size * width;
    const bool tiled = page_tiled(a.page_size, a.kv_rank, a.rope_dim);
    for (long long e = blockIdx.x * 256LL + threadIdx.x; e < total; e += 256LL * gridDim.x) {
        const int t = (int)(e / width), c = (int)(e % width);
        const int slot = a.slot_mapping[t];
        const int page = slot / a.page_size, off = slot % a.page_size;
        if (slot < 0 || page >= a.num_pool_pages)
            continue;
        uint16_t* base = a.pages + page * rec;
        if (c < a.kv_rank)
            base[latent_word(tiled, off, c, a.page_size, a.kv_rank)] =
                T::from_float(a.ckv[(long long)t * a.kv_rank + c]);
        else {
            const int j = c - a.kv_rank;
            base[rope_word(tiled, off, j, a.page_size, a.kv_rank, a.rope_dim)] =
                T::from_float(a.krope[(long long)t * a.rope_dim + j]);
        }
    }
}

}  // namespace

hipError_t launch_build_metadata(const MetadataArgs& a, hipStream_t stream) {
    if (a.B <= kMetaLdsCap && (long long)a.B * a.max_pages <= kMetaSmallPt)
        hipLaunchKernelGGL(build_metadata_lds_kernel, dim3(1), dim3(kMetaThreads), 0, stream, a);
    else if (a.B <= kMetaLdsCap)
        hipLaunchKernelGGL(build_metadata_kernel<true>, dim3(1), dim3(kMetaThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(build_metadata_kernel<false>, dim3(1), dim3(kMetaThreads), 0, stream,
                           a);
    return hipGetLastError();
}

// XCD of each workgroup of a launch (the XCC_ID hardware register), for the placement probe.
__global__ __launch_bounds__(64) void xcd_probe_kernel(int32_t* out) {
    if (threadIdx.x == 0) {
        unsigned x;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
        out[blockIdx.x] = (int32_t)x;
    }
}

int xcd_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || n < 1)
        return 0;
    return n;
}

// Whether the workgroups w of a launch with one residue w % n run on one XCD, and the n
// residues on n different XCDs, on the current device: ids of 16 rounds of n workgroups,
// launched twice.  Empty string when it holds, else the reason.  (Which XCD takes
// residue 0 differs between hardware queues: each queue starts its round-robin on an XCD
// of its own, which placement does not depend on.)
std::string probe_xcd_placement() {
    const int n = xcd_count();
    if (n < 1 || n > kPlaceMaxXcds)
        return "XCD count " + std::to_string(n) + " outside 1.." + std::to_string(kPlaceMaxXcds);
    const int G = 16 * n;
    int32_t* d = nullptr;
    std::vector<int32_t> h(G);
    std::string why;
    if (hipMalloc(&d, G * sizeof(int32_t)) != hipSuccess)
        return "probe allocation failed";
    for (int rep = 0; rep < 2 && why.empty(); ++rep) {
        hipLaunchKernelGGL(xcd_probe_kernel, dim3(G), dim3(64), 0, nullptr, d);
        if (hipMemcpy(h.data(), d, G * sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess) {
            why = "probe launch failed";
            break;
        }
        for (int w = 0; w < G && why.empty(); ++w)
            if (h[w] != h[w % n] || (w < n && std::count(h.begin(), h.begin() + n, h[w]) != 1) ||
                h[w] < 0 || h[w] > 15)
                why = "workgroup " + std::to_string(w) + " ran on XCD " + std::to_string(h[w]);
    }
    (void)hipFree(d);
    return why;
}

hipError_t launch_append(const AppendArgs& a, int dtype, hipStream_t stream) {
    const long long total = (long long)a.T * (a.kv_rank + a.rope_dim);
    if (total == 0)
        return hipSuccess;
    const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    if (dtype == 0)
        hipLaunchKernelGGL(append_kernel<F16>, dim3(blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(append_kernel<BF16>, dim3(blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla
