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
//   flattens (query, head) into q-rows r = i*H + h: a workgroup of 4 waves owns 128
//   consecutive q-rows of one session (16 queries at H = 8), a wave QT 16-row tiles.
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

constexpr int kPfWaves = 4;

template <typename T, int KV, int RP, int PS, int QT>
__global__ __launch_bounds__(64 * kPfWaves) void prefill_page_kernel(PrefillArgs a) {
    static_assert(KV % 32 == 0 && RP % 8 == 0 && RP <= 32 && PS % 32 == 0, "tile shape");
    constexpr int KS = KV / 32;               // latent k-steps of the score MFMAs
    constexpr int TT = PS / 16;               // 16-token tiles per page
    constexpr int UPP = PS / 32;              // 32-token k-steps of O^T per page
    constexpr int RT = KV / 16;               // 16-row (latent) tiles of O^T
    constexpr int REC = PS * (KV + RP);       // words of a page record
    constexpr int CHUNKS = REC / 8;           // 16-byte chunks of a record
    constexpr int THREADS = 64 * kPfWaves;
    constexpr int CPT = (CHUNKS + THREADS - 1) / THREADS;
    constexpr int WG_ROWS = kPfWaves * QT * 16;
    static_assert(KV % 16 == 0 && (PS * KV) % 8 == 0, "record chunks");
    using V8 = typename T::vec8;
    __shared__ __attribute__((aligned(16))) uint16_t buf[2][REC];

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
    const int wave = tid >> 6;
    // keys [0, k_hi) are visible to some q-row of this workgroup
    const int last_q = min(n_rows - 1, rb + WG_ROWS - 1) / H;
    const int k_hi = ctx + last_q + 1;
    const int n_pages = (k_hi + PS - 1) / PS;
    const int32_t* ptab = a.page_table + (long long)b * a.max_pages;

    // ---- page staging: 16-byte chunks, slots at or past k_len zeroed ----
    u32x4 stage[CPT];
    auto load_page = [&](int p) {
        const int page = ptab[p];
        const bool ok = (unsigned)page < (unsigned)a.num_pool_pages;
        const uint16_t* base = a.pages + (long long)(ok ? page : 0) * REC;
        const int tok0 = p * PS;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + k * THREADS;
            stage[k] = u32x4{0, 0, 0, 0};
            if (c < CHUNKS) {
                // slot of chunk c: latent chunks run (t, j, g, n), rope chunks (t, ch, n)
                const int slot = c < PS * KV / 8 ? (c / (16 * 4 * KS)) * 16 + (c & 15)
                                                 : ((c - PS * KV / 8) / (16 * (RP / 8))) * 16 +
                                                       (c & 15);
                if (ok && tok0 + slot < k_len)
                    stage[k] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4*>(base + (long long)c * 8));
            }
        }
    };
    auto store_page = [&](uint16_t* dst) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + k * THREADS;
            if (c < CHUNKS)
                *reinterpret_cast<u32x4*>(dst + c * 8) = stage[k];
        }
    };

    // ---- this wave's q-tiles: Q^T operands, causal limits ----
    const int wr0 = rb + wave * QT * 16;  // first session q-row of the wave
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
    const int rope_off = (16 * (rope_lane ? g : g % (RP / 8)) + n) * 8;
    // transpose-read address of lane (g, j=n) inside a token tile: token 4g + n/4,
    // latent 4*(n%4) + (row-tile offset)
    const int tr_lane = (((n & 3) >> 1) * 128) + (4 * g + (n >> 2)) * 8 + 4 * (n & 1);

    float m_run[QT], l_run[QT];
    floatx4 acc[QT][RT];
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        m_run[q] = -INFINITY;
        l_run[q] = 0.0f;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            acc[q][rt] = floatx4{0, 0, 0, 0};
    }

    load_page(0);
    store_page(buf[0]);
    __syncthreads();
    for (int p = 0; p < n_pages; ++p) {
        const bool more = p + 1 < n_pages;
        if (more)
            load_page(p + 1);  // in flight while this page is consumed
        const uint16_t* pg = buf[p & 1];
        const int tok0 = p * PS;
        // S^T tiles
        floatx4 sc[TT][QT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int q = 0; q < QT; ++q)
                sc[t][q] = floatx4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                const V8 ka = *reinterpret_cast<const V8*>(pg + (t * KS + j) * 512 + lane * 8);
#pragma unroll
                for (int q = 0; q < QT; ++q)
                    sc[t][q] = T::mma32(ka, qv[q][j], sc[t][q]);
            }
            const V8 kr =
                *reinterpret_cast<const V8*>(pg + PS * KV + t * (RP / 8) * 128 + rope_off);
#pragma unroll
            for (int q = 0; q < QT; ++q)
                sc[t][q] = T::mma32(kr, qv[q][KS], sc[t][q]);
        }
        // mask + online softmax per q-row (lane column n)
        V8 pb[QT][UPP], pl[QT][UPP];  // P^T operands (pl: the low part, bf16 only)
#pragma unroll
        for (int q = 0; q < QT; ++q) {
            float mp = -INFINITY;
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tok = tok0 + 16 * t + 4 * g + i;
                    const float x = tok <= lim[q] ? sc[t][q][i] * a.scale_log2 : -INFINITY;
                    sc[t][q][i] = x;
                    mp = fmaxf(mp, x);
                }
            mp = fmaxf(mp, __shfl_xor(mp, 16, 64));
            mp = fmaxf(mp, __shfl_xor(mp, 32, 64));
            const float m_new = fmaxf(m_run[q], mp);
            if (m_new > m_run[q]) {
                const float alpha = m_run[q] == -INFINITY ? 0.0f : exp2_fast(m_run[q] - m_new);
                l_run[q] *= alpha;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    acc[q][rt] *= alpha;
                m_run[q] = m_new;
            }
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = m_new == -INFINITY ? 0.0f : exp2_fast(sc[t][q][i] - m_new);
                    psum += e;
                    const auto hi = static_cast<typename T::scalar>(e);
                    pb[q][t / 2][4 * (t % 2) + i] = hi;
                    if constexpr (T::split_p)
                        pl[q][t / 2][4 * (t % 2) + i] =
                            static_cast<typename T::scalar>(e - static_cast<float>(hi));
                }
            l_run[q] += psum;  // per lane; summed over the 4 lane groups at the end
        }
        // O^T += C^T . P^T
#pragma unroll
        for (int u = 0; u < UPP; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int blk = ((rt >> 1) * 4 + 2 * (rt & 1)) * 128;  // latent rows 16rt..
                const u32x2 lo = lds_read_tr16(pg + (2 * u) * KS * 512 + blk + tr_lane);
                const u32x2 hi = lds_read_tr16(pg + (2 * u + 1) * KS * 512 + blk + tr_lane);
                const V8 ca = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
                for (int q = 0; q < QT; ++q) {
                    acc[q][rt] = T::mma32(ca, pb[q][u], acc[q][rt]);
                    if constexpr (T::split_p)
                        acc[q][rt] = T::mma32(ca, pl[q][u], acc[q][rt]);
                }
            }
        if (more)
            store_page(buf[(p + 1) & 1]);  // last read of that buffer was before the barrier
        __syncthreads();
    }

    // ---- normalise and store ----
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        float l = l_run[q];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const int r = wr0 + q * 16 + n;
        if (r >= n_rows)
            continue;
        const long long fr = (long long)q0 * H + r;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            *reinterpret_cast<floatx4*>(a.out + fr * KV + 16 * rt + 4 * g) = acc[q][rt] * inv;
        if (a.lse && g == 0)
            a.lse[fr] = (m_run[q] + __log2f(l)) * kLn2;
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

constexpr int kPfQT = 2;

template <typename T>
hipError_t launch_prefill_page(const PrefillArgs& a, int max_q_len, hipStream_t stream) {
    constexpr int rows = kPfWaves * kPfQT * 16;
    const long long gx = ((long long)max_q_len * a.H + rows - 1) / rows;
    hipLaunchKernelGGL((prefill_page_kernel<T, 128, 16, 64, kPfQT>), dim3((unsigned)gx, a.B),
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
