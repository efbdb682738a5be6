// Shared device helpers for the gfx950 MLA kernels: 16-bit element types,
// MFMA operand vectors, RNE conversions and wave reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mla {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element-type traits: 16-bit storage dtype code 0 = fp16, 1 = bf16 (the cache
// stores raw 16-bit words; the tag picks the MFMA flavour and conversions).
struct F16 {
    using scalar = _Float16;
    using vec8 = half8;
    static constexpr int code = 0;
    // Softmax probabilities enter the P.C MFMA as one fp16 operand (2^-11 relative).
    static constexpr bool split_p = false;
    __device__ static float to_float(uint16_t bits) {
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    }
    __device__ static uint16_t from_float(float x) {  // IEEE RNE (v_cvt_f16_f32)
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    __device__ static floatx4 mma32(vec8 a, vec8 b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    __device__ static vec8 ones8() { return vec8{1, 1, 1, 1, 1, 1, 1, 1}; }
};

struct BF16 {
    using scalar = __bf16;
    using vec8 = bf8;
    static constexpr int code = 1;
    // bf16 keeps 8 mantissa bits: probabilities enter the P.C MFMA as hi + lo bf16
    // parts (two MFMAs, about 16 bits), so the output stays within the fp32 tolerance.
    static constexpr bool split_p = true;
    __device__ static float to_float(uint16_t bits) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
    }
    __device__ static uint16_t from_float(float x) {  // RNE, quiet NaN
        uint32_t u = __builtin_bit_cast(uint32_t, x);
        if ((u & 0x7fffffffu) > 0x7f800000u)
            return static_cast<uint16_t>((u >> 16) | 0x40u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return static_cast<uint16_t>(u >> 16);
    }
    __device__ static floatx4 mma32(vec8 a, vec8 b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static vec8 ones8() {
        const __bf16 one = __builtin_bit_cast(__bf16, static_cast<uint16_t>(0x3f80));
        return vec8{one, one, one, one, one, one, one, one};
    }
};

__device__ inline float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ inline float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off, 64);
    return v;
}

// Max / sum over lanes n, n+16, n+32, n+48 of a wave (its four 16-lane rows), left in
// every lane.  gfx950's v_permlane16_swap exchanges rows between the row pairs {0,1} and
// {2,3}, v_permlane32_swap the two 32-lane halves: two VALU swaps instead of two LDS
// permute round trips.  Each stage combines the two rows of a pair, so the result is
// the one __shfl_xor(., 16) then __shfl_xor(., 32) gives (max and + are commutative).
// Every lane of the wave must be active.
// (The swap results are copied out element by element: a __builtin_bit_cast of an
// element of the returned vector reads element 0 in this toolchain.)
__device__ __forceinline__ void swap_rows16(float x, float& a, float& b) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const unsigned r0 = r[0], r1 = r[1];
    a = __uint_as_float(r0);
    b = __uint_as_float(r1);
}
__device__ __forceinline__ void swap_halves32(float x, float& a, float& b) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const unsigned r0 = r[0], r1 = r[1];
    a = __uint_as_float(r0);
    b = __uint_as_float(r1);
}
__device__ __forceinline__ float rows_max(float x) {
    float a, b;
    swap_rows16(x, a, b);
    swap_halves32(fmaxf(a, b), a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float rows_sum(float x) {
    float a, b;
    swap_rows16(x, a, b);
    swap_halves32(a + b, a, b);
    return a + b;
}

// One wave copies 1 KB from global memory to LDS: lane l's 16 bytes, read at
// base + off bytes (base uniform, off the lane's own), land at dst + 16 l bytes (gfx950
// global_load_lds_dwordx4 in its scalar-base form; the LDS address goes in M0, which no
// other code here uses).  Written as inline assembly so that the compiler, which cannot
// tell which LDS bytes such a copy writes, does not wait for every copy in flight before
// each later LDS access (it did, before the first transpose read after a prefetch).
// The copy counts in vmcnt: the caller waits for it (s_waitcnt vmcnt) and orders its
// LDS reads after the wait (wave_lds_fence or a barrier) before reading what it wrote.
// Any vmcnt wait of the compiler's own (for a global load, or a register reload) also
// waits for the copies issued before it, so the copies go out after such loads.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy_block_to_lds(const void* base, uint32_t off, void* dst) {
    // readfirstlane returns int: each half goes through uint32_t before widening (a
    // sign-extended low half would set the upper 32 bits of the address).
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((uint32_t)b));
    const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
    const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)dst));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0), "v"(off), "s"(reinterpret_cast<const void*>(sb))
                 : "memory", "m0");
}
// The 32-bit LDS address of a __shared__ object, for copy_block_to_lds_at: a caller that
// issues several copies converts its destination once and adds byte offsets, instead of
// paying the generic-to-LDS conversion (a null check on a 64-bit pointer) per copy.
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)p));
}
// copy_block_to_lds with the destination given as an LDS address (uniform).
__device__ __forceinline__ void copy_block_to_lds_at(const void* base, uint32_t off, uint32_t lds) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((uint32_t)b));
    const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
    const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lds));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0), "v"(off), "s"(reinterpret_cast<const void*>(sb))
                 : "memory", "m0");
}
// Four consecutive 1 KB blocks, base + k KB -> lds + k KB (k < 4), through the
// instruction offset, which global_load_lds applies to the global and the LDS address
// alike: one M0 and one base for the four copies.
__device__ __forceinline__ void copy_4blocks_to_lds_at(const void* base, uint32_t off, uint32_t lds) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((uint32_t)b));
    const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
    const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lds));
    asm volatile(
        "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "global_load_lds_dwordx4 %1, %2 offset:1024\n\t"
        "global_load_lds_dwordx4 %1, %2 offset:2048\n\t"
        "global_load_lds_dwordx4 %1, %2 offset:3072"
        :
        : "s"(m0), "v"(off), "s"(reinterpret_cast<const void*>(sb))
        : "memory", "m0");
}
#pragma clang diagnostic pop

// Orders this wave's LDS accesses: nothing before it moves after it, or after it before.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace mla

namespace mla {

// ---- Page record layout ------------------------------------------------------
// A page record holds page_size tokens of one layer: the latent section
// (page_size * kv_rank words) followed by the rope-key section (page_size *
// rope_dim words), 16-bit words.  When page_size % 16 == 0, kv_rank % 32 == 0 and
// rope_dim % 8 == 0 the record is TILED in MFMA-operand order, so that one 64-lane
// 16-byte load reads 1 KB contiguously:
//   latent (slot, r): tile t = slot/16, n = slot%16, j = r/32, g = (r%32)/8,
//                     e = r%8  ->  ((t*(kv_rank/32) + j)*4 + g)*128 + n*8 + e
//   rope (slot, c):   ch = c/8, e = c%8
//                     ->  page_size*kv_rank + (t*(rope_dim/8) + ch)*128 + n*8 + e
// Otherwise the record is row-major: latent slot*kv_rank + r, rope
// page_size*kv_rank + slot*rope_dim + c.
__host__ __device__ inline bool page_tiled(int page_size, int kv_rank, int rope_dim) {
    return page_size % 16 == 0 && kv_rank % 32 == 0 && rope_dim % 8 == 0;
}
__host__ __device__ inline long long latent_word(bool tiled, int slot, int r, int page_size,
                                                 int kv_rank) {
    (void)page_size;
    if (!tiled)
        return (long long)slot * kv_rank + r;
    const int t = slot >> 4, n = slot & 15, j = r >> 5, g = (r & 31) >> 3, e = r & 7;
    return ((long long)(t * (kv_rank >> 5) + j) * 4 + g) * 128 + n * 8 + e;
}
__host__ __device__ inline long long rope_word(bool tiled, int slot, int c, int page_size,
                                               int kv_rank, int rope_dim) {
    const long long base = (long long)page_size * kv_rank;
    if (!tiled)
        return base + (long long)slot * rope_dim + c;
    const int t = slot >> 4, n = slot & 15, ch = c >> 3, e = c & 7;
    return base + (long long)(t * (rope_dim >> 3) + ch) * 128 + n * 8 + e;
}

}  // namespace mla
