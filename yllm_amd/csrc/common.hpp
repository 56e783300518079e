// common.hpp -- shared device helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yhip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kF16 = 0, kF32 = 1, kBF16 = 2;
// RoPE kinds (the public YHIP_ROPE_* values)
constexpr uint32_t kRopeNone = 0, kRopePairs = 1, kRopeHalf = 2, kRopeMrope = 3;

// KV cache geometry (per sequence, per layer):
//   K: [n_kv][kv_stride][D]                  row = position
//   V: [n_kv][kv_stride/32][D][32]           32-position tiles, each stored
//                                            transposed (d-major)
// A block of 32 consecutive positions is then one contiguous run of 32*D
// halfs in K and one in V, and a V tile is directly the A operand layout of
// the P.V MFMA (a lane reads 8 consecutive positions of one dimension).
constexpr uint32_t kVTile = 32;

__host__ __device__ inline size_t k_index(uint32_t kvh, uint32_t pos, uint32_t d, uint32_t D,
                                          uint32_t kv_stride)
{
    return ((size_t)kvh * kv_stride + pos) * D + d;
}

__host__ __device__ inline size_t v_index(uint32_t kvh, uint32_t pos, uint32_t d, uint32_t D,
                                          uint32_t kv_stride)
{
    return (((size_t)kvh * (kv_stride / kVTile) + pos / kVTile) * D + d) * kVTile + (pos % kVTile);
}

// float -> f16 bits with the reference CPU rounding (platform.c:340-379):
// the magnitude gets half an f16 ulp added and is truncated, so ties go away
// from zero; f32 subnormals become signed zero; overflow becomes inf; NaN
// keeps a quiet payload of 0x200.  Integer-only, identical on host and device.
__host__ __device__ inline uint16_t f32_to_f16_ref(float f)
{
    uint32_t bits = __builtin_bit_cast(uint32_t, f);
    uint32_t s = (bits >> 16) & 0x8000u;
    uint32_t be = (bits >> 23) & 0xffu;
    uint32_t frac = bits & 0x7fffffu;
    if (be == 0u) return (uint16_t)s;
    if (be == 0xffu) return (uint16_t)(s | 0x7c00u | (frac ? 0x0200u : 0u));
    int he = (int)be - 112;
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)s;
        uint32_t m = frac | 0x800000u;
        uint32_t sh = (uint32_t)(14 - he);
        return (uint16_t)(s | ((m + (1u << (sh - 1))) >> sh));
    }
    uint32_t r = frac + 0x1000u;
    if (r & 0x800000u) {
        he += 1;
        if (he >= 31) return (uint16_t)(s | 0x7c00u);
        return (uint16_t)(s | ((uint32_t)he << 10));
    }
    return (uint16_t)(s | ((uint32_t)he << 10) | (r >> 13));
}

__host__ __device__ inline float bf16_bits_to_f32(uint16_t b)
{
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__host__ __device__ inline float f16_bits_to_f32(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}

// one element of a q/k/v source of element type dt, widened to float exactly
__device__ inline float load_as_f32(const void* p, size_t i, uint32_t dt)
{
    if (dt == kF32) return reinterpret_cast<const float*>(p)[i];
    uint16_t b = reinterpret_cast<const uint16_t*>(p)[i];
    return dt == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Workgroup barrier for LDS traffic only: it waits for this thread's LDS
// accesses (lgkmcnt(0)) and nothing else.  __syncthreads(), and a fence on
// LDS alone, also wait for every outstanding global or buffer load of the
// thread (vmcnt(0)), which stalls on loads issued ahead for later use;
// loads whose data another thread reads through LDS must be waited for
// explicitly before the barrier that publishes them.  The empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ inline void lds_barrier()
{
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt at their maxima (no wait)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x op x from lane ^ 16 (rows 0 <-> 1, 2 <-> 3) and lane ^ 32 (halves), by
// gfx950's permlane swaps in the VALU rather than ds_bpermute through the LDS
// unit; with a commutative op every lane gets the value the lane ^ mask
// exchange gives.
__device__ inline float max_xor16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ inline float max_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ inline float sum_xor16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ inline float sum_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

template <int CTRL>
__device__ inline float dpp_mov(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// The sum over each aligned group of N lanes (N = 16, 32, 64) in the order
// of the __shfl_xor butterfly with masks N/2, ..., 2, 1, bit for bit its
// result, by VALU lane exchanges instead of ds_bpermute round trips through
// the LDS unit: permlane swaps for 32 and 16, a row rotation by 8 for xor 8,
// a row rotation by 4 for xor 4 (after the xor-8 step lanes l and l ^ 8 hold
// the same value, so lane (l + 4) mod 16 holds lane l ^ 4's), quad
// permutations for 2 and 1.  (x + p and p + x are the same float.)
template <int N>
__device__ inline float xor_sum(float x)
{
    static_assert(N == 16 || N == 32 || N == 64, "groups of 16, 32 or 64 lanes");
    if constexpr (N == 64) x = sum_xor32(x);
    if constexpr (N >= 32) x = sum_xor16(x);
    x += dpp_mov<0x128>(x);  // row_ror:8
    x += dpp_mov<0x124>(x);  // row_ror:4
    x += dpp_mov<0x4e>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp_mov<0xb1>(x);   // quad_perm [1, 0, 3, 2]
    return x;
}

}  // namespace yhip
