// synth.cpp -- seeded synthetic inputs and host conversions (host code).
//
// Generator: splitmix64 with the constants of the reference's yrng
// (platform.c:411-417).  Draw i of a stream (0-based) uses the state
// seed + (i+1)*0x9e3779b97f4a7c15, i.e. the value yrng returns on its
// (i+1)-th call after ysrand(seed) (platform.c:405-409: seed 0 -> golden
// constant), so any range of a stream can be produced independently.
#include "../../include/yllm_hip.h"
#include "common.hpp"

#include <math.h>

namespace {

constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ull;

inline uint64_t mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// uniform in (0, 1): 24 random bits, offset by half a step so log() is finite
inline double uniform_of(uint64_t r) { return ((double)(r >> 40) + 0.5) * (1.0 / 16777216.0); }

}  // namespace

extern "C" {

void yhip_synth_normal(uint64_t seed, uint64_t first, float sigma, float* out, uint64_t n)
{
    if (seed == 0) seed = kGolden;
    const double two_pi = 6.283185307179586476925286766559;
    // value k uses draws 2*(k/2) and 2*(k/2)+1 of the stream (one Box-Muller pair)
    for (uint64_t k = 0; k < n; ++k) {
        const uint64_t idx = first + k;
        const uint64_t pair = idx >> 1;
        const uint64_t d0 = 2 * pair, d1 = 2 * pair + 1;
        const double u1 = uniform_of(mix(seed + (d0 + 1) * kGolden));
        const double u2 = uniform_of(mix(seed + (d1 + 1) * kGolden));
        const double rad = sqrt(-2.0 * log(u1));
        const double z = (idx & 1) ? rad * sin(two_pi * u2) : rad * cos(two_pi * u2);
        out[k] = (float)(sigma * z);
    }
}

void yhip_synth_round_f16(float* x, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) x[i] = (float)__builtin_bit_cast(_Float16, yhip::f32_to_f16_ref(x[i]));
}

void yhip_synth_round_bf16(float* x, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t b = __builtin_bit_cast(uint32_t, x[i]);
        b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
        x[i] = __builtin_bit_cast(float, b);
    }
}

void yhip_host_f32_to_f16(const float* src, uint16_t* dst, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) dst[i] = yhip::f32_to_f16_ref(src[i]);
}

void yhip_host_f16_to_f32(const uint16_t* src, float* dst, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) dst[i] = (float)__builtin_bit_cast(_Float16, src[i]);
}

void yhip_host_f32_to_bf16(const float* src, uint16_t* dst, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t b = __builtin_bit_cast(uint32_t, src[i]);
        dst[i] = (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
    }
}

}  // extern "C"
