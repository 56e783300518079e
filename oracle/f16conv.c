/* f16conv.c -- half/bfloat conversions of the CPU oracle (TEST INFRASTRUCTURE).
 *
 * Kept in a translation unit of its own so that, as in the reference
 * (inference/core/platform.c:316 is out of line in platform.c), every f16
 * decode inside the attention loops is a real call and the loops stay scalar.
 */
#include "yref.h"
#include <string.h>

/* platform.c:316-338 */
float yo_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t he = (h >> 10) & 0x1fu;
    uint32_t frac = h & 0x3ffu;
    uint32_t bits;
    if (he == 0x1fu) {
        /* inf, or a quiet NaN carrying the reference's fixed payload */
        bits = sign | 0x7f800000u | (frac ? 0x7fc000u : 0u);
    } else if (he != 0u) {
        bits = sign | ((he + 112u) << 23) | (frac << 13);
    } else if (frac == 0u) {
        bits = sign;
    } else {
        /* subnormal half: shift the leading one up to bit 10 */
        int lead = 0;
        while (!(frac & 0x400u)) { frac <<= 1; lead++; }
        bits = sign | ((uint32_t)(113 - lead) << 23) | ((frac & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* platform.c:340-379 */
uint16_t yo_f32_to_f16(float f)
{
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint16_t s = (uint16_t)((bits >> 16) & 0x8000u);
    uint32_t be = (bits >> 23) & 0xffu;
    uint32_t frac = bits & 0x7fffffu;
    if (be == 0u) return s;                                       /* zero, f32 subnormal */
    if (be == 0xffu) return (uint16_t)(s | 0x7c00u | (frac ? 0x0200u : 0u));
    int he = (int)be - 112;                                       /* rebias 127 -> 15 */
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return s;
        uint32_t m = frac | 0x800000u;
        uint32_t sh = (uint32_t)(14 - he);
        return (uint16_t)(s | ((m + (1u << (sh - 1))) >> sh));
    }
    /* add half an f16 ulp and truncate: ties round away from zero */
    uint32_t r = frac + 0x1000u;
    if (r & 0x800000u) {
        he += 1;
        if (he >= 31) return (uint16_t)(s | 0x7c00u);
        return (uint16_t)(s | ((uint32_t)he << 10));
    }
    return (uint16_t)(s | ((uint32_t)he << 10) | (r >> 13));
}

/* platform.c:381-391 */
uint16_t yo_bf16_to_f16(uint16_t b)
{
    uint16_t s = b & 0x8000u;
    int be = (b >> 7) & 0xff;
    uint16_t frac = b & 0x7fu;
    if (be == 0xff) return (uint16_t)(s | (frac ? 0x7e00u : 0x7c00u));
    int he = be - 112;
    if (he <= 0) return s;
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    return (uint16_t)(s | ((uint16_t)he << 10) | (uint16_t)(frac << 3));
}

float yo_bf16_to_f32(uint16_t b)
{
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void yo_f32_to_f16_buf(const float* src, uint16_t* dst, size_t n)
{
    size_t i;
    for (i = 0; i < n; i++) dst[i] = yo_f32_to_f16(src[i]);
}
