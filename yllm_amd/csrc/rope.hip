// rope.hip -- rotary position embedding of q and k fused with the K and V
// stores into the head-major HBM cache: the step before attention
// (engine.c:1054-1072 llama / qwen, engine.c:910-934 qwen35).
//
// Kinds (matvec.c:890-939), per head of head_dim d, position pos, pair j:
//   PAIRS  (rope_inplace, llama):        (v[2j], v[2j+1]),        j < d/2
//   HALF   (rope_inplace_qwen, qwen):    (v[j], v[j+d/2]),        j < d/2
//   MROPE  (rope_inplace_mrope, qwen35): (v[j], v[j+n_rot/2]),    j < n_rot/2,
//          dims n_rot..d-1 unchanged
// with freq = powf(theta, -2j/dn) (dn = d, or n_rot for MROPE),
// ang = freq * pos, (a, b) -> (a cos - b sin, a sin + b cos), in float like
// the reference.  The frequencies come in the launch arguments, computed by
// the host C library's powf as in the reference: a 1-ulp frequency error
// would grow to about pos * 6e-8 rad at position pos (8e-3 rad at 131071).
// The angle is then bit for bit the reference's; the device cosf / sinf
// differ from the host library by an ulp or two.
//
// One launch, two kinds of workgroup:
//  * rotation blocks: a wave per token (for few tokens, a few waves per
//    token, each with a range of its heads).  Its lanes own the token's
//    pairs (two heads per pass at d = 64, two pairs per lane at d = 256);
//    each lane computes its angles' sine and cosine once and applies them to
//    the pair in every head of its range, loading four passes ahead of
//    their stores.  Loads and stores are 8 / 4 bytes per lane where the
//    pair is two adjacent elements.  q goes to
//    q_out (f32 / f16 / bf16); k is rounded with the reference f32->f16
//    rounding (platform.c:340-379) into the token's K row of each kv head.
//    For a few tokens (decode) the same wave also writes the token's V
//    elements into the tiles.
//  * V tile blocks (more than kScatterRows tokens): 64 tokens x 64 channels
//    staged in LDS, read along source rows and written along tile rows,
//    rounded the same way.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace yhip {
namespace {

constexpr uint32_t kScatterRows = 16;  // up to this many tokens the rotation waves write V too

__device__ inline uint16_t bf16_bits(float x)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ inline uint16_t half_bits(float x, uint32_t dt)
{
    return dt == kF16 ? __builtin_bit_cast(uint16_t, (_Float16)x) : bf16_bits(x);
}

// two elements e0, e1 of q_out row `o`
__device__ inline void store_q_pair(void* out, size_t o, uint32_t e0, uint32_t e1, uint32_t dt, float x0, float x1)
{
    if (dt == kF32) {
        float* p = reinterpret_cast<float*>(out) + o;
        if (e1 == e0 + 1) {
            *reinterpret_cast<float2*>(p + e0) = make_float2(x0, x1);
        } else {
            p[e0] = x0;
            p[e1] = x1;
        }
    } else {
        uint16_t* p = reinterpret_cast<uint16_t*>(out) + o;
        const uint16_t h0 = half_bits(x0, dt), h1 = half_bits(x1, dt);
        if (e1 == e0 + 1) {
            *reinterpret_cast<uint32_t*>(p + e0) = (uint32_t)h0 | ((uint32_t)h1 << 16);
        } else {
            p[e0] = h0;
            p[e1] = h1;
        }
    }
}

template <int D>
__device__ void v_tile_block(const RopeArgs& a, uint32_t vb)
{
    __shared__ uint16_t tile[64][66];
    const uint32_t kv_dim = a.n_kv * D;
    const uint32_t ntx = (kv_dim + 63u) / 64u;
    const uint32_t j0 = (vb % ntx) * 64u, b0 = (vb / ntx) * 64u;
    const uint32_t tx = threadIdx.x & 63u, ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64u; r += 4u) {
        const uint32_t b = b0 + r, j = j0 + tx;
        if (b < a.B && j < kv_dim) tile[r][tx] = f32_to_f16_ref(__builtin_nontemporal_load(a.v + (size_t)b * a.v_stride + j));
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64u; r += 4u) {
        const uint32_t j = j0 + r, b = b0 + tx;
        if (b < a.B && j < kv_dim) {
            const uint32_t h = j / D, d = j - h * D;
            a.vc[v_index(h, a.pos_start + b, d, D, a.kv_stride)] = tile[tx][r];
        }
    }
}

template <uint32_t KIND, int D>
__global__ __launch_bounds__(256) void rope_kv_kernel(RopeArgs a)
{
    // products and differences rounded separately, as the reference
#pragma clang fp contract(off)
    // the two roles alternate over the first 2 * min(rotation, tile) workgroups,
    // so the V tiles stream alongside the rotation instead of after it
    uint32_t blk = blockIdx.x;
    {
        const uint32_t m = min(a.rope_blocks, a.v_blocks);
        bool tile_role;
        if (blk < 2 * m) {
            tile_role = blk & 1u;
            blk >>= 1;
        } else {
            tile_role = a.v_blocks > a.rope_blocks;
            blk -= m;
        }
        if (tile_role) {  // workgroup-uniform
            v_tile_block<D>(a, blk);
            return;
        }
    }
    constexpr uint32_t P = D / 2;                  // pairs per head
    constexpr uint32_t HPI = P >= 64 ? 1 : 64 / P;  // heads per pass
    constexpr uint32_t PPL = P >= 64 ? P / 64 : 1;  // pairs per lane
    constexpr uint32_t U = 4;                      // passes whose loads are issued together
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = blk * 4u + (threadIdx.x >> 6);
    const uint32_t b = w / a.groups, g = w % a.groups;
    if (b >= a.B) return;  // wave-uniform; no barrier follows in this role
    const uint32_t pos = a.pos_start + b;
    const uint32_t sub = HPI > 1 ? lane / P : 0;

    uint32_t e0[PPL], e1[PPL];
    float c[PPL], s[PPL];
    bool rot[PPL];
#pragma unroll
    for (uint32_t r = 0; r < PPL; ++r) {
        const uint32_t p = HPI > 1 ? lane % P : lane + 64u * r;
        const uint32_t nr2 = a.n_rot / 2;
        if (KIND == kRopeHalf) {
            e0[r] = p;
            e1[r] = p + P;
            rot[r] = true;
        } else if (KIND == kRopeMrope && p < nr2) {
            e0[r] = p;
            e1[r] = p + nr2;
            rot[r] = true;
        } else {  // PAIRS, and the unrotated dims of MROPE / NONE
            e0[r] = 2 * p;
            e1[r] = 2 * p + 1;
            rot[r] = KIND == kRopePairs;
        }
        c[r] = 1.0f;
        s[r] = 0.0f;
        if (rot[r]) sincosf(a.freq[p] * (float)pos, &s[r], &c[r]);
    }

    // this wave's heads: [h_lo, h_hi) of q heads then kv heads (kv heads only without q_out)
    const uint32_t heads = a.n_heads + a.n_kv;
    const uint32_t h_first = a.q_out ? 0u : a.n_heads;
    const uint32_t h_lo = h_first + g * a.heads_per_wave;
    const uint32_t h_hi = min(heads, h_lo + a.heads_per_wave);
    for (uint32_t h0 = h_lo; h0 < h_hi; h0 += HPI * U) {
        // loads of U passes first, then their stores (q_out may be q: every
        // lane reads its own elements before it writes them)
        float x0[U][PPL], x1[U][PPL];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t h = h0 + u * HPI + sub;
            if (h >= h_hi) break;
            const bool is_q = h < a.n_heads;
            const float* src = is_q ? a.q + (size_t)b * a.q_stride + (size_t)h * D
                                    : a.k + (size_t)b * a.k_stride + (size_t)(h - a.n_heads) * D;
#pragma unroll
            for (uint32_t r = 0; r < PPL; ++r) {
                if (e1[r] == e0[r] + 1) {
                    typedef float f32x2_ __attribute__((ext_vector_type(2)));
                    const f32x2_ v = __builtin_nontemporal_load(reinterpret_cast<const f32x2_*>(src + e0[r]));
                    x0[u][r] = v[0];
                    x1[u][r] = v[1];
                } else {
                    x0[u][r] = __builtin_nontemporal_load(src + e0[r]);
                    x1[u][r] = __builtin_nontemporal_load(src + e1[r]);
                }
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t h = h0 + u * HPI + sub;
            if (h >= h_hi) break;
            const bool is_q = h < a.n_heads;
#pragma unroll
            for (uint32_t r = 0; r < PPL; ++r) {
                float y0 = x0[u][r], y1 = x1[u][r];
                if (rot[r]) {
                    y0 = x0[u][r] * c[r] - x1[u][r] * s[r];
                    y1 = x0[u][r] * s[r] + x1[u][r] * c[r];
                }
                if (is_q) {
                    store_q_pair(a.q_out, (size_t)b * a.q_out_stride + (size_t)h * D, e0[r], e1[r], a.q_out_dtype,
                                 y0, y1);
                } else {
                    uint16_t* row = a.kc + k_index(h - a.n_heads, pos, 0, D, a.kv_stride);
                    const uint16_t k0 = f32_to_f16_ref(y0), k1 = f32_to_f16_ref(y1);
                    if (e1[r] == e0[r] + 1) {
                        *reinterpret_cast<uint32_t*>(row + e0[r]) = (uint32_t)k0 | ((uint32_t)k1 << 16);
                    } else {
                        row[e0[r]] = k0;
                        row[e1[r]] = k1;
                    }
                }
            }
        }
    }
    if (a.B <= kScatterRows) {
        // few tokens: the token's waves write its V elements (2-byte scatters into the tiles)
        const uint32_t kv_dim = a.n_kv * D;
        for (uint32_t j = g * 64u + lane; j < kv_dim; j += 64u * a.groups) {
            const uint32_t h = j / D, d = j - h * D;
            a.vc[v_index(h, pos, d, D, a.kv_stride)] = f32_to_f16_ref(a.v[(size_t)b * a.v_stride + j]);
        }
    }
}

template <uint32_t KIND>
hipError_t launch_kind(const RopeArgs& a, dim3 grid, hipStream_t st)
{
    switch (a.D) {
    case 64: hipLaunchKernelGGL((rope_kv_kernel<KIND, 64>), grid, dim3(256), 0, st, a); break;
    case 128: hipLaunchKernelGGL((rope_kv_kernel<KIND, 128>), grid, dim3(256), 0, st, a); break;
    case 256: hipLaunchKernelGGL((rope_kv_kernel<KIND, 256>), grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rope_kv(RopeArgs a, hipStream_t st)
{
    // waves per token: one (all heads share the token's sines and cosines)
    // unless there are too few tokens to give the chip about 1024 waves;
    // then the heads are split over up to one wave per pass
    const uint32_t hpi = a.D >= 128 ? 1u : 64u / (a.D / 2);
    const uint32_t active = a.q_out ? a.n_heads + a.n_kv : a.n_kv;
    const uint32_t passes = (active + hpi - 1) / hpi;
    uint32_t groups = a.B >= 1024u ? 1u : (1024u + a.B - 1) / a.B;
    groups = groups < passes ? groups : passes;
    const uint32_t per = (passes + groups - 1) / groups;  // passes per wave
    a.heads_per_wave = per * hpi;
    a.groups = (passes + per - 1) / per;
    a.rope_blocks = (uint32_t)(((uint64_t)a.B * a.groups + 3u) / 4u);
    a.v_blocks = a.B > kScatterRows ? ((a.n_kv * a.D + 63u) / 64u) * ((a.B + 63u) / 64u) : 0u;
    const dim3 grid(a.rope_blocks + a.v_blocks);
    switch (a.kind) {
    case kRopeNone: return launch_kind<kRopeNone>(a, grid, st);
    case kRopePairs: return launch_kind<kRopePairs>(a, grid, st);
    case kRopeHalf: return launch_kind<kRopeHalf>(a, grid, st);
    case kRopeMrope: return launch_kind<kRopeMrope>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace yhip
