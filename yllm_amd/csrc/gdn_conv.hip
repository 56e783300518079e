// gdn_conv.hip -- the Gated DeltaNet layer's neighbours of the recurrence on
// gfx950: the causal conv1d + silu ahead of it and the gated RMSNorm after it.
//
// conv1d (matvec.c:956-968, called per token at engine.c:805-812).  The
// engine keeps a delay line state[kwidth][dim]; per token it drops row 0,
// appends the input as row kwidth-1 and replaces the input by
// sum_i state[i][ch] * w[ch*kwidth + i] (i in order), then applies silu.
// Unrolled over T tokens that is a causal FIR filter per channel,
//     out[t][ch] = sum_i w[ch][i] * X(t - kwidth + 1 + i),
// X(tau) = x[tau] for tau >= 0 and the old delay-line row tau + kwidth
// before the first token; afterwards row r holds X(T - kwidth + r).  Every
// output depends on kwidth known inputs only, so the tokens run in parallel
// (no recurrence): a thread owns a run of kRun tokens of one channel and
// slides its window through registers.  Products and sums are separate
// roundings in the reference's order (its ISO C build does not contract
// them; here contraction is switched off in the kernel), so the conv values
// are bit for bit the reference's; silu uses the
// device expf.  The new delay line goes to state_out.  In place
// (state_out == state) with T > kRun it is written by a second launch, after
// every read of the old one; for T <= kRun (a decode step) each thread owns
// all of its channel's tokens and writes the channel's new rows itself, and
// out of place the thread of a channel's last run does.
//
// rmsnorm_gated (matvec.c:1007-1021, engine.c:845-847 per v-head):
//     y = x * w * (1 / sqrtf(sum(x^2) / n + eps)) * (z / (1 + expf(-z)))
// one wave per (token, head); the sum of squares is a wave reduction (the
// reference sums in order, so results agree to rounding, not bit for bit).
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace yhip {
namespace {

constexpr int kRun = 8;  // tokens per thread in the conv

template <int KW, bool OWN_STATE>
__global__ __launch_bounds__(256) void gdn_conv_kernel(GdnConvArgs a)
{
    // separate product and sum roundings, as the reference (contraction
    // would fuse them into one fma)
#pragma clang fp contract(off)
    const uint32_t ch = blockIdx.x * 256 + threadIdx.x;
    const uint32_t t0 = blockIdx.y * kRun;
    if (ch >= a.dim) return;
    float w[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) w[i] = a.w[(size_t)ch * KW + i];
    // window X(t0 - KW + 1 .. t0 + kRun - 1)
    float xw[KW - 1 + kRun];
#pragma unroll
    for (int j = 0; j < KW - 1 + kRun; ++j) {
        const int64_t tau = (int64_t)t0 - (KW - 1) + j;
        if (tau < 0)
            xw[j] = a.state[(size_t)(tau + KW) * a.dim + ch];
        else if (tau < (int64_t)a.T)
            xw[j] = a.x[(size_t)tau * a.x_stride + ch];
        else
            xw[j] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < kRun; ++r) {
        const uint32_t t = t0 + r;
        if (t >= a.T) break;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < KW; ++i) acc = acc + xw[r + i] * w[i];
        a.out[(size_t)t * a.out_stride + ch] = a.silu ? acc / (1.0f + expf(-acc)) : acc;
    }
    // The new delay line, row r = X(T - KW + r) = xw[T - 1 - t0 + r].  With
    // T <= kRun (OWN_STATE) this thread read every input of its channel; out
    // of place, the thread of the channel's last run holds every input the
    // new rows need (they start at X(T - KW) >= X(t0 - KW + 1)) and no other
    // thread reads state_out.  In place with several runs, the second
    // launch writes it after every read of the old line.
    if (OWN_STATE || (a.state_out != a.state && t0 + kRun >= a.T)) {
#pragma unroll
        for (int j = 0; j < KW - 1 + kRun; ++j) {
            const int r = j - ((int)a.T - 1 - (int)t0);
            if (r >= 0 && r < KW) a.state_out[(size_t)r * a.dim + ch] = xw[j];
        }
    }
}

// new delay line of an in-place call: row r = X(T - kwidth + r).  One thread
// per channel reads the channel's old rows before it writes any.
template <int KW>
__global__ __launch_bounds__(256) void gdn_conv_state_kernel(GdnConvArgs a)
{
    const uint32_t ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= a.dim) return;
    float nw[KW];
#pragma unroll
    for (int r = 0; r < KW; ++r) {
        const int64_t tau = (int64_t)a.T - KW + r;
        nw[r] = tau >= 0 ? a.x[(size_t)tau * a.x_stride + ch] : a.state[(size_t)(tau + KW) * a.dim + ch];
    }
#pragma unroll
    for (int r = 0; r < KW; ++r) a.state_out[(size_t)r * a.dim + ch] = nw[r];
}

// One wave per (token, head); PER = head_dim / 64 elements per lane.  x, z
// and the weight are loaded together, before the sum (loaded after it, z and
// the weight were a second memory round trip per wave).
template <int W_F16, int PER>
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(GdnNormArgs a)
{
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);  // (token, head) pair
    const int lane = threadIdx.x & 63;
    if (row >= a.T * a.n_heads) return;  // wave-uniform
    const uint32_t t = row / a.n_heads, h = row % a.n_heads;
    const float* x = a.x + (size_t)t * a.x_stride + (size_t)h * a.head_dim;
    const float* z = a.z + (size_t)t * a.z_stride + (size_t)h * a.head_dim;
    float* y = a.y + (size_t)t * a.y_stride + (size_t)h * a.head_dim;
    float xv[PER], zv[PER], wv[PER], ss = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t i = k * 64 + lane;
        xv[k] = x[i];
        zv[k] = z[i];
        wv[k] = W_F16 ? (float)reinterpret_cast<const _Float16*>(a.w)[i] : reinterpret_cast<const float*>(a.w)[i];
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) ss += xv[k] * xv[k];
    ss = xor_sum<64>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)a.head_dim + a.eps);
#pragma unroll
    for (int k = 0; k < PER; ++k) y[k * 64 + lane] = xv[k] * wv[k] * inv * (zv[k] / (1.0f + expf(-zv[k])));
}

template <int KW>
hipError_t launch_conv_kw(const GdnConvArgs& a, hipStream_t st)
{
    const dim3 grid((a.dim + 255) / 256, (a.T + kRun - 1) / kRun);
    if (a.T <= (uint32_t)kRun) {  // one run per channel (a decode step): one launch
        hipLaunchKernelGGL((gdn_conv_kernel<KW, true>), grid, dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((gdn_conv_kernel<KW, false>), grid, dim3(256), 0, st, a);
        if (a.state_out == a.state)  // in place: the new line after every read of the old one
            hipLaunchKernelGGL(gdn_conv_state_kernel<KW>, dim3((a.dim + 255) / 256), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gdn_conv(const GdnConvArgs& a, hipStream_t st)
{
    hipError_t e;
    switch (a.kwidth) {
    case 1: e = launch_conv_kw<1>(a, st); break;
    case 2: e = launch_conv_kw<2>(a, st); break;
    case 3: e = launch_conv_kw<3>(a, st); break;
    case 4: e = launch_conv_kw<4>(a, st); break;
    case 5: e = launch_conv_kw<5>(a, st); break;
    case 6: e = launch_conv_kw<6>(a, st); break;
    case 7: e = launch_conv_kw<7>(a, st); break;
    case 8: e = launch_conv_kw<8>(a, st); break;
    default: return hipErrorInvalidValue;
    }
    return e;
}

template <int PER>
void launch_norm_per(const GdnNormArgs& a, hipStream_t st)
{
    const dim3 grid((a.T * a.n_heads + 3) / 4);
    if (a.w_f16)
        hipLaunchKernelGGL((gdn_gated_norm_kernel<1, PER>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((gdn_gated_norm_kernel<0, PER>), grid, dim3(256), 0, st, a);
}

hipError_t launch_gdn_gated_norm(const GdnNormArgs& a, hipStream_t st)
{
    switch (a.head_dim) {
    case 64: launch_norm_per<1>(a, st); break;
    case 128: launch_norm_per<2>(a, st); break;
    case 192: launch_norm_per<3>(a, st); break;
    case 256: launch_norm_per<4>(a, st); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace yhip
