// gdn_decode.hip -- one decode token of a Gated DeltaNet layer
// (engine.c:786-847 for a single token): the gates (788-793), conv1d +
// silu over the projected qkv row (805-812, conv1d_update matvec.c:956-968),
// l2norm of q and k per k head (826-827, matvec.c:942-949), the state update
// and output (gdn_state_update, matvec.c:975-1004) and the gated RMSNorm of
// each v head (845-847, rmsnorm_gated matvec.c:1007-1021).
//
// The default is one launch, gdn_decode_head_kernel (below): a 1024-thread
// workgroup per v head with the gated RMSNorm fused.  The two-launch form
// (YHIP_GDN_DECODE2=1): gdn_decode_kernel, a workgroup (256 threads) owns 16 state
// columns of v head h (D/16 workgroups per head, as gdn_step_kernel), which
// reads k head kh = h % n_k:
//  1. every thread issues its loads at once: its slice of the state, one q
//     and one k channel of head kh (conv weights and delay line), and for 16
//     threads one of the workgroup's v channels;
//  2. conv + silu of those channels (products and sums rounded separately
//     in the reference's order, so the conv is bit for bit the
//     reference's), the gates, the l2norm of q and k through LDS (every
//     workgroup of the head computes the whole q and k head, 2 D channels);
//  3. the state update of its 16 columns by 16 threads each (decay, delta
//     rule, output) and the raw outputs into y.
// Then the gated RMSNorm kernel (gdn_conv.hip) normalises each head of y in
// place: its sum over the head's D outputs spans the head's workgroups.
// The delay line is read from conv_in and written to conv_out (separate
// buffers, swapped by the caller every token), so no workgroup can read a
// row that another one has already replaced.  q/k channels of head kh are
// written by the workgroups of v head kh (n_v >= n_k, so it exists), 16 per
// workgroup; v channels by the workgroup that owns them.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>

namespace yhip {
namespace {

constexpr int kThreads = 256;
constexpr int kCols = 16;  // state columns per workgroup
constexpr int kMaxKw = 8;

// Cross-lane sums in the VALU (DPP row permutations and gfx950's permlane
// swaps) instead of ds_bpermute round trips through the LDS unit: every lane
// of the group ends with the same total, added in the same order.
template <int CTRL>
__device__ inline float dpp_f(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
// over each 8-lane group: xor 1, xor 2 (quad permutations), then the other
// quad of the group (half-row mirror)
__device__ inline float sum8(float x)
{
    x += dpp_f<0xb1>(x);   // quad_perm [1, 0, 3, 2]
    x += dpp_f<0x4e>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp_f<0x141>(x);  // row_half_mirror
    return x;
}
__device__ inline float sum16(float x)
{
    x = sum8(x);
    return x + dpp_f<0x140>(x);  // row_mirror: the other half of the row
}
__device__ inline float sum64(float x)
{
    x = sum16(x);
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);  // rows 0 + 1, 2 + 3
    x = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    const auto hv = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                     false, false);  // halves
    return __builtin_bit_cast(float, (uint32_t)hv[0]) + __builtin_bit_cast(float, (uint32_t)hv[1]);
}

template <int D>
__global__ __launch_bounds__(kThreads) void gdn_decode_kernel(GdnDecodeArgs a)
{
    // separate product and sum roundings in the conv, as the reference
#pragma clang fp contract(off)
    constexpr int TPC = kThreads / kCols;  // threads per state column (16)
    constexpr int SL = D / TPC;            // state elements per thread
    constexpr uint32_t nblk = D / kCols;   // workgroups per head
    __shared__ float qs[D], ks[D], vs[kCols];
    __shared__ float red[2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = blockIdx.x / nblk, blk = blockIdx.x % nblk;
    const uint32_t kh = h % a.n_k;
    const uint32_t key_dim = a.n_k * D;
    const uint32_t col = tid / TPC, part = tid % TPC, j = blk * kCols + col;

    // 1. loads: state slice, then this thread's conv channels
    const float* Sp = a.S + ((size_t)h * D + j) * D + part * SL;
    float* So = a.S_out + ((size_t)h * D + j) * D + part * SL;
    float s[SL];
#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(Sp + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[i + e] = x[e];
    }
    // channel c of the 2 D q/k channels (q: c < D, k: c >= D) and, for
    // tid < kCols, v channel j0 + tid
    struct Chan {
        float X[kMaxKw], w[kMaxKw];
        uint32_t ch;
    };
    auto load = [&](Chan& c, uint32_t ch) {
        c.ch = ch;
#pragma unroll
        for (int r = 0; r < kMaxKw; ++r) {
            if (r >= (int)a.kwidth) break;
            c.w[r] = a.conv_w[(size_t)ch * a.kwidth + r];
            c.X[r] = r + 1 < (int)a.kwidth ? a.conv_in[(size_t)(r + 1) * a.conv_dim + ch] : a.qkv[ch];
        }
    };
    auto conv = [&](const Chan& c) {
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < kMaxKw; ++r) {
            if (r >= (int)a.kwidth) break;
            acc = acc + c.X[r] * c.w[r];
        }
        return acc / (1.0f + expf(-acc));
    };
    auto store_line = [&](const Chan& c) {
#pragma unroll
        for (int r = 0; r < kMaxKw; ++r) {
            if (r >= (int)a.kwidth) break;
            a.conv_out[(size_t)r * a.conv_dim + c.ch] = c.X[r];
        }
    };
    constexpr int QK_PER = 2 * D / kThreads;  // q/k channels per thread (1 at D = 128)
    Chan cq[QK_PER > 0 ? QK_PER : 1];
    const bool qk_thread = QK_PER > 0 || tid < 2 * D;
#pragma unroll
    for (int u = 0; u < (QK_PER > 0 ? QK_PER : 1); ++u) {
        const uint32_t c = tid + u * kThreads;  // 0 .. 2D-1
        if (qk_thread) load(cq[u], c < (uint32_t)D ? kh * D + c : key_dim + kh * D + (c - D));
    }
    Chan cv;
    const bool v_thread = tid < kCols;
    if (v_thread) load(cv, 2 * key_dim + h * D + blk * kCols + tid);
    // gates (engine.c:788-793), read with the other loads: after a barrier
    // their loads would add a memory round trip to the token's chain
    const float bt = 1.0f / (1.0f + expf(-a.beta_raw[h]));
    const float g = expf(log1pf(expf(a.alpha[h] + a.dt_bias[h])) * a.ssm_a[h]);

    // 2. conv + silu; the new delay line row r is X[r]
#pragma unroll
    for (int u = 0; u < (QK_PER > 0 ? QK_PER : 1); ++u) {
        if (!qk_thread) break;
        const uint32_t c = tid + u * kThreads;
        const float y = conv(cq[u]);
        if (c < (uint32_t)D) qs[c] = y;
        else ks[c - D] = y;
        // head kh's q/k channels: 16 of them per workgroup of v head kh
        if (h == kh && (c % D) / kCols == blk) store_line(cq[u]);
    }
    if (v_thread) {
        vs[tid] = conv(cv);
        store_line(cv);
    }
    lds_barrier();
    // l2 norms: wave 0 sums q^2, wave 1 sums k^2 (the reference sums in order;
    // this is a tree, equal to rounding)
    if (wave < 2) {
        const float* src = wave == 0 ? qs : ks;
        float ss = 0.0f;
        for (int i = lane; i < D; i += 64) ss += src[i] * src[i];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        if (lane == 0) red[wave] = 1.0f / fmaxf(sqrtf(ss), a.l2_eps);
    }
    lds_barrier();
    const float rq = red[0], rk = red[1];

    // 3. state update of column j (matvec.c:975-1004, as gdn_step_kernel)
    float k[SL], q[SL];
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        k[i] = ks[part * SL + i] * rk;
        q[i] = qs[part * SL + i] * rq;
    }
    auto sum_tpc = [](float x) {
#pragma unroll
        for (int m = TPC / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
        return x;
    };
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        s[i] *= g;
        p = fmaf(s[i], k[i], p);
    }
    const float delta = (vs[col] - sum_tpc(p)) * bt;
    float p2 = 0.0f;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        s[i] = fmaf(k[i], delta, s[i]);
        p2 = fmaf(s[i], q[i], p2);
    }
    const float o = sum_tpc(p2) * (1.0f / sqrtf((float)D));
#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        f32x4 x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = s[i + e];
        *reinterpret_cast<f32x4*>(So + i) = x;
    }
    if (part == 0) a.y[(size_t)h * D + j] = o;
}

// One launch for the whole token: a workgroup of 1024 threads computes a
// whole v head (TPC = 1024 / D threads per state column, SL = D / TPC
// elements each), so the gated RMSNorm's sum over the head's D outputs stays
// in the workgroup.  Every thread issues its loads at once (one conv channel:
// threads 0..2D-1 the q/k channels of k head kh, 2D..3D-1 the v channels of
// head h; z and the norm weight; its state slice last), one wave forms the
// gates while they are in flight, then conv + silu, l2 norms, the outputs,
// the new state and the normalised, gated outputs.  The barriers order LDS only: a
// __syncthreads before the norm's sum waited for the state stores to
// complete (~1.3 us of a ~5.4 us workgroup).
//
// NP workgroups per head: each computes the whole head -- the RMSNorm needs
// every column's output -- and stores only its D / NP columns of the new
// state, their outputs and their v channels of the delay line, so the
// head's 64 KiB of state stores (D = 128) spread over NP CUs while its loads
// are shared through the L2 of one XCD (workgroup b runs on XCD b mod 8, so
// b = h mod 8 + 8 (part + NP (h / 8)) puts a head's parts on one XCD).
// Measured at 16 heads, d 128, in graphs of 400 tokens: 6.6 us per token
// with NP = 1, 5.75 with NP = 8.  With NP > 1 a part reads columns other
// parts write, so the state must go out of place (S_out != S).
template <int D, int NP, int KWM>
__global__ __launch_bounds__(1024) void gdn_decode_head_kernel(GdnDecodeArgs a)
{
#pragma clang fp contract(off)
    constexpr int NT = 1024;
    constexpr int TPC = NT / D;   // threads per state column
    constexpr int SL = D / TPC;   // state elements per thread
    constexpr uint32_t CPP = D / NP;  // columns stored per part
    static_assert(3 * D <= NT, "one conv channel per thread");
    static_assert(D % NP == 0, "whole columns per part");
    static_assert(TPC == 8 || TPC == 16, "a state column's threads sum in one row");
    __shared__ float qs[D], ks[D], vs[D];
    __shared__ float l2p[3 * (2 * D / 64)];  // per q/k wave: its q.q, k.k and q.k
    __shared__ float ssq[NT / 64];
    __shared__ float s_gate[2];  // beta, g of the head
    constexpr int GW = 3 * D / 64;  // the first wave without a conv channel computes the gates
    static_assert(GW < NT / 64, "a wave without a conv channel");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t b = blockIdx.x, h = (b % 8u) + 8u * (b / (8u * NP)), pt = (b / 8u) % NP;
    if (h >= a.n_v) return;  // uniform over the workgroup
    const uint32_t kh = h % a.n_k;
    const uint32_t key_dim = a.n_k * D;
    const uint32_t j = tid / TPC, part = tid % TPC;
    const uint32_t own0 = pt * CPP;
    const bool own_col = j - own0 < CPP;  // this part stores column j

    // the head's gate inputs (engine.c:788-793) first: every load of the
    // token is issued before any wait, so its chain holds one memory round
    // trip
    const float beta_raw = a.beta_raw[h], alpha = a.alpha[h], dt_bias = a.dt_bias[h], ssm_a = a.ssm_a[h];
    // a thread's SL elements of row j: float4 r at 4 (r TPC + part), so one
    // 16-byte load instruction of a row's TPC threads covers 16 TPC whole,
    // consecutive bytes (as consecutive SL-element runs per thread, every
    // instruction took every other 16-byte chunk of its rows)
    const float* Sp = a.S + ((size_t)h * D + j) * D + part * 4;
    float* So = a.S_out + ((size_t)h * D + j) * D + part * 4;
    auto el = [&](int i) -> uint32_t { return (uint32_t)(i / 4) * 4u * TPC + part * 4u + (uint32_t)(i % 4); };
    // this thread's conv channel: q_i (tid = 2i < 2D) and k_i (tid = 2i + 1)
    // of head kh side by side, so one lane pair holds both for the q.k sum;
    // v (2D <= tid < 3D) of head h
    const bool has_ch = tid < 3 * D, qk_ch = tid < 2 * D, is_k = qk_ch && (tid & 1);
    const uint32_t ci = (uint32_t)tid >> 1;
    const uint32_t ch = !has_ch ? 0u
                        : qk_ch ? (is_k ? key_dim : 0u) + kh * D + ci
                                : 2 * key_dim + h * D + (tid - 2 * D);
    // KWM taps are loaded by every thread from valid addresses (taps past
    // kwidth repeat the last weight and the current row, and are not used): a
    // load under a condition, into a register that starts at zero, made the
    // compiler wait for every earlier load before the next one was issued
    const uint32_t kw = a.kwidth;
    float X[KWM], w[KWM];
#pragma unroll
    for (int r = 0; r < KWM; ++r) {
        w[r] = a.conv_w[(size_t)ch * kw + min((uint32_t)r, kw - 1u)];
        const float* src = (uint32_t)r + 1u < kw ? a.conv_in + (size_t)(r + 1) * a.conv_dim : a.qkv;
        X[r] = src[ch];
    }
    // z and the norm weight of column j, for every thread (part 0 uses them);
    // the weight as two 16-bit loads whose indices are in bounds for both
    // dtypes, joined where it is used
    const float zv = a.z[(size_t)h * D + j];
    const uint16_t* nw16 = reinterpret_cast<const uint16_t*>(a.norm_w);
    const uint16_t w_lo = nw16[a.norm_w_f16 ? j : 2 * j], w_hi = nw16[a.norm_w_f16 ? j : 2 * j + 1];
    // the state slice last: the conv channels, z and the weight are used first,
    // and with in-order completion a wait for them does not wait for the state
    float s[SL];
#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(Sp + i * TPC);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[i + e] = x[e];
    }
    // the gates once per workgroup, by a wave that has no conv channel (every
    // wave computing them cost ~0.3 us of VALU issue per SIMD), from scalar
    // loads, while the vector loads are in flight
    if (wave == GW) {
        const float bt_ = 1.0f / (1.0f + expf(-beta_raw));
        const float g_ = expf(log1pf(expf(alpha + dt_bias)) * ssm_a);
        if (lane == 0) {
            s_gate[0] = bt_;
            s_gate[1] = g_;
        }
    }
    float y = 0.0f;
    if (has_ch) {
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < KWM; ++r)
            if ((uint32_t)r < kw) acc = acc + X[r] * w[r];
        y = acc * __builtin_amdgcn_rcpf(1.0f + expf(-acc));
        if (!qk_ch) vs[tid - 2 * D] = y;
        else if (is_k) ks[ci] = y;
        else qs[ci] = y;
    }
    // the norm weight and z's silu, while their loads have just landed: used
    // only at the end, their waits there also waited for the state stores
    // (in-order memory counter), and the output store's latency added to
    // theirs.  Only the lanes that write y form them (no memory instruction
    // inside, so waves without such a lane skip it).
    const bool writes_y = part == 0 && own_col;
    float wv = 0.0f, zs = 0.0f;
    if (writes_y) {
        wv = a.norm_w_f16 ? (float)__builtin_bit_cast(_Float16, w_lo)
                          : __builtin_bit_cast(float, (uint32_t)w_lo | (uint32_t)w_hi << 16);
        zs = zv * __builtin_amdgcn_rcpf(1.0f + expf(-zv));
    }
    asm volatile("" : "+v"(wv), "+v"(zs));
    // l2 norms and q.k: the q/k channels are waves 0 .. 2D/64-1; each wave
    // sums its q.q, k.k and q.k (q_i k_i from the lane pair), one barrier
    // publishes them (the reference sums in order; this is a tree, equal to
    // rounding)
    if (__builtin_amdgcn_readfirstlane(wave) < 2 * D / 64) {  // the q/k waves only (uniform)
        const float yo = dpp_mov<0xb1>(y);  // the lane pair's other channel
        const float sqq = sum64(is_k ? 0.0f : y * y), skk = sum64(is_k ? y * y : 0.0f);
        const float sqk = sum64(is_k ? 0.0f : y * yo);
        if (lane == 0) {
            l2p[3 * wave] = sqq;
            l2p[3 * wave + 1] = skk;
            l2p[3 * wave + 2] = sqk;
        }
    }
    lds_barrier();
    float qq = 0.0f, kk = 0.0f, pkq = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < 2 * D / 64; ++w2) {
        qq += l2p[3 * w2];
        kk += l2p[3 * w2 + 1];
        pkq += l2p[3 * w2 + 2];
    }
    // 1 / max(sqrt(x), eps) as min(rsq(x), 1 / eps) (x = 0 gives 1 / eps)
    const float rq = fminf(__builtin_amdgcn_rsqf(qq), a.l2_inv_eps);
    const float rk = fminf(__builtin_amdgcn_rsqf(kk), a.l2_inv_eps);

    const float bt = s_gate[0], g = s_gate[1];

    auto sum_tpc = [](float x) { return TPC == 8 ? sum8(x) : sum16(x); };
    float kr[SL], qr[SL];  // the thread's slice of the raw q, k rows
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        kr[i] = ks[el(i)];
        qr[i] = qs[el(i)];
    }
    // Column j's output from the state before the token:
    // o_j = (g rq (S_j . q) + d_j rk rq (k . q)) / sqrt(D) with
    // d_j = (v_j - g rk (S_j . k)) beta -- the update's algebra in another
    // order, equal to q . S_j' / sqrt(D) within rounding, at two FMAs per
    // state element.  Every part forms it for every column (the norm needs
    // all D outputs; in place as out of place, so both give the same bits).
    float pa = 0.0f, pb = 0.0f;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        pa = fmaf(s[i], qr[i], pa);
        pb = fmaf(s[i], kr[i], pb);
    }
    pa = sum_tpc(pa);
    pb = sum_tpc(pb);
    const float dn = (vs[j] - g * rk * pb) * bt;
    const float on = (g * rq * pa + dn * (rk * rq * pkq)) * (1.0f / sqrtf((float)D));

    // the new state of the part's own columns (CPP * TPC consecutive threads:
    // whole waves): the decay and delta rule of gdn_state_update
    // (matvec.c:975-1004) with the normalisations factored out of the sums --
    // k . (g S_j) = g rk (kr . S_j) is the pb above, so the rule's delta is
    // dn, and S_j' = g S_j + kr (rk dn).  The output q . S_j' / sqrt(D) is then
    // on by the same algebra, so y takes on for every column.
    if (own_col) {
        const float kd = rk * dn;
#pragma unroll
        for (int i = 0; i < SL; ++i) s[i] = fmaf(kr[i], kd, s[i] * g);
#pragma unroll
        for (int i = 0; i < SL; i += 4) {
            f32x4 x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = s[i + e];
            *reinterpret_cast<f32x4*>(So + i * TPC) = x;
        }
    }
    // rmsnorm_gated over the head's D outputs (matvec.c:1007-1021), as
    // gdn_gated_norm_kernel computes it
    const float sq = sum64(part == 0 ? on * on : 0.0f);
    if (lane == 0) ssq[wave] = sq;
    lds_barrier();
    if (writes_y) {
        float ss = 0.0f;
#pragma unroll
        for (int wv2 = 0; wv2 < NT / 64; ++wv2) ss += ssq[wv2];
        const float inv = __builtin_amdgcn_rsqf(ss / (float)D + a.norm_eps);
        a.y[(size_t)h * D + j] = on * wv * inv * zs;
    }
    // the delay line last (nothing here reads it; stored earlier, a wait for a
    // load issued before it waited for the store too): head kh's q/k channels
    // by part 0 of v head kh (n_v >= n_k), v channels by the part of their
    // own head that stores that column
    if (has_ch && (tid >= 2 * D ? (uint32_t)(tid - 2 * D) - own0 < CPP : (h == kh && pt == 0))) {
#pragma unroll
        for (int r = 0; r < KWM; ++r)
            if ((uint32_t)r < kw) a.conv_out[(size_t)r * a.conv_dim + ch] = X[r];
    }
}

}  // namespace

template <int D, int NP>
void launch_head(const GdnDecodeArgs& a, hipStream_t st)
{
    const uint32_t grid = 8u * NP * ((a.n_v + 7u) / 8u);
    if (a.kwidth <= 4)
        hipLaunchKernelGGL((gdn_decode_head_kernel<D, NP, 4>), dim3(grid), dim3(1024), 0, st, a);
    else
        hipLaunchKernelGGL((gdn_decode_head_kernel<D, NP, kMaxKw>), dim3(grid), dim3(1024), 0, st, a);
}

hipError_t launch_gdn_decode(const GdnDecodeArgs& a, hipStream_t st)
{
    // The norm fused (one launch): NP = 8 workgroups per v head when the
    // state goes out of place, one in place.  YHIP_GDN_DECODE2=1 selects the
    // two-launch form (16-column workgroups + the norm kernel);
    // YHIP_GDN_DECODE_NP = 1, 2, 4, 8 or 16 sets NP for out-of-place calls.
    static const int two = [] {
        const char* e = getenv("YHIP_GDN_DECODE2");
        return e ? atoi(e) : 0;
    }();
    static const int np_env = [] {
        const char* e = getenv("YHIP_GDN_DECODE_NP");
        return e ? atoi(e) : 8;
    }();
    if (!two) {
        // the l2norm's 1 / eps once here, not by a division in every wave
        GdnDecodeArgs b = a;
        b.l2_inv_eps = 1.0f / a.l2_eps;
        const int np = a.S_out == a.S ? 1 : np_env;
        switch (a.D * 100 + np) {
        case 6401: launch_head<64, 1>(b, st); break;
        case 6402: launch_head<64, 2>(b, st); break;
        case 6404: launch_head<64, 4>(b, st); break;
        case 6408: launch_head<64, 8>(b, st); break;
        case 6416: launch_head<64, 16>(b, st); break;
        case 12801: launch_head<128, 1>(b, st); break;
        case 12802: launch_head<128, 2>(b, st); break;
        case 12804: launch_head<128, 4>(b, st); break;
        case 12808: launch_head<128, 8>(b, st); break;
        case 12816: launch_head<128, 16>(b, st); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (a.D) {
    case 64: hipLaunchKernelGGL(gdn_decode_kernel<64>, dim3(a.n_v * (64 / kCols)), dim3(kThreads), 0, st, a); break;
    case 128:
        hipLaunchKernelGGL(gdn_decode_kernel<128>, dim3(a.n_v * (128 / kCols)), dim3(kThreads), 0, st, a);
        break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // gated RMSNorm of each head, in place on y
    GdnNormArgs n = {};
    n.y = a.y;
    n.x = a.y;
    n.z = a.z;
    n.w = a.norm_w;
    n.y_stride = n.x_stride = n.z_stride = a.n_v * a.D;
    n.T = 1;
    n.n_heads = a.n_v;
    n.head_dim = a.D;
    n.w_f16 = a.norm_w_f16;
    n.eps = a.norm_eps;
    return launch_gdn_gated_norm(n, st);
}

}  // namespace yhip
