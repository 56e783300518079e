// gdn.hip -- Gated DeltaNet (qwen35 linear attention) recurrence on gfx950.
//
// Semantics: per token, q and k are L2-normalised per k-head
// (l2norm_inplace, matvec.c:942-949, called at engine.c:826-827), then
// gdn_state_update (matvec.c:975-1004): v-head h reads k-head h % n_k; its
// state is stored transposed, S[h][j][i] (column j of the d_k x d_v matrix
// is contiguous), and for every column j
//     S[h][j][:] *= g,   g = exp(gate[h])
//     delta_j = (v[j] - S[h][j][:] . k) * beta[h]
//     S[h][j][:] += delta_j * k
//     out[j] = (S[h][j][:] . q) / sqrt(d_v)
// Columns never interact, so the state parallelises over (head, column)
// without communication; only the time dimension is sequential.
//
// Three kernels.  A single token (a decode step) runs gdn_step_kernel; the
// token-by-token kernel (gdn_kernel) serves short sequences and callers
// without a workspace; the chunked form below (gdn_prep_kernel, then
// gdn_chain_kernel) serves prefill.
//
// Token by token.  A workgroup (4 waves) owns 64 columns of one head for the
// whole sequence; lane l holds column j0+l and wave w the d_k slice
// [w*D/4, (w+1)*D/4) of it, in registers (32 floats at D = 128).  Inputs are
// staged through LDS in chunks of 32 tokens, double buffered (the next
// chunk's global loads are in flight while the current chunk runs), and q/k
// rows are normalised once in LDS.  Per token a wave reads its k and q
// slices with broadcast LDS loads, updates its slice, and the two dot
// products over d_k are completed across the 4 waves through LDS (two
// barriers per token).  Arithmetic is fp32 throughout, as in the reference.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace yhip {
namespace {

constexpr int kChunk = 32;  // tokens staged per LDS buffer
constexpr int kCols = 64;   // state columns per workgroup (one per lane)

template <int D>
__global__ __launch_bounds__(256, 1) void gdn_kernel(GdnArgs a)
{
    constexpr int SL = D / 4;  // d_k elements per lane (one wave's slice)
    __shared__ float Kc[2][kChunk][D];
    __shared__ float Qc[2][kChunk][D];
    __shared__ float Vc[2][kChunk][kCols];
    __shared__ float Gc[2][kChunk];
    __shared__ float Bc[2][kChunk];
    __shared__ float red[2][2][4][kCols];  // [parity][which dot][wave][column]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int nblk = D / kCols;
    const uint32_t h = blockIdx.x / nblk;
    const uint32_t j0 = (blockIdx.x % nblk) * kCols;
    const uint32_t kh = h % a.n_k;  // matvec.c:983
    const float scale = 1.0f / sqrtf((float)D);

    // this lane's slice of column j0+lane
    const float* Sp = a.S + ((size_t)h * D + j0 + lane) * D + wave * SL;
    float* So = a.S_out + ((size_t)h * D + j0 + lane) * D + wave * SL;
    float s[SL];
#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(Sp + i);
        s[i] = x[0];
        s[i + 1] = x[1];
        s[i + 2] = x[2];
        s[i + 3] = x[3];
    }

    // staging: per chunk, k and q rows of D floats (kChunk*D/4 float4 each),
    // 64 v values per token, and the two gates
    constexpr int KQ4 = kChunk * D / 4 / 256;  // float4 per thread per matrix
    constexpr int V4 = kChunk * kCols / 4 / 256;
    f32x4 rk[KQ4], rq[KQ4], rv[V4];
    float rg = 0.0f, rb = 0.0f;
    auto load_chunk = [&](uint32_t c) {
        const uint32_t t0 = c * kChunk;
#pragma unroll
        for (int u = 0; u < KQ4; ++u) {
            const int e = (tid + 256 * u) * 4, t = e / D, i = e % D;
            if (t0 + t < a.T) {
                const size_t off = (size_t)(t0 + t) * a.qk_stride + (size_t)kh * D + i;
                rk[u] = *reinterpret_cast<const f32x4*>(a.k + off);
                rq[u] = *reinterpret_cast<const f32x4*>(a.q + off);
            } else {
                rk[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                rq[u] = rk[u];
            }
        }
#pragma unroll
        for (int u = 0; u < V4; ++u) {
            const int e = (tid + 256 * u) * 4, t = e / kCols, j = e % kCols;
            rv[u] = t0 + t < a.T
                        ? *reinterpret_cast<const f32x4*>(a.v + (size_t)(t0 + t) * a.v_stride + (size_t)h * D + j0 + j)
                        : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (tid < kChunk && t0 + tid < a.T) {
            rg = a.gate[(size_t)(t0 + tid) * a.n_v + h];
            rb = a.beta[(size_t)(t0 + tid) * a.n_v + h];
        }
    };
    auto store_chunk = [&](int b) {
#pragma unroll
        for (int u = 0; u < KQ4; ++u) {
            const int e = (tid + 256 * u) * 4, t = e / D, i = e % D;
            *reinterpret_cast<f32x4*>(&Kc[b][t][i]) = rk[u];
            *reinterpret_cast<f32x4*>(&Qc[b][t][i]) = rq[u];
        }
#pragma unroll
        for (int u = 0; u < V4; ++u) {
            const int e = (tid + 256 * u) * 4, t = e / kCols, j = e % kCols;
            *reinterpret_cast<f32x4*>(&Vc[b][t][j]) = rv[u];
        }
        if (tid < kChunk) {
            Gc[b][tid] = expf(rg);
            Bc[b][tid] = rb;
        }
    };
    // l2 normalisation of the chunk's q and k rows (2*kChunk rows, one wave
    // per row at a time): x / max(sqrt(sum x^2), eps)
    auto normalise = [&](int b) {
        if (a.eps <= 0.0f) return;
        for (int r = wave; r < 2 * kChunk; r += 4) {
            float* row = r < kChunk ? Kc[b][r] : Qc[b][r - kChunk];
            float x[D / 64], ss = 0.0f;
#pragma unroll
            for (int u = 0; u < D / 64; ++u) {
                x[u] = row[lane + 64 * u];
                ss += x[u] * x[u];
            }
            ss = xor_sum<64>(ss);
            const float rs = 1.0f / fmaxf(sqrtf(ss), a.eps);
#pragma unroll
            for (int u = 0; u < D / 64; ++u) row[lane + 64 * u] = x[u] * rs;
        }
    };

    const uint32_t nchunks = (a.T + kChunk - 1) / kChunk;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    normalise(0);
    __syncthreads();

    int par = 0;
    for (uint32_t c = 0; c < nchunks; ++c) {
        const int b = c & 1;
        if (c + 1 < nchunks) load_chunk(c + 1);
        const uint32_t t0 = c * kChunk;
        const int nt = min((uint32_t)kChunk, a.T - t0);
        for (int t = 0; t < nt; ++t) {
            const float g = Gc[b][t], bt = Bc[b][t];
            float kr[SL], qr[SL];
#pragma unroll
            for (int i = 0; i < SL; i += 4) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(&Kc[b][t][wave * SL + i]);
                const f32x4 y = *reinterpret_cast<const f32x4*>(&Qc[b][t][wave * SL + i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kr[i + e] = x[e];
                    qr[i + e] = y[e];
                }
            }
            float p = 0.0f;
#pragma unroll
            for (int i = 0; i < SL; ++i) {
                s[i] *= g;
                p = fmaf(s[i], kr[i], p);
            }
            red[par][0][wave][lane] = p;
            __syncthreads();
            const float dot = (red[par][0][0][lane] + red[par][0][1][lane]) +
                              (red[par][0][2][lane] + red[par][0][3][lane]);
            const float delta = (Vc[b][t][lane] - dot) * bt;
            float p2 = 0.0f;
#pragma unroll
            for (int i = 0; i < SL; ++i) {
                s[i] = fmaf(kr[i], delta, s[i]);
                p2 = fmaf(s[i], qr[i], p2);
            }
            red[par][1][wave][lane] = p2;
            __syncthreads();
            if (wave == 0) {
                const float o = (red[par][1][0][lane] + red[par][1][1][lane]) +
                                (red[par][1][2][lane] + red[par][1][3][lane]);
                a.out[(size_t)(t0 + t) * a.out_stride + (size_t)h * D + j0 + lane] = o * scale;
            }
            par ^= 1;
        }
        if (c + 1 < nchunks) {
            // buffer b^1 was last read by chunk c-1, whose final barrier has passed
            store_chunk(b ^ 1);
            __syncthreads();
            normalise(b ^ 1);
            __syncthreads();
        }
    }

#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        f32x4 x;
        x[0] = s[i];
        x[1] = s[i + 1];
        x[2] = s[i + 2];
        x[3] = s[i + 3];
        *reinterpret_cast<f32x4*>(So + i) = x;
    }
}

// ---------------------------------------------------------------------------
// Chunked form.  For a chunk of kC tokens t = 0..kC-1 starting from the
// state M0 (M[j][i] = S[h][j][i], d_v x d_k), with cumulative log-decays
// G_t = sum_{s<=t} gate_s, gamma_t = exp(G_t) and e_t = exp(G_last - G_t),
// the per-token recurrence unrolls to
//     (I + A) Delta = diag(beta) V - diag(beta*gamma) K M0^T
//     A[t][s] = beta_t exp(G_t - G_s) (k_t . k_s)            s < t
//     O       = diag(gamma) Q M0^T + P Delta,  P[t][s] = exp(G_t - G_s) (q_t . k_s), s <= t
//     M_last  = gamma_last M0 + Delta^T diag(e) K
// (rows of Delta, V, K, Q, O are tokens).  With T = (I + A)^-1, U = T
// diag(beta) V and W = T diag(beta*gamma) K, Delta = U - W M0^T.
// Two launches: gdn_prep_kernel computes, for every (v-head, chunk) at
// once, W, Q~ = diag(gamma) Q, K~ = diag(e) K, P, U and gamma_last;
// gdn_chain_kernel walks the chunks in order (Delta = U - W M^T, the output
// O = Q~ M^T + P Delta, M <- gamma_last M + Delta^T K~).  The prep's Gram
// products are fp32 MFMA (v_mfma_f32_16x16x4_f32); the chain's are split
// bf16 (mfma_x3 below; -W rounded to bf16); every accumulation, stored
// value and the state are fp32.
constexpr int kC = 64;  // tokens per chunk of the chunked form

__device__ inline f32x4 mfma_f32(float a, float b, const f32x4& c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Split-bf16 products (the chain kernel): x = hi + lo with hi = bf16(x) and
// lo = bf16(x - hi), each rounded to nearest even, so |x - hi - lo| <=
// 2^-18 |x|; a.b is taken as hi.hi + hi.lo + lo.hi (the dropped lo.lo and
// the splits leave ~2^-16 of each product) with fp32 accumulation, on the
// bf16 MFMA at 16x the rate of the fp32 one.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ inline void split_bf16(const float (&x)[8], bf16x8& hi, bf16x8& lo)
{
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        hi[j] = (__bf16)x[j];
        lo[j] = (__bf16)(x[j] - (float)hi[j]);
    }
}
__device__ inline f32x4 mfma_x3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl, f32x4 c)
{
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
}

template <int D>
struct ChunkWs {
    // per (v-head, chunk):
    //   Wb  [kC * D / 2]  -W rounded to bf16 in the chain kernel's register
    //                 order: the 16 bytes (w * D/32 + s) * 64 + l hold
    //                 -W[16w + l%16][(l/16) D/4 + 8s .. +7]
    //   Qb  [kC * D]  Q~ as bf16 hi / lo in the chain kernel's register order:
    //                 the 16 bytes ((w * D/32 + s) * 2 + hl) * 64 + l hold part
    //                 hl of Q~[16w + l%16][(l/16) D/4 + 8s .. +7]
    //   Kb  [kC * D]  K~ likewise: the 16 bytes ((b * 2 + s) * 2 + hl) * 64 + l
    //                 hold part hl of K~[16 (l/16) + 8s .. +7][16b + l%16]
    //   Pb  [kC * kC] P likewise: the 16 bytes ((w * 2 + s) * 2 + hl) * 64 + l
    //                 hold part hl of P[16w + l%16][16 (l/16) + 8s .. +7]
    //   U^T [D][kC], gamma_last (+3 floats of padding, where chain lanes
    //                 with no output to write store theirs)
    static constexpr size_t floats = (size_t)kC * D / 2 + (size_t)2 * kC * D + (size_t)kC * kC + (size_t)kC * D + 4;
    float* Wb;
    float* Q;
    float* Kb;
    float* P;
    float* U;
    float* gl;
    __device__ ChunkWs(float* ws, uint32_t h, uint32_t c, uint32_t n_chunks)
    {
        Wb = ws + ((size_t)h * n_chunks + c) * floats;
        Q = Wb + kC * D / 2;
        Kb = Q + kC * D;
        P = Kb + kC * D;
        U = P + kC * kC;
        gl = U + kC * D;
    }
};

template <int D>
__global__ __launch_bounds__(256, 2) void gdn_prep_kernel(GdnArgs a)
{
    constexpr int KP = D + 4;  // LDS row stride of the q / k rows (16-byte rows, staggered banks)
    constexpr int AP = kC + 4;
    constexpr int KQ = D / 4;  // contraction indices per lane group in the Gram MFMAs
    // A and P share their LDS with the q rows: once Q~ is written out and
    // each wave holds its Gram rows of Q in registers, Qn is dead.  84 -> 68
    // KiB at D = 128, two workgroups per CU.
    constexpr int QAN = kC * KP > kC * AP + kC * kC ? kC * KP : kC * AP + kC * kC;
    __shared__ float Kn[kC][KP];
    __shared__ float QA[QAN];
    __shared__ float sg[kC], sb[kC], sgam[kC], see[kC];
    float(*Qn)[KP] = reinterpret_cast<float(*)[KP]>(QA);
    float(*Am)[AP] = reinterpret_cast<float(*)[AP]>(QA);
    float(*Pm)[kC] = reinterpret_cast<float(*)[kC]>(QA + kC * AP);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const uint32_t c = blockIdx.x, h = blockIdx.y, kh = h % a.n_k;
    const uint32_t t0 = c * kC;
    const int nt = (int)min((uint32_t)kC, a.T - t0);
    ChunkWs<D> w(a.ws, h, c, a.n_chunks);

    // the chunk's gates and betas (token = lane, clamped to the last token;
    // wave 0 masks them): read with the q / k rows, unconditionally -- read
    // under lane < nt they came after a wait for every q / k load, a second
    // memory round trip
    const size_t gi = (size_t)(t0 + min(lane, nt - 1)) * a.n_v + h;
    const float g_raw = a.gate[gi], b_raw = a.beta[gi];

    // q and k rows of the chunk (zero past the last token): all loads issued
    // before any LDS store; the l2 norms are taken in registers (a row's D/4
    // float4s sit in D/4 consecutive lanes)
    {
        constexpr int NE = kC * D / 4 / 256;
        constexpr int RL = D / 4;
        f32x4 kv[NE], qv[NE];
#pragma unroll
        for (int u = 0; u < NE; ++u) {
            const int e = tid + 256 * u, t = e / (D / 4), i = (e % (D / 4)) * 4;
            const size_t off = (size_t)(t0 + min(t, nt - 1)) * a.qk_stride + (size_t)kh * D + i;
            kv[u] = *reinterpret_cast<const f32x4*>(a.k + off);
            qv[u] = *reinterpret_cast<const f32x4*>(a.q + off);
        }
        if (a.eps > 0.0f) {
#pragma unroll
            for (int u = 0; u < NE; ++u) {
                float kk = 0.0f, qq = 0.0f;
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    kk += kv[u][x] * kv[u][x];
                    qq += qv[u][x] * qv[u][x];
                }
                kk = xor_sum<RL>(kk);
                qq = xor_sum<RL>(qq);
                kv[u] *= 1.0f / fmaxf(sqrtf(kk), a.eps);
                qv[u] *= 1.0f / fmaxf(sqrtf(qq), a.eps);
            }
        }
#pragma unroll
        for (int u = 0; u < NE; ++u) {
            const int e = tid + 256 * u, t = e / (D / 4), i = (e % (D / 4)) * 4;
            const float keep = t < nt ? 1.0f : 0.0f;
            *reinterpret_cast<f32x4*>(&Kn[t][i]) = kv[u] * keep;
            *reinterpret_cast<f32x4*>(&Qn[t][i]) = qv[u] * keep;
        }
    }
    // gates: inclusive prefix sum of the log-decays over the chunk
    if (wave == 0) {
        float gv = lane < nt ? g_raw : 0.0f;
        const float bv = lane < nt ? b_raw : 0.0f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float x = __shfl_up(gv, o, 64);
            if (lane >= o) gv += x;
        }
        const float glast = __shfl(gv, 63, 64);
        sg[lane] = gv;
        sb[lane] = bv;
        sgam[lane] = expf(gv);
        see[lane] = expf(glast - gv);
        if (lane == 0) w.gl[0] = expf(glast);
    }
    __syncthreads();

    // Q~ = diag(gamma) Q and K~ = diag(e) K as bf16 hi / lo in the chain
    // kernel's register order (ChunkWs)
    for (int e = tid; e < 4 * (D / 32) * 64; e += 256) {
        const int l = e % 64, ws_ = e / 64, sk = ws_ % (D / 32), wt = ws_ / (D / 32);
        const int t = 16 * wt + (l & 15), i = (l >> 4) * (D / 4) + 8 * sk;
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(&Qn[t][i]);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(&Qn[t][i + 4]);
        float x[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {  // rounded products (not contracted into the split)
            x[u] = __fmul_rn(x0[u], sgam[t]);
            x[u + 4] = __fmul_rn(x1[u], sgam[t]);
        }
        bf16x8 hi, lo;
        split_bf16(x, hi, lo);
        bf16x8* dst = reinterpret_cast<bf16x8*>(w.Q) + (size_t)ws_ * 128 + l;
        dst[0] = hi;
        dst[64] = lo;
    }
    for (int e = tid; e < (D / 16) * 2 * 64; e += 256) {
        const int l = e % 64, bs = e / 64, sk = bs % 2, b = bs / 2;
        const int tk = 16 * (l >> 4) + 8 * sk, ik = 16 * b + (l & 15);
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = Kn[tk + u][ik] * see[tk + u];
        bf16x8 hi, lo;
        split_bf16(x, hi, lo);
        bf16x8* dst = reinterpret_cast<bf16x8*>(w.Kb) + (size_t)bs * 128 + l;
        dst[0] = hi;
        dst[64] = lo;
    }

    // Gram matrices K K^T and Q K^T over the ten 16x16 tiles (tb, sb) with
    // sb <= tb (A needs s < t, P needs s <= t; P is zero above); wave w takes
    // tiles w, w+4, w+8.  Lane group g contracts over d_k indices g*KQ ..
    // g*KQ+KQ-1.  The sums stay in registers until every read of Qn is done,
    // then A overwrites Qn.
    {
        static_assert(kC == 64, "four 16-token blocks per chunk");
        constexpr int NTL = 10, TPW = 3;
        f32x4 gkk[TPW], gqk[TPW];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const int ti = wave + 4 * j;
            gkk[j] = gqk[j] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (ti < NTL) {  // uniform over the wave
                const int tb = ti >= 6 ? 3 : ti >= 3 ? 2 : ti >= 1 ? 1 : 0, sbk = ti - tb * (tb + 1) / 2;
                f32x4 skk[2], sqk[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) skk[e] = sqk[e] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < KQ; kb += 4) {
                    const f32x4 x = *reinterpret_cast<const f32x4*>(&Kn[16 * tb + r][g * KQ + kb]);
                    const f32x4 y = *reinterpret_cast<const f32x4*>(&Qn[16 * tb + r][g * KQ + kb]);
                    const f32x4 b = *reinterpret_cast<const f32x4*>(&Kn[16 * sbk + r][g * KQ + kb]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        skk[e & 1] = mfma_f32(x[e], b[e], skk[e & 1]);
                        sqk[e & 1] = mfma_f32(y[e], b[e], sqk[e & 1]);
                    }
                }
                gkk[j] = skk[0] + skk[1];
                gqk[j] = sqk[0] + sqk[1];
            }
        }
        __syncthreads();  // every read of Qn is done: A may overwrite it
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const int ti = wave + 4 * j;
            if (ti < NTL) {
                const int tb = ti >= 6 ? 3 : ti >= 3 ? 2 : ti >= 1 ? 1 : 0, sbk = ti - tb * (tb + 1) / 2;
                const int s = 16 * sbk + r;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * tb + 4 * g + i;
                    const float dec = s <= t ? expf(sg[t] - sg[s]) : 0.0f;
                    Am[t][s] = s < t ? sb[t] * dec * gkk[j][i] : 0.0f;
                    Pm[t][s] = dec * gqk[j][i];
                }
            }
        }
        // P above the diagonal blocks: row block `wave`, column blocks wave+1 ..
        for (int cb = wave + 1; cb < kC / 16; ++cb)
#pragma unroll
            for (int i = 0; i < 4; ++i) Pm[16 * wave + 4 * g + i][16 * cb + r] = 0.0f;
    }
    __syncthreads();

    // Forward substitution (I + A) X = [diag(beta) V | diag(beta*gamma) K]
    // in 16-row blocks on fp32 MFMA: X_i = T_ii (B_i - sum_{j<i} A_ij X_j),
    // T_ii = (I + A_ii)^-1.  The four T_ii come first, by substitution
    // (threads 0..63: column tid % 16 of block tid / 16), and replace the
    // diagonal blocks of A.  Wave w then owns the 16-column tiles w, w + 4,
    // ... of X as MFMA accumulators (lane (g, r): rows 4g .. 4g+3 of each
    // block, column r); in the products the contraction over the 16 rows of
    // X_j runs in the order the accumulators hold them (step e takes row
    // 4g + e from lane group g, against A_ij[m][4g + e]), so X stays in
    // registers.  The column-per-thread substitution this replaces read
    // every A row through LDS in every thread (11.5 us of a ~32 us
    // workgroup).
    constexpr int CTW = 2 * D / 64;  // 16-column tiles per wave
    {
        const int bi = tid >> 4, cc = tid & 15;
        float tc[16];
        if (tid < 64) {
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                float acc = m == cc ? 1.0f : 0.0f;
#pragma unroll
                for (int k = 0; k < m; ++k) acc = fmaf(-Am[16 * bi + m][16 * bi + k], tc[k], acc);
                tc[m] = acc;
            }
        } else {
            // meanwhile the other three waves write P as bf16 hi / lo in the
            // chain kernel's register order (ChunkWs)
            for (int e = tid - 64; e < 4 * 2 * 64; e += 192) {
                const int l = e % 64, ws_ = e / 64, sk = ws_ % 2, wt = ws_ / 2;
                const int t = 16 * wt + (l & 15), s = 16 * (l >> 4) + 8 * sk;
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(&Pm[t][s]);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(&Pm[t][s + 4]);
                float x[8];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    x[u] = x0[u];
                    x[u + 4] = x1[u];
                }
                bf16x8 hi, lo;
                split_bf16(x, hi, lo);
                bf16x8* dst = reinterpret_cast<bf16x8*>(w.P) + (size_t)ws_ * 128 + l;
                dst[0] = hi;
                dst[64] = lo;
            }
        }
        __syncthreads();
        if (tid < 64) {
#pragma unroll
            for (int m = 0; m < 16; ++m) Am[16 * bi + m][16 * bi + cc] = tc[m];
        }
    }
    // right-hand sides: tiles ct < CTW / 2 are V columns (tile w + 4 ct < D / 16
    // for every wave), the rest K columns; rows past the last token have
    // beta = 0, so their (clamped, valid) V rows contribute nothing
    f32x4 X[CTW][4];
    {
        const float* vp = a.v + (size_t)h * D;
#pragma unroll
        for (int ct = 0; ct < CTW / 2; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = 16 * i + 4 * g + e;
                    X[ct][i][e] = vp[(size_t)(t0 + min(t, nt - 1)) * a.v_stride + 16 * (wave + 4 * ct) + r];
                }
#pragma unroll
        for (int ct = CTW / 2; ct < CTW; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = 16 * i + 4 * g + e;
                    X[ct][i][e] = sgam[t] * Kn[t][16 * (wave + 4 * ct) + r - D];
                }
#pragma unroll
        for (int ct = 0; ct < CTW; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) X[ct][i][e] *= sb[16 * i + 4 * g + e];
    }
    __syncthreads();  // T_ii in place
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < i; ++j) {
            const f32x4 av = *reinterpret_cast<const f32x4*>(&Am[16 * i + r][16 * j + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ct = 0; ct < CTW; ++ct) X[ct][i] = mfma_f32(-av[e], X[ct][j][e], X[ct][i]);
        }
        const f32x4 tv = *reinterpret_cast<const f32x4*>(&Am[16 * i + r][16 * i + 4 * g]);
#pragma unroll
        for (int ct = 0; ct < CTW; ++ct) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = mfma_f32(tv[e], X[ct][i][e], acc);
            X[ct][i] = acc;
        }
    }
    // U^T rows (the V columns): four consecutive tokens per lane
#pragma unroll
    for (int ct = 0; ct < CTW / 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<f32x4*>(w.U + (size_t)(16 * (wave + 4 * ct) + r) * kC + 16 * i + 4 * g) = X[ct][i];
    // -W through LDS (A is dead once every wave has read it)
    __syncthreads();
#pragma unroll
    for (int ct = CTW / 2; ct < CTW; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) QA[(16 * i + 4 * g + e) * KP + 16 * (wave + 4 * ct) + r - D] = -X[ct][i][e];
    __syncthreads();
    // -W as bf16 in the chain kernel's register order (ChunkWs)
    for (int e = tid; e < 4 * (D / 32) * 64; e += 256) {
        const int l = e % 64, ws_ = e / 64, sk = ws_ % (D / 32), wt = ws_ / (D / 32);
        const float* src = QA + (16 * wt + (l & 15)) * KP + (l >> 4) * (D / 4) + 8 * sk;
        float x[8];
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(src), x1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            x[u] = x0[u];
            x[u + 4] = x1[u];
        }
        bf16x8 hi;
#pragma unroll
        for (int u = 0; u < 8; ++u) hi[u] = (__bf16)x[u];
        reinterpret_cast<bf16x8*>(w.Wb)[(size_t)ws_ * 64 + l] = hi;
    }
}

// The recurrence across chunks with each chunk's output: per chunk,
// Delta = U - W M^T, O = (Q~ M^T + P Delta) / sqrt(d) and then
// M <- gamma_last M + Delta^T K~.  A workgroup of four waves owns J = 16
// state rows (d_v indices j0..j0+15) of one head, walks the chunks in order
// and writes the output columns j0..j0+15.  Both output products reuse
// operands the recurrence already holds: Q~ M^T has phase A's state
// operands (B) and P Delta has phase B's Delta^T operands; only Q~ and P
// rows are extra loads.  (A separate output pass over all chunks needed the
// chunk's starting state and Delta recorded in the workspace: 96 KB written
// and read again per chunk and head, and a third launch.)
//
// Every operand element of a chunk is read by exactly one wave, so each wave
// loads its own straight into registers, two chunks ahead (three register
// sets): phase A, wave w forms the Delta tile of tokens 16w..16w+15 from -W
// rows (its A operand), the U^T slice (the accumulator's start) and the state
// rows in LDS (B); phase B, wave w updates the state tiles of d_k blocks
// w D/64 .. (kept in its registers in fp32) from Delta^T in LDS (A) and K~
// (B).  Only the state slice and the Delta tile pass through LDS, as bf16
// hi / lo pairs; two barriers per chunk.  The products are split-bf16
// (mfma_x3: three bf16 MFMAs per product, fp32 accumulation; the state,
// Delta and the outputs themselves stay fp32), except that -W enters rounded
// to bf16 (W M^T as W.Mhi + W.Mlo): an error in W M^T only perturbs the
// prediction the delta rule subtracts, which the following tokens correct,
// so its rounding shows in the outputs at ~1e-5 relative (K~ feeds the
// state directly and keeps both parts), and it halves the bytes of -W each
// chunk moves.  The prep kernel writes -W, K~, Q~ and P in the order the
// lanes read them (ChunkWs).
//
// An output tile (16 tokens x the 16 columns) is two halves summed in fp32:
// half 0 is Q~ M^T over the first D/2 of d_k plus P Delta over the first
// k-step of the chunk's tokens, half 1 the rest.  PARTS = 1: wave w forms
// both halves of token tile w.  PARTS = 2 (two workgroups per slice, both
// running the recurrence): part p writes token tiles 2p and 2p + 1, wave w
// forms half w / 2 of tile 2p + w % 2, and the two halves meet in LDS.  The
// chain is bound by the bytes each CU loads per chunk (the -W, K~ and U^T
// operands 52 KB, the Q~ and P rows 48 KB); with two parts a CU loads 76 KB.
// Both forms give the same bits.
template <int D, int PARTS>
__global__ __launch_bounds__(256, 1) void gdn_chain_kernel(GdnArgs a)
{
    constexpr int J = 16;          // state rows (d_v indices) per workgroup
    constexpr int NSA = D / 32;    // phase A k-steps (d_k, 8 per lane group each)
    constexpr int NBW = D / 64;    // phase B: 16-wide d_k blocks per wave
    constexpr int NQ = NSA / PARTS, NP = 2 / PARTS;  // Q~ and P k-steps per wave
    static_assert(kC == 64 && D % 64 == 0, "four token tiles and four waves of d_k blocks");
    static_assert(PARTS == 1 || PARTS == 2, "one or two workgroups per slice");
    constexpr int MP = D + 8, DP = kC + 8;  // bf16 row strides (16-byte rows, staggered banks)
    __shared__ __attribute__((aligned(16))) __bf16 Mh[J][MP], Mlo[J][MP];   // the state slice, rows j
    __shared__ __attribute__((aligned(16))) __bf16 Dh[J][DP], Dlo[J][DP];   // Delta^T of the chunk, rows j
    __shared__ f32x4 Ox[PARTS == 2 ? 4 : 1][64];                            // output halves (PARTS = 2)

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    // workgroup b = (part * D/16 + slice) * n_v + h: consecutive workgroups
    // go to different XCDs, so the slices of one head (b mod 8 fixed when n_v
    // is a multiple of 8) share an L2 and read the head's chunk data once
    const uint32_t h = blockIdx.x % a.n_v, sl = blockIdx.x / a.n_v, jt = sl % (D / 16), j0 = jt * J;
    const int part = (int)(sl / (D / 16));
    const int ot = PARTS == 1 ? wave : 2 * part + (wave & 1);  // the wave's output token tile
    const int oh = PARTS == 1 ? 0 : wave >> 1;                 // and half (PARTS = 2)
    const float* S = a.S + ((size_t)h * D + j0) * D;
    float* So = a.S_out + ((size_t)h * D + j0) * D;
    const uint32_t nlast = a.n_chunks - 1;
    const float scale = 1.0f / sqrtf((float)D);

    // one chunk's register operands of this wave
    struct Ops {
        bf16x8 w[NSA];        // -W[16 wave + r][g D/4 + 8s .. +7] (bf16)
        f32x4 u;              // U^T[j0 + r][16 wave + 4g .. +3]
        bf16x8 q[NQ][2];      // Q~[16 ot + r][g D/4 + 8s .. +7] of its k-steps, hi and lo
        bf16x8 k[NBW][2][2];  // K~[16g + 8s .. +7][16 (NBW wave + bb) + r], hi and lo
        bf16x8 p[NP][2];      // P[16 ot + r][16g + 8s .. +7] of its k-steps, hi and lo
        float gl;
    };
    // the loads of one register set in two halves (-W, U and Q~; K~, P and
    // gamma_last)
    auto load_a = [&](Ops& o, uint32_t c) {
        ChunkWs<D> w(a.ws, h, c, a.n_chunks);
        const bf16x8* wb = reinterpret_cast<const bf16x8*>(w.Wb);
#pragma unroll
        for (int sk = 0; sk < NSA; ++sk) o.w[sk] = wb[(size_t)(wave * NSA + sk) * 64 + lane];
        o.u = *reinterpret_cast<const f32x4*>(w.U + (size_t)(j0 + r) * kC + 16 * wave + 4 * g);
        const bf16x8* qb = reinterpret_cast<const bf16x8*>(w.Q);
#pragma unroll
        for (int i = 0; i < NQ; ++i)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) o.q[i][hl] = qb[((size_t)(ot * NSA + oh * NQ + i) * 2 + hl) * 64 + lane];
    };
    auto load_b = [&](Ops& o, uint32_t c) {
        ChunkWs<D> w(a.ws, h, c, a.n_chunks);
        const bf16x8* kb = reinterpret_cast<const bf16x8*>(w.Kb);
#pragma unroll
        for (int bb = 0; bb < NBW; ++bb)
#pragma unroll
            for (int sk = 0; sk < 2; ++sk)
#pragma unroll
                for (int hl = 0; hl < 2; ++hl)
                    o.k[bb][sk][hl] = kb[((size_t)((NBW * wave + bb) * 2 + sk) * 2 + hl) * 64 + lane];
        const bf16x8* pb = reinterpret_cast<const bf16x8*>(w.P);
#pragma unroll
        for (int i = 0; i < NP; ++i)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) o.p[i][hl] = pb[((size_t)(ot * 2 + oh * NP + i) * 2 + hl) * 64 + lane];
        o.gl = w.gl[0];
    };
    auto load = [&](Ops& o, uint32_t c) {
        load_a(o, c);
        load_b(o, c);
    };
    // the state tiles of this wave in fp32: mt[bb][e] = M[j0 + 4g + e][16 (NBW wave + bb) + r]
    f32x4 mt[NBW];
    auto put_state = [&] {
#pragma unroll
        for (int bb = 0; bb < NBW; ++bb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 16 * (NBW * wave + bb) + r;
                const __bf16 hi = (__bf16)mt[bb][e];
                Mh[4 * g + e][i] = hi;
                Mlo[4 * g + e][i] = (__bf16)(mt[bb][e] - (float)hi);
            }
    };
    // output rows 16 ot + 4g + i of chunk c, column j0 + r, for i in [i0, i0
    // + n); with PARTS = 2 the half of a previous chunk in LDS is added first
    // (its partner wave stored it before the last barrier).  Lanes with
    // nothing to write (chunk c < 0, or a token past the last) store to the
    // chunk's padding word, so every chunk runs the same memory instructions.
    auto put_out = [&](int64_t c, f32x4 o) {
        if (PARTS == 2) o = o + Ox[(wave & 1) * 2 + (oh ^ 1)][lane];
        const uint32_t cc = c < 0 ? 0u : (uint32_t)c;
        float* pad = ChunkWs<D>(a.ws, h, cc, a.n_chunks).gl + 1;
#pragma unroll
        for (int i = 0; i < 4 / PARTS; ++i) {
            const int ii = PARTS == 1 ? i : 2 * oh + i;
            const uint32_t t = cc * kC + 16 * ot + 4 * g + ii;
            float* dst = c >= 0 && t < a.T ? a.out + (size_t)t * a.out_stride + (size_t)h * D + j0 + r : pad;
            *dst = o[ii] * scale;
        }
    };
#pragma unroll
    for (int bb = 0; bb < NBW; ++bb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mt[bb][e] = S[(size_t)(4 * g + e) * D + 16 * (NBW * wave + bb) + r];
    put_state();
    Ops oa, ob, oc;  // chunks c, c+1, c+2 of a round of three
    load(oa, 0);
    load(ob, min(1u, nlast));
    __syncthreads();
    f32x4 oprev = f32x4{0.f, 0.f, 0.f, 0.f};  // PARTS = 2: this wave's half of the previous chunk

    // One chunk with operand set o; the loads of the set for chunk cf go out
    // in between the MFMAs (the -W / Q~ half in phase A, the K~ / P half in
    // phase B): a wave that issued its loads in one burst waited for the
    // CU's memory pipeline instead of issuing MFMAs.
    auto chunk = [&](uint32_t c, const Ops& o, Ops& of, uint32_t cf) {
        // phase A: Delta rows 16 wave + 4g + e, column j0 + r = U - W M^T;
        // then the Q~ M^T part of the output halves
        f32x4 o0 = f32x4{0.f, 0.f, 0.f, 0.f}, o1 = o0;
        {
            f32x4 acc = o.u;
            bf16x8 bh[NSA], bl[NSA];
#pragma unroll
            for (int sk = 0; sk < NSA; ++sk) {
                bh[sk] = *reinterpret_cast<const bf16x8*>(&Mh[r][g * (D / 4) + 8 * sk]);
                bl[sk] = *reinterpret_cast<const bf16x8*>(&Mlo[r][g * (D / 4) + 8 * sk]);
            }
            if (PARTS == 2) put_out((int64_t)c - 1, oprev);
            load_a(of, cf);
#pragma unroll
            for (int sk = 0; sk < NSA; ++sk) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.w[sk], bl[sk], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.w[sk], bh[sk], acc, 0, 0, 0);
            }
#pragma unroll
            for (int k = 0; k < 2 * NSA; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
            }
            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
            bf16x4 dh, dl;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dh[e] = (__bf16)acc[e];
                dl[e] = (__bf16)(acc[e] - (float)dh[e]);
            }
            *reinterpret_cast<bf16x4*>(&Dh[r][16 * wave + 4 * g]) = dh;
            *reinterpret_cast<bf16x4*>(&Dlo[r][16 * wave + 4 * g]) = dl;
            if (PARTS == 1) {
#pragma unroll
                for (int i = 0; i < NSA / 2; ++i) o0 = mfma_x3(o.q[i][0], o.q[i][1], bh[i], bl[i], o0);
#pragma unroll
                for (int i = NSA / 2; i < NSA; ++i) o1 = mfma_x3(o.q[i][0], o.q[i][1], bh[i], bl[i], o1);
            } else if (oh == 0) {  // uniform over the wave; the B operands are k-steps oh NQ ..
#pragma unroll
                for (int i = 0; i < NQ; ++i) o0 = mfma_x3(o.q[i][0], o.q[i][1], bh[i], bl[i], o0);
            } else {
#pragma unroll
                for (int i = 0; i < NQ; ++i) o0 = mfma_x3(o.q[i][0], o.q[i][1], bh[NQ + i], bl[NQ + i], o0);
            }
        }
        lds_barrier();
        // phase B: M <- gamma_last M + Delta^T K~ on this wave's d_k blocks;
        // then the P Delta part of the output halves
        bf16x8 ah[2], al[2];
#pragma unroll
        for (int sk = 0; sk < 2; ++sk) {
            ah[sk] = *reinterpret_cast<const bf16x8*>(&Dh[r][16 * g + 8 * sk]);
            al[sk] = *reinterpret_cast<const bf16x8*>(&Dlo[r][16 * g + 8 * sk]);
        }
        load_b(of, cf);
#pragma unroll
        for (int bb = 0; bb < NBW; ++bb) {
            f32x4 acc = mt[bb] * o.gl;
#pragma unroll
            for (int sk = 0; sk < 2; ++sk) acc = mfma_x3(ah[sk], al[sk], o.k[bb][sk][0], o.k[bb][sk][1], acc);
            mt[bb] = acc;
        }
#pragma unroll
        for (int k = 0; k < 6 * NBW; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
        }
        put_state();
        if (PARTS == 1) {
            o0 = mfma_x3(o.p[0][0], o.p[0][1], ah[0], al[0], o0);
            o1 = mfma_x3(o.p[1][0], o.p[1][1], ah[1], al[1], o1);
            put_out(c, o0 + o1);
        } else {
            if (oh == 0)
                o0 = mfma_x3(o.p[0][0], o.p[0][1], ah[0], al[0], o0);
            else
                o0 = mfma_x3(o.p[0][0], o.p[0][1], ah[1], al[1], o0);
            Ox[(wave & 1) * 2 + oh][lane] = o0;  // the partner adds it after the barrier
            oprev = o0;
        }
        lds_barrier();
    };
    // chunk c's operands are in a register set loaded two chunks before.
    // Whole rounds of three chunks in a loop without exits in between, the
    // rest after it: with an exit test after every chunk the compiler's
    // waits for the register sets at the loop head covered every load in
    // flight (vmcnt(1)), once per round.
    const uint32_t rounds = a.n_chunks / 3;
    uint32_t c = 0;
    for (uint32_t rd = 0; rd < rounds; ++rd, c += 3) {
        chunk(c, oa, oc, min(c + 2, nlast));
        chunk(c + 1, ob, oa, min(c + 3, nlast));
        chunk(c + 2, oc, ob, min(c + 4, nlast));
    }
    if (c <= nlast) {
        chunk(c, oa, oc, min(c + 2, nlast));
        if (c + 1 <= nlast) chunk(c + 1, ob, oa, min(c + 3, nlast));
    }
    if (PARTS == 2) put_out(nlast, oprev);

    if (part == 0) {
#pragma unroll
        for (int bb = 0; bb < NBW; ++bb)
#pragma unroll
            for (int e = 0; e < 4; ++e) So[(size_t)(4 * g + e) * D + 16 * (NBW * wave + bb) + r] = mt[bb][e];
    }
}

// One token (a decode step).  A workgroup of 256 threads owns 16 columns of
// one head; the 16 lanes of a column hold D/16 elements each, so both dot
// products over d_k are a 16-lane butterfly and nothing goes through LDS.
// All of a lane's loads (state slice, q/k slices, v, gates) are issued
// together: one memory round trip, then the update, then the stores.
template <int D>
__global__ __launch_bounds__(256) void gdn_step_kernel(GdnArgs a)
{
    constexpr int SL = D / 16;
    const int tid = threadIdx.x, part = tid & 15, col = tid >> 4;
    constexpr uint32_t nblk = D / 16;
    const uint32_t h = blockIdx.x / nblk, j = (blockIdx.x % nblk) * 16 + col;
    const uint32_t kh = h % a.n_k;
    const float scale = 1.0f / sqrtf((float)D);
    const float* Sp = a.S + ((size_t)h * D + j) * D + part * SL;
    float* So = a.S_out + ((size_t)h * D + j) * D + part * SL;
    const float* kp = a.k + (size_t)kh * D + part * SL;
    const float* qp = a.q + (size_t)kh * D + part * SL;
    float s[SL], k[SL], q[SL];
#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(Sp + i);
        const f32x4 y = *reinterpret_cast<const f32x4*>(kp + i);
        const f32x4 z = *reinterpret_cast<const f32x4*>(qp + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s[i + e] = x[e];
            k[i + e] = y[e];
            q[i + e] = z[e];
        }
    }
    const float vj = a.v[(size_t)h * D + j];
    const float g = expf(a.gate[h]), bt = a.beta[h];
    auto sum16 = [](float x) { return xor_sum<16>(x); };
    if (a.eps > 0.0f) {
        float kk = 0.0f, qq = 0.0f;
#pragma unroll
        for (int i = 0; i < SL; ++i) {
            kk += k[i] * k[i];
            qq += q[i] * q[i];
        }
        const float rk = 1.0f / fmaxf(sqrtf(sum16(kk)), a.eps), rq = 1.0f / fmaxf(sqrtf(sum16(qq)), a.eps);
#pragma unroll
        for (int i = 0; i < SL; ++i) {
            k[i] *= rk;
            q[i] *= rq;
        }
    }
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        s[i] *= g;
        p = fmaf(s[i], k[i], p);
    }
    const float delta = (vj - sum16(p)) * bt;
    float p2 = 0.0f;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
        s[i] = fmaf(k[i], delta, s[i]);
        p2 = fmaf(s[i], q[i], p2);
    }
    const float o = sum16(p2) * scale;
#pragma unroll
    for (int i = 0; i < SL; i += 4) {
        f32x4 x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = s[i + e];
        *reinterpret_cast<f32x4*>(So + i) = x;
    }
    if (part == 0) a.out[(size_t)h * D + j] = o;
}

// engine.c:788-793: beta <- sigmoid(beta), gate <- softplus(alpha + dt) * a,
// softplus as log1p(exp(.)) like the reference
__global__ void gdn_gates_kernel(float* beta, float* gate, const float* alpha, const float* dt,
                                 const float* ssm_a, uint32_t n, uint32_t n_v)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t h = i % n_v;
    beta[i] = 1.0f / (1.0f + expf(-beta[i]));
    gate[i] = log1pf(expf(alpha[i] + dt[h])) * ssm_a[h];
}

template <int D>
hipError_t launch_gdn_d(const GdnArgs& a, hipStream_t st)
{
    if (a.T == 1) {
        hipLaunchKernelGGL(gdn_step_kernel<D>, dim3(a.n_v * (D / 16)), dim3(256), 0, st, a);
    } else if (a.ws) {
        hipLaunchKernelGGL(gdn_prep_kernel<D>, dim3(a.n_chunks, a.n_v), dim3(256), 0, st, a);
        // two workgroups per state slice when they fit the GPU and the state
        // goes out of place (in place, one part's final state could reach S
        // before the other part has read it)
        const uint32_t slices = a.n_v * (D / 16);
        if (a.S_out != a.S && 2 * slices <= (uint32_t)n_cus())
            hipLaunchKernelGGL((gdn_chain_kernel<D, 2>), dim3(2 * slices), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((gdn_chain_kernel<D, 1>), dim3(slices), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(gdn_kernel<D>, dim3(a.n_v * (D / kCols)), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gdn(const GdnArgs& a, hipStream_t st)
{
    switch (a.D) {
    case 64: return launch_gdn_d<64>(a, st);
    case 128: return launch_gdn_d<128>(a, st);
    default: return hipErrorInvalidValue;
    }
}

size_t gdn_chunk_workspace(uint32_t T, uint32_t n_v, uint32_t D)
{
    const size_t n_chunks = (T + kC - 1) / kC;
    const size_t per = D == 64 ? ChunkWs<64>::floats : ChunkWs<128>::floats;
    return n_chunks * n_v * per * sizeof(float);
}

uint32_t gdn_chunk_tokens() { return kC; }

hipError_t launch_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt, const float* ssm_a,
                            uint32_t T, uint32_t n_v, hipStream_t st)
{
    const uint32_t n = T * n_v;
    hipLaunchKernelGGL(gdn_gates_kernel, dim3((n + 255) / 256), dim3(256), 0, st, beta, gate, alpha, dt, ssm_a, n,
                       n_v);
    return hipGetLastError();
}

}  // namespace yhip
