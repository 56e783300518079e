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
// Decomposition.  A workgroup (4 waves) owns 64 columns of one head for the
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
    float* Sp = a.S + ((size_t)h * D + j0 + lane) * D + wave * SL;
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
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
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
        *reinterpret_cast<f32x4*>(Sp + i) = x;
    }
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
    hipLaunchKernelGGL(gdn_kernel<D>, dim3(a.n_v * (D / kCols)), dim3(256), 0, st, a);
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

hipError_t launch_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt, const float* ssm_a,
                            uint32_t T, uint32_t n_v, hipStream_t st)
{
    const uint32_t n = T * n_v;
    hipLaunchKernelGGL(gdn_gates_kernel, dim3((n + 255) / 256), dim3(256), 0, st, beta, gate, alpha, dt, ssm_a, n,
                       n_v);
    return hipGetLastError();
}

}  // namespace yhip
