// o_proj.hip -- the step after attention: x[b] += W_o . att[b]
// (engine.c:969-973: matmul(att_out, x2, SLOT_O) then the residual add;
// matmul_f16 / matmul_f32, matvec.c:98-122).
//
// W_o is [hidden][qdim] (f16 or f32), att [B][qdim] f32 (or f16 when the
// attention kernel wrote f16; f16 att takes f16 weights), x [B][hidden] f32.
//  * Few tokens (decode, B <= kGemvRows): oproj_gemv_kernel reads W_o once
//    from HBM and applies it to all B rows; activations stay f32 and every
//    product and sum is f32 (the reference's arithmetic, summed in another
//    order).  A wave owns kRows output rows; its lanes take 8 consecutive
//    inputs each (16-byte weight loads at f16), eight iterations of loads in
//    flight (all of a 4096-wide row), then a shuffle reduction and the
//    residual add.
//  * More tokens: hipBLASLt GEMMs (TN, f32 accumulate, beta = 1 for the
//    residual).  f16 weights: att is split into f16 hi + lo parts
//    (hi = f16(att), lo = f16(att - hi)) and multiplied twice, which keeps
//    about 22 bits of each activation; attention outputs are convex
//    combinations of f16 V rows (times a gate <= 1), so |att| <= 65504 and
//    hi never overflows.  f16 att: one f16 GEMM.  f32 weights: one f32 GEMM
//    on att itself.
#include "common.hpp"
#include "internal.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace yhip {
namespace {

constexpr uint32_t kRows = 2;  // output rows per wave

template <int W_F16, int A_F16, int NB>
__global__ __launch_bounds__(256) void oproj_gemv_kernel(OProjArgs a)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t o0 = (blockIdx.x * 4u + (threadIdx.x >> 6)) * kRows;
    if (o0 >= a.hidden) return;  // wave-uniform
    float acc[kRows][NB];
#pragma unroll
    for (uint32_t r = 0; r < kRows; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = 0.0f;

#pragma unroll 8
    for (uint32_t i0 = lane * 8u; i0 < a.qdim; i0 += 512u) {
        float w[kRows][8];
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r) {
            const uint32_t o = min(o0 + r, a.hidden - 1);  // a missing last row repeats a real one, unused
            if (W_F16) {
                const f16x8 v = *reinterpret_cast<const f16x8*>(reinterpret_cast<const _Float16*>(a.w) +
                                                                (size_t)o * a.qdim + i0);
#pragma unroll
                for (int e = 0; e < 8; ++e) w[r][e] = (float)v[e];
            } else {
                const float* p = reinterpret_cast<const float*>(a.w) + (size_t)o * a.qdim + i0;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(p);
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w[r][e] = v0[e];
                    w[r][4 + e] = v1[e];
                }
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if ((uint32_t)b >= a.B) break;  // uniform
            float xv[8];
            if (A_F16) {
                const f16x8 v = *reinterpret_cast<const f16x8*>(reinterpret_cast<const _Float16*>(a.att) +
                                                                (size_t)b * a.att_stride + i0);
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = (float)v[e];
            } else {
                const float* p = reinterpret_cast<const float*>(a.att) + (size_t)b * a.att_stride + i0;
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(p);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xv[e] = x0[e];
                    xv[4 + e] = x1[e];
                }
            }
#pragma unroll
            for (uint32_t r = 0; r < kRows; ++r) {
                float s = acc[r][b];
#pragma unroll
                for (int e = 0; e < 8; ++e) s += xv[e] * w[r][e];
                acc[r][b] = s;
            }
        }
    }
#pragma unroll
    for (uint32_t r = 0; r < kRows; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) acc[r][b] += __shfl_xor(acc[r][b], m, 64);
    if (lane == 0) {
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r) {
            if (o0 + r >= a.hidden) break;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if ((uint32_t)b >= a.B) break;
                a.x[(size_t)b * a.x_stride + o0 + r] += acc[r][b];
            }
        }
    }
}

// att rows -> f16 hi and lo parts, [B][qdim] contiguous
__global__ __launch_bounds__(256) void oproj_split_kernel(_Float16* hi, _Float16* lo, const float* att,
                                                          uint32_t att_stride, uint32_t B, uint32_t qdim)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint64_t)B * qdim) return;
    const uint32_t b = (uint32_t)(idx / qdim), i = (uint32_t)(idx % qdim);
    const float v = att[(size_t)b * att_stride + i];
    const _Float16 h = (_Float16)v;
    hi[idx] = h;
    lo[idx] = (_Float16)(v - (float)h);
}

template <int W_F16, int A_F16>
hipError_t launch_gemv(const OProjArgs& a, hipStream_t st)
{
    const uint32_t waves = (a.hidden + kRows - 1) / kRows;
    const dim3 grid((waves + 3) / 4);
    if (a.B <= 1)
        hipLaunchKernelGGL((oproj_gemv_kernel<W_F16, A_F16, 1>), grid, dim3(256), 0, st, a);
    else if (a.B <= 2)
        hipLaunchKernelGGL((oproj_gemv_kernel<W_F16, A_F16, 2>), grid, dim3(256), 0, st, a);
    else if (a.B <= 4)
        hipLaunchKernelGGL((oproj_gemv_kernel<W_F16, A_F16, 4>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((oproj_gemv_kernel<W_F16, A_F16, 8>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

// ---- hipBLASLt: one handle per device, one plan per shape -----------------

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo;
};

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<std::tuple<int, int, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t>, Plan> g_plans;

const char* lt_err(hipblasStatus_t s)
{
    switch (s) {
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "hipBLASLt not initialised";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "hipBLASLt allocation failed";
    case HIPBLAS_STATUS_INVALID_VALUE: return "hipBLASLt invalid value";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "hipBLASLt: no kernel for this problem";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "hipBLASLt execution failed";
    default: return "hipBLASLt error";
    }
}

// D = C = x^T (hidden x B, ld x_stride) += op_T(W) . Bm  with W [hidden][k] row-major
// (= k x hidden column-major, lda k) and Bm k x n column-major (ldb)
const char* gemm_tn(int w_f16, const void* w, const void* bm, uint32_t ldb, float* x, uint32_t x_stride, uint32_t m,
                    uint32_t n, uint32_t k, void* ws, size_t ws_bytes, hipStream_t st)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return "hipGetDevice failed";
    std::lock_guard<std::mutex> lock(g_mu);
    hipblasLtHandle_t h;
    auto hit = g_handles.find(dev);
    if (hit == g_handles.end()) {
        hipblasStatus_t s = hipblasLtCreate(&h);
        if (s != HIPBLAS_STATUS_SUCCESS) return lt_err(s);
        g_handles[dev] = h;
    } else {
        h = hit->second;
    }
    const auto key = std::make_tuple(dev, w_f16, m, n, k, ldb, x_stride, (uint32_t)(ws_bytes >> 20));
    auto pit = g_plans.find(key);
    if (pit == g_plans.end()) {
        Plan p;
        const hipDataType ab = w_f16 ? HIP_R_16F : HIP_R_32F;
        hipblasStatus_t s = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        if (s == HIPBLAS_STATUS_SUCCESS)
            s = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
        if (s == HIPBLAS_STATUS_SUCCESS)
            s = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
        if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&p.la, ab, k, m, k);
        if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&p.lb, ab, k, n, ldb);
        if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, m, n, x_stride);
        hipblasLtMatmulPreference_t pref = nullptr;
        if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatmulPreferenceCreate(&pref);
        const uint64_t wsb = ws_bytes;
        if (s == HIPBLAS_STATUS_SUCCESS)
            s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                      sizeof(wsb));
        hipblasLtMatmulHeuristicResult_t res;
        int found = 0;
        if (s == HIPBLAS_STATUS_SUCCESS)
            s = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, &res, &found);
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        if (s == HIPBLAS_STATUS_SUCCESS && found < 1) s = HIPBLAS_STATUS_NOT_SUPPORTED;
        if (s != HIPBLAS_STATUS_SUCCESS) {
            if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
            if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
            if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
            if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
            return lt_err(s);
        }
        p.algo = res.algo;
        pit = g_plans.emplace(key, p).first;
    }
    const Plan& p = pit->second;
    const float alpha = 1.0f, beta = 1.0f;
    const hipblasStatus_t s = hipblasLtMatmul(h, p.desc, &alpha, w, p.la, bm, p.lb, &beta, x, p.lc, x, p.lc, &p.algo,
                                              ws, ws_bytes, st);
    return s == HIPBLAS_STATUS_SUCCESS ? nullptr : lt_err(s);
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

size_t oproj_workspace(uint32_t B, uint32_t qdim, uint32_t w_f16, uint32_t att_f16)
{
    if (B <= kGemvRows) return 0;
    return (w_f16 && !att_f16 ? 2 * align256((size_t)B * qdim * 2) : 0) + kGemmWorkspace;
}

const char* launch_oproj(const OProjArgs& a, void* ws, size_t ws_bytes, hipStream_t st)
{
    if (a.B <= kGemvRows) {
        hipError_t e;
        if (a.w_f16)
            e = a.att_f16 ? launch_gemv<1, 1>(a, st) : launch_gemv<1, 0>(a, st);
        else
            e = a.att_f16 ? launch_gemv<0, 1>(a, st) : launch_gemv<0, 0>(a, st);
        return e == hipSuccess ? nullptr : hipGetErrorString(e);
    }
    if (a.att_f16) {  // f16 weights and f16 activations: one GEMM
        return gemm_tn(1, a.w, a.att, a.att_stride, a.x, a.x_stride, a.hidden, a.B, a.qdim, ws, kGemmWorkspace, st);
    }
    if (!a.w_f16) {
        return gemm_tn(0, a.w, a.att, a.att_stride, a.x, a.x_stride, a.hidden, a.B, a.qdim, ws, kGemmWorkspace, st);
    }
    const size_t part = align256((size_t)a.B * a.qdim * 2);
    _Float16* hi = reinterpret_cast<_Float16*>(ws);
    _Float16* lo = reinterpret_cast<_Float16*>(reinterpret_cast<char*>(ws) + part);
    void* lt_ws = reinterpret_cast<char*>(ws) + 2 * part;
    const uint64_t n = (uint64_t)a.B * a.qdim;
    hipLaunchKernelGGL(oproj_split_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, hi, lo,
                       reinterpret_cast<const float*>(a.att), a.att_stride, a.B, a.qdim);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hipGetErrorString(e);
    const char* msg = gemm_tn(1, a.w, hi, a.qdim, a.x, a.x_stride, a.hidden, a.B, a.qdim, lt_ws, kGemmWorkspace, st);
    if (msg) return msg;
    return gemm_tn(1, a.w, lo, a.qdim, a.x, a.x_stride, a.hidden, a.B, a.qdim, lt_ws, kGemmWorkspace, st);
}

}  // namespace yhip
