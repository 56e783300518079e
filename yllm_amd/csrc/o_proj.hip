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
//  * More tokens: oproj_gemm_kernel, an f16 MFMA GEMM with f32 accumulation
//    and the residual add in its epilogue.  f16 att: one product.  f32 att
//    with f16 weights: att is split into f16 hi + lo parts (hi = f16(att),
//    lo = f16(att - hi)) and both products accumulate in the same registers,
//    which keeps about 22 bits of each activation; attention outputs are
//    convex combinations of f16 V rows (times a gate <= 1), so |att| <= 65504
//    and hi never overflows.  f32 weights: the weights are split the same
//    way and hi.Whi + lo.Whi + hi.Wlo accumulate.
#include "common.hpp"
#include "internal.hpp"


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
        // the weights are read once per call: non-temporal loads (one token,
        // 4096 x 4096 f16: 9.3 -> 8.8 us)
        float w[kRows][8];
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r) {
            const uint32_t o = min(o0 + r, a.hidden - 1);  // a missing last row repeats a real one, unused
            if (W_F16) {
                const f16x8 v = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(reinterpret_cast<const _Float16*>(a.w) +
                                                                (size_t)o * a.qdim + i0));
#pragma unroll
                for (int e = 0; e < 8; ++e) w[r][e] = (float)v[e];
            } else {
                const float* p = reinterpret_cast<const float*>(a.w) + (size_t)o * a.qdim + i0;
                const f32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
                const f32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
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
            acc[r][b] = xor_sum<64>(acc[r][b]);
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

// f32 rows -> f16 hi and lo parts, hi = f16(v), lo = f16(v - hi), each a
// contiguous [rows][cols] matrix
__global__ __launch_bounds__(256) void oproj_split_kernel(_Float16* hi, _Float16* lo, const float* src,
                                                          uint32_t src_stride, uint32_t rows, uint32_t cols)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint64_t)rows * cols) return;
    const uint32_t r = (uint32_t)(idx / cols), i = (uint32_t)(idx % cols);
    const float v = src[(size_t)r * src_stride + i];
    const _Float16 h = (_Float16)v;
    hi[idx] = h;
    lo[idx] = (_Float16)(v - (float)h);
}

// ---- the GEMM: x[t][o] += sum_k T[t][k] * O[o][k] over nseg K segments ----
//
// T (tokens, the MFMA A operand) and O (W_o rows, the B operand) are f16
// rows with K innermost; segment s multiplies T_s by O_s over k in [0, K)
// (f32 attention: T_s = hi, lo against O_s = W, W; f32 weights: T_s = hi,
// lo, hi against O_s = Whi, Whi, Wlo), so the hi + lo products accumulate in
// registers and x is read and written once.
//
// A workgroup (4 waves, 2 x 2) owns BT tokens x BO outputs; a wave owns
// (TM x 32) x (TN x 32) of them in TM x TN v_mfma_f32_32x32x16_f16
// accumulators.  K advances 32 at a time through LDS: both tiles go from HBM
// straight into LDS (buffer loads with the LDS destination, 16 bytes per
// lane), rows of 64 bytes with XOR-swizzled 16-byte chunks so the fragment
// reads are free of bank conflicts, in three stages: the tiles of the next
// two steps load while this step's MFMAs run.  Output: lane l holds output
// o = l % 32 of its 32 x 32 block and 16 tokens; the residual add is a float
// atomic add per element at L2 (one add per element, so the result is the
// load, add and store's), which keeps x's read off the kernel's tail.
struct GemmArgs {
    const _Float16* t[3];  // token rows, ld t_ld (elements)
    const _Float16* o[3];  // output rows (W_o), ld K
    float* x;
    uint32_t t_ld, x_stride, N, M, K, nseg;
};

constexpr int kBK = 32;     // K per step: rows of 4 chunks of 16 bytes
constexpr int kStages = 3;  // LDS stages: the loads of 2 steps ahead are in flight

// 16-byte chunk swizzle of a 64-byte LDS row: 8 consecutive rows hit 8
// distinct bank groups (32 banks, b128 reads in groups of 8 lanes), and 16
// consecutive rows 16 (64 banks, groups of 16 lanes)
__device__ inline int gemm_swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// s_waitcnt vmcnt(n), no wait on the other counters
template <int N>
__device__ inline void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

__device__ inline f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// one 16-byte HBM -> LDS load per lane (lane i writes at lds + 16 i)
__device__ inline void gemm_lds_load16(__amdgpu_buffer_rsrc_t r, _Float16* lds, int voff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

template <int TM, int TN>
__global__ __launch_bounds__(256, 2) void oproj_gemm_kernel(GemmArgs a)
{
    constexpr int BT = 2 * TM * 32, BO = 2 * TN * 32;  // workgroup tile
    constexpr int ROWS = BT + BO;                       // LDS rows per stage (128 B each)
    constexpr int CPR = kBK / 8;                         // chunks per row
    constexpr int NLD = ROWS * CPR / 256;               // 16-byte loads per thread per step
    constexpr int NLD_T = BT * CPR / 256;               // of which token rows
    static_assert(BT * CPR % 256 == 0 && BO * CPR % 256 == 0, "whole load instructions per operand");
    __shared__ __attribute__((aligned(16))) _Float16 lds[kStages * ROWS * kBK];

    // the wave index in a scalar register: the LDS destination of a
    // direct-to-LDS load (M0) must be uniform, and with a per-lane index the
    // compiler wrapped every such load in a loop over the lanes' values
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r32 = lane & 31, hh = lane >> 5;
    const int wt = wave >> 1, wo = wave & 1;
    // Tile order: the hardware deals consecutive workgroups to the 8 XCDs in
    // turn; workgroup x takes position (x % 8) * (grid / 8) + x / 8 of the
    // order below, so each XCD works through a contiguous run of it, and the
    // order walks groups of 4 token tiles across the output tiles, so the
    // workgroups an XCD runs at once share a few token and weight tiles in
    // its L2 (grid is a multiple of 8).
    const uint32_t n_ot = (a.M + BO - 1) / BO, n_tt = (a.N + BT - 1) / BT;
    const uint32_t per_xcd = gridDim.x / 8u;
    const uint32_t pid = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    const uint32_t grp = pid / (4u * n_ot), in_g = pid % (4u * n_ot);
    const uint32_t g_rows = min(4u, n_tt - grp * 4u);
    if (pid >= n_ot * n_tt) return;
    const uint32_t t0 = (grp * 4u + in_g % g_rows) * BT, o0 = (in_g / g_rows) * BO;
    const uint32_t ksteps = (a.K + kBK - 1) / kBK, nsteps = ksteps * a.nseg;

    // per load instruction i: the LDS chunk this lane fills and its row / column
    int goff[NLD];  // byte offset of the chunk within its operand, k0 = 0 (0x80000000: outside)

#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int Lc = 256 * i + 64 * wave + lane;
        const int R = Lc / CPR, c = (Lc % CPR) ^ gemm_swz(R);
        if (i < NLD_T) {
            const uint32_t t = t0 + R;
            goff[i] = (int)(t * a.t_ld * 2u + c * 16u) | (t < a.N ? 0 : (int)0x80000000);
        } else {
            const uint32_t o = o0 + (R - BT);
            goff[i] = (int)(o * a.K * 2u + c * 16u) | (o < a.M ? 0 : (int)0x80000000);
        }
    }
    auto rsrc = [&](const _Float16* p, uint32_t bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(p), 0, bytes, 0x00020000);
    };
    const uint32_t t_bytes = ((a.N - 1) * a.t_ld + a.K) * 2u, o_bytes = a.M * a.K * 2u;
    // the segments' base addresses as offsets from segment 0's, read once
    // (indexing a.t[seg] in the loop reads the kernel arguments from memory at
    // every step and waits for them; a select chain over the pointers went
    // through scratch memory)
    const uint64_t tb0 = (uint64_t)a.t[0], ob0 = (uint64_t)a.o[0];
    const uint64_t td1 = (uint64_t)a.t[1] - tb0, td2 = (uint64_t)a.t[2] - tb0;
    const uint64_t od1 = (uint64_t)a.o[1] - ob0, od2 = (uint64_t)a.o[2] - ob0;
    auto issue = [&](_Float16* buf, uint32_t st) {
        const bool past = st >= nsteps;  // workgroup-uniform
        const uint32_t seg = past ? 0 : st / ksteps, k0 = past ? 0 : (st % ksteps) * kBK;
        const uint64_t s1 = seg == 1, s2 = seg == 2;
        const __amdgpu_buffer_rsrc_t rt = rsrc((const _Float16*)(tb0 + s1 * td1 + s2 * td2), t_bytes);
        const __amdgpu_buffer_rsrc_t ro = rsrc((const _Float16*)(ob0 + s1 * od1 + s2 * od2), o_bytes);
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            // a chunk past K (the last step of a K that is no multiple of 64)
            // reads zeros, not the next row
            const int Lc = 256 * i + 64 * wave + lane;
            const int kc = ((Lc % CPR) ^ gemm_swz(Lc / CPR)) * 8;
            const int off = (past || goff[i] < 0 || k0 + kc >= a.K) ? (int)0x80000000 : goff[i] + (int)k0 * 2;
            gemm_lds_load16(i < NLD_T ? rt : ro, buf + (256 * i + 64 * wave) * 8, off);
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int m = 0; m < TM; ++m)
#pragma unroll
        for (int n = 0; n < TN; ++n)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[m][n][i] = 0.0f;

    // MFMA fragments: row row0 + r32 of a stage, 16-byte chunk (2 kk + hh) ^
    // swz(r32) (row0 is a multiple of 32, so the swizzle is r32's).  The
    // lane's part of the address goes through an opaque move each step, so
    // the compiler keeps one base per k chunk instead of hoisting an address
    // per fragment out of the loop.
    auto compute = [&](uint32_t stage) {
        int lane_row;
        asm volatile("v_mov_b32 %0, %1" : "=v"(lane_row) : "v"(r32 * kBK * 2 + (int)(stage * ROWS * kBK * 2)));
        const int sw = gemm_swz(r32);
        const char* base = reinterpret_cast<const char*>(lds) + lane_row;
        constexpr int KK = kBK / 16;
        f16x8 ft[2][TM], fo[2][TN];
        auto load = [&](int kk) {
            const char* b = base + (((2 * kk + hh) ^ sw) << 4);
#pragma unroll
            for (int n = 0; n < TN; ++n)
                fo[kk & 1][n] = *reinterpret_cast<const f16x8*>(b + (BT + (wo * TN + n) * 32) * kBK * 2);
#pragma unroll
            for (int m = 0; m < TM; ++m)
                ft[kk & 1][m] = *reinterpret_cast<const f16x8*>(b + ((wt * TM + m) * 32) * kBK * 2);
        };
        load(0);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (kk + 1 < KK) load(kk + 1);  // in flight under this k chunk's MFMAs
#pragma unroll
            for (int m = 0; m < TM; ++m)
#pragma unroll
                for (int n = 0; n < TN; ++n) acc[m][n] = mfma32(ft[kk & 1][m], fo[kk & 1][n], acc[m][n]);
        }
    };

    // Steps 0..kStages-2 load ahead; step st waits for its own tiles (the
    // loads of the kStages-2 later steps may stay in flight: a count, issued
    // in order, of NLD loads per step, every one of them issued -- past the
    // end they read zeros), then, after the barrier that orders the last
    // reads of stage (st-1) % kStages before it, loads step st+kStages-1 there.
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue(lds + s * ROWS * kBK, s);
    for (uint32_t st = 0; st < nsteps; ++st) {
        wait_vm<(kStages - 2) * NLD>();
        lds_barrier();
        issue(lds + ((st + kStages - 1) % kStages) * ROWS * kBK, st + kStages - 1);
        compute(st % kStages);
    }
    wait_vm<0>();  // the loads past the end land before the workgroup ends

    // x[t][o] += acc with float atomics at L2 (each element receives one
    // add: the result equals a load, add and store), no load of x on the way
#pragma unroll
    for (int m = 0; m < TM; ++m)
#pragma unroll
        for (int n = 0; n < TN; ++n) {
            const uint32_t o = o0 + (wo * TN + n) * 32 + r32;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t t = t0 + (wt * TM + m) * 32 + 8 * (i / 4) + 4 * hh + (i % 4);
                if (t < a.N && o < a.M) unsafeAtomicAdd(a.x + (size_t)t * a.x_stride + o, acc[m][n][i]);
            }
        }
}

template <int TM, int TN>
hipError_t launch_gemm_tiles(const GemmArgs& a, hipStream_t st)
{
    constexpr uint32_t BT = 2 * TM * 32, BO = 2 * TN * 32;
    const uint32_t tiles = ((a.N + BT - 1) / BT) * ((a.M + BO - 1) / BO);
    hipLaunchKernelGGL((oproj_gemm_kernel<TM, TN>), dim3((tiles + 7) / 8 * 8), dim3(256), 0, st, a);
    return hipGetLastError();
}

// Tile choice: 128 x 256 workgroup tiles for large batches, two workgroups
// per CU (MFMA-bound; one workgroup's barrier wait is covered by the other's
// MFMAs: 8192 x 4096 x 4096 ran 787 TFLOP/s against 771 for 256 x 256 tiles
// at one workgroup per CU); 64 x 64 for small ones (the engine's chunks of
// up to 64 tokens: the weights are read once and the launch is
// bandwidth-bound, so more, smaller workgroups stream them).  Token rows are
// launched in pieces whose byte offsets stay below 2 GiB.
hipError_t launch_gemm(GemmArgs a, hipStream_t st)
{
    const uint64_t row_bytes = (uint64_t)a.t_ld * 2;
    uint64_t per = ((1ull << 31) - 1 - (uint64_t)a.K * 2) / row_bytes;
    per = per / 256 * 256;
    const uint32_t N = a.N;
    for (uint32_t n0 = 0; n0 < N; n0 += (uint32_t)per) {
        GemmArgs b = a;
        b.N = (uint32_t)(N - n0 < per ? N - n0 : per);
        for (uint32_t s = 0; s < a.nseg; ++s) b.t[s] = a.t[s] + (size_t)n0 * a.t_ld;
        b.x = a.x + (size_t)n0 * a.x_stride;
        const hipError_t e = b.N > 128 ? launch_gemm_tiles<2, 4>(b, st) : launch_gemm_tiles<1, 1>(b, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
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

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

size_t oproj_workspace(uint32_t B, uint32_t qdim, uint32_t w_f16, uint32_t att_f16, uint32_t hidden)
{
    if (B <= kGemvRows || att_f16) return 0;
    // f32 att as f16 hi and lo matrices; f32 weights as f16 hi and lo too
    return 2 * align256((size_t)B * qdim * 2) + (w_f16 ? 0 : 2 * align256((size_t)hidden * qdim * 2));
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
    (void)ws_bytes;
    GemmArgs g = {};
    g.x = a.x;
    g.x_stride = a.x_stride;
    g.N = a.B;
    g.M = a.hidden;
    g.K = a.qdim;
    const _Float16* w16 = reinterpret_cast<const _Float16*>(a.w);
    if (a.att_f16) {  // f16 weights and f16 activations: one segment
        g.nseg = 1;
        g.t[0] = reinterpret_cast<const _Float16*>(a.att);
        g.t_ld = a.att_stride;
        g.o[0] = w16;
        const hipError_t e = launch_gemm(g, st);
        return e == hipSuccess ? nullptr : hipGetErrorString(e);
    }
    // f32 activations (and f32 weights): f16 hi / lo parts in the workspace
    const size_t tpart = align256((size_t)a.B * a.qdim * 2);
    _Float16* thi = reinterpret_cast<_Float16*>(ws);
    _Float16* tlo = reinterpret_cast<_Float16*>(reinterpret_cast<char*>(ws) + tpart);
    const uint64_t n = (uint64_t)a.B * a.qdim;
    hipLaunchKernelGGL(oproj_split_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, thi, tlo,
                       reinterpret_cast<const float*>(a.att), a.att_stride, a.B, a.qdim);
    g.t_ld = a.qdim;
    if (a.w_f16) {
        g.nseg = 2;
        g.t[0] = thi;  // hi . W
        g.t[1] = tlo;  // lo . W
        g.o[0] = g.o[1] = w16;
    } else {
        const size_t wpart = align256((size_t)a.hidden * a.qdim * 2);
        _Float16* whi = reinterpret_cast<_Float16*>(reinterpret_cast<char*>(ws) + 2 * tpart);
        _Float16* wlo = reinterpret_cast<_Float16*>(reinterpret_cast<char*>(ws) + 2 * tpart + wpart);
        const uint64_t nw = (uint64_t)a.hidden * a.qdim;
        hipLaunchKernelGGL(oproj_split_kernel, dim3((uint32_t)((nw + 255) / 256)), dim3(256), 0, st, whi, wlo,
                           reinterpret_cast<const float*>(a.w), a.qdim, a.hidden, a.qdim);
        g.nseg = 3;  // hi.Whi + lo.Whi + hi.Wlo (the lo.lo term is below f32 rounding)
        g.t[0] = thi;
        g.t[1] = tlo;
        g.t[2] = thi;
        g.o[0] = whi;
        g.o[1] = whi;
        g.o[2] = wlo;
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = launch_gemm(g, st);
    return e == hipSuccess ? nullptr : hipGetErrorString(e);
}

}  // namespace yhip
