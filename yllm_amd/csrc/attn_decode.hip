// attn_decode.hip -- split-K flash decoding over the head-major HBM KV cache.
//
// Semantics: engine.c:1074-1096 (one query token per head attends to keys
// 0..pos, scores scaled by 1/sqrt(d), softmax, weighted sum of V), optionally
// followed by the qwen35 sigmoid gate (engine.c:959-960).
//
// Work decomposition.  A workgroup (4 waves; two per CU for d <= 128) owns
// one (sequence, kv head,
// split of split_keys keys).  The whole GQA group of query heads that reads
// that kv head is processed together, so every K/V byte is read from HBM
// once.  The split's keys are walked in blocks of 32 -- one contiguous 8 KB
// run of K and one of V for d = 128 -- and wave w takes blocks w, w+W, ...
// with the next block's loads in flight while the current one is computed
// (two register fragment sets for d <= 128): two waves per SIMD, each with
// up to 32 KB outstanding.  Measured on MI355X at 32k keys: this beats a
// 4-deep ring at one wave per SIMD and 8-wave workgroups.  On splits of up
// to kLdsSplitKeys keys a block's K goes to LDS in whole-row 1 KB loads and
// the score operands are read from there (see kLdsSplitKeys).
//
// MFMA formulation (v_mfma_f32_16x16x32_f16, per wave, per 32-key block):
//   S^T[key][head] = K[key][:] . Q^T[:][head]       A = K rows, B = q (16 head
//                                                    slots, group padded)
//   O^T[d][head]  += V^T[d][key] . P^T[key][head]   A = the V tile (stored
//                                                    d-major), B = P^T
// Lane l owns head slot l%16 in every accumulator, so the softmax statistics
// of a head live in one column of lanes: the max needs two cross-lane steps,
// the running sum none until the end.  K rows are loaded in the order
// 8*(m/4) + 4t + m%4 (row m of half t) so that the score layout of lane group
// g is keys 8g..8g+7, exactly the k-slots of the P^T operand: P never leaves
// registers.  q is split into f16 hi + lo parts (two MFMAs) so scores keep
// ~fp32 accuracy for fp32 queries; the kernel is HBM-bound and the extra
// MFMAs are free.
//
// Splits write (max, sum, unnormalised O) partials in the log2 domain to the
// workspace; a merge kernel combines them per (sequence, head).  With a single
// split the workgroup writes the final output directly.  (Merging inside the
// split kernel by the last workgroup to arrive was measured slower both
// ways: with a device-scope release per workgroup, which writes back the
// XCD's whole L2, 4x slower; with write-through partial stores, an arrival
// counter and coherent reloads, 36.0 vs 32.3 us at 32k keys -- that chain
// sits on the tail of the kernel, where the separate merge kernel costs less.)
#include "common.hpp"
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>

#include <type_traits>

namespace yhip {
namespace {

// Cache policies of the K/V block loads (the buffer load's aux operand):
// 0, the default, or 2, non-temporal.  Every K/V byte of a decode step is
// read once; when a launch reads more than the caches keep from one step to
// the next (8 rotating layer caches of 32k keys, 134 MB each), streamed
// non-temporally the split kernel runs 9-14 % faster (32k keys 28.9 -> 26.4
// us, 128k 94.0 -> 81.3, 64 ragged sequences 792 -> 738); a small cache the
// next token reads again (one layer of 8.9 MB in the hybrid group) is faster
// kept (8.12 against 8.23 ms per group step).  decode_policy() picks.
constexpr int kKvDefault = 0, kKvStream = 2;

constexpr int kKeysPerBlock = 32;

// waves per workgroup, register fragment sets per wave, workgroups per CU
template <int D> constexpr int waves_of() { return 4; }
template <int D> constexpr int nbuf_of() { return D <= 128 ? 2 : 1; }
template <int D> constexpr int wg_per_cu() { return D <= 128 ? 2 : 1; }
// K blocks staged through LDS (the LK instantiations) for splits of at most
// this many keys, instead of loaded as MFMA operands.  Same box: 32k keys
// (splits of 1024) 23.9 -> 23.1 us, 14/2 heads, d 64, 512 keys (one split)
// 5.07 -> 4.37 us, 16/2 heads, d 256, 4352 keys (splits of 128) 10.6 ->
// 10.0 us; on longer splits the staged form ran slower
// (128k keys, splits of 4096: 79.5 -> 82.5 us; the 64-sequence batch,
// ~3000: 703 -> 706 us), so those keep the operand loads.
constexpr uint32_t kLdsSplitKeys = 1024;

// Staged K block of one wave: 32 rows of D halves, each 16-byte chunk at
// column c ^ kswz(r) of its row.  The score MFMA reads 16 rows (krow + 4t
// below: rows {0-3, 8-11, 16-19, 24-27}, + 4 for t = 1) at one column per
// 16-lane group; the swizzle gives those 16 rows 16 distinct 16-byte bank
// columns of a 256-byte bank window (64 banks): at d = 128 (256-byte rows)
// r & 15 with bit 4 folded into bit 2, at d = 64 (128-byte rows, two per
// window) bits 1, 3, 4 of r for the 8 rows of each parity.
template <int D>
__device__ inline uint32_t kswz(uint32_t r)
{
    if constexpr (D >= 128) return (r & 15u) ^ (((r >> 4) & 1u) << 2);
    else return ((r >> 1) & 1u) | (((r >> 3) & 1u) << 1) | (((r >> 4) & 1u) << 2);
}

// One 16-byte HBM -> LDS load per lane (lane i writes at lds + 16 i), with
// the launch's cache policy.  A __device__ function: lambdas in a kernel are
// host-device, and the host pass drops a kernel whose lambda calls this
// gfx950-only builtin.
template <int POL>
__device__ inline void k_dma16(__amdgpu_buffer_rsrc_t r, _Float16* lds, uint32_t voff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, POL);
}

// s_waitcnt vmcnt(N) (lgkmcnt, expcnt not waited for), fenced against moves
// of memory operations and of the scheduler across it
template <int N>
__device__ inline void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

__device__ inline f32x4 mfma16(const f16x8& a, const f16x8& b, const f32x4& c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float sigmoid_ref(float g) { return 1.0f / (1.0f + expf(-g)); }

// The by-value RoPE table (~1 KB of kernel arguments) is an argument of the
// ROPE instantiations only; the others take this stand-in with the same
// member names, whose fields they never read.
struct DecodeRopeNone {
    const float* k;
    const float* v;
    uint16_t* kc;
    uint16_t* vc;
    uint32_t kind, n_rot;
    float cs[2][1];
};
template <bool ROPE>
using DecodeRopeArg = typename std::conditional<ROPE, DecodeRope, DecodeRopeNone>::type;
static_assert(offsetof(DecodeRope, cs) % 8 == 0 && alignof(DecodeRope) == 8,
              "the cosine table is read with 8-byte loads from the kernel arguments");

// one 32-key block of K and V as MFMA operands of one lane
template <int D>
struct Frag {
    f16x8 k[2][D / 32];
    f16x8 v[D / 16];
};

// ROPE: the query arrives unrotated and the token at position len0 - 1 is
// neither rotated nor stored yet (yhip_attn_decode_rope): every workgroup
// rotates the query heads it stages (each thread loads its float4 and, for
// pairs half a span apart, the partner float4), and the workgroup whose split
// holds the token rotates the token's key, stores key and value into the
// cache and substitutes them for the cache rows it loaded.  The cosines and
// sines come from the host's cosf / sinf, as the reference computes them.
template <int D, bool ROPE, int POL, bool KVM, bool LK>
__global__ __launch_bounds__(64 * waves_of<D>(), wg_per_cu<D>()) void decode_split_kernel(DecodeArgs a,
                                                                                            DecodeRopeArg<ROPE> rp)
{
    constexpr int kWaves = waves_of<D>();
    constexpr int kThreads = 64 * kWaves;
    constexpr int NC = D / 32;  // 32-wide d chunks of the QK contraction
    constexpr int NB = D / 16;  // 16-row d blocks of the PV output
    // LK: each wave's two staged K blocks (separate variables, so the
    // compiler can tell a read of one from the loads in flight into the
    // other); after the key loop a wave's combine rows take their place
    // (d = 256: one block per wave, and the combine rows keep their own area)
    constexpr int NBUF = nbuf_of<D>();
    constexpr bool OK_ROWS = LK && NBUF == 2;  // combine rows in the staged blocks
    constexpr int KBH = LK ? kKeysPerBlock * D : 8;  // halves of one staged block
    __shared__ __attribute__((aligned(16))) _Float16 s_k0[kWaves][KBH];
    __shared__ __attribute__((aligned(16))) _Float16 s_k1[kWaves][NBUF == 2 ? KBH : 8];
    __shared__ __attribute__((aligned(16))) _Float16 s_qk[OK_ROWS ? 2 * 16 * (D + 8) : 8];
    __shared__ __attribute__((aligned(16))) float s_o[OK_ROWS ? 1 : kWaves][16][D + 4];
    __shared__ float s_m[kWaves][16];
    __shared__ float s_l[kWaves][16];
    // the token's K bits by dimension, and its V bits by lane: element
    // d = 16 b + n at [n][b], so lane n reads its NB values in one go
    __shared__ __attribute__((aligned(16))) uint16_t s_knew[ROPE ? D : 8];
    __shared__ __attribute__((aligned(16))) uint16_t s_vt[ROPE ? 16 : 1][ROPE ? D / 16 : 8];

    // grid (n_splits, n_kv, n_seq), or (n_kv, n_splits, n_seq) with KVM
    const uint32_t kvh = KVM ? blockIdx.x : blockIdx.y, split = KVM ? blockIdx.y : blockIdx.x, seq = blockIdx.z;
    // a length beyond the planned maximum is clamped, never read past
    const uint32_t len = min(min(a.lens ? a.lens[seq] : a.len0, a.kv_stride), a.split_keys * a.n_splits);
    const uint32_t kbeg = split * a.split_keys;
    // query heads h with h*n_kv/n_heads == kvh form [h0, h1) (engine.c:1079)
    // (KVM launches have whole groups of gmax heads: no division)
    const uint32_t h0 = KVM ? kvh * a.gmax : (kvh * a.n_heads + a.n_kv - 1) / a.n_kv;
    const uint32_t h1 = KVM ? h0 + a.gmax : ((kvh + 1) * a.n_heads + a.n_kv - 1) / a.n_kv;
    const uint32_t G = h1 - h0;
    if (kbeg >= len) {  // uniform over the workgroup
        // a sequence without keys gets zeros (times the gate), as the merge
        // kernel writes them when there are several splits
        if (len == 0 && a.n_splits == 1)
            for (uint32_t idx = threadIdx.x; idx < G * D; idx += kThreads) {
                const uint32_t h = h0 + idx / D, d = idx % D;
                float r = 0.0f;
                if (a.gate) r *= sigmoid_ref(a.gate[(size_t)seq * a.gate_stride + (size_t)h * D + d]);
                a.out[(size_t)seq * a.out_stride + (size_t)h * D + d] = r;
            }
        return;
    }
    const uint32_t kend = min(len, kbeg + a.split_keys);

    const uint16_t* K = (a.kptrs ? a.kptrs[seq] : a.k0) + k_index(kvh, 0, 0, D, a.kv_stride);
    const uint16_t* Vt = (a.vptrs ? a.vptrs[seq] : a.v0) + v_index(kvh, 0, 0, D, a.kv_stride);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;

    float m = -INFINITY, l = 0.0f;
    f32x4 o[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int krow = 8 * (n >> 2) + (n & 3);  // + 4t for half t

    // Block loads go through buffer resources over this kv head's K rows and
    // V tiles, and every prefetch is issued, valid or not: with a fixed
    // number of loads per block the compiler waits for exactly the block a
    // step reads (a conditional prefetch makes it wait for all loads,
    // including the one just issued for the next block).  A block past the
    // split gets an offset beyond the resource; the hardware returns zeros
    // for it without a memory access.
    const uint32_t nblk = (kend - kbeg + kKeysPerBlock - 1) / kKeysPerBlock;
    const uint32_t head_bytes = a.kv_stride * D * 2;
    const __amdgpu_buffer_rsrc_t rK =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(K), 0, head_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rV =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Vt), 0, head_bytes, 0x00020000);
    const uint32_t k_lane = (krow * D + g * 8) * 2;      // bytes within a block's K rows
    const uint32_t v_lane = (n * kVTile + g * 8) * 2;    // row d = n (+16b), positions 8g..8g+7
    // LK: a block's K rows are NJ loads of 1 KB each (whole rows, contiguous
    // in HBM); load j, lane l fills chunk 64 j + l of the staged block, i.e.
    // row r = (64 j + l) / CPR at column p = (64 j + l) % CPR, and so reads
    // the row's chunk p ^ kswz(r).  The score MFMA's operands are then read
    // from LDS.  (Loaded directly as operands, every load instruction covers
    // 16 rows x 64 bytes, and the same stream ran ~5 % slower.)
    static_assert(!LK || D == 64 || D == 128 || D == 256, "the swizzle's row widths");
    constexpr int CPR = D / 8;                 // 16-byte chunks per K row
    constexpr int NJ = kKeysPerBlock * CPR / 64;
    constexpr int NL = (LK ? NJ : 2 * NC) + NB;  // loads per block and lane
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave, in a scalar register
    auto kdma_off = [&](int j) -> uint32_t {
        const uint32_t P = 64u * j + lane, r = P / CPR, p = P % CPR;
        return r * D * 2 + ((p ^ kswz<D>(r)) * 16);
    };
    auto load = [&](Frag<D>& f, uint32_t blk, int slot) {
        const uint32_t key0 = kbeg + blk * kKeysPerBlock;
        const bool ok = blk < nblk;
        const uint32_t vb = ok ? (key0 / kVTile) * D * kVTile * 2 + v_lane : 0x80000000u;
        if constexpr (LK) {
            // the slot's fragment reads of the previous block are complete
            // (their MFMAs have consumed them; this wait only pins that down)
            __builtin_amdgcn_s_waitcnt(0xc07f);
            _Float16* dst = slot == 0 ? &s_k0[wv][0] : &s_k1[wv][0];
            const uint32_t kb0 = ok ? key0 * D * 2 : 0x80000000u;
#pragma unroll
            for (int j = 0; j < NJ; ++j) k_dma16<POL>(rK, dst + 512 * j, kb0 + kdma_off(j));
            // K before V in issue order: the score MFMAs wait for K alone
            __builtin_amdgcn_sched_barrier(0);
        } else {
            const uint32_t kb = ok ? key0 * D * 2 + k_lane : 0x80000000u;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    f.k[t][c] = __builtin_bit_cast(
                        f16x8, __builtin_amdgcn_raw_buffer_load_b128(rK, kb + (4 * t * D + c * 32) * 2, 0, POL));
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
            f.v[b] = __builtin_bit_cast(f16x8,
                                        __builtin_amdgcn_raw_buffer_load_b128(rV, vb + b * 16 * kVTile * 2, 0, POL));
    };

    // q is read once per workgroup: each thread loads float4s of the G heads'
    // rows (issued before the first blocks, so waiting for q does not wait
    // for K/V), splits them into f16 hi + lo parts and stages both in LDS
    // (rows padded by 16 bytes against bank conflicts; zeros for the padded
    // head slots).  The staging area is the one the wave combine uses after
    // the key loop.
    constexpr int D4 = D / 4;
    constexpr int QROW = D + 8;                                 // halves per staged row
    constexpr int QPT = (16 * D4 + kThreads - 1) / kThreads;   // float4s per thread
    static_assert(OK_ROWS || sizeof(s_o) >= 2 * 16 * QROW * sizeof(_Float16), "q staging fits the combine area");
    // [2][16][QROW]: hi, lo (combine rows in the staged blocks: its own area;
    // the K blocks' loads are in flight meanwhile)
    _Float16* s_q;
    if constexpr (OK_ROWS) s_q = s_qk;
    else s_q = reinterpret_cast<_Float16*>(&s_o[0][0][0]);
    // ROPE: pairs (d, d + half) of the first `span` dims for HALF / MROPE
    // (half = span / 2), (d, d + 1) for PAIRS; a thread rotating a float4 of
    // the first kind also loads its partner float4 at d +- half
    const uint32_t rkind = ROPE ? rp.kind : kRopeNone;
    const uint32_t span = (rkind == kRopeMrope) ? rp.n_rot : (uint32_t)D, half = span / 2;
    const bool far_pairs = rkind == kRopeHalf || rkind == kRopeMrope;
    // a rotated element's pair index (the cosine and sine it needs)
    auto pair_of = [&](uint32_t d) -> uint32_t { return far_pairs ? (d < half ? d : d - half) : d >> 1; };
    auto rotated = [&](uint32_t d) -> bool { return far_pairs ? d < span : rkind == kRopePairs; };
    // Every lane issues its q loads unconditionally, from a row that is valid
    // for every lane (the padded head slots read head 0's and are zeroed
    // afterwards): a load issued on some lanes only, into a zero-initialised
    // register, made the compiler copy the result right after the load and
    // wait for it -- before the K/V block loads were even issued (+1 us per
    // launch at 16/2 heads of 256).
    static_assert(16 * D4 % kThreads == 0, "whole rows of float4s per thread");
    const float* qbase = a.q + (size_t)seq * a.q_stride + (size_t)h0 * D;
    f32x4 qv[QPT];
#pragma unroll
    for (int r = 0; r < QPT; ++r) {
        const uint32_t idx = threadIdx.x + r * kThreads, hn = idx / D4, d = (idx % D4) * 4;
        qv[r] = *reinterpret_cast<const f32x4*>(qbase + (size_t)(hn < G ? hn : 0u) * D + d);
    }
    // ROPE: the new token (key len0 - 1) is stored by the workgroup whose
    // split holds it
    const uint32_t tpos = len - 1;
    const bool owns_tok = ROPE && kbeg <= tpos && tpos < kend;  // uniform over the workgroup

    // ROPE: the rotation's own loads go out with q, before the blocks (the
    // staging below then waits for them and q only; issued after the blocks,
    // in-order completion made it wait for the whole first round of blocks,
    // +1.2 us per launch at 16/2 heads of 256 and 4352 keys): per float4, its
    // partner float4 for pairs half a span apart, and its cosines and sines
    // (kernel arguments) in 8-byte loads -- four consecutive pairs pj .. pj + 3
    // half a span apart (half is a multiple of 4), or two adjacent pairs
    // d / 2, d / 2 + 1 for PAIRS -- from clamped, always-valid indices; the
    // kind selects afterwards.  The owner also loads the token's raw key
    // element d, its partner and its value element (thread d < D), with that
    // element's pair.
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    constexpr int RQ = ROPE ? QPT : 1;
    f32x4 qp[RQ];
    f32x2 tc[RQ][2], ts[RQ][2];
    float kraw = 0.0f, kpart = 0.0f, vraw = 0.0f, kc1 = 1.0f, ks1 = 0.0f;
    if constexpr (ROPE) {
#pragma unroll
        for (int r = 0; r < QPT; ++r) {
            const uint32_t idx = threadIdx.x + r * kThreads, hn = idx / D4, d = (idx % D4) * 4;
            qp[r] = *reinterpret_cast<const f32x4*>(qbase + (size_t)(hn < G ? hn : 0u) * D +
                                                    (d < half ? d + half : (d - half) % D));
            const uint32_t pj = min(far_pairs ? (d < half ? d : d - half) : d >> 1, 124u);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                tc[r][u] = *reinterpret_cast<const f32x2*>(&rp.cs[0][pj + 2 * u]);
                ts[r][u] = *reinterpret_cast<const f32x2*>(&rp.cs[1][pj + 2 * u]);
            }
        }
        if (owns_tok && threadIdx.x < (uint32_t)D) {
            const uint32_t d = threadIdx.x;
            const uint32_t pr = far_pairs ? (d < span ? (d < half ? d + half : d - half) : d) : (d ^ 1u);
            kraw = rp.k[(size_t)kvh * D + d];
            kpart = rp.k[(size_t)kvh * D + pr];
            vraw = rp.v[(size_t)kvh * D + d];
            const uint32_t pj = min(pair_of(d), 127u);
            kc1 = rp.cs[0][pj];
            ks1 = rp.cs[1][pj];
        }
    }

    // NBUF blocks of this wave in flight
    Frag<D> f[NBUF];
#pragma unroll
    for (int i = 0; i < NBUF; ++i) load(f[i], wave + i * kWaves, i);
    // nothing below moves above the block loads (a use of q or the rotation's
    // loads scheduled among them waits for them before the rest are issued)
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (ROPE) {
        // element d with value x, partner value p and its pair's cosine c and
        // sine sn: the reference's (a, b) -> (a c - b s, a s + b c), a the
        // pair's first element; unrotated elements pass through unchanged
        // (x c - p sn for a pair's first element, p sn + x c = x c + p sn for
        // its second: two rounded products and one rounded sum either way,
        // formed without a branch)
        auto rotate = [&](float x, float p, float c, float sn, bool first, bool rot) {
#pragma clang fp contract(off)
            const float u = x * c, t = p * sn;
            const float r = first ? u - t : u + t;
            return rot ? r : x;
        };
#pragma unroll
        for (int r = 0; r < QPT; ++r) {
            const uint32_t idx = threadIdx.x + r * kThreads, hn = idx / D4, d = (idx % D4) * 4;
            const f32x4 c4 = far_pairs ? f32x4{tc[r][0][0], tc[r][0][1], tc[r][1][0], tc[r][1][1]}
                                       : f32x4{tc[r][0][0], tc[r][0][0], tc[r][0][1], tc[r][0][1]};
            const f32x4 s4 = far_pairs ? f32x4{ts[r][0][0], ts[r][0][1], ts[r][1][0], ts[r][1][1]}
                                       : f32x4{ts[r][0][0], ts[r][0][0], ts[r][0][1], ts[r][0][1]};
            // span and half are multiples of 4: one answer per float4 for the
            // kinds with pairs half a span apart
            const bool rot = rotated(d), first4 = d < half;
            f16x4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // partner: the same lane's float4 for PAIRS (element e ^ 1), else the loaded one
                const float y = rotate(qv[r][e], far_pairs ? qp[r][e] : qv[r][e ^ 1], c4[e], s4[e],
                                       far_pairs ? first4 : (e & 1) == 0, rot);
                const float x = hn < G ? y : 0.0f;
                const _Float16 h = (_Float16)x;
                hi[e] = h;
                lo[e] = (_Float16)(x - (float)h);
            }
            *reinterpret_cast<f16x4*>(s_q + hn * QROW + d) = hi;
            *reinterpret_cast<f16x4*>(s_q + (16 + hn) * QROW + d) = lo;
        }
        if (owns_tok && threadIdx.x < (uint32_t)D) {
            // the token's key and value with the reference rounding, into LDS
            // for the substitution below; they go to the cache after the key
            // loop (issued here, the loop's waits for its blocks waited for
            // these scattered 2-byte stores too)
            const uint32_t d = threadIdx.x;
            s_knew[d] = f32_to_f16_ref(rotate(kraw, kpart, kc1, ks1, far_pairs ? d < half : (d & 1u) == 0, rotated(d)));
            s_vt[d % 16][d / 16] = f32_to_f16_ref(vraw);
        }
    } else {
#pragma unroll
        for (int r = 0; r < QPT; ++r) {
            const uint32_t idx = threadIdx.x + r * kThreads, hn = idx / D4, d = (idx % D4) * 4;
            f16x4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x = hn < G ? qv[r][e] : 0.0f;
                const _Float16 h = (_Float16)x;
                hi[e] = h;
                lo[e] = (_Float16)(x - (float)h);
            }
            *reinterpret_cast<f16x4*>(s_q + hn * QROW + d) = hi;
            *reinterpret_cast<f16x4*>(s_q + (16 + hn) * QROW + d) = lo;
        }
    }
    lds_barrier();
    // B operand of the score MFMA: head slot n, dims c*32 + 8g .. +7
    f16x8 qhi[NC], qlo[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        qhi[c] = *reinterpret_cast<const f16x8*>(s_q + n * QROW + c * 32 + g * 8);
        qlo[c] = *reinterpret_cast<const f16x8*>(s_q + (16 + n) * QROW + c * 32 + g * 8);
    }
    // ROPE: the token's score for head slot n, by the MFMA chain of the key
    // loop with every A row the token's key (each output element is the same
    // dot product, in the same order, as the one of the token's own row)
    float stok = 0.0f;
    if constexpr (ROPE) {
        if (owns_tok) {
            f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const f16x8 kn = *reinterpret_cast<const f16x8*>(&s_knew[c * 32 + g * 8]);
                st = mfma16(kn, qhi[c], st);
                st = mfma16(kn, qlo[c], st);
            }
            stok = st[0];
        }
    }

    // LK: the lane's fragment offsets in a staged block -- row krow + 4t,
    // dims c*32 + 8g .. +7, i.e. chunk 4c + g of the row
    uint32_t koff[2][NC];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint32_t r = krow + 4 * t;
            koff[t][c] = r * D + (((4u * c + g) ^ kswz<D>(r)) * 8);  // in halves
        }

    auto compute = [&](Frag<D>& f, uint32_t key0, int slot) {
        // ROPE: the block holding the token (uniform over the wave)
        const bool tok_here = ROPE && owns_tok && tpos >= key0 && tpos < key0 + kKeysPerBlock;
        const uint32_t rr = tpos - key0;
        f32x4 s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                f16x8 kf;
                if constexpr (LK)
                    kf = *reinterpret_cast<const f16x8*>((slot == 0 ? &s_k0[wv][0] : &s_k1[wv][0]) + koff[t][c]);
                else
                    kf = f.k[t][c];
                s[t] = mfma16(kf, qhi[c], s[t]);
                s[t] = mfma16(kf, qlo[c], s[t]);
            }
        }
        // s[t][i] is head n, key key0 + 8g + 4t + i
        float x[8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[4 * t + i] = s[t][i] * a.c;
        if constexpr (ROPE) {
            // the block holding the token: its K and V rows came from the cache
            // before the token was stored.  The token's score replaces the one
            // of its row (key rr: lane group rr >> 3, element rr % 8 of x), and
            // after the softmax its V bits replace the loaded ones.
            if (tok_here) {
                const uint32_t jt = rr & 7u;
                const bool grp_here = (uint32_t)g == rr >> 3;
                const float xt = stok * a.c;
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = grp_here && (uint32_t)j == jt ? xt : x[j];
            }
        }
        const bool tail = key0 + kKeysPerBlock > kend;
        if (tail) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (key0 + 8 * g + j >= kend) x[j] = -INFINITY;
        }
        float mx = x[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) mx = fmaxf(mx, x[j]);
        mx = max_xor16(mx);
        mx = max_xor32(mx);
        const float mn = fmaxf(m, mx);
        const float alpha = fast_exp2(m - mn);
        float p[8], ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            p[j] = fast_exp2(x[j] - mn);
            ps += p[j];
        }
        l = l * alpha + ps;
        m = mn;
#pragma unroll
        for (int b = 0; b < NB; ++b) o[b] *= alpha;
        if (tail) {
            // keys past the end carry P = 0; their V must not be NaN/inf
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (key0 + 8 * g + j >= kend) f.v[b][j] = (_Float16)0.0f;
        }
        if constexpr (ROPE) {
            if (tok_here) {
                // V: the token is element e = rr % 8 -- the same for every lane
                // of the wave -- of the lanes of group rr >> 3, so only dword
                // e / 2 of each fragment changes, in its half e % 2: masked
                // merges with the lane's token values read unconditionally (a
                // select on a value read from LDS became a branch per fragment,
                // +1 us for the owner's wave at d = 256)
                constexpr int NBH = NB / 8 > 0 ? NB / 8 : 1;  // 16-byte reads per lane
                uint16_t vrow[NBH * 8];
#pragma unroll
                for (int u = 0; u < NBH; ++u) {
                    if constexpr (NB >= 8) {
                        const u32x4 w4 = *reinterpret_cast<const u32x4*>(&s_vt[n][8 * u]);
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            vrow[8 * u + 2 * k] = (uint16_t)(w4[k] & 0xffffu);
                            vrow[8 * u + 2 * k + 1] = (uint16_t)(w4[k] >> 16);
                        }
                    } else {
#pragma unroll
                        for (int k = 0; k < NB; ++k) vrow[k] = s_vt[n][k];
                    }
                }
                const uint32_t e = rr & 7u, sh = (e & 1u) * 16u;
                const uint32_t msk = (uint32_t)g == rr >> 3 ? 0xffffu << sh : 0u;
                auto put_v = [&](auto W) {
                    constexpr int w = decltype(W)::value;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        u32x4 x4 = __builtin_bit_cast(u32x4, f.v[b]);
                        x4[w] = (x4[w] & ~msk) | (((uint32_t)vrow[b] << sh) & msk);
                        f.v[b] = __builtin_bit_cast(f16x8, x4);
                    }
                };
                switch (e >> 1) {  // uniform over the wave
                case 0: put_v(std::integral_constant<int, 0>{}); break;
                case 1: put_v(std::integral_constant<int, 1>{}); break;
                case 2: put_v(std::integral_constant<int, 2>{}); break;
                default: put_v(std::integral_constant<int, 3>{}); break;
                }
            }
        }
        f16x8 pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = (_Float16)p[j];
#pragma unroll
        for (int b = 0; b < NB; ++b) o[b] = mfma16(f.v[b], pf, o[b]);
    };

    // Ring of NBUF fragment sets over this wave's blocks (wave, wave+W, ...):
    // while a block NBUF ahead exists, compute slot i and refill it; the last
    // NBUF blocks are computed without refills.  (Refills past the split are
    // not free even though they read nothing: the buffer unit still takes
    // each lane's 16 bytes through its pipeline, ~1.4 us for one d = 256
    // block, which dominates a launch of one block per wave.)
    const uint32_t nbw = nblk > (uint32_t)wave ? (nblk - wave + kWaves - 1) / kWaves : 0;
    uint32_t j = 0;
    for (; j + NBUF < nbw; j += NBUF) {
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
            const uint32_t b = wave + (j + i) * kWaves;
            // LK: the block's K has landed once at most its own V loads and
            // the NBUF - 1 blocks issued after it are in flight (issue order
            // is pinned by the waits' scheduling barriers and those in load;
            // the compiler waits for V itself before the P.V MFMAs)
            if constexpr (LK) wait_vm<(NBUF - 1) * NL + NB>();
            compute(f[i], kbeg + b * kKeysPerBlock, i);
            load(f[i], b + NBUF * kWaves, i);
            if constexpr (LK) __builtin_amdgcn_sched_barrier(0);
        }
    }
    if constexpr (LK && NBUF == 1) {
        if (j < nbw) {
            wait_vm<NB>();
            compute(f[0], kbeg + (wave + j * kWaves) * kKeysPerBlock, 0);
        }
    } else if constexpr (LK) {  // two slots; the second's loads are the last issued
        if (j < nbw) {
            wait_vm<NL + NB>();
            compute(f[0], kbeg + (wave + j * kWaves) * kKeysPerBlock, 0);
        }
        if (j + 1 < nbw) {
            wait_vm<NB>();
            compute(f[1], kbeg + (wave + (j + 1) * kWaves) * kKeysPerBlock, 1);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NBUF; ++i)
            if (j + i < nbw) compute(f[i], kbeg + (wave + (j + i) * kWaves) * kKeysPerBlock, i);
    }
    // LK: every load into the staged blocks has landed (a slot past the
    // wave's blocks may still be taking zeros) before the combine rows
    // overwrite them
    if constexpr (LK) wait_vm<0>();

    if (ROPE && owns_tok && threadIdx.x < (uint32_t)D) {  // the token's K and V into the cache
        const uint32_t d = threadIdx.x;
        rp.kc[k_index(kvh, tpos, d, D, a.kv_stride)] = s_knew[d];
        rp.vc[v_index(kvh, tpos, d, D, a.kv_stride)] = s_vt[d % 16][d / 16];
    }
    // per-lane partial sums -> per head (the four lane groups hold one head)
    l = sum_xor16(l);
    l = sum_xor32(l);
    // Combine the four waves in one LDS round: each wave stages its own
    // (m, l) and, for the group's G heads only (the padded slots' writes were
    // most of the combine's LDS traffic at G <= 8), its unscaled
    // accumulators; after one barrier the threads that form an output float4
    // rescale the four waves' float4s to the head's maximum as they sum them.
    // (Rescaling in the staging waves took a second barrier and LDS round.)
    // combine row r of wave w: LK, rows 0-7 in the wave's first staged
    // block and rows 8-15 in its second (8 (D + 4) floats fit one block)
    static_assert(!OK_ROWS || 8 * (D + 4) * 4 <= KBH * 2, "combine rows fit a staged block");
    auto orow = [&](uint32_t w, uint32_t r) -> float* {
        if constexpr (OK_ROWS)
            return reinterpret_cast<float*>(r < 8 ? &s_k0[w][0] : &s_k1[w][0]) + (r & 7u) * (D + 4);
        else
            return &s_o[w][r][0];
    };
    if (g == 0) {
        s_m[wave][n] = m;
        s_l[wave][n] = l;
    }
    if ((uint32_t)n < G) {
#pragma unroll
        for (int b = 0; b < NB; ++b) *reinterpret_cast<f32x4*>(orow(wave, n) + b * 16 + 4 * g) = o[b];
    }
    // an LDS-only barrier: a full barrier also waited for the owner's token
    // stores (scattered 2-byte K/V writes issued before the loop), which made
    // that workgroup the launch's straggler (+1.6 us)
    lds_barrier();

    // a single split writes the result directly, otherwise a partial
    const size_t grp = (size_t)seq * a.n_kv + kvh;  // (sequence, kv head) group
    for (uint32_t idx = threadIdx.x; idx < G * D4; idx += kThreads) {
        const uint32_t hn = idx / D4, d = (idx - hn * D4) * 4;
        // every LDS read first (one round trip), then the arithmetic
        float mw[kWaves], lw[kWaves];
        f32x4 ow[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            mw[w] = s_m[w][hn];
            lw[w] = s_l[w][hn];
            ow[w] = *reinterpret_cast<const f32x4*>(orow(w, hn) + d);
        }
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mw[w]);
        f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            // a wave without keys holds m = -inf, l = 0 and zero accumulators
            const float c = mw[w] == -INFINITY ? 0.0f : fast_exp2(mw[w] - M);
            O += ow[w] * c;
            L += lw[w] * c;
        }
        if (a.n_splits == 1) {
            const uint32_t h = h0 + hn;
            f32x4 r = O * (1.0f / L);
            if (a.gate) {
                const float* gp = a.gate + (size_t)seq * a.gate_stride + (size_t)h * D + d;
#pragma unroll
                for (int e = 0; e < 4; ++e) r[e] *= sigmoid_ref(gp[e]);
            }
            *reinterpret_cast<f32x4*>(a.out + (size_t)seq * a.out_stride + (size_t)h * D + d) = r;
        } else {
            const size_t slot = (grp * a.n_splits + split) * a.gmax + hn;
            *reinterpret_cast<f32x4*>(a.part_o + slot * D + d) = O;
            if (d == 0) {
                a.part_ml[slot * 2] = M;
                a.part_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// One workgroup per (query head, 64-dimension slice, sequence): 16 float4
// columns x 16 split subsets.  Thread t owns 4 output dimensions and the
// splits sg, sg+16, ...; it loads their (max, sum) pairs and partial outputs
// together (one memory round trip for up to 16 * kRound splits), combines
// them against its own running max, and the 16 subsets are then combined in
// LDS with one more rescale.  The gate is loaded first, beside the partials.
constexpr uint32_t kMergeSlice = 64;
constexpr uint32_t kMergeRound = 8;  // partial loads per thread and round of the merge

template <int D, uint32_t NG, bool KVM>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a)
{
    constexpr uint32_t SL = D < kMergeSlice ? D : kMergeSlice;  // dimensions per workgroup
    constexpr uint32_t E4 = SL / 4;     // float4 columns of the slice
    constexpr uint32_t NS = D / SL;     // slices per head
    static_assert(E4 * NG <= 256, "at most 256 threads");
    __shared__ f32x4 s_o[E4 * NG];      // NG split subsets, combined at the end
    __shared__ float s_m[E4 * NG], s_l[E4 * NG];
    // grid (n_heads * NS, n_seq), or (n_kv, G * NS, n_seq) with KVM (G query
    // heads per kv head)
    const uint32_t t = threadIdx.x;
    const uint32_t h = KVM ? blockIdx.x * a.gmax + blockIdx.y / NS : blockIdx.x / NS;
    const uint32_t d0 = ((KVM ? blockIdx.y : blockIdx.x) % NS) * SL;
    const uint32_t seq = KVM ? blockIdx.z : blockIdx.y;
    const uint32_t kvh = KVM ? blockIdx.x : h * a.n_kv / a.n_heads;
    const uint32_t hn = KVM ? blockIdx.y / NS : h - (kvh * a.n_heads + a.n_kv - 1) / a.n_kv;
    const uint32_t len = min(min(a.lens ? a.lens[seq] : a.len0, a.kv_stride), a.split_keys * a.n_splits);
    const uint32_t ns = (len + a.split_keys - 1) / a.split_keys;
    const size_t sbase = ((size_t)seq * a.n_kv + kvh) * a.n_splits;
    const uint32_t e4 = t % E4, sg = t / E4;
    const uint32_t d = d0 + 4 * e4;

    // Every load below is issued unconditionally from a valid address (the
    // output row stands in for a missing gate; slots past n_splits read slot 0,
    // and every split past ns is masked by selects, so the addresses wait for
    // no division), the first round's partials and the gate before
    // any wait: a load under a condition, into a register set beforehand, made
    // the compiler wait for it before issuing the next one (one memory round
    // trip per round of splits, 3.4 us per merge at 34 splits), and a loop
    // around the first round waited for the gate first.  Gate rows need not be
    // 16-byte aligned.
    constexpr uint32_t kRound = kMergeRound;
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    f32x2 ml[kRound];
    f32x4 ov[kRound];
    float M = -INFINITY, L = 0.0f;
    f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
    // The thread's slots are whole splits apart: one 64-bit address for its
    // slot of split 0, then 32-bit offsets (a split past n_splits reads split
    // 0's slot); a 64-bit index product per load had the round's last load
    // issued ~400 instructions after its first.
    const size_t slot0 = sbase * a.gmax + hn;
    const float* const pml = a.part_ml + slot0 * 2;
    const float* const po = a.part_o + slot0 * D + d;
    const uint32_t sm = a.gmax * 2u, so = a.gmax * (uint32_t)D;  // floats per split
    auto issue = [&](uint32_t s0) {
        const uint32_t om0 = s0 * sm, oo0 = s0 * so;
#pragma unroll
        for (uint32_t r = 0; r < kRound; ++r) {
            const bool in = s0 + r * NG < a.n_splits;
            const uint32_t om = in ? om0 + r * NG * sm : 0u, oo = in ? oo0 + r * NG * so : 0u;
            ml[r] = *reinterpret_cast<const f32x2*>(pml + om);
            ov[r] = *reinterpret_cast<const f32x4*>(po + oo);
        }
    };
    auto fold = [&](uint32_t s0) {
        float ms[kRound], ls[kRound];
        f32x4 os[kRound];
#pragma unroll
        for (uint32_t r = 0; r < kRound; ++r) {
            const bool ok = s0 + r * NG < ns;
            ms[r] = ok ? ml[r][0] : -INFINITY;
            ls[r] = ok ? ml[r][1] : 0.0f;
            os[r] = ok ? ov[r] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        float mr = M;
#pragma unroll
        for (uint32_t r = 0; r < kRound; ++r) mr = fmaxf(mr, ms[r]);
        if (mr != -INFINITY) {
            const float c_old = fast_exp2(M - mr);
            L *= c_old;
            O *= c_old;
#pragma unroll
            for (uint32_t r = 0; r < kRound; ++r) {
                const float c = fast_exp2(ms[r] - mr);
                L += ls[r] * c;
                O += os[r] * c;
            }
            M = mr;
        }
    };
    issue(sg);
    const float* gp = a.gate ? a.gate + (size_t)seq * a.gate_stride + (size_t)h * D + d
                             : a.out + (size_t)seq * a.out_stride + (size_t)h * D + d;
    f32x4 gt;
#pragma unroll
    for (int e = 0; e < 4; ++e) gt[e] = gp[e];
    __builtin_amdgcn_sched_barrier(0);  // the round's loads and the gate in flight before any use
    fold(sg);
    for (uint32_t s0 = sg + NG * kRound; s0 < ns; s0 += NG * kRound) {  // more than NG * kRound splits
        issue(s0);
        __builtin_amdgcn_sched_barrier(0);
        fold(s0);
    }
    // the gate's sigmoid before the barrier, off the combine's tail (only
    // with a gate: without one the stand-in row may hold any bits)
    f32x4 gs = f32x4{1.f, 1.f, 1.f, 1.f};
    if (a.gate) {
#pragma unroll
        for (int e = 0; e < 4; ++e) gs[e] = sigmoid_ref(gt[e]);
    }
    s_o[t] = O;
    s_m[t] = M;
    s_l[t] = L;
    lds_barrier();  // the gate's load may still be in flight
    if (t < E4) {
        // every subset's (m, l, O) read first (one LDS round trip)
        float mg[NG], lg[NG];
        f32x4 og[NG];
#pragma unroll
        for (uint32_t g2 = 0; g2 < NG; ++g2) {
            mg[g2] = s_m[g2 * E4 + t];
            lg[g2] = s_l[g2 * E4 + t];
            og[g2] = s_o[g2 * E4 + t];
        }
        float Mt = -INFINITY;
#pragma unroll
        for (uint32_t g2 = 0; g2 < NG; ++g2) Mt = fmaxf(Mt, mg[g2]);
        float Lt = 0.0f;
        f32x4 Ot = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t g2 = 0; g2 < NG; ++g2) {
            // a subset without splits holds m = -inf, l = 0 and O = 0
            const float c = mg[g2] == -INFINITY ? 0.0f : fast_exp2(mg[g2] - Mt);
            Lt += lg[g2] * c;
            Ot += og[g2] * c;
        }
        f32x4 r = ns ? Ot * (1.0f / Lt) * gs : f32x4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f32x4*>(a.out + (size_t)seq * a.out_stride + (size_t)h * D + d) = r;
    }
}

// Non-temporal K/V loads when the launch reads at least 32 MiB of K and V
// (an upper bound for a batch with device-side lengths); YHIP_DECODE_NT=0 or
// 1 forces the choice.
bool decode_streams(const DecodeArgs& a)
{
    static const int env = [] {
        const char* e = getenv("YHIP_DECODE_NT");
        return e ? atoi(e) : -1;
    }();
    if (env == 0 || env == 1) return env == 1;
    const uint64_t keys = a.lens ? (uint64_t)a.split_keys * a.n_splits : a.len0;
    const uint64_t bytes = (uint64_t)a.n_seq * a.n_kv * keys * a.D * 4u;
    return bytes >= (32ull << 20);
}

template <int D, uint32_t NG, bool KVM>
void launch_merge(const DecodeArgs& a, hipStream_t st)
{
    constexpr uint32_t slices = D < kMergeSlice ? 1 : D / kMergeSlice;
    constexpr uint32_t e4 = (D < kMergeSlice ? D : kMergeSlice) / 4;
    const dim3 grid = KVM ? dim3(a.n_kv, a.n_heads / a.n_kv * slices, a.n_seq) : dim3(a.n_heads * slices, a.n_seq);
    hipLaunchKernelGGL((decode_merge_kernel<D, NG, KVM>), grid, dim3(e4 * NG), 0, st, a);
}

template <int D, bool ROPE, bool KVM, bool LK>
void launch_split(const DecodeArgs& a, const DecodeRopeArg<ROPE>& rr, hipStream_t st)
{
    const dim3 grid = KVM ? dim3(a.n_kv, a.n_splits, a.n_seq) : dim3(a.n_splits, a.n_kv, a.n_seq);
    if (decode_streams(a))
        hipLaunchKernelGGL((decode_split_kernel<D, ROPE, kKvStream, KVM, LK>), grid, dim3(64 * waves_of<D>()), 0, st,
                           a, rr);
    else
        hipLaunchKernelGGL((decode_split_kernel<D, ROPE, kKvDefault, KVM, LK>), grid, dim3(64 * waves_of<D>()), 0, st,
                           a, rr);
}

template <int D, bool ROPE, bool KVM>
hipError_t launch_decode_o(const DecodeArgs& a, const DecodeRope& r, hipStream_t st)
{
    DecodeRopeArg<ROPE> rr{};
    if constexpr (ROPE) rr = r;
    if (a.split_keys <= kLdsSplitKeys) launch_split<D, ROPE, KVM, true>(a, rr, st);
    else launch_split<D, ROPE, KVM, false>(a, rr, st);
    if (a.n_splits > 1) {
        // the fewest split subsets whose one round of loads (kMergeRound per
        // thread) covers every split: one memory round trip and the smallest
        // LDS combine (32 splits: 4 subsets, 25.2 us at 32k keys against 26.4
        // with 16; 34 splits: 8, the d 256 token 11.25 against 12.0 us)
        const uint32_t rounds = (a.n_splits + kMergeRound - 1) / kMergeRound;
        if (rounds <= 1) launch_merge<D, 1, KVM>(a, st);
        else if (rounds <= 2) launch_merge<D, 2, KVM>(a, st);
        else if (rounds <= 4) launch_merge<D, 4, KVM>(a, st);
        else if (rounds <= 8) launch_merge<D, 8, KVM>(a, st);
        else launch_merge<D, 16, KVM>(a, st);
    }
    return hipGetLastError();
}

// The hardware deals workgroups to the 8 XCDs in turn by their linear id.
// With the kv head first in both grids (KVM, for kv head counts that are
// multiples of 8 and whole query-head groups), a kv head's splits and the
// merges of its query heads share XCDs (XCD kvh mod 8), so its q rows and
// the partials the merges read stay in those XCDs' L2: 32k keys, 32 / 8 heads
// 25.3 -> 24.6 us, 64 sequences 731 -> 706 us, 128k unchanged.  With 2 kv
// heads the same order was slower (the hybrid group's d 256 token 11.2 ->
// 11.6 us), so other shapes keep the split-major order.
template <int D, bool ROPE>
hipError_t launch_decode_d(const DecodeArgs& a, const DecodeRope& r, hipStream_t st)
{
    if (a.n_kv % 8u == 0 && a.n_heads % a.n_kv == 0) return launch_decode_o<D, ROPE, true>(a, r, st);
    return launch_decode_o<D, ROPE, false>(a, r, st);
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

}  // namespace

namespace {

// The plan's two tunables: the workgroup target of a launch and the smallest
// split (a multiple of 128 keys).  YHIP_DECODE_WG / YHIP_DECODE_MINSK
// override them for tuning sweeps.
uint64_t plan_target_wg(uint32_t n_seq)
{
    static const long env_wg = [] {
        const char* e = getenv("YHIP_DECODE_WG");
        return e ? atol(e) : 0L;
    }();
    return env_wg > 0 ? (uint64_t)env_wg : (n_seq == 1 ? 256 : 3072);
}

// A context whose K and V take at most this many bytes per kv head is not
// split: one workgroup per (sequence, kv head) writes the output directly,
// without partials and the merge launch (~4.5 us of launch gap and merge).
// Measured on MI355X, graph-replayed: 64 KiB 3.8 vs 6.5 us, 128 KiB 5.1-5.6
// vs 6.6-8.1 us (14/2 d 64, 32/8 d 128, 8/8 d 64), 256 KiB a tie (7.8-10.2
// both ways), 512 KiB 13-16 vs 7-10 us.  YHIP_DECODE_ONE_SPLIT overrides it.
uint64_t plan_one_split_bytes()
{
    static const uint64_t b = [] {
        const char* e = getenv("YHIP_DECODE_ONE_SPLIT");
        return e ? (uint64_t)atoll(e) : (uint64_t)160 * 1024;
    }();
    return b;
}

uint64_t plan_min_split()
{
    static const uint64_t min_sk = [] {
        const char* e = getenv("YHIP_DECODE_MINSK");
        const long v = e ? atol(e) : 0;
        return (uint64_t)(v > 0 ? v : 128);
    }();
    return min_sk;
}

size_t partial_bytes(uint32_t n_seq, uint32_t n_splits, uint32_t n_heads, uint32_t n_kv, uint32_t D)
{
    if (n_splits <= 1) return 0;
    const size_t gmax = (n_heads + n_kv - 1) / n_kv;
    const size_t groups = (size_t)n_seq * n_kv;
    return align256(groups * n_splits * gmax * 2 * sizeof(float)) + groups * n_splits * gmax * D * sizeof(float);
}

}  // namespace

size_t decode_plan(uint32_t n_seq, uint32_t max_len, uint64_t total_len, uint32_t n_heads,
                   uint32_t n_kv, uint32_t D, uint32_t* split_keys, uint32_t* n_splits)
{
    // A single sequence splits evenly: about one workgroup per CU (256), each
    // streaming an equal run, is fastest (measured at 32k and 128k keys).  A
    // ragged batch needs finer splits: its workgroups have unequal work and
    // their count is quantised by the resident slots (512 at d <= 128), so a
    // split size that leaves a nearly empty last round costs a whole round
    // (64 sequences of 1k..32k keys: 4.5 TB/s at 2048 workgroups, 5.9 at
    // 3072).  A split is a multiple of 128 keys (one 32-key block per wave);
    // longer contexts with few kv heads get splits down to 128 keys so they
    // still spread over many CUs; short ones are not split at all.
    const uint64_t target_wg = plan_target_wg(n_seq), min_sk = plan_min_split();
    const uint64_t work = total_len * (uint64_t)n_kv;
    uint64_t sk = (work + target_wg - 1) / target_wg;
    if (sk < min_sk) sk = min_sk;
    if (sk < (max_len + kMaxSplits - 1) / kMaxSplits) sk = ((uint64_t)max_len + kMaxSplits - 1) / kMaxSplits;
    sk = (sk + 127) / 128 * 128;
    uint32_t ns;
    if (sk >= max_len || (uint64_t)max_len * D * 4 <= plan_one_split_bytes()) {
        sk = ((uint64_t)max_len + 31) / 32 * 32;
        if (sk < 32) sk = 32;
        ns = 1;
    } else {
        ns = (uint32_t)((max_len + sk - 1) / sk);
    }
    *split_keys = (uint32_t)sk;
    *n_splits = ns;
    return partial_bytes(n_seq, ns, n_heads, n_kv, D);
}

size_t decode_workspace_bound(uint32_t n_seq, uint32_t max_len, uint64_t total_len, uint32_t n_heads,
                              uint32_t n_kv, uint32_t D)
{
    uint32_t sk, ns;
    const size_t exact = decode_plan(n_seq, max_len, total_len, n_heads, n_kv, D, &sk, &ns);
    if (n_seq != 1) return exact;
    // Every single-sequence call with len <= max_len: the split size is at
    // least len*n_kv/target, at least the minimum split and at least
    // len/kMaxSplits, so the split count is at most the smallest of
    // target/n_kv, max_len/min split and kMaxSplits (rounded up).  The count
    // itself is not monotone in len (the split size is rounded up to 128
    // keys), so a workspace sized for max_len alone can be too small for a
    // shorter call.
    const uint64_t target_wg = plan_target_wg(1), min_sk = plan_min_split();
    uint64_t nsb = (target_wg + n_kv - 1) / n_kv;
    const uint64_t by_len = ((uint64_t)max_len + min_sk - 1) / min_sk;
    if (by_len < nsb) nsb = by_len;
    if (nsb > kMaxSplits) nsb = kMaxSplits;
    const size_t bound = partial_bytes(1, (uint32_t)nsb, n_heads, n_kv, D);
    return bound > exact ? bound : exact;
}

void decode_bind_workspace(DecodeArgs& a, void* workspace)
{
    a.gmax = (a.n_heads + a.n_kv - 1) / a.n_kv;
    if (a.n_splits == 1 || !workspace) {
        a.part_ml = a.part_o = nullptr;
        return;
    }
    const size_t groups = (size_t)a.n_seq * a.n_kv;
    char* p = reinterpret_cast<char*>(workspace);
    a.part_ml = reinterpret_cast<float*>(p);
    p += align256(groups * a.n_splits * a.gmax * 2 * sizeof(float));
    a.part_o = reinterpret_cast<float*>(p);
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t st)
{
    const DecodeRope none{};
    switch (a.D) {
    case 64: return launch_decode_d<64, false>(a, none, st);
    case 128: return launch_decode_d<128, false>(a, none, st);
    case 256: return launch_decode_d<256, false>(a, none, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode_rope(const DecodeArgs& a, const DecodeRope& r, hipStream_t st)
{
    if (a.n_seq != 1 || a.lens || a.len0 == 0) return hipErrorInvalidValue;
    switch (a.D) {
    case 64: return launch_decode_d<64, true>(a, r, st);
    case 128: return launch_decode_d<128, true>(a, r, st);
    case 256: return launch_decode_d<256, true>(a, r, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace yhip
