// attn_prefill.hip -- causal grouped-query attention for a batch of prompt
// tokens on gfx950 MFMA.
//
// Semantics: engine.c:532-563 (token b at position pos_start+b attends to
// keys 0..pos_start+b; scores scaled by 1/sqrt(d); softmax; weighted V),
// with the optional qwen35 sigmoid gate (engine.c:959-960).
//
// Tiling.  A workgroup owns 128 consecutive queries of one query head; each
// of its 4-wave key groups (one or two, see prefill_groups) gives wave w 32
// of them.  Keys stream through LDS in tiles of 64 (K rows [64][D] and V^T
// [D][64], straight from the cache layout), loaded with buffer
// instructions into registers -- K two tiles ahead, V one -- and stored to
// padded LDS rows.  With two groups, group g takes tiles g, g+2, ... and
// the partial (max, sum, O) of the groups merge through LDS at the end.
// Workgroups are issued heaviest (latest queries) first so the causal
// triangle drains evenly.
//
// MFMA formulation (v_mfma_f32_32x32x16_f16), everything transposed so that a
// lane owns one query for the whole kernel:
//   S^T[key][q] = K[key][:] . Q^T[:][q]        A = K tile (LDS), B = Q (regs)
//   O^T[d][q]  += V^T[d][key] . P^T[key][q]    A = V^T tile (LDS), B = P (regs)
// Softmax statistics of a query are in one lane pair (l, l+32): row max over
// a tile is 31 in-lane maxes and one exchange, the running sum is per lane
// until the end.  K rows are written to LDS with rows 4..7 and 8..11 of every
// 16 swapped, which turns the 32x32 accumulator layout (rows 8(i/4)+4(l/32)+
// i%4) into contiguous key runs 8(l/32)+i: the score registers are then
// exactly the k-slots of the P^T operand and P stays in registers.
// Scores use exp2 with log2(e)/sqrt(d) folded into one multiply.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>
#include <stdlib.h>

namespace yhip {
namespace {

constexpr int BM = 128;  // queries per workgroup
constexpr int BN = 64;   // keys per tile

__device__ inline f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ inline float sigmoid_ref(float g) { return 1.0f / (1.0f + expf(-g)); }

// key row r of a tile lives in LDS row perm(r): rows 4..7 <-> 8..11 of each 16
__device__ inline int lds_row_of_key(int r)
{
    return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

// key (within a 32-key half) of accumulator element i for lane half hh
__device__ inline int key_of_acc(int i, int hh) { return i < 8 ? 8 * hh + i : 16 + 8 * hh + (i - 8); }

__device__ inline void load_q8(f16x8& dst, const void* q, size_t off, uint32_t dt)
{
    if (dt == kF32) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(q) + off);
        const f32x4 b = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(q) + off + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dst[j] = (_Float16)a[j];
            dst[j + 4] = (_Float16)b[j];
        }
    } else if (dt == kF16) {
        dst = *reinterpret_cast<const f16x8*>(reinterpret_cast<const uint16_t*>(q) + off);
    } else {
        const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(q) + off);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dst[2 * j] = (_Float16)__builtin_bit_cast(float, w[j] << 16);
            dst[2 * j + 1] = (_Float16)__builtin_bit_cast(float, w[j] & 0xffff0000u);
        }
    }
}

__device__ inline void store_out4(void* out, size_t off, uint32_t dt, f32x4 v)
{
    if (dt == kF32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + off) = v;
    } else if (dt == kF16) {
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        f16x4 h;
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = (_Float16)v[j];
        *reinterpret_cast<f16x4*>(reinterpret_cast<uint16_t*>(out) + off) = h;
    } else {
        // round to nearest even; each element goes through a scalar float
        // (bit-casting an ext-vector element directly reads element 0)
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float f = v[j];
            const uint32_t x = __builtin_bit_cast(uint32_t, f);
            h[j] = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
        }
        u32x2 w;
        w[0] = h[0] | (h[1] << 16);
        w[1] = h[2] | (h[3] << 16);
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(out) + off) = w;
    }
}

template <int D, int NG>
__global__ __launch_bounds__(256 * NG, (NG == 1 && D <= 128) ? 2 : 1) void prefill_kernel(PrefillArgs a)
{
    constexpr int KS = D + 8;     // K tile row stride (halfs), 16 B pad
    constexpr int VS = BN + 8;    // V tile row stride (halfs)
    constexpr int NKK = D / 16;   // k-chunks of the score MFMA
    constexpr int NDB = D / 32;   // d-blocks of the output MFMA
    constexpr int CH = D / 32;    // 16-byte chunks per thread per tile (K and V each)
    constexpr int KCH = D / 8;    // 16-byte chunks per K row
    constexpr float kSlack = 8.0f;
    // NG key groups of 4 waves share the workgroup's 128 queries: group g
    // walks key tiles g, g+NG, g+2NG, ... with its own LDS buffers, and the
    // groups' partial results are merged at the end, so the longest chain
    // of dependent tiles a wave walks is 1/NG of the causal row.  Within a
    // group K is staged two of its tiles ahead (the score MFMAs of its next
    // tile run during the softmax of the current one) and V one tile ahead,
    // each double buffered; every buffer is rewritten only after the
    // barrier that ends its last reader's step, so one barrier per step
    // suffices (plus one in the first step, after the prologue's scores).
    __shared__ _Float16 Kl[2][NG][BN * KS];
    __shared__ _Float16 Vl[2][NG][D * VS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int grp = tid >> 8, gtid = tid & 255, wave = gtid >> 6;
    const int r32 = lane & 31, hh = lane >> 5;

    const uint32_t nqb = (a.B + BM - 1) / BM;
    uint32_t qb, h;
    if (a.xcd_map) {
        // Consecutive workgroups go to the 8 XCDs in turn.  XCD x serves kv
        // head x % n_kv, so the query heads that read one kv head share an
        // L2 and its K/V tiles are fetched from HBM once per XCD group, not
        // once per XCD; within an XCD the order stays heaviest first.
        const uint32_t x = blockIdx.x % 8u, slot = blockIdx.x / 8u;
        const uint32_t per = 8u / a.n_kv, G = a.n_heads / a.n_kv;
        const uint32_t g = x % a.n_kv, i = slot * per + x / a.n_kv;
        qb = nqb - 1 - i / G;
        h = g * G + i % G;
    } else {
        qb = nqb - 1 - blockIdx.x / a.n_heads;
        h = blockIdx.x % a.n_heads;
    }
    const uint32_t kvh = h * a.n_kv / a.n_heads;  // engine.c:537

    const uint32_t qi0 = qb * BM;
    const uint32_t qlast = min(a.B, qi0 + BM) - 1;
    const uint32_t kmax = a.pos_start + qlast;  // last key any query here reads
    const uint32_t ntiles = kmax / BN + 1;
    const uint32_t nsteps = (ntiles + NG - 1) / NG;  // loop steps (workgroup-uniform)
    // this group's tiles: kt = grp + NG*st for st < gsteps
    const uint32_t gsteps = ntiles > (uint32_t)grp ? (ntiles - grp + NG - 1) / NG : 0;

    const uint32_t wq0 = qi0 + wave * 32;
    const bool wave_active = wq0 < a.B;
    const uint32_t wpos_first = a.pos_start + wq0;
    const uint32_t wpos_last = a.pos_start + min(wq0 + 31, a.B - 1);
    const uint32_t my_pos = a.pos_start + wq0 + r32;
    const uint32_t my_q = min(wq0 + r32, a.B - 1);
    // tiles this wave computes: 0 .. wtiles-1, of which this group's are st < wsteps
    const uint32_t wtiles = wave_active ? wpos_last / BN + 1 : 0;
    const uint32_t wsteps = wtiles > (uint32_t)grp ? (wtiles - grp + NG - 1) / NG : 0;
    auto tile_of = [&](uint32_t st) { return (uint32_t)grp + NG * st; };

    f16x8 qf[NKK];
    {
        const size_t base = (size_t)my_q * a.q_stride + (size_t)h * D + hh * 8;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) load_q8(qf[kk], a.q, base + kk * 16, a.q_dtype);
        // Complete the query loads here.  Their first reader is the first
        // score MFMA inside the key loop, whose tile loads are conditional;
        // left pending, the wait the compiler places before that MFMA cannot
        // count the tile loads and becomes a full vmcnt(0) on every step,
        // exposing the next tile's global latency each time.
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    }

    // Buffer resources over this kv head's K rows and V tiles (reads past the
    // cache return zeros).  Per-thread offsets are fixed; a tile adds the
    // scalar kt*BN*D*2 bytes (the same for K rows and 32-position V tiles).
    const uint32_t head_bytes = a.kv_stride * D * 2;
    const __amdgpu_buffer_rsrc_t rK = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kc + k_index(kvh, 0, 0, D, a.kv_stride)), 0, head_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rV = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.vc + v_index(kvh, 0, 0, D, a.kv_stride)), 0, head_bytes, 0x00020000);
    int kgo[CH], klo[CH], vlo[CH], vkey[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = gtid + 256 * i;
        const int row = c / KCH, col = c % KCH;
        kgo[i] = (row * D + col * 8) * 2;
        klo[i] = lds_row_of_key(row) * KS + col * 8;
        // V chunk c: 32-position tile c/(4D), row d, 8 positions
        const int t = c / (4 * D), r = c % (4 * D);
        vkey[i] = t * (int)kVTile + (r & 3) * 8;  // key of the chunk within the 64-key tile
        vlo[i] = (r >> 2) * VS + vkey[i];
    }
    u32x4 kreg[CH], vreg[CH];
    auto load_k = [&](uint32_t st) {
        const uint32_t off = tile_of(st) * BN * D * 2;
#pragma unroll
        for (int i = 0; i < CH; ++i)
            kreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rK, kgo[i], off, 0));
    };
    auto load_v = [&](uint32_t st) {
        const uint32_t off = tile_of(st) * BN * D * 2;
#pragma unroll
        for (int i = 0; i < CH; ++i)
            vreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rV, gtid * 16 + i * 4096, off, 0));
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CH; ++i) *reinterpret_cast<u32x4*>(&Kl[buf][grp][klo[i]]) = kreg[i];
    };
    auto store_v = [&](int buf, uint32_t st) {
        const uint32_t k0 = tile_of(st) * BN;
        const bool tail = k0 + BN - 1 > kmax;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            u32x4 v = vreg[i];
            if (tail) {
                // keys past kmax were never stored: their P is 0, their V must be finite
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t key = k0 + vkey[i] + 2 * e;
                    if (key > kmax) v[e] = 0u;
                    else if (key + 1 > kmax) v[e] &= 0xffffu;
                }
            }
            *reinterpret_cast<u32x4*>(&Vl[buf][grp][vlo[i]]) = v;
        }
    };

    // running max (log2 domain): finite so that a tile whose keys are all in
    // the lane's future (possible as a group's first tile) leaves l and O at
    // zero instead of forming -inf - -inf
    float m = -1e30f, l = 0.0f;
    f32x16 o[NDB];
#pragma unroll
    for (int b = 0; b < NDB; ++b)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[b][i] = 0.0f;

    // scores of step st's tile into S (both 32-key halves)
    auto qk = [&](f32x16 (&S)[2], uint32_t st) {
        const _Float16* kr = &Kl[st & 1][grp][r32 * KS + hh * 8];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const f16x8 kf = *reinterpret_cast<const f16x8*>(kr + 32 * j * KS + kk * 16);
                S[j] = kk == 0 ? mfma32(kf, qf[0], f32x16{}) : mfma32(kf, qf[kk], S[j]);
            }
    };
    // running max update of the lane's query from tile scores S (raw, masked)
    auto update_max = [&](const f32x16 (&S)[2]) {
        float mx = S[0][0];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, S[j][i]);
        mx = wave_max_xor(mx, 32) * a.c;
        if (__ballot(mx > m + kSlack)) {  // wave-uniform: some query's max moved
            const float mn = mx > m + kSlack ? mx : m;
            const float alpha = fast_exp2(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int b = 0; b < NDB; ++b) o[b] *= alpha;
        }
    };
    auto probs = [&](const f32x16 (&S)[2], f16x8 (&pf)[4]) {
        const float nm = -m;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float p = fast_exp2(fmaf(S[i >> 4][i & 15], a.c, nm));
            l += p;
            pf[i >> 3][i & 7] = (_Float16)p;
        }
    };
    auto pv = [&](const f16x8 (&pf)[4], uint32_t st) {
        const _Float16* vr = &Vl[st & 1][grp][r32 * VS + hh * 8];
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
            for (int b = 0; b < NDB; ++b)  // independent accumulators back to back
                o[b] = mfma32(*reinterpret_cast<const f16x8*>(vr + b * 32 * VS + kc * 16), pf[kc], o[b]);
    };
    // scores of step st's tile into Snext while the probabilities of Scur are
    // formed: each score MFMA is followed by the exp2 work it can hide
    auto qk_probs = [&](f32x16 (&Snext)[2], uint32_t st, const f32x16 (&Scur)[2], f16x8 (&pf)[4]) {
        constexpr int PPM = 32 / (2 * NKK);  // probabilities per MFMA
        const _Float16* kr = &Kl[st & 1][grp][r32 * KS + hh * 8];
        const float nm = -m;
        // MFMA n = kk*2 + j (halves alternate, so neighbours are independent);
        // its K fragment is read one MFMA ahead
        f16x8 kf = *reinterpret_cast<const f16x8*>(kr);
#pragma unroll
        for (int n = 0; n < 2 * NKK; ++n) {
            const int kk = n >> 1, j = n & 1;
            f16x8 kn = kf;
            if (n + 1 < 2 * NKK) {
                const int kk1 = (n + 1) >> 1, j1 = (n + 1) & 1;
                kn = *reinterpret_cast<const f16x8*>(kr + 32 * j1 * KS + kk1 * 16);
            }
            Snext[j] = kk == 0 ? mfma32(kf, qf[0], f32x16{}) : mfma32(kf, qf[kk], Snext[j]);
#pragma unroll
            for (int u = 0; u < PPM; ++u) {
                const int i = n * PPM + u;
                const float p = fast_exp2(fmaf(Scur[i >> 4][i & 15], a.c, nm));
                l += p;
                pf[i >> 3][i & 7] = (_Float16)p;
            }
            kf = kn;
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);        // next fragment's LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // this MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4 * PPM, 0);  // softmax work it hides
        }
    };
    // a tile that reaches past the wave's first query: keys beyond the
    // lane's position get -inf
    auto mask = [&](f32x16 (&S)[2], uint32_t st) {
        const uint32_t k0 = tile_of(st) * BN;
        if (k0 + BN - 1 > wpos_first) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (k0 + 32 * j + key_of_acc(i, hh) > my_pos) S[j][i] = -INFINITY;
        }
    };

    // prologue: the group's first K, V and second K in LDS; scores of step 0
    if (gsteps > 0) {
        load_k(0);
        load_v(0);
        store_k(0);
        store_v(0, 0);
    }
    if (gsteps > 1) {
        load_k(1);
        store_k(1);
    }
    __syncthreads();
    f32x16 Sa[2], Sb[2];
    if (wsteps > 0) qk(Sa, 0);

    // step st: loads K(st+2), V(st+1); scores of st+1 overlap the softmax of
    // st; P.V of st; stores K(st+2) over K(st) and V(st+1) over V(st-1); one
    // barrier.  With pos_start not a multiple of 32 a wave's queries straddle
    // a tile boundary, so a tile with a successor may still need the mask.
    auto step = [&](uint32_t st, f32x16 (&Scur)[2], f32x16 (&Snext)[2]) {
        if (st + 2 < gsteps) load_k(st + 2);
        if (st + 1 < gsteps) load_v(st + 1);
        if (st + 1 < wsteps) {
            mask(Scur, st);
            update_max(Scur);
            f16x8 pf[4];
            qk_probs(Snext, st + 1, Scur, pf);
            pv(pf, st);
        } else if (st < wsteps) {
            mask(Scur, st);
            update_max(Scur);
            f16x8 pf[4];
            probs(Scur, pf);
            pv(pf, st);
        }
        // K(0)'s last reader is the prologue's score pass, which no barrier
        // separates from the first store over it
        if (st == 0) __syncthreads();
        if (st + 2 < gsteps) store_k(st & 1);
        if (st + 1 < gsteps) store_v((st + 1) & 1, st + 1);
        __syncthreads();
    };
    for (uint32_t st = 0; st < nsteps; st += 2) {
        step(st, Sa, Sb);
        if (st + 1 < nsteps) step(st + 1, Sb, Sa);
    }

    l += __shfl_xor(l, 32, 64);
    if (NG > 1) {
        // groups 1..NG-1 hand (m, l, O) to group 0 through LDS; the tile
        // buffers are free after the last step's barrier
        constexpr int NV = NDB * 16 + 2;  // floats per lane
        static_assert(NV * 256 * 4 * (NG - 1) <= (int)sizeof(Kl), "merge area");
        float* xo = reinterpret_cast<float*>(&Kl[0][0][0]) + (size_t)(grp > 0 ? grp - 1 : 0) * NV * 256;
        if (grp > 0) {
            xo[gtid] = m;
            xo[256 + gtid] = l;
#pragma unroll
            for (int b = 0; b < NDB; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) xo[(2 + b * 16 + i) * 256 + gtid] = o[b][i];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < NG; ++g) {
            const float* xi = reinterpret_cast<const float*>(&Kl[0][0][0]) + (size_t)(g - 1) * NV * 256;
            const float m1 = xi[gtid], l1 = xi[256 + gtid];
            const float mg = fmaxf(m, m1);
            const float a0 = fast_exp2(m - mg), a1 = fast_exp2(m1 - mg);
            m = mg;
            l = l * a0 + l1 * a1;
#pragma unroll
            for (int b = 0; b < NDB; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[b][i] = o[b][i] * a0 + xi[(2 + b * 16 + i) * 256 + gtid] * a1;
        }
    }
    if (!wave_active) return;
    const uint32_t qi = wq0 + r32;
    if (qi >= a.B) return;
    const float inv = 1.0f / l;
#pragma unroll
    for (int b = 0; b < NDB; ++b) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const uint32_t d = b * 32 + 8 * i4 + 4 * hh;
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[b][4 * i4 + e] * inv;
            if (a.gate) {
                const float* gp = a.gate + (size_t)qi * a.gate_stride + (size_t)h * D + d;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] *= sigmoid_ref(gp[e]);
            }
            store_out4(a.out, (size_t)qi * a.out_stride + (size_t)h * D + d, a.out_dtype, v);
        }
    }
}

template <int D, int NG>
hipError_t launch_prefill_d(PrefillArgs a, hipStream_t st)
{
    // the XCD mapping needs whole kv groups per XCD group and an equal share
    // per XCD (measured 470 -> 478 TFLOP/s at 2048 tokens x 28 heads)
    static const int env = [] {
        const char* e = getenv("YHIP_PREFILL_XCD");
        return e ? atoi(e) : 1;
    }();
    const uint32_t nqb0 = (a.B + BM - 1) / BM;
    a.xcd_map = env != 0 && a.n_kv <= 8 && 8 % a.n_kv == 0 && a.n_heads % a.n_kv == 0 &&
                ((uint64_t)nqb0 * (a.n_heads / a.n_kv)) % (8 / a.n_kv) == 0;
    const uint32_t nqb = (a.B + BM - 1) / BM;
    hipLaunchKernelGGL((prefill_kernel<D, NG>), dim3(nqb * a.n_heads), dim3(256 * NG), 0, st, a);
    return hipGetLastError();
}

// Key groups per workgroup.  Two groups halve the longest chain of tiles a
// wave walks, which is what bounds a grid that fills the machine only once
// (2048 tokens x 28 heads: 448 workgroups on 256 CUs, 420 -> 479 TFLOP/s);
// with many workgroups per CU two independent 4-wave workgroups hide latency
// better than one 8-wave workgroup under one barrier (8192 tokens: 888 vs
// 790 TFLOP/s).  Two groups need the LDS of two groups' tiles (head_dim <=
// 128).  YHIP_PREFILL_NG=1/2 forces the choice for comparisons.
int prefill_groups(const PrefillArgs& a)
{
    static const int env = [] {
        const char* e = getenv("YHIP_PREFILL_NG");
        return e ? atoi(e) : 0;
    }();
    static const int n_cu = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    if (a.D > 128) return 1;
    if (env == 1 || env == 2) return env;
    const uint64_t wgs = (uint64_t)((a.B + BM - 1) / BM) * a.n_heads;
    return wgs <= 2 * (uint64_t)n_cu ? 2 : 1;
}

}  // namespace

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t st)
{
    const int ng = prefill_groups(a);
    switch (a.D) {
    case 64: return ng == 2 ? launch_prefill_d<64, 2>(a, st) : launch_prefill_d<64, 1>(a, st);
    case 128: return ng == 2 ? launch_prefill_d<128, 2>(a, st) : launch_prefill_d<128, 1>(a, st);
    case 256: return launch_prefill_d<256, 1>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace yhip
