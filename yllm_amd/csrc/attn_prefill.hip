// attn_prefill.hip -- causal grouped-query attention for a batch of prompt
// tokens on gfx950 MFMA.
//
// Semantics: engine.c:532-563 (token b at position pos_start+b attends to
// keys 0..pos_start+b; scores scaled by 1/sqrt(d); softmax; weighted V),
// with the optional qwen35 sigmoid gate (engine.c:959-960).
//
// Tiling.  A work item is 128 consecutive queries of one query head; each
// of the workgroup's 4-wave key groups (one or two, see prefill_groups)
// gives wave w 32 of them.  Keys stream through LDS in tiles of 64 (K rows
// [64][D] and V^T [D][64], straight from the cache layout), loaded from HBM
// directly into LDS -- K two tiles ahead, V one -- as unpadded rows with
// XOR-swizzled 16-byte chunks.  With two groups, group g takes tiles g,
// g+2, ... and the partial (max, sum, O) of the groups merge through LDS at
// the end.  Items are taken heaviest (latest queries) first so the causal
// triangle drains evenly; with one 8-wave workgroup per CU the grid is the
// resident workgroups, each walking its items in snake order with the next
// item's first loads issued during the current item's last key step.
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
// Keys per tile: 64 up to head_dim 128; 32 at 256, so that a workgroup's
// double-buffered K and V tiles take 64 KB of LDS and two workgroups (two
// waves per SIMD) fit on a CU.
__host__ __device__ constexpr int bn_of(int D) { return D > 128 ? 32 : 64; }

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

// fp32 query elements off..off+7 as f16 hi + lo parts: hi = f16(x), lo =
// f16(x - hi), so hi + lo carries ~22 bits of x and K.hi + K.lo (two MFMAs
// into one fp32 accumulator) keeps the score at fp32-level error
__device__ inline void load_q8_split(f16x8& hi, f16x8& lo, const float* q, size_t off)
{
    const f32x4 a = *reinterpret_cast<const f32x4*>(q + off);
    const f32x4 b = *reinterpret_cast<const f32x4*>(q + off + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hi[j] = (_Float16)a[j];
        lo[j] = (_Float16)(a[j] - (float)hi[j]);
        hi[j + 4] = (_Float16)b[j];
        lo[j + 4] = (_Float16)(b[j] - (float)hi[j + 4]);
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

// One 16-byte HBM -> LDS load per lane: lane i writes at lds + 16 i.  A
// __device__ function, not a lambda: lambdas in a kernel are host-device, and
// the host compilation pass silently drops a kernel whose lambdas call this
// gfx950-only builtin.
__device__ inline void lds_load16(__amdgpu_buffer_rsrc_t r, _Float16* lds, int voff, uint32_t soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// 16-byte chunk swizzle of an LDS tile row (XOR into the chunk index).  For
// rows of 8 chunks (128 B) the swizzle is (r & 7) ^ bit 3 of r: 8 consecutive
// rows then hit 8 distinct chunk columns (32-bank LDS, b128 reads in groups
// of 8 lanes) and 16 consecutive rows give each half of a 256-byte bank
// window 8 distinct columns (64 banks, groups of 16 lanes).  Rows of 4
// chunks (64 B, the V^T rows of 32-key tiles) take (bit 1 ^ bit 3, bit 2):
// a bijection of bits 1, 2 for the four rows of one parity among 8 (32
// banks) and of bits 2, 3 for the four rows r, r+4, r+8, r+12 that share a
// 256-byte window (64 banks).  Rows of 16 or more chunks (256 B and up) use
// r & 15.  All depend on bits 0..3 of the row only, so rows 32 apart share
// the swizzle.
template <int NCH>
__device__ inline int chunk_swz(int r)
{
    if constexpr (NCH >= 16) return r & 15;
    else if constexpr (NCH == 8) return (r & 7) ^ ((r >> 3) & 1);
    else return (((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2);
}

// Schedule of one key step's MFMAs: NQ score MFMAs of the next tile and NPV
// P.V MFMAs of this tile (k-slot kc = n / NDB of NKC uses the probabilities
// 8 kc .. 8 kc + 7), with the tile's 8 NKC probabilities spread over them.
// The exp2 of a probability is quarter rate (about as long as half a
// 32x32x16 MFMA with its fma, add and convert), so one to two per MFMA hide
// under the matrix pipe, where 32 under the score MFMAs alone or under the
// PV MFMAs alone would not.  Slot order: the first NQ/2 score MFMAs under
// k-slot 0's probabilities; then for kc = 0..NKC-1 k-slot kc's PV MFMAs
// interleaved with the next score MFMAs under k-slot kc+1's probabilities.
struct FSlot {
    int8_t pv;  // 0: score MFMA n, 1: PV MFMA n
    int8_t n;
    int8_t p0;  // probabilities p0 .. p0+np-1 formed after this MFMA
    int8_t np;
};
template <int NQ, int NPV, int NDB, int NKC>
struct FusedSchedule {
    static_assert(NPV == NKC * NDB && NKC >= 2, "k-slots of 16 keys");
    static constexpr int N = NQ + NPV;
    FSlot s[N];
    constexpr FusedSchedule() : s{}
    {
        const int QA = NQ / 2, QB = (NQ - QA + NKC - 2) / (NKC - 1);
        int k = 0, q = 0, v = 0;
        for (int t = 0; t < QA; ++t)
            s[k++] = FSlot{0, (int8_t)q++, (int8_t)(t * 8 / QA), (int8_t)((t + 1) * 8 / QA - t * 8 / QA)};
        for (int kc = 0; kc < NKC; ++kc) {
            const bool more = kc < NKC - 1;
            const int nq = more ? (QB < NQ - q ? QB : NQ - q) : NQ - q;
            const int tot = NDB + nq;
            for (int t = 0; t < tot; ++t) {
                const bool is_pv = (t + 1) * NDB / tot > t * NDB / tot;
                const int p0 = more ? 8 * (kc + 1) + t * 8 / tot : 0;
                const int np = more ? (t + 1) * 8 / tot - t * 8 / tot : 0;
                s[k++] = FSlot{(int8_t)is_pv, (int8_t)(is_pv ? v++ : q++), (int8_t)p0, (int8_t)np};
            }
        }
    }
};

// first query head of kv head g: heads h with h*n_kv/n_heads == g are
// [head0(g), head0(g+1)) (engine.c:537)
__device__ inline uint32_t head0(const PrefillArgs& a, uint32_t g) { return (g * a.n_heads + a.n_kv - 1) / a.n_kv; }

// A work item: query block qb (plain rows) or row block qb (packed rows) of
// kv head kvh, key split `split`; h is the query head of plain rows.
struct PItem {
    uint32_t qb, h, kvh, split;
};

// Row r (0..127) of an item -> query index b and head; valid is false for
// rows past the item's end (their loads are clamped to the last row).
struct PRow {
    uint32_t b, h;
    bool valid;
};
template <bool SPLIT>
__device__ inline PRow row_of(const PrefillArgs& a, const PItem& I, uint32_t r)
{
    if (!(SPLIT && a.pack)) {
        const uint32_t q = I.qb * BM + r;
        return PRow{min(q, a.B - 1), I.h, q < a.B};
    }
    const uint32_t h0 = head0(a, I.kvh), nrows = (head0(a, I.kvh + 1) - h0) * a.B;
    const uint32_t rr = I.qb * BM + r, rc = min(rr, nrows - 1);
    return PRow{rc % a.B, h0 + rc / a.B, rr < nrows};
}

// The query indices a wave's 32 rows span (wave-uniform): [first, last].
template <bool SPLIT>
__device__ inline bool wave_span(const PrefillArgs& a, const PItem& I, int wave, uint32_t& first, uint32_t& last)
{
    if (!(SPLIT && a.pack)) {
        const uint32_t q0 = I.qb * BM + wave * 32;
        first = q0;
        last = min(q0 + 31, a.B - 1);
        return q0 < a.B;
    }
    const uint32_t nrows = (head0(a, I.kvh + 1) - head0(a, I.kvh)) * a.B;
    const uint32_t r0 = I.qb * BM + wave * 32, rl = min(r0 + 31, nrows - 1);
    if (r0 / a.B == rl / a.B) {
        first = r0 % a.B;
        last = rl % a.B;
    } else {  // the rows cross into the next head: its first queries, the previous head's last
        first = 0;
        last = a.B - 1;
    }
    return r0 < nrows;
}

// Key tiles of an item: [t0, t0 + nt).  The item's last key is kmax (its
// last query's position; with packed rows (B < 128) every item holds some
// head's query B-1).
template <int BN, bool SPLIT>
__device__ inline void item_keys(const PrefillArgs& a, const PItem& I, uint32_t& kmax, uint32_t& t0, uint32_t& nt)
{
    kmax = a.pos_start + ((SPLIT && a.pack) ? a.B - 1 : min(a.B, I.qb * BM + BM) - 1);
    const uint32_t all = kmax / BN + 1;
    if (SPLIT) {
        t0 = I.split * a.split_tiles;
        const uint32_t t1 = min(all, t0 + a.split_tiles);
        nt = t1 > t0 ? t1 - t0 : 0;
    } else {
        t0 = 0;
        nt = all;
    }
}

// SPLIT: the split mode (one item per workgroup, packed rows, a key range
// per split); a separate instantiation keeps the plain mode's registers.
// QS: fp32 queries as f16 hi + lo parts, two score MFMAs per k-chunk (32 more
// registers per lane at d = 128: one workgroup of 4 waves per CU, one key
// group).
template <int D, int NG, bool SPLIT, bool QS = false>
__global__ __launch_bounds__(256 * NG * (D > 128 ? 2 : 1), (NG == 1 && D <= 128 && !QS) ? 2 : 1) void prefill_kernel(
    PrefillArgs a)
{
    static_assert(NG == 1 || NG == 2, "one or two key groups");
    static_assert(!SPLIT || NG == 1, "the split mode runs one key group");
    static_assert(!QS || NG == 1, "split queries run one key group");
    // Pair mode (head_dim 256): a wave's 32 queries with all 256 dimensions
    // need 64 registers of Q and 128 of O, which leaves one wave per SIMD.
    // Instead two waves share 32 queries and each owns half the dimensions
    // of Q and O; each forms the scores over its half, the halves meet
    // through LDS at the step barrier (the sum is formed in the same order by
    // both waves, so both hold the same scores, maximum and probabilities),
    // and each accumulates its half of O.  The workgroup is 8 waves over the
    // same 128 queries, one per CU, two waves per SIMD.
    constexpr bool PAIR = D > 128;
    static_assert(!PAIR || NG == 1, "pair mode runs one key group");
    constexpr int LT = PAIR ? 512 : 256;  // threads of a key group (they share the tile loads)
    constexpr int DQ = PAIR ? D / 2 : D;  // dimensions of Q and O a wave holds
    constexpr int BN = bn_of(D);  // keys per tile
    constexpr int NS = BN / 32;   // 32-key halves of a tile (score accumulators)
    constexpr int NKC = BN / 16;  // k-slots of the output MFMA per tile
    constexpr int NKK = DQ / 16;  // k-chunks of the score MFMA
    constexpr int NDB = DQ / 32;  // d-blocks of the output MFMA
    constexpr int CH = BN * D / (8 * LT);  // 16-byte chunks per thread per tile (K and V each)
    constexpr int KCH = D / 8;    // 16-byte chunks per K row
    constexpr int VCH = BN / 8;   // 16-byte chunks per V row
    constexpr float kSlack = 8.0f;
    // NG key groups of 4 waves share the workgroup's 128 queries: group g
    // walks key tiles g, g+NG, g+2NG, ... with its own LDS buffers, and the
    // groups' partial results are merged at the end, so the longest chain
    // of dependent tiles a wave walks is 1/NG of the causal row.
    //
    // Tiles go from HBM straight into LDS (buffer loads with the LDS
    // destination; lane i of a load writes 16 bytes at base + 16 i), K rows
    // [64][D] and V^T rows [D][64], unpadded with swizzled 16-byte chunks.
    // Within a group K is loaded two of its tiles ahead (the score MFMAs of
    // its next tile run during the softmax of the current one) and V one
    // tile ahead, each double buffered.  Buffers of parity 0 and 1 are
    // separate variables, so the compiler can see that a step's loads in
    // flight (into one parity) never alias its LDS reads (of the other) and
    // does not wait for them; each thread waits for its own loads before the
    // barrier that ends the step.
    //
    // Pair mode keeps three buffers of each (K three tiles ahead, V two), so
    // that every tile load has two steps to land: its steps are short (16
    // MFMAs per wave) and all eight waves meet at each step's barrier.
    constexpr int NB = PAIR ? 3 : 2;  // K buffers and V buffers
    __shared__ __attribute__((aligned(16))) _Float16 Kl0[NG][BN * D];
    __shared__ __attribute__((aligned(16))) _Float16 Kl1[NG][BN * D];
    __shared__ __attribute__((aligned(16))) _Float16 Kl2[NB > 2 ? BN * D : 8];
    __shared__ __attribute__((aligned(16))) _Float16 Vl0[NG][D * BN];
    __shared__ __attribute__((aligned(16))) _Float16 Vl1[NG][D * BN];
    __shared__ __attribute__((aligned(16))) _Float16 Vl2[NB > 2 ? D * BN : 8];
    // Pair mode: each wave's partial scores of a tile, by tile parity, as
    // [parity][wave][float4 j][lane] (consecutive lanes, consecutive 16
    // bytes).  Two key groups: (max, sum) of group 1's queries for the merge.
    // (One array: pair mode fills the 160 KB of LDS exactly.)
    __shared__ f32x4 Xl[PAIR ? 2 * 8 * 4 * NS * 64 : NG > 1 ? 128 : 1];
    float* const s_ml = reinterpret_cast<float*>(&Xl[0]);

    // Items (query block, head) in heaviest-first order are dealt to the
    // resident workgroups in snake order (item slot it*W + j on even rounds,
    // it*W + W-1-j on odd ones), which balances the causal triangle's
    // linearly decreasing costs; the grid is one item per workgroup when
    // there are no more items than resident slots.
    const uint32_t nqb = (a.B + BM - 1) / BM;
    // item `it` of this workgroup; false past the last
    auto item_of = [&](uint32_t it, PItem& I) -> bool {
        if (SPLIT) {
            // one item per workgroup.  The items of a (kv head, split) tile
            // group read the same K/V tiles: XCD x serves tile groups x, x+8,
            // ... (consecutive workgroups go to the 8 XCDs in turn), so they
            // share its L2.
            if (it > 0) return false;
            const uint32_t x = blockIdx.x % 8u, j = blockIdx.x / 8u;
            const uint32_t ipg = a.n_rb * (a.pack ? 1u : a.gmax);
            const uint32_t tg = (j / ipg) * 8u + x, w = j % ipg;
            if (tg >= a.n_kv * a.n_split) return false;
            I.kvh = tg % a.n_kv;
            I.split = tg / a.n_kv;
            const uint32_t h0 = head0(a, I.kvh), h1 = head0(a, I.kvh + 1);
            if (a.pack) {
                I.qb = w;
                I.h = h0;
                return w * BM < (h1 - h0) * a.B;
            }
            I.qb = a.n_rb - 1 - w / a.gmax;  // heaviest first
            I.h = h0 + w % a.gmax;
            return I.h < h1;
        }
        I.split = 0;
        if (a.xcd_map) {
            // Consecutive workgroups go to the 8 XCDs in turn.  XCD x serves
            // kv head x % n_kv, so the query heads that read one kv head
            // share an L2 and its K/V tiles are fetched from HBM once per XCD
            // group, not once per XCD; the XCD's own workgroups take its items.
            const uint32_t x = blockIdx.x % 8u, j = blockIdx.x / 8u, W = gridDim.x / 8u;
            const uint32_t slot = it * W + ((it & 1u) ? W - 1u - j : j);
            if (slot >= nqb * a.n_heads / 8u) return false;
            const uint32_t per = 8u / a.n_kv, G = a.n_heads / a.n_kv;
            const uint32_t g = x % a.n_kv, i = slot * per + x / a.n_kv;
            I.qb = nqb - 1 - i / G;
            I.h = g * G + i % G;
        } else {
            const uint32_t W = gridDim.x;
            const uint32_t slot = it * W + ((it & 1u) ? W - 1u - blockIdx.x : blockIdx.x);
            if (slot >= nqb * a.n_heads) return false;
            I.qb = nqb - 1 - slot / a.n_heads;
            I.h = slot % a.n_heads;
        }
        I.kvh = I.h * a.n_kv / a.n_heads;  // engine.c:537
        return true;
    };
    // An item's first loads are issued during the previous item: its
    // group's first K, V and second K tiles in the previous item's last key
    // step, into buffers that step no longer reads (the V tile only after
    // the step when that step reads V buffer 0), and, for f16 queries, the
    // query fragments after the key loop (registers the key loop reads
    // cannot be loaded inside it without the compiler waiting for them
    // there).  Their latency hides under that step, the merge and the output
    // stores.  With a gate the epilogue loads the gate values, which would
    // then wait behind these loads; such items issue their loads at their
    // own start.
    const bool early = a.gate == nullptr && !PAIR;
    PItem cur;
    if (!item_of(0, cur)) return;  // uniform over the workgroup
    for (uint32_t it = 0;; ++it) {
        // Thread indices pass through an opaque move each item so that nothing
        // derived from them is hoisted out of the item loop: the key loop's
        // register budget stays that of a single item.
        int tid;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
        const int lane = tid & 63;
        // with one key group the group is a constant, so the LDS tile bases are
        // too and fold into the reads' offset fields; with two it is read into
        // a scalar register (the LDS destination of a direct-to-LDS load must
        // be uniform, and from a per-lane group index the compiler wrapped
        // every such load in a loop over the lanes' values)
        const int grp = NG > 1 ? (int)__builtin_amdgcn_readfirstlane(tid / LT) : 0,
                  gtid = NG > 1 ? tid % LT : tid, wave = gtid >> 6;
        // the wave's 32 queries (qw) and, in pair mode, its half of the dimensions (hf)
        const int qw = PAIR ? wave >> 1 : wave, hf = PAIR ? wave & 1 : 0;
        const int r32 = lane & 31, hh = lane >> 5;
        PItem nxt{};
        const bool has_next = item_of(it + 1, nxt);

        // Chunk L = LT i + gtid of a tile is the 16 bytes this thread loads
        // with its i-th instruction.  K: LDS row R = L / KCH holds key row
        // lds_row_of_key(R) (an involution), column chunk (L % KCH) ^ swz(R).
        // V: LDS row d = L / VCH holds positions 8c..8c+7 in chunk
        // (L % VCH) ^ swz(d), from 32-position tile c / 4.
        int kgo[CH], vgo[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int L = gtid + LT * i;
            const int R = L / KCH, kc = (L % KCH) ^ chunk_swz<KCH>(R);
            kgo[i] = (lds_row_of_key(R) * D + kc * 8) * 2;
            const int d = L / VCH, vc = (L % VCH) ^ chunk_swz<VCH>(d);
            vgo[i] = (vc >> 2) * (D * (int)kVTile * 2) + d * (int)kVTile * 2 + (vc & 3) * 16;
        }
        const int ksw = chunk_swz<KCH>(r32), vsw = chunk_swz<VCH>(r32);
        // buffers by parity (a constant at every call after inlining)
        auto kbuf = [&](int par) { return par == 0 ? &Kl0[grp][0] : par == 1 ? &Kl1[grp][0] : &Kl2[0]; };
        auto vbuf = [&](int par) { return par == 0 ? &Vl0[grp][0] : par == 1 ? &Vl1[grp][0] : &Vl2[0]; };
        // Buffer resources over a kv head's K rows and V tiles.  A tile adds
        // the scalar offset kt*BN*D*2 bytes (the same for K rows and two
        // 32-position V tiles); every tile lies inside the cache (kv_stride is a
        // multiple of 64 above kmax).
        const uint32_t head_bytes = a.kv_stride * D * 2;
        auto rsrc_k = [&](uint32_t kv) {
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kc + k_index(kv, 0, 0, D, a.kv_stride)), 0,
                                                     head_bytes, 0x00020000);
        };
        auto rsrc_v = [&](uint32_t kv) {
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vc + v_index(kv, 0, 0, D, a.kv_stride)), 0,
                                                     head_bytes, 0x00020000);
        };
        // tile kt of a K (V) resource into K (V) buffer par
        auto dma_k_of = [&](__amdgpu_buffer_rsrc_t r, int par, uint32_t kt) {
#pragma unroll
            for (int i = 0; i < CH; ++i) lds_load16(r, kbuf(par) + (LT * i + 64 * wave) * 8, kgo[i], kt * BN * D * 2);
        };
        auto dma_v_of = [&](__amdgpu_buffer_rsrc_t r, int par, uint32_t kt) {
#pragma unroll
            for (int i = 0; i < CH; ++i) lds_load16(r, vbuf(par) + (LT * i + 64 * wave) * 8, vgo[i], kt * BN * D * 2);
        };
        auto dma_done = [] { __builtin_amdgcn_s_waitcnt(0x0f70); };  // vmcnt(0): this thread's loads landed
        // all but this thread's last n tile loads landed (n of 0, CH or 2 CH:
        // an immediate; memory loads retire in order)
        auto dma_wait_but = [](uint32_t n) {
            if (n >= 2 * CH) __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * CH));
            else if (n >= CH) __builtin_amdgcn_s_waitcnt(0x0f70 | CH);
            else __builtin_amdgcn_s_waitcnt(0x0f70);
        };
        f16x8 qf[NKK];
        f16x8 ql[QS ? NKK : 1];  // QS: the lo parts
        // the first loads of an item, see above: the K tiles, the first V
        // tile and the queries
        auto item_steps = [&](const PItem& I, uint32_t& t0) {
            uint32_t km, nt;
            item_keys<BN, SPLIT>(a, I, km, t0, nt);
            return nt > (uint32_t)grp ? (nt - grp + NG - 1) / NG : 0u;  // this group's tiles
        };
        auto issue_item_k = [&](const PItem& I) {
            uint32_t t0;
            const uint32_t igsteps = item_steps(I, t0);
            const __amdgpu_buffer_rsrc_t rk = rsrc_k(I.kvh);
            if (igsteps > 0) dma_k_of(rk, 0, t0 + grp);
            if (igsteps > 1) dma_k_of(rk, 1, t0 + grp + NG);
        };
        auto issue_item_q = [&](const PItem& I) {
            if (a.q_dtype == kF16) {
                const PRow rw = row_of<SPLIT>(a, I, qw * 32 + r32);
                const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + (size_t)rw.b * a.q_stride +
                                     (size_t)rw.h * D + hf * DQ + hh * 8;
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) qf[kk] = *reinterpret_cast<const f16x8*>(qp + kk * 16);
            }
        };
        auto issue_item_v = [&](const PItem& I) {
            uint32_t t0;
            if (item_steps(I, t0) > 0) dma_v_of(rsrc_v(I.kvh), 0, t0 + grp);
        };
        // pair mode, after the first loads: K(2) and V(1); returns their count
        auto issue_item_deep = [&](const PItem& I) -> uint32_t {
            uint32_t t0;
            const uint32_t n = item_steps(I, t0);
            if (n > 2) dma_k_of(rsrc_k(I.kvh), 2, t0 + 2);
            if (n > 1) dma_v_of(rsrc_v(I.kvh), 1, t0 + 1);
            return (n > 2 ? CH : 0) + (n > 1 ? CH : 0);
        };
        uint32_t deep_loads = 0;  // loads the prologue need not wait for
        if (it == 0 || !early) {
            if (it > 0) __syncthreads();  // the previous item's epilogue read LDS these loads overwrite
            issue_item_k(cur);
            issue_item_v(cur);
            issue_item_q(cur);
            if constexpr (NB > 2) deep_loads = issue_item_deep(cur);
        }

        const uint32_t kvh = cur.kvh;
        uint32_t kmax, t0, ntiles;  // this item's keys end at kmax; its tiles are t0 .. t0+ntiles-1
        item_keys<BN, SPLIT>(a, cur, kmax, t0, ntiles);
        const uint32_t nsteps = (ntiles + NG - 1) / NG;  // loop steps (workgroup-uniform)
        // this group's tiles: kt = t0 + grp + NG*st for st < gsteps
        const uint32_t gsteps = ntiles > (uint32_t)grp ? (ntiles - grp + NG - 1) / NG : 0;

        uint32_t wfirst, wlast;
        const bool wave_active = wave_span<SPLIT>(a, cur, qw, wfirst, wlast);
        const uint32_t wpos_first = a.pos_start + wfirst;
        const uint32_t wpos_last = a.pos_start + wlast;
        const PRow myrow = row_of<SPLIT>(a, cur, qw * 32 + r32);
        const uint32_t my_pos = a.pos_start + myrow.b;
        // tiles this wave computes: t0 .. t0+wtiles-1, of which this group's are st < wsteps
        const uint32_t wend = wave_active ? wpos_last / BN + 1 : 0;  // one past the wave's last tile
        const uint32_t wtiles = wend > t0 ? min(wend - t0, ntiles) : 0;
        const uint32_t wsteps = wtiles > (uint32_t)grp ? (wtiles - grp + NG - 1) / NG : 0;
        auto tile_of = [&](uint32_t st) { return t0 + (uint32_t)grp + NG * st; };

        const __amdgpu_buffer_rsrc_t rK = rsrc_k(kvh), rV = rsrc_v(kvh);
        auto dma_k = [&](int par, uint32_t st) { dma_k_of(rK, par, tile_of(st)); };
        auto dma_v = [&](int par, uint32_t st) { dma_v_of(rV, par, tile_of(st)); };

        // MFMA operands from LDS.  K fragment (j, kk): key row r32 + 32 j, dims
        // DQ hf + 16 kk + 8 hh .. +7 = chunk 2 (kk + NKK hf) + hh.  V fragment
        // (b, kc): row d = DQ hf + 32 b + r32, positions 16 kc + 8 hh .. +7 =
        // chunk 2 kc + hh.
        auto read_k = [&](int par, int j, int kk) {
            return *reinterpret_cast<const f16x8*>(kbuf(par) + (r32 + 32 * j) * D +
                                                   (((2 * (kk + NKK * hf) + hh) ^ ksw) << 3));
        };
        auto read_v = [&](int par, int b, int kc) {
            return *reinterpret_cast<const f16x8*>(vbuf(par) + (DQ * hf + 32 * b + r32) * BN +
                                                   (((2 * kc + hh) ^ vsw) << 3));
        };
        // pair mode: publish this wave's partial scores of a tile (before the
        // step barrier), add the partner's (after it)
        auto xwrite = [&](const f32x16 (&S)[NS], int par) {
            if constexpr (PAIR) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4)
                        Xl[((par * 8 + wave) * 4 * NS + 4 * j + q4) * 64 + lane] =
                            f32x4{S[j][4 * q4], S[j][4 * q4 + 1], S[j][4 * q4 + 2], S[j][4 * q4 + 3]};
            }
        };
        auto xadd = [&](f32x16 (&S)[NS], int par) {
            if constexpr (PAIR) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        const f32x4 o4 = Xl[((par * 8 + (wave ^ 1)) * 4 * NS + 4 * j + q4) * 64 + lane];
#pragma unroll
                        for (int e = 0; e < 4; ++e) S[j][4 * q4 + e] += o4[e];
                    }
            }
        };
        // Keys past kmax in the workgroup's last tile were never stored and may
        // hold any bits: their P is 0, but their V must be finite.  The group
        // that owns that tile zeroes them in LDS once, in the step that reads it.
        auto zero_v_tail = [&](int par, uint32_t st) {
            const uint32_t k0 = tile_of(st) * BN;
            const uint32_t valid = kmax - k0 + 1;  // keys 0..valid-1 of the tile are stored
            _Float16* vb = vbuf(par);
            for (int idx = gtid; idx < D * VCH; idx += LT) {
                const int d = idx / VCH, c = idx % VCH;  // logical chunk c: keys 8c..8c+7
                if ((uint32_t)(8 * c + 7) < valid) continue;
                f16x8* ch = reinterpret_cast<f16x8*>(vb + d * BN + ((c ^ chunk_swz<VCH>(d)) << 3));
                f16x8 v = *ch;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if ((uint32_t)(8 * c + e) >= valid) v[e] = (_Float16)0.0f;
                *ch = v;
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

        // scores of the tile in K buffer P into S (its 32-key halves)
        auto qk = [&](f32x16 (&S)[NS], int par) {
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
                for (int j = 0; j < NS; ++j) {
                    const f16x8 kf = read_k(par, j, kk);
                    S[j] = kk == 0 ? mfma32(kf, qf[0], f32x16{}) : mfma32(kf, qf[kk], S[j]);
                    if constexpr (QS) S[j] = mfma32(kf, ql[kk], S[j]);
                }
        };
        // running max update of the lane's query from tile scores S (raw, masked)
        auto update_max = [&](const f32x16 (&S)[NS]) {
            float mx = S[0][0];
#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, S[j][i]);
            // the lane pair (l, l+32) holds one query: exchange the halves
            const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx),
                                                             __builtin_bit_cast(uint32_t, mx), false, false);
            mx = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1])) * a.c;
            if (__ballot(mx > m + kSlack)) {  // wave-uniform: some query's max moved
                const float mn = mx > m + kSlack ? mx : m;
                const float alpha = fast_exp2(m - mn);
                m = mn;
                l *= alpha;
#pragma unroll
                for (int b = 0; b < NDB; ++b) o[b] *= alpha;
            }
        };
        auto probs = [&](const f32x16 (&S)[NS], f16x8 (&pf)[NKC]) {
            const float nm = -m;
#pragma unroll
            for (int i = 0; i < 16 * NS; ++i) {
                const float p = fast_exp2(fmaf(S[i >> 4][i & 15], a.c, nm));
                l += p;
                pf[i >> 3][i & 7] = (_Float16)p;
            }
        };
        // O^T += V^T P^T over the tile in V buffer P; fragments are read two
        // MFMAs ahead (three in a ring)
        auto pv = [&](const f16x8 (&pf)[NKC], int par) {
            constexpr int NM = NKC * NDB;  // MFMA n: kc = n / NDB, b = n % NDB
            f16x8 vf[3];
            vf[0] = read_v(par, 0, 0);
            vf[1] = read_v(par, 1 % NDB, 1 / NDB);
#pragma unroll
            for (int n = 0; n < NM; ++n) {
                if (n + 2 < NM) vf[(n + 2) % 3] = read_v(par, (n + 2) % NDB, (n + 2) / NDB);
                o[n % NDB] = mfma32(vf[n % 3], pf[n / NDB], o[n % NDB]);
            }
        };
        // Scores of the next tile (K buffer kpar) into Snext and P.V of this tile
        // (V buffer vpar), with this tile's probabilities (from Scur) formed
        // between them per FusedSchedule; K and V fragments are read two MFMAs
        // ahead in their own streams.
        auto qk_pv = [&](f32x16 (&Snext)[NS], int kpar, const f32x16 (&Scur)[NS], int vpar) {
            constexpr int NQ = NS * NKK, NPV = NKC * NDB;  // score MFMA n: half n % NS, k-chunk n / NS
            constexpr FusedSchedule<NQ, NPV, NDB, NKC> sch{};
            constexpr int MAXP = 8;
            const float nm = -m;
            f16x8 pf[NKC], kf[3], vf[3];
            kf[0] = read_k(kpar, 0, 0);
            kf[1] = read_k(kpar, 1 % NS, 1 / NS);
            vf[0] = read_v(vpar, 0, 0);
            vf[1] = read_v(vpar, 1 % NDB, 1 / NDB);
#pragma unroll
            for (int t = 0; t < sch.N; ++t) {
                const int n = sch.s[t].n;
                if (sch.s[t].pv) {
                    if (n + 2 < NPV) vf[(n + 2) % 3] = read_v(vpar, (n + 2) % NDB, (n + 2) / NDB);
                    o[n % NDB] = mfma32(vf[n % 3], pf[n / NDB], o[n % NDB]);
                } else {
                    if (n + 2 < NQ) kf[(n + 2) % 3] = read_k(kpar, (n + 2) % NS, (n + 2) / NS);
                    Snext[n % NS] = n < NS ? mfma32(kf[n % 3], qf[0], f32x16{})
                                           : mfma32(kf[n % 3], qf[n / NS], Snext[n % NS]);
                    if constexpr (QS) Snext[n % NS] = mfma32(kf[n % 3], ql[n / NS], Snext[n % NS]);
                }
#pragma unroll
                for (int u = 0; u < MAXP; ++u) {
                    if (u < sch.s[t].np) {
                        const int i = sch.s[t].p0 + u;
                        const float p = fast_exp2(fmaf(Scur[i >> 4][i & 15], a.c, nm));
                        l += p;
                        pf[i >> 3][i & 7] = (_Float16)p;
                    }
                }
            }
        };
        // a tile that reaches past the wave's first query: keys beyond the
        // lane's position get -inf
        auto mask = [&](f32x16 (&S)[NS], uint32_t st) {
            const uint32_t k0 = tile_of(st) * BN;
            if (k0 + BN - 1 > wpos_first) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (k0 + 32 * j + key_of_acc(i, hh) > my_pos) S[j][i] = -INFINITY;
            }
        };

        // prologue: this item's first loads are in flight (issued above or at the
        // end of the previous item); f32 and bf16 queries are loaded and
        // converted here.  All loads are complete before the key loop, whose
        // waits then count only tile loads (in pair mode K(2) and V(1) may
        // still be in flight; the first step waits for them).
        dma_wait_but(deep_loads);
        if (a.q_dtype != kF16) {
            const size_t qbase = (size_t)myrow.b * a.q_stride + (size_t)myrow.h * D + hf * DQ + hh * 8;
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                if constexpr (QS) load_q8_split(qf[kk], ql[kk], reinterpret_cast<const float*>(a.q), qbase + kk * 16);
                else load_q8(qf[kk], a.q, qbase + kk * 16, a.q_dtype);
            }
            if (NB == 2) dma_done();
        }
        if constexpr (NB > 2) lds_barrier();
        else __syncthreads();
        f32x16 Sa[NS], Sb[NS];
        if (wsteps > 0) {
            qk(Sa, 0);
            xwrite(Sa, 0);
        }
        // step 0 loads K(NB) over K(0), whose last readers are the scores above
        if constexpr (NB > 2) lds_barrier();
        else __syncthreads();

        // step st (buffer phase ph = st % NB, score parity sp = st % 2): loads
        // K(st+NB) into K buffer ph (it held K(st), last read by the previous
        // step's scores) and V(st+NB-1) into V buffer (ph+NB-1) % NB (it held
        // V(st-1)); scores of st+1 (K buffer (ph+1) % NB) overlap the softmax
        // of st; P.V of st (V buffer ph); one barrier.  With pos_start not a
        // multiple of 32 a wave's queries straddle a tile boundary, so a tile
        // with a successor may still need the mask.
        // the step that reads the tile holding kmax (the item's last tile, unless
        // a later split owns it), in this group's buffers
        const bool has_tail = ntiles > 0 && t0 + ntiles == kmax / BN + 1 && (kmax + 1) % BN != 0;
        const uint32_t tail_step = (ntiles - 1) / NG;
        const int tail_grp = (int)((ntiles - 1) % NG);
        const bool prefetch = has_next && early;
        // the group's last step (or, for a group without tiles, the first) issues
        // the next item's loads
        const uint32_t last_st = gsteps > 0 ? gsteps - 1 : 0;
        auto step = [&](int ph, int sp, uint32_t st, f32x16 (&Scur)[NS], f32x16 (&Snext)[NS]) {
            const bool lk = st + NB < gsteps, lv = st + NB - 1 < gsteps;
            if (lk) dma_k(ph, st + NB);
            if (lv) dma_v((ph + NB - 1) % NB, st + NB - 1);
            if (prefetch && st == last_st) {
                // K buffers are free (no scores follow), V buffer 1-p too
                issue_item_k(nxt);
                if (ph == 1 || gsteps == 0) issue_item_v(nxt);
            }
            if (has_tail && st == tail_step) {  // workgroup-uniform
                if (grp == tail_grp) zero_v_tail(ph, st);
                lds_barrier();
            }
            if (st + 1 < wsteps) {
                xadd(Scur, sp);
                mask(Scur, st);
                update_max(Scur);
                qk_pv(Snext, (ph + 1) % NB, Scur, ph);
                xwrite(Snext, 1 - sp);
            } else if (st < wsteps) {
                xadd(Scur, sp);
                mask(Scur, st);
                update_max(Scur);
                f16x8 pf[NKC];
                probs(Scur, pf);
                pv(pf, ph);
            }
            if constexpr (NB > 2) {
                // the previous steps' loads (this step's have two steps to land)
                dma_wait_but((lk ? CH : 0) + (lv ? CH : 0));
            } else {
                // this step's own loads (none from the group's last step on, whose
                // next-item loads are waited for by the next item)
                if (!(prefetch && st >= last_st)) dma_done();
            }
            lds_barrier();
        };
        if constexpr (NB == 2) {
            for (uint32_t st = 0; st < nsteps; st += 2) {
                step(0, 0, st, Sa, Sb);
                if (st + 1 < nsteps) step(1, 1, st + 1, Sb, Sa);
            }
        } else {
            // buffer phase period 3, score parity period 2
            for (uint32_t st = 0; st < nsteps; st += 6) {
                step(0, 0, st, Sa, Sb);
                if (st + 1 >= nsteps) break;
                step(1, 1, st + 1, Sb, Sa);
                if (st + 2 >= nsteps) break;
                step(2, 0, st + 2, Sa, Sb);
                if (st + 3 >= nsteps) break;
                step(0, 1, st + 3, Sb, Sa);
                if (st + 4 >= nsteps) break;
                step(1, 0, st + 4, Sa, Sb);
                if (st + 5 >= nsteps) break;
                step(2, 1, st + 5, Sb, Sa);
            }
        }

        // the next item's first V tile when the last step still read V buffer 0,
        // and its queries
        if (prefetch) {
            if (gsteps > 0 && (last_st & 1u) == 0) issue_item_v(nxt);
            issue_item_q(nxt);
        }
        {
            // the lane pair (l, l+32) holds one query: add the halves
            const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, l),
                                                             __builtin_bit_cast(uint32_t, l), false, false);
            l = __builtin_bit_cast(float, (uint32_t)sw[0]) + __builtin_bit_cast(float, (uint32_t)sw[1]);
        }
        // Thread indices for the epilogue from a fresh opaque read, so that the
        // ones of the item's start need not stay live through the key loop.
        int tid_e;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tid_e) : "v"((int)threadIdx.x));
        const int gtid_e = NG > 1 ? tid_e % LT : tid_e, lane_e = tid_e & 63;
        const int qw_e = PAIR ? gtid_e >> 7 : gtid_e >> 6, hf_e = PAIR ? (gtid_e >> 6) & 1 : 0;
        int b_lo = 0, b_hi = NDB;  // the O blocks this thread stores
        if constexpr (NG > 1) {
            // The two groups' (m, l, O) meet through LDS: m, l in s_ml and O
            // through V buffer 1 of both groups (the one buffer the next item's
            // first loads leave free; 32 KB at d = 128), half the blocks at a
            // time.  Group 1 hands over blocks 0 .. HB-1, which group 0 merges
            // and stores; then group 0 hands over blocks HB .., which group 1
            // merges and stores, so both groups issue half of the output.
            constexpr int HB = NDB / 2;  // O blocks per round
            static_assert(HB * 16 * 256 * 4 <= (int)sizeof(Vl1), "merge area");
            float* oarea = reinterpret_cast<float*>(&Vl1[0][0]);
            if (grp == 1) {
                s_ml[gtid_e] = m;
                s_ml[256 + gtid_e] = l;
#pragma unroll
                for (int b = 0; b < HB; ++b)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oarea[(b * 16 + i) * 256 + gtid_e] = o[b][i];
            }
            lds_barrier();
            float mo = m, lo = l;  // the other group's (m, l)
            auto merge_half = [&](int r) {
                const float mg = fmaxf(m, mo);
                const float cs = fast_exp2(m - mg), co = fast_exp2(mo - mg);
#pragma unroll
                for (int b = 0; b < HB; ++b)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        o[r * HB + b][i] = o[r * HB + b][i] * cs + oarea[(b * 16 + i) * 256 + gtid_e] * co;
            };
            if (grp == 0) {
                mo = s_ml[gtid_e];
                lo = s_ml[256 + gtid_e];
                merge_half(0);
            }
            lds_barrier();  // round 0 read before round 1 overwrites
            if (grp == 0) {
                s_ml[gtid_e] = m;
                s_ml[256 + gtid_e] = l;
#pragma unroll
                for (int b = 0; b < HB; ++b)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oarea[(b * 16 + i) * 256 + gtid_e] = o[HB + b][i];
            }
            lds_barrier();
            if (grp == 1) {
                mo = s_ml[gtid_e];
                lo = s_ml[256 + gtid_e];
                merge_half(1);
            }
            const float mg = fmaxf(m, mo);
            l = l * fast_exp2(m - mg) + lo * fast_exp2(mo - mg);
            m = mg;
            b_lo = grp * HB;
            b_hi = b_lo + HB;
        }
        const PRow rw = row_of<SPLIT>(a, cur, qw_e * 32 + (lane_e & 31));
        if (rw.valid) {
            if (SPLIT && a.n_split > 1) {
                // split partials: (max, sum) and the unnormalised O of this
                // row over this split's keys
                const size_t pr = ((size_t)cur.split * a.n_heads + rw.h) * a.B + rw.b;
                if ((lane_e >> 5) == 0 && hf_e == 0) {
                    typedef float f32x2 __attribute__((ext_vector_type(2)));
                    *reinterpret_cast<f32x2*>(a.part_ml + 2 * pr) = f32x2{m, l};
                }
#pragma unroll
                for (int b = 0; b < NDB; ++b) {
                    if (b < b_lo || b >= b_hi) continue;
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4) {
                        const uint32_t d = hf_e * DQ + b * 32 + 8 * i4 + 4 * (lane_e >> 5);
                        f32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = o[b][4 * i4 + e];
                        *reinterpret_cast<f32x4*>(a.part_o + pr * D + d) = v;
                    }
                }
            } else {
                const float inv = 1.0f / l;
#pragma unroll
                for (int b = 0; b < NDB; ++b) {
                    if (b < b_lo || b >= b_hi) continue;
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4) {
                        const uint32_t d = hf_e * DQ + b * 32 + 8 * i4 + 4 * (lane_e >> 5);
                        f32x4 v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = o[b][4 * i4 + e] * inv;
                        if (a.gate) {
                            const float* gp = a.gate + (size_t)rw.b * a.gate_stride + (size_t)rw.h * D + d;
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] *= sigmoid_ref(gp[e]);
                        }
                        store_out4(a.out, (size_t)rw.b * a.out_stride + (size_t)rw.h * D + d, a.out_dtype, v);
                    }
                }
            }
        }
        if (!has_next) break;
        cur = nxt;
    }  // items
}

// One thread per (row, 4 output dimensions) of the split mode: the splits'
// (max, sum, O) partials of query b of head h are combined in the log2
// domain, then normalised, gated and stored.  Rows are b * n_heads + h, so a
// workgroup's output stores are contiguous; each round of 8 splits issues
// its loads together.
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    constexpr uint32_t C4 = D / 4;
    constexpr uint32_t kRound = 8;
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    const uint32_t row = idx / C4, c4 = idx % C4;
    if (row >= a.B * a.n_heads) return;
    const uint32_t b = row / a.n_heads, h = row % a.n_heads;
    const size_t split_stride = (size_t)a.n_heads * a.B;
    const size_t p0 = (size_t)h * a.B + b;
    const uint32_t d = 4 * c4;
    // the gate is read with the partials, not after them (a second memory
    // round trip); without a gate the output row stands in as a valid address
    const float* gp = a.gate ? a.gate + (size_t)b * a.gate_stride + (size_t)h * D + d
                             : reinterpret_cast<const float*>(a.out);
    f32x4 gt;
#pragma unroll
    for (int e = 0; e < 4; ++e) gt[e] = gp[e];
    float M = -1e30f, L = 0.0f;
    f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t s0 = 0; s0 < a.n_split; s0 += kRound) {
        f32x2 ml[kRound];
        f32x4 os[kRound];
#pragma unroll
        for (uint32_t r = 0; r < kRound; ++r) {
            if (s0 + r < a.n_split) {
                const size_t p = (s0 + r) * split_stride + p0;
                ml[r] = *reinterpret_cast<const f32x2*>(a.part_ml + 2 * p);
                os[r] = *reinterpret_cast<const f32x4*>(a.part_o + p * D + 4 * c4);
            } else {
                ml[r] = f32x2{-1e30f, 0.0f};
                os[r] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        float mr = M;
#pragma unroll
        for (uint32_t r = 0; r < kRound; ++r) mr = fmaxf(mr, ml[r][0]);
        const float co = fast_exp2(M - mr);
        L *= co;
        O *= co;
#pragma unroll
        for (uint32_t r = 0; r < kRound; ++r) {
            const float c = fast_exp2(ml[r][0] - mr);
            L += ml[r][1] * c;
            O += os[r] * c;
        }
        M = mr;
    }
    // every query has key 0 in split 0, so L > 0
    f32x4 v = O * (1.0f / L);
    if (a.gate) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= sigmoid_ref(gt[e]);
    }
    store_out4(a.out, (size_t)b * a.out_stride + (size_t)h * D + d, a.out_dtype, v);
}

}  // namespace

int n_cus()
{
    static const int n_cu = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return n_cu;
}

namespace {

// threads of a prefill workgroup: 4 waves per key group, 8 in pair mode
constexpr int prefill_threads(int D, int NG) { return 256 * NG * (D > 128 ? 2 : 1); }

template <int D, int NG, bool QS>
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
    const uint32_t items = nqb0 * a.n_heads;
    // resident workgroups: one round of the grid fills every slot once
    static const int per_cu = [] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<D, NG, false, QS>, prefill_threads(D, NG),
                                                         0) != hipSuccess ||
            n < 1)
            n = 1;
        return n;
    }();
    // Resident workgroups walking the item list pay off with one 8-wave
    // workgroup per CU (two key groups), where nothing else on the CU covers
    // a workgroup's start and end (2048 tokens x 28 heads: 57.1 -> 55.7 us);
    // with two 4-wave workgroups per CU the hardware's own dispatch of the
    // next workgroup already overlaps them and is about 1 % faster (8192
    // tokens).  YHIP_PREFILL_PERSIST=0/1 forces the choice for comparisons.
    static const int persist = [] {
        const char* e = getenv("YHIP_PREFILL_PERSIST");
        return e ? atoi(e) : -1;
    }();
    uint32_t grid = items;
    if (persist > 0 || (persist < 0 && prefill_threads(D, NG) > 256)) {
        const uint64_t slots = (uint64_t)per_cu * (uint64_t)n_cus();
        if (slots < grid) grid = (uint32_t)slots;
        if (a.xcd_map) grid = grid / 8u * 8u;  // whole XCD groups (items are a multiple of 8)
        if (grid == 0) grid = items;
    }
    hipLaunchKernelGGL((prefill_kernel<D, NG, false, QS>), dim3(grid), dim3(prefill_threads(D, NG)), 0, st, a);
    return hipGetLastError();
}

template <int D, bool QS>
hipError_t launch_prefill_split_d(const PrefillArgs& a, hipStream_t st)
{
    const uint32_t ipg = a.n_rb * (a.pack ? 1u : a.gmax);
    const uint32_t groups = a.n_kv * a.n_split;
    const uint32_t grid = (groups + 7u) / 8u * 8u * ipg;
    hipLaunchKernelGGL((prefill_kernel<D, 1, true, QS>), dim3(grid), dim3(prefill_threads(D, 1)), 0, st, a);
    if (a.n_split > 1) {
        const uint64_t threads = (uint64_t)a.B * a.n_heads * (D / 4);
        hipLaunchKernelGGL(prefill_merge_kernel<D>, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, st, a);
    }
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
    const int n_cu = n_cus();
    if (a.D > 128) return 1;
    if (env == 1 || env == 2) return env;
    const uint64_t wgs = (uint64_t)((a.B + BM - 1) / BM) * a.n_heads;
    return wgs <= 2 * (uint64_t)n_cu ? 2 : 1;
}

}  // namespace

namespace {

size_t align256p(size_t x) { return (x + 255) / 256 * 256; }

// Split-mode tunables (YHIP_PREFILL_SPLIT=0 turns the mode off; the others
// bound the split count and the tiles per split, for sweeps).
struct SplitTune {
    int on;
    uint32_t max_split, min_tiles;
};
const SplitTune& split_tune()
{
    static const SplitTune t = [] {
        SplitTune r{1, 16, 4};
        if (const char* e = getenv("YHIP_PREFILL_SPLIT")) r.on = atoi(e) != 0;
        if (const char* e = getenv("YHIP_PREFILL_MAXSPLIT")) r.max_split = (uint32_t)(atoi(e) > 0 ? atoi(e) : 1);
        if (const char* e = getenv("YHIP_PREFILL_MINTILES")) r.min_tiles = (uint32_t)(atoi(e) > 0 ? atoi(e) : 1);
        return r;
    }();
    return t;
}

size_t split_bytes(uint32_t n_split, uint32_t B, uint32_t n_heads, uint32_t D)
{
    if (n_split <= 1) return 0;
    const size_t rows = (size_t)n_split * n_heads * B;
    return align256p(rows * 2 * sizeof(float)) + rows * D * sizeof(float);
}

// Items of a split-mode launch before splitting, and the workgroups that
// fill the GPU once.
void split_shape(uint32_t B, uint32_t n_heads, uint32_t n_kv, uint32_t D, uint32_t& pack, uint32_t& n_rb,
                 uint32_t& gmax, uint64_t& base, uint64_t& target)
{
    gmax = (n_heads + n_kv - 1) / n_kv;
    pack = B < (uint32_t)BM;
    n_rb = pack ? (gmax * B + BM - 1) / BM : (B + BM - 1) / BM;
    base = (uint64_t)n_kv * n_rb * (pack ? 1u : gmax);
    target = (uint64_t)(D <= 128 ? 2 : 1) * (uint64_t)n_cus();  // resident workgroups per CU
}

}  // namespace

size_t prefill_plan(PrefillArgs& a)
{
    a.split_mode = a.pack = 0;
    a.n_split = 1;
    a.split_tiles = 0;
    a.n_rb = 0;
    a.gmax = 0;
    const SplitTune& t = split_tune();
    // The plain mode, (query block, head) items, fills the GPU when there
    // are at least as many items as CUs (prompts of a few hundred tokens and
    // up).  Fewer items -- the engine's 64-token chunks over a long prefix
    // -- would leave most CUs idle while each walks the whole prefix: the
    // split mode packs a kv head's query heads into full 128-row items and
    // splits the keys so that the launch fills the GPU.
    if (!t.on || (uint64_t)((a.B + BM - 1) / BM) * a.n_heads >= (uint64_t)n_cus()) return 0;
    uint64_t base, target;
    split_shape(a.B, a.n_heads, a.n_kv, a.D, a.pack, a.n_rb, a.gmax, base, target);
    a.split_mode = 1;
    const uint32_t ntiles = (a.pos_start + a.B - 1) / bn_of((int)a.D) + 1;
    uint64_t S = target / base;
    if (S > t.max_split) S = t.max_split;
    const uint32_t by_tiles = (ntiles + t.min_tiles - 1) / t.min_tiles;
    if (S > by_tiles) S = by_tiles;
    if (S < 1) S = 1;
    a.split_tiles = (ntiles + (uint32_t)S - 1) / (uint32_t)S;
    a.n_split = (ntiles + a.split_tiles - 1) / a.split_tiles;
    return split_bytes(a.n_split, a.B, a.n_heads, a.D);
}

size_t prefill_workspace_bound(uint32_t B, uint32_t max_end, uint32_t n_heads, uint32_t n_kv, uint32_t D)
{
    // the plan for any pos_start <= max_end - B: its split count is at most
    // min(target/base, max_split, ceil(tiles/min_tiles)) with the most tiles
    const SplitTune& t = split_tune();
    if (!t.on || B == 0 || n_kv == 0 || max_end < B || (uint64_t)((B + BM - 1) / BM) * n_heads >= (uint64_t)n_cus())
        return 0;
    uint32_t pack, n_rb, gmax;
    uint64_t base, target;
    split_shape(B, n_heads, n_kv, D, pack, n_rb, gmax, base, target);
    const uint32_t ntiles = (max_end - 1) / bn_of((int)D) + 1;
    uint64_t S = target / base;
    if (S > t.max_split) S = t.max_split;
    const uint32_t by_tiles = (ntiles + t.min_tiles - 1) / t.min_tiles;
    if (S > by_tiles) S = by_tiles;
    return split_bytes((uint32_t)(S < 1 ? 1 : S), B, n_heads, D);
}

uint32_t prefill_tile_keys(uint32_t D) { return (uint32_t)bn_of((int)D); }

void prefill_bind_workspace(PrefillArgs& a, void* workspace)
{
    if (a.n_split <= 1 || !workspace) {
        a.part_ml = a.part_o = nullptr;
        return;
    }
    char* p = reinterpret_cast<char*>(workspace);
    a.part_ml = reinterpret_cast<float*>(p);
    a.part_o = reinterpret_cast<float*>(p + align256p((size_t)a.n_split * a.n_heads * a.B * 2 * sizeof(float)));
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t st)
{
    // fp32 queries keep fp32-level scores (hi + lo parts, one key group)
    const bool qs = a.q_dtype == kF32;
    if (a.split_mode) {
        switch (a.D) {
        case 64: return qs ? launch_prefill_split_d<64, true>(a, st) : launch_prefill_split_d<64, false>(a, st);
        case 128: return qs ? launch_prefill_split_d<128, true>(a, st) : launch_prefill_split_d<128, false>(a, st);
        case 256: return qs ? launch_prefill_split_d<256, true>(a, st) : launch_prefill_split_d<256, false>(a, st);
        default: return hipErrorInvalidValue;
        }
    }
    const int ng = prefill_groups(a);
    switch (a.D) {
    case 64:
        return qs ? launch_prefill_d<64, 1, true>(a, st)
                  : ng == 2 ? launch_prefill_d<64, 2, false>(a, st) : launch_prefill_d<64, 1, false>(a, st);
    case 128:
        return qs ? launch_prefill_d<128, 1, true>(a, st)
                  : ng == 2 ? launch_prefill_d<128, 2, false>(a, st) : launch_prefill_d<128, 1, false>(a, st);
    case 256: return qs ? launch_prefill_d<256, 1, true>(a, st) : launch_prefill_d<256, 1, false>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace yhip
