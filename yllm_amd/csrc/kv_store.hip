// kv_store.hip -- writes K/V rows into the head-major HBM cache and converts
// between the engine layout and the head-major layout.
//
// Geometry: common.hpp (K rows per head; V in 32-position tiles stored
// d-major).  Rounding is the reference CPU f32->f16 (platform.c:340-379), so
// a cache filled here holds the same bits as the engine's (engine.c:1068-1072).
#include "common.hpp"
#include "internal.hpp"

namespace yhip {
namespace {

// source element -> f16 bits: f16 sources are copied, f32/bf16 sources are
// widened exactly and rounded the way the reference rounds
__device__ inline uint16_t to_cache_bits(const void* p, size_t i, uint32_t dt)
{
    if (dt == kF16) return reinterpret_cast<const uint16_t*>(p)[i];
    return f32_to_f16_ref(load_as_f32(p, i, dt));
}

// K rows: one thread per element, consecutive threads walk head_dim, so both
// the source row and the destination row are read/written contiguously.
__global__ __launch_bounds__(256) void k_store_kernel(uint16_t* __restrict__ kc,
                                                      const void* __restrict__ k, uint32_t dt,
                                                      uint32_t pos_start, uint32_t B,
                                                      uint32_t n_kv, uint32_t D,
                                                      uint32_t kv_stride)
{
    const uint32_t kv_dim = n_kv * D;
    const uint64_t idx = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint64_t)B * kv_dim) return;
    const uint32_t b = (uint32_t)(idx / kv_dim), j = (uint32_t)(idx - (uint64_t)b * kv_dim);
    const uint32_t h = j / D, d = j - h * D;
    kc[k_index(h, pos_start + b, d, D, kv_stride)] = to_cache_bits(k, (size_t)b * kv_dim + j, dt);
}

// V rows go to d-major tiles.  A 64(pos) x 64(dim) block is staged in LDS so
// that reads walk source rows and writes walk positions inside a tile.
__global__ __launch_bounds__(256) void v_store_kernel(uint16_t* __restrict__ vc,
                                                      const void* __restrict__ v, uint32_t dt,
                                                      uint32_t v_stride, uint32_t pos_start, uint32_t B,
                                                      uint32_t n_kv, uint32_t D,
                                                      uint32_t kv_stride)
{
    __shared__ uint16_t tile[64][66];
    const uint32_t kv_dim = n_kv * D;
    const uint32_t j0 = blockIdx.x * 64u, b0 = blockIdx.y * 64u;
    const uint32_t tx = threadIdx.x & 63u, ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64u; r += 4u) {
        const uint32_t b = b0 + r, j = j0 + tx;
        if (b < B && j < kv_dim) tile[r][tx] = to_cache_bits(v, (size_t)b * v_stride + j, dt);
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64u; r += 4u) {
        const uint32_t j = j0 + r, b = b0 + tx;
        if (b < B && j < kv_dim) {
            const uint32_t h = j / D, d = j - h * D;
            vc[v_index(h, pos_start + b, d, D, kv_stride)] = tile[tx][r];
        }
    }
}

// Bulk store, K and V in one launch.  A workgroup owns 64 destination
// positions (aligned to 64, so a V group of 8 positions never straddles a
// 32-position tile) times 64 dimensions of one kv head.  Each thread takes
// groups of 8 consecutive dimensions of a row: two 16-byte f32 loads (or
// one f16 / bf16 load), the reference rounding, one 16-byte K store; the V
// group goes through LDS, from which groups of 8 consecutive positions of
// one dimension are read back and stored as 16 bytes into the tile.
// Positions outside [pos_start, pos_start + B) are neither read nor
// written.  Sources are 16-byte aligned rows of n_kv * D elements.
template <uint32_t DT>
__global__ __launch_bounds__(256) void kv_block_kernel(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                       const void* __restrict__ k, const void* __restrict__ v,
                                                       uint32_t pos_start, uint32_t B, uint32_t n_kv, uint32_t D,
                                                       uint32_t kv_stride)
{
    __shared__ uint16_t tv[64][72];  // [position][dimension], rows 144 bytes apart
    const uint32_t kv_dim = n_kv * D;
    const uint32_t j0 = blockIdx.x * 64u;                          // first dimension (one kv head)
    const uint32_t p0 = (pos_start & ~63u) + blockIdx.y * 64u;     // first destination position
    const uint32_t h = j0 / D, d0 = j0 - h * D;
    typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
    auto load8 = [&](const void* src, size_t off, u16x8& out) {
        if constexpr (DT == kF32) {
            const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(src) + off));
            const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(src) + off + 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                out[e] = f32_to_f16_ref(a[e]);
                out[e + 4] = f32_to_f16_ref(b[e]);
            }
        } else {
            const u16x8 w = __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(reinterpret_cast<const uint16_t*>(src) + off));
            if constexpr (DT == kF16) {
                out = w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) out[e] = f32_to_f16_ref(bf16_bits_to_f32(w[e]));
            }
        }
    };
    // both rows' loads go out before any wait: from clamped, always-valid
    // rows (a load under the bounds test waited for the first row's round
    // trip before the second row's was issued); the stores keep the test.
    // The source rows are read once: non-temporal loads (4.34 -> 4.52 TB/s
    // at 8192 rows of 8 kv heads x 128)
    u16x8 kb[2], vb[2];
#pragma unroll
    for (uint32_t it = 0; it < 2; ++it) {
        const uint32_t g = threadIdx.x + 256u * it;  // row g / 8, dimensions 8 (g % 8) ..
        const uint32_t r = g >> 3, c = (g & 7u) * 8u;
        const uint32_t pos = min(max(p0 + r, pos_start), pos_start + B - 1u);
        const size_t off = (size_t)(pos - pos_start) * kv_dim + j0 + c;
        load8(k, off, kb[it]);
        load8(v, off, vb[it]);
    }
#pragma unroll
    for (uint32_t it = 0; it < 2; ++it) {
        const uint32_t g = threadIdx.x + 256u * it;
        const uint32_t r = g >> 3, c = (g & 7u) * 8u;
        const uint32_t pos = p0 + r;
        if (pos < pos_start || pos >= pos_start + B) continue;
        *reinterpret_cast<u16x8*>(kc + k_index(h, pos, d0 + c, D, kv_stride)) = kb[it];
        *reinterpret_cast<u16x8*>(&tv[r][c]) = vb[it];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t it = 0; it < 2; ++it) {
        const uint32_t g = threadIdx.x + 256u * it;  // dimension g / 8, positions 8 (g % 8) ..
        const uint32_t dl = g >> 3, r0 = (g & 7u) * 8u;
        const uint32_t pos0 = p0 + r0;
        u16x8 w;
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = tv[r0 + e][dl];
        uint16_t* dst = vc + v_index(h, pos0, d0 + dl, D, kv_stride);
        if (pos0 >= pos_start && pos0 + 8u <= pos_start + B) {
            *reinterpret_cast<u16x8*>(dst) = w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (pos0 + e >= pos_start && pos0 + e < pos_start + B) dst[e] = w[e];
        }
    }
}

// A few rows (decode appends one per step): K and V elements in one launch,
// one thread per (row, element); the V writes are 2-byte scatters into the
// tiles, which is cheap at this size and saves the second launch.
__global__ __launch_bounds__(256) void kv_rows_kernel(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                      const void* __restrict__ k, const void* __restrict__ v,
                                                      uint32_t dt, uint32_t pos_start, uint32_t B, uint32_t n_kv,
                                                      uint32_t D, uint32_t kv_stride)
{
    const uint32_t kv_dim = n_kv * D;
    const uint64_t idx = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint64_t)B * kv_dim) return;
    const uint32_t b = (uint32_t)(idx / kv_dim), j = (uint32_t)(idx - (uint64_t)b * kv_dim);
    const uint32_t h = j / D, d = j - h * D;
    kc[k_index(h, pos_start + b, d, D, kv_stride)] = to_cache_bits(k, (size_t)b * kv_dim + j, dt);
    vc[v_index(h, pos_start + b, d, D, kv_stride)] = to_cache_bits(v, (size_t)b * kv_dim + j, dt);
}

// V tiles -> engine V rows (bits copied)
__global__ __launch_bounds__(256) void v_to_engine_kernel(uint16_t* __restrict__ ev,
                                                          const uint16_t* __restrict__ vc,
                                                          uint32_t rows, uint32_t n_kv, uint32_t D,
                                                          uint32_t kv_stride)
{
    __shared__ uint16_t tile[64][66];
    const uint32_t kv_dim = n_kv * D;
    const uint32_t j0 = blockIdx.x * 64u, b0 = blockIdx.y * 64u;
    const uint32_t tx = threadIdx.x & 63u, ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64u; r += 4u) {
        const uint32_t j = j0 + r, b = b0 + tx;
        if (b < rows && j < kv_dim) {
            const uint32_t h = j / D, d = j - h * D;
            tile[r][tx] = vc[v_index(h, b, d, D, kv_stride)];
        }
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64u; r += 4u) {
        const uint32_t b = b0 + r, j = j0 + tx;
        if (b < rows && j < kv_dim) ev[(size_t)b * kv_dim + j] = tile[tx][r];
    }
}

// K: engine rows <-> head-major rows (bits copied); dir 0 = to head-major
__global__ __launch_bounds__(256) void k_copy_kernel(uint16_t* __restrict__ kc,
                                                     uint16_t* __restrict__ ek, uint32_t rows,
                                                     uint32_t n_kv, uint32_t D,
                                                     uint32_t kv_stride, int dir)
{
    const uint32_t kv_dim = n_kv * D;
    const uint64_t idx = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint64_t)rows * kv_dim) return;
    const uint32_t b = (uint32_t)(idx / kv_dim), j = (uint32_t)(idx - (uint64_t)b * kv_dim);
    const uint32_t h = j / D, d = j - h * D;
    const size_t hm = k_index(h, b, d, D, kv_stride);
    const size_t en = (size_t)b * kv_dim + j;
    if (dir == 0) kc[hm] = ek[en];
    else ek[en] = kc[hm];
}

}  // namespace

hipError_t launch_kv_store(uint16_t* kc, uint16_t* vc, const void* k, const void* v, uint32_t dt,
                           uint32_t pos_start, uint32_t B, uint32_t n_kv, uint32_t D,
                           uint32_t kv_stride, hipStream_t st)
{
    const uint32_t kv_dim = n_kv * D;
    dim3 gk((uint32_t)(((uint64_t)B * kv_dim + 255u) / 256u));
    if (B <= 4) {
        hipLaunchKernelGGL(kv_rows_kernel, gk, dim3(256), 0, st, kc, vc, k, v, dt, pos_start, B, n_kv, D, kv_stride);
        return hipGetLastError();
    }
    const bool aligned = ((uintptr_t)k % 16u) == 0 && ((uintptr_t)v % 16u) == 0 && ((uintptr_t)kc % 16u) == 0 &&
                         ((uintptr_t)vc % 16u) == 0;
    if (aligned && D % 64u == 0) {
        // K and V in one launch, 64 aligned destination positions x 64 dimensions per workgroup
        const dim3 gb(kv_dim / 64u, ((pos_start & 63u) + B + 63u) / 64u);
        switch (dt) {
        case kF32: hipLaunchKernelGGL(kv_block_kernel<kF32>, gb, dim3(256), 0, st, kc, vc, k, v, pos_start, B, n_kv,
                                      D, kv_stride); break;
        case kF16: hipLaunchKernelGGL(kv_block_kernel<kF16>, gb, dim3(256), 0, st, kc, vc, k, v, pos_start, B, n_kv,
                                      D, kv_stride); break;
        default: hipLaunchKernelGGL(kv_block_kernel<kBF16>, gb, dim3(256), 0, st, kc, vc, k, v, pos_start, B, n_kv,
                                    D, kv_stride); break;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_store_kernel, gk, dim3(256), 0, st, kc, k, dt, pos_start, B, n_kv, D,
                       kv_stride);
    dim3 gv((kv_dim + 63u) / 64u, (B + 63u) / 64u);
    hipLaunchKernelGGL(v_store_kernel, gv, dim3(256), 0, st, vc, v, dt, kv_dim, pos_start, B, n_kv, D,
                       kv_stride);
    return hipGetLastError();
}

hipError_t launch_kv_from_engine(uint16_t* kc, uint16_t* vc, const uint16_t* ek, const uint16_t* ev,
                                 uint32_t rows, uint32_t n_kv, uint32_t D, uint32_t kv_stride,
                                 hipStream_t st)
{
    // f16 engine rows are a store of f16 sources (their bits are copied)
    return launch_kv_store(kc, vc, ek, ev, kF16, 0u, rows, n_kv, D, kv_stride, st);
}

hipError_t launch_kv_to_engine(uint16_t* ek, uint16_t* ev, const uint16_t* kc, const uint16_t* vc,
                               uint32_t rows, uint32_t n_kv, uint32_t D, uint32_t kv_stride,
                               hipStream_t st)
{
    const uint32_t kv_dim = n_kv * D;
    dim3 gk((uint32_t)(((uint64_t)rows * kv_dim + 255u) / 256u));
    hipLaunchKernelGGL(k_copy_kernel, gk, dim3(256), 0, st, const_cast<uint16_t*>(kc), ek, rows, n_kv,
                       D, kv_stride, 1);
    dim3 gv((kv_dim + 63u) / 64u, (rows + 63u) / 64u);
    hipLaunchKernelGGL(v_to_engine_kernel, gv, dim3(256), 0, st, ev, vc, rows, n_kv, D, kv_stride);
    return hipGetLastError();
}

}  // namespace yhip
