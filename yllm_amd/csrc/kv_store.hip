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
    const uint32_t kv_dim = n_kv * D;
    dim3 gk((uint32_t)(((uint64_t)rows * kv_dim + 255u) / 256u));
    hipLaunchKernelGGL(k_copy_kernel, gk, dim3(256), 0, st, kc, const_cast<uint16_t*>(ek), rows, n_kv,
                       D, kv_stride, 0);
    // f16 bits through the same tiler as the store (f16 sources are copied)
    dim3 gv((kv_dim + 63u) / 64u, (rows + 63u) / 64u);
    hipLaunchKernelGGL(v_store_kernel, gv, dim3(256), 0, st, vc, (const void*)ev, kF16, kv_dim, 0u, rows, n_kv,
                       D, kv_stride);
    return hipGetLastError();
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
