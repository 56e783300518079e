// decode_noalloc.hip -- yhip_attn_decode_batch_noalloc: the batched decode
// with its split-K partials in a fixed device array of this library instead
// of a caller's workspace, for callers that cannot allocate (code under HIP
// graph capture, serving loops that forbid hipMalloc).  It shares the
// checks, plan and kernels of yhip_attn_decode_batch.
#include "../../include/yllm_hip.h"
#include "internal.hpp"

#include <mutex>
#include <stdio.h>

namespace {

// Each GPU holds its own copy of this array until the process ends.  In host
// code the name is only a stand-in for the device symbol: its device address
// comes from hipGetSymbolAddress, once per device with that device current,
// and only that address is handed to kernels.
constexpr size_t kScratchBytes = YHIP_DECODE_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];  // device address of `scratch`, per device

// The current device's address of `scratch`, resolved on the first call on
// that device; null with *rc and the message set on failure.
void* scratch_of_current_device(const char* fn, int* rc)
{
    char msg[256];
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        snprintf(msg, sizeof msg, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
        *rc = yhip::api_fail(YHIP_EDEVICE, msg);
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        snprintf(msg, sizeof msg, "%s: device %d beyond the %d supported", fn, dev, kMaxDevices);
        *rc = yhip::api_fail(YHIP_EDEVICE, msg);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            snprintf(msg, sizeof msg, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
            *rc = yhip::api_fail(YHIP_EDEVICE, msg);
            return nullptr;
        }
        g_ptr[dev] = ptr;
    }
    return g_ptr[dev];
}

}  // namespace

extern "C" int yhip_attn_decode_batch_noalloc(float* att_out, uint32_t out_stride, const float* q,
                                              uint32_t q_stride, const uint16_t* const* kcaches,
                                              const uint16_t* const* vcaches, const uint32_t* lens,
                                              uint32_t n_seq, uint32_t max_len, uint64_t total_len,
                                              uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                              uint32_t kv_stride, const float* gate, uint32_t gate_stride,
                                              void* stream)
{
    const char* fn = "yhip_attn_decode_batch_noalloc";
    // The scratch is resolved only when the plan has partials that fit it;
    // shapes that do not fit fail in the shared checks (after the argument
    // checks) with YHIP_ENOSPC.  The partials need no initialisation: the
    // merge reads only the splits the split kernel of the same call wrote.
    void* ws = nullptr;
    if (n_kv_heads != 0 && n_seq != 0 && max_len != 0) {
        uint32_t sk = 0, ns = 0;
        const size_t need = yhip::decode_plan(n_seq, max_len, total_len, n_heads, n_kv_heads, head_dim, &sk, &ns);
        if (need > 0 && need <= kScratchBytes) {
            int rc = 0;
            ws = scratch_of_current_device(fn, &rc);
            if (!ws) return rc;
        }
    }
    return yhip::decode_batch_common(fn, att_out, out_stride, q, q_stride, kcaches, vcaches, lens, n_seq, max_len,
                                     total_len, n_heads, n_kv_heads, head_dim, kv_stride, gate, gate_stride, ws,
                                     kScratchBytes, "library's fixed scratch (call yhip_attn_decode_batch with a "
                                     "workspace instead)", stream);
}
