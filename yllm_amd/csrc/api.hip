// api.hip -- the extern "C" entry points declared in include/yllm_hip.h:
// argument validation, split planning and kernel launches.  No allocation
// happens here: workspaces come from the caller.
#include "../../include/yllm_hip.h"
#include "internal.hpp"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace {

thread_local char g_err[512];

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int done(hipError_t e, const char* what)
{
    if (e != hipSuccess) return fail(YHIP_EDEVICE, "%s: %s", what, hipGetErrorString(e));
    g_err[0] = 0;
    return YHIP_OK;
}

bool valid_head_dim(uint32_t d) { return d == 64 || d == 128 || d == 256; }
bool valid_dtype(uint32_t t) { return t == YHIP_F16 || t == YHIP_F32 || t == YHIP_BF16; }

// shared shape checks of the attention entry points
int check_heads(const char* fn, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t kv_stride)
{
    if (!valid_head_dim(head_dim)) return fail(YHIP_EINVAL, "%s: head_dim %u not in {64,128,256}", fn, head_dim);
    if (n_heads == 0 || n_kv == 0 || n_kv > n_heads)
        return fail(YHIP_EINVAL, "%s: need 1 <= n_kv_heads (%u) <= n_heads (%u)", fn, n_kv, n_heads);
    if ((n_heads + n_kv - 1) / n_kv > 16)
        return fail(YHIP_EINVAL, "%s: more than 16 query heads per kv head (%u/%u)", fn, n_heads, n_kv);
    if (kv_stride == 0 || kv_stride % 64 != 0)
        return fail(YHIP_EINVAL, "%s: kv_stride %u must be a positive multiple of 64", fn, kv_stride);
    // the kernels address one kv head's K rows or V tiles with 32-bit buffer
    // offsets and use offsets from 2 GiB up as "past the end"
    if ((uint64_t)kv_stride * head_dim * 2 >= 0x80000000ull)
        return fail(YHIP_EINVAL, "%s: one kv head's cache (kv_stride %u x head_dim %u) must stay under 2 GiB", fn,
                    kv_stride, head_dim);
    return 0;
}

}  // namespace

extern "C" {

const char* yhip_last_error(void) { return g_err; }

const char* yhip_version(void) { return "yllm-hip 0.1 (gfx950)"; }

uint64_t yhip_kv_layer_elems(uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride)
{
    return (uint64_t)n_kv_heads * head_dim * kv_stride;
}

int yhip_kv_store(uint16_t* kcache, uint16_t* vcache, const void* k, const void* v,
                  uint32_t src_dtype, uint32_t pos_start, uint32_t B, uint32_t n_kv_heads,
                  uint32_t head_dim, uint32_t kv_stride, void* stream)
{
    if (!kcache || !vcache || !k || !v) return fail(YHIP_EINVAL, "yhip_kv_store: null pointer");
    if (!valid_dtype(src_dtype)) return fail(YHIP_EINVAL, "yhip_kv_store: bad src_dtype %u", src_dtype);
    if (!valid_head_dim(head_dim) || n_kv_heads == 0)
        return fail(YHIP_EINVAL, "yhip_kv_store: bad n_kv_heads %u / head_dim %u", n_kv_heads, head_dim);
    if (kv_stride == 0 || kv_stride % 64 != 0)
        return fail(YHIP_EINVAL, "yhip_kv_store: kv_stride %u must be a positive multiple of 64", kv_stride);
    if ((uint64_t)pos_start + B > kv_stride)
        return fail(YHIP_EINVAL, "yhip_kv_store: rows %u..%u exceed kv_stride %u", pos_start,
                    pos_start + B, kv_stride);
    if (B == 0) return done(hipSuccess, "");
    return done(yhip::launch_kv_store(kcache, vcache, k, v, src_dtype, pos_start, B, n_kv_heads,
                                      head_dim, kv_stride, (hipStream_t)stream),
                "yhip_kv_store");
}

int yhip_kv_from_engine(uint16_t* kcache, uint16_t* vcache, const uint16_t* eng_k,
                        const uint16_t* eng_v, uint32_t n_rows, uint32_t n_kv_heads,
                        uint32_t head_dim, uint32_t kv_stride, void* stream)
{
    if (!kcache || !vcache || !eng_k || !eng_v) return fail(YHIP_EINVAL, "yhip_kv_from_engine: null pointer");
    if (!valid_head_dim(head_dim) || n_kv_heads == 0 || kv_stride % 64 != 0 || n_rows > kv_stride)
        return fail(YHIP_EINVAL, "yhip_kv_from_engine: bad shape");
    if (n_rows == 0) return done(hipSuccess, "");
    return done(yhip::launch_kv_from_engine(kcache, vcache, eng_k, eng_v, n_rows, n_kv_heads, head_dim,
                                            kv_stride, (hipStream_t)stream),
                "yhip_kv_from_engine");
}

int yhip_kv_to_engine(uint16_t* eng_k, uint16_t* eng_v, const uint16_t* kcache,
                      const uint16_t* vcache, uint32_t n_rows, uint32_t n_kv_heads,
                      uint32_t head_dim, uint32_t kv_stride, void* stream)
{
    if (!kcache || !vcache || !eng_k || !eng_v) return fail(YHIP_EINVAL, "yhip_kv_to_engine: null pointer");
    if (!valid_head_dim(head_dim) || n_kv_heads == 0 || kv_stride % 64 != 0 || n_rows > kv_stride)
        return fail(YHIP_EINVAL, "yhip_kv_to_engine: bad shape");
    if (n_rows == 0) return done(hipSuccess, "");
    return done(yhip::launch_kv_to_engine(eng_k, eng_v, kcache, vcache, n_rows, n_kv_heads, head_dim,
                                          kv_stride, (hipStream_t)stream),
                "yhip_kv_to_engine");
}

size_t yhip_attn_decode_workspace(uint32_t n_seq, uint32_t max_len, uint64_t total_len,
                                  uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim)
{
    if (n_kv_heads == 0) return 0;
    return yhip::decode_workspace_bound(n_seq, max_len, total_len, n_heads, n_kv_heads, head_dim);
}

}  // extern "C"

namespace yhip {

int decode_batch_common(const char* fn, float* att_out, uint32_t out_stride, const float* q, uint32_t q_stride,
                        const uint16_t* const* kcaches, const uint16_t* const* vcaches, const uint32_t* lens,
                        uint32_t n_seq, uint32_t max_len, uint64_t total_len, uint32_t n_heads,
                        uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride, const float* gate,
                        uint32_t gate_stride, void* workspace, size_t workspace_bytes, const char* ws_name,
                        void* stream)
{
    if (!att_out || !q || !kcaches || !vcaches || !lens) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    int rc = check_heads(fn, n_heads, n_kv_heads, head_dim, kv_stride);
    if (rc) return rc;
    if (n_seq == 0) return done(hipSuccess, "");
    if (n_seq > 65535) return fail(YHIP_EINVAL, "%s: n_seq %u > 65535", fn, n_seq);
    if (max_len == 0 || max_len > kv_stride)
        return fail(YHIP_EINVAL, "%s: max_len %u must be in 1..kv_stride (%u)", fn, max_len, kv_stride);
    const uint32_t row = n_heads * head_dim;
    if (q_stride < row || out_stride < row || q_stride % 4 || out_stride % 4)
        return fail(YHIP_EINVAL, "%s: q_stride/out_stride must be >= n_heads*head_dim and a multiple of 4", fn);
    if (gate && gate_stride < row) return fail(YHIP_EINVAL, "%s: gate_stride too small", fn);
    yhip::DecodeArgs a = {};
    const size_t need = yhip::decode_plan(n_seq, max_len, total_len, n_heads, n_kv_heads, head_dim,
                                          &a.split_keys, &a.n_splits);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(YHIP_ENOSPC, "%s: these shapes need %zu bytes of split partials, the %s holds %zu", fn, need,
                    ws_name, workspace_bytes);
    a.q = q;
    a.kptrs = kcaches;
    a.vptrs = vcaches;
    a.lens = lens;
    a.out = att_out;
    a.gate = gate;
    a.n_seq = n_seq;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.D = head_dim;
    a.kv_stride = kv_stride;
    a.q_stride = q_stride;
    a.out_stride = out_stride;
    a.gate_stride = gate_stride;
    a.c = (float)(1.4426950408889634 / sqrt((double)head_dim));
    yhip::decode_bind_workspace(a, workspace);
    return done(yhip::launch_decode(a, (hipStream_t)stream), fn);
}

int api_fail(int code, const char* msg) { return fail(code, "%s", msg); }

}  // namespace yhip

namespace {

// The reference's frequency formula (matvec.c:895) with the host powf, for
// the rotated pairs j < span / 2; the last table is kept per thread.
void rope_freqs(float* freq, uint32_t rope, uint32_t span, float theta)
{
    if (rope == YHIP_ROPE_NONE) return;
    thread_local float t_theta = 0.0f;
    thread_local uint32_t t_span = 0;
    thread_local float t_freq[128];
    if (t_span != span || !(t_theta == theta)) {
        for (uint32_t j = 0; j < span / 2; ++j) t_freq[j] = powf(theta, -2.0f * (float)j / (float)span);
        t_span = span;
        t_theta = theta;
    }
    memcpy(freq, t_freq, sizeof(float) * (span / 2));
}

}  // namespace

extern "C" {

int yhip_attn_decode_batch(float* att_out, uint32_t out_stride, const float* q,
                           uint32_t q_stride, const uint16_t* const* kcaches,
                           const uint16_t* const* vcaches, const uint32_t* lens,
                           uint32_t n_seq, uint32_t max_len, uint64_t total_len,
                           uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                           uint32_t kv_stride, const float* gate, uint32_t gate_stride,
                           void* workspace, size_t workspace_bytes, void* stream)
{
    return yhip::decode_batch_common("yhip_attn_decode_batch", att_out, out_stride, q, q_stride, kcaches, vcaches, lens,
                               n_seq, max_len, total_len, n_heads, n_kv_heads, head_dim, kv_stride, gate,
                               gate_stride, workspace, workspace_bytes, "workspace", stream);
}


int yhip_attn_decode(float* att_out, const float* q, const uint16_t* kcache,
                     const uint16_t* vcache, uint32_t pos, uint32_t n_heads,
                     uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride,
                     const float* gate, void* workspace, size_t workspace_bytes, void* stream)
{
    const char* fn = "yhip_attn_decode";
    if (!att_out || !q || !kcache || !vcache) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    int rc = check_heads(fn, n_heads, n_kv_heads, head_dim, kv_stride);
    if (rc) return rc;
    if (pos >= kv_stride) return fail(YHIP_EINVAL, "%s: pos %u >= kv_stride %u", fn, pos, kv_stride);
    yhip::DecodeArgs a = {};
    const uint32_t len = pos + 1;
    const size_t need = yhip::decode_plan(1, len, len, n_heads, n_kv_heads, head_dim, &a.split_keys,
                                          &a.n_splits);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(YHIP_ENOSPC, "%s: workspace %zu < %zu bytes", fn, workspace_bytes, need);
    a.q = q;
    a.k0 = kcache;
    a.v0 = vcache;
    a.len0 = len;
    a.out = att_out;
    a.gate = gate;
    a.n_seq = 1;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.D = head_dim;
    a.kv_stride = kv_stride;
    a.q_stride = n_heads * head_dim;
    a.out_stride = n_heads * head_dim;
    a.gate_stride = n_heads * head_dim;
    a.c = (float)(1.4426950408889634 / sqrt((double)head_dim));
    yhip::decode_bind_workspace(a, workspace);
    return done(yhip::launch_decode(a, (hipStream_t)stream), fn);
}

int yhip_attn_decode_rope(float* att_out, const float* q, const float* k, const float* v, uint16_t* kcache,
                          uint16_t* vcache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t kv_stride, uint32_t rope, uint32_t n_rot, float theta, const float* gate,
                          void* workspace, size_t workspace_bytes, void* stream)
{
    const char* fn = "yhip_attn_decode_rope";
    if (!att_out || !q || !k || !v || !kcache || !vcache) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    int rc = check_heads(fn, n_heads, n_kv_heads, head_dim, kv_stride);
    if (rc) return rc;
    if (pos >= kv_stride) return fail(YHIP_EINVAL, "%s: pos %u >= kv_stride %u", fn, pos, kv_stride);
    if (rope > YHIP_ROPE_MROPE) return fail(YHIP_EINVAL, "%s: unknown rope kind %u", fn, rope);
    if (rope == YHIP_ROPE_MROPE && (n_rot == 0 || n_rot % 8 || n_rot > head_dim))
        return fail(YHIP_EINVAL, "%s: n_rot %u must be a multiple of 8 and at most head_dim", fn, n_rot);
    if ((uintptr_t)q % 16 || (uintptr_t)att_out % 16)
        return fail(YHIP_EINVAL, "%s: q and att_out must be 16-byte aligned", fn);
    yhip::DecodeArgs a = {};
    const uint32_t len = pos + 1;
    const size_t need = yhip::decode_plan(1, len, len, n_heads, n_kv_heads, head_dim, &a.split_keys,
                                          &a.n_splits);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(YHIP_ENOSPC, "%s: workspace %zu < %zu bytes", fn, workspace_bytes, need);
    a.q = q;
    a.k0 = kcache;
    a.v0 = vcache;
    a.len0 = len;
    a.out = att_out;
    a.gate = gate;
    a.n_seq = 1;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.D = head_dim;
    a.kv_stride = kv_stride;
    a.q_stride = n_heads * head_dim;
    a.out_stride = n_heads * head_dim;
    a.gate_stride = n_heads * head_dim;
    a.c = (float)(1.4426950408889634 / sqrt((double)head_dim));
    yhip::decode_bind_workspace(a, workspace);
    yhip::DecodeRope r = {};
    r.k = k;
    r.v = v;
    r.kc = kcache;
    r.vc = vcache;
    r.kind = rope;
    r.n_rot = rope == YHIP_ROPE_MROPE ? n_rot : head_dim;
    if (rope != YHIP_ROPE_NONE) {
        // the angles and their cosines and sines as the reference forms them
        // (matvec.c:895-898: host powf, float product, cosf, sinf)
        float freq[128];
        rope_freqs(freq, rope, r.n_rot, theta);
        for (uint32_t j = 0; j < r.n_rot / 2; ++j) {
            const float ang = freq[j] * (float)pos;
            r.cs[0][j] = cosf(ang);
            r.cs[1][j] = sinf(ang);
        }
    }
    return done(yhip::launch_decode_rope(a, r, (hipStream_t)stream), fn);
}

size_t yhip_attn_prefill_workspace(uint32_t B, uint32_t max_end, uint32_t n_heads, uint32_t n_kv_heads,
                                   uint32_t head_dim)
{
    if (n_kv_heads == 0 || !valid_head_dim(head_dim)) return 0;
    return yhip::prefill_workspace_bound(B, max_end, n_heads, n_kv_heads, head_dim);
}

int yhip_attn_prefill(void* att_out, uint32_t out_dtype, uint32_t out_stride, const void* q,
                      uint32_t q_dtype, uint32_t q_stride, const uint16_t* kcache,
                      const uint16_t* vcache, uint32_t pos_start, uint32_t B, uint32_t n_heads,
                      uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride,
                      const float* gate, uint32_t gate_stride, void* workspace, size_t workspace_bytes,
                      void* stream)
{
    const char* fn = "yhip_attn_prefill";
    if (!att_out || !q || !kcache || !vcache) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (!valid_dtype(out_dtype) || !valid_dtype(q_dtype)) return fail(YHIP_EINVAL, "%s: bad dtype", fn);
    int rc = check_heads(fn, n_heads, n_kv_heads, head_dim, kv_stride);
    if (rc) return rc;
    if ((uint64_t)pos_start + B > kv_stride)
        return fail(YHIP_EINVAL, "%s: positions %u..%u exceed kv_stride %u", fn, pos_start, pos_start + B,
                    kv_stride);
    const uint32_t row = n_heads * head_dim;
    if (q_stride < row || out_stride < row || q_stride % 8 || out_stride % 8)
        return fail(YHIP_EINVAL, "%s: q_stride/out_stride must be >= n_heads*head_dim and a multiple of 8", fn);
    if (gate && gate_stride < row) return fail(YHIP_EINVAL, "%s: gate_stride too small", fn);
    if (B == 0) return done(hipSuccess, "");
    const uint64_t nblocks = (uint64_t)(B + 127) / 128 * n_heads;
    if (nblocks > 0x7fffffffull) return fail(YHIP_EINVAL, "%s: grid too large", fn);
    yhip::PrefillArgs a = {};
    a.q = q;
    a.q_dtype = q_dtype;
    a.q_stride = q_stride;
    a.kc = kcache;
    a.vc = vcache;
    a.kv_stride = kv_stride;
    a.out = att_out;
    a.out_dtype = out_dtype;
    a.out_stride = out_stride;
    a.gate = gate;
    a.gate_stride = gate_stride;
    a.pos_start = pos_start;
    a.B = B;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.D = head_dim;
    a.c = (float)(1.4426950408889634 / sqrt((double)head_dim));
    // a launch with few work items splits the keys when a workspace is given
    // for the partials; without one it runs unsplit
    size_t need = yhip::prefill_plan(a);
    if (need > 0 && !workspace) {
        a.n_split = 1;
        a.split_tiles = (pos_start + B - 1) / yhip::prefill_tile_keys(head_dim) + 1;
        need = 0;
    }
    if (need > 0 && (workspace_bytes < need || (uintptr_t)workspace % 16))
        return fail(YHIP_ENOSPC, "%s: the key split needs %zu bytes of workspace (16-byte aligned), %zu given", fn,
                    need, workspace_bytes);
    yhip::prefill_bind_workspace(a, workspace);
    return done(yhip::launch_prefill(a, (hipStream_t)stream), fn);
}

// S_out: NULL (or S) updates S in place; otherwise the state after the call
// goes to S_out, which must not overlap S, and S is left as it was.
static int state_out_ok(const char* fn, const float* S, float*& S_out, size_t floats)
{
    if (!S_out) S_out = const_cast<float*>(S);
    if (S_out == S) return 0;
    if ((uintptr_t)S_out & 15) return fail(YHIP_EINVAL, "%s: S_out must be 16-byte aligned", fn);
    const char *a0 = (const char*)S, *a1 = a0 + floats * sizeof(float);
    const char *b0 = (const char*)S_out, *b1 = b0 + floats * sizeof(float);
    if (b0 < a1 && a0 < b1) return fail(YHIP_EINVAL, "%s: S_out overlaps S without being S", fn);
    return 0;
}

static int gdn_common(const char* fn, float* S, float* S_out, float* out, uint32_t out_stride, const float* q,
                      const float* k, uint32_t qk_stride, const float* v, uint32_t v_stride, const float* gate,
                      const float* beta, uint32_t T, uint32_t n_k, uint32_t n_v, uint32_t head_dim, float eps,
                      void* workspace, size_t workspace_bytes, void* stream)
{
    if (!S || !out || !q || !k || !v || !gate || !beta) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (head_dim != 64 && head_dim != 128) return fail(YHIP_EINVAL, "%s: head_dim %u not in {64,128}", fn, head_dim);
    if (n_k == 0 || n_v == 0) return fail(YHIP_EINVAL, "%s: need n_k_heads >= 1 and n_v_heads >= 1", fn);
    if (qk_stride < n_k * head_dim || v_stride < n_v * head_dim || out_stride < n_v * head_dim ||
        qk_stride % 4 || v_stride % 4 || out_stride % 4)
        return fail(YHIP_EINVAL, "%s: strides must cover the heads and be multiples of 4", fn);
    if (((uintptr_t)S | (uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15)
        return fail(YHIP_EINVAL, "%s: S, q, k, v must be 16-byte aligned", fn);
    const size_t state_floats = (size_t)n_v * head_dim * head_dim;
    if (int rc = state_out_ok(fn, S, S_out, state_floats)) return rc;
    if (T == 0)  // no token: the state after the call is the state before it
        return done(S_out == S ? hipSuccess
                               : hipMemcpyAsync(S_out, S, state_floats * sizeof(float), hipMemcpyDeviceToDevice,
                                                (hipStream_t)stream),
                    fn);
    yhip::GdnArgs a = {};
    a.S = S;
    a.S_out = S_out;
    a.out = out;
    a.q = q;
    a.k = k;
    a.v = v;
    a.gate = gate;
    a.beta = beta;
    a.T = T;
    a.n_k = n_k;
    a.n_v = n_v;
    a.D = head_dim;
    a.qk_stride = qk_stride;
    a.v_stride = v_stride;
    a.out_stride = out_stride;
    a.eps = eps;
    // the chunked form runs when a workspace is given and the sequence fills a chunk
    if (workspace && T >= yhip::gdn_chunk_tokens()) {
        const size_t need = yhip::gdn_chunk_workspace(T, n_v, head_dim);
        if (workspace_bytes < need)
            return fail(YHIP_ENOSPC, "%s: workspace of %zu bytes, need %zu", fn, workspace_bytes, need);
        if ((uintptr_t)workspace & 15) return fail(YHIP_EINVAL, "%s: workspace must be 16-byte aligned", fn);
        a.ws = reinterpret_cast<float*>(workspace);
        a.n_chunks = (T + yhip::gdn_chunk_tokens() - 1) / yhip::gdn_chunk_tokens();
    }
    return done(yhip::launch_gdn(a, (hipStream_t)stream), fn);
}

int yhip_gdn_step(float* S, float* out, const float* q, const float* k, const float* v, const float* gate,
                  const float* beta, uint32_t n_k_heads, uint32_t n_v_heads, uint32_t head_dim, float l2_eps,
                  void* stream)
{
    return gdn_common("yhip_gdn_step", S, S, out, n_v_heads * head_dim, q, k, n_k_heads * head_dim, v,
                      n_v_heads * head_dim, gate, beta, 1, n_k_heads, n_v_heads, head_dim, l2_eps, nullptr, 0,
                      stream);
}

int yhip_gdn_chunk(float* S, float* S_out, float* out, uint32_t out_stride, const float* q, const float* k,
                   uint32_t qk_stride, const float* v, uint32_t v_stride, const float* gate, const float* beta,
                   uint32_t T, uint32_t n_k_heads, uint32_t n_v_heads, uint32_t head_dim, float l2_eps,
                   void* workspace, size_t workspace_bytes, void* stream)
{
    return gdn_common("yhip_gdn_chunk", S, S_out, out, out_stride, q, k, qk_stride, v, v_stride, gate, beta, T,
                      n_k_heads, n_v_heads, head_dim, l2_eps, workspace, workspace_bytes, stream);
}

size_t yhip_gdn_chunk_workspace(uint32_t T, uint32_t n_v_heads, uint32_t head_dim)
{
    if ((head_dim != 64 && head_dim != 128) || T < yhip::gdn_chunk_tokens()) return 0;
    return yhip::gdn_chunk_workspace(T, n_v_heads, head_dim);
}

int yhip_rope_kv_store(void* q_out, uint32_t q_out_dtype, uint32_t q_out_stride, const float* q, uint32_t q_stride,
                       const float* k, uint32_t k_stride, const float* v, uint32_t v_stride, uint16_t* kcache,
                       uint16_t* vcache, uint32_t pos_start, uint32_t B, uint32_t n_heads, uint32_t n_kv_heads,
                       uint32_t head_dim, uint32_t kv_stride, uint32_t rope, uint32_t n_rot, float theta,
                       void* stream)
{
    const char* fn = "yhip_rope_kv_store";
    int rc = check_heads(fn, n_heads, n_kv_heads, head_dim, kv_stride);
    if (rc) return rc;
    if (!k || !v || !kcache || !vcache || (q_out && !q)) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (rope > YHIP_ROPE_MROPE) return fail(YHIP_EINVAL, "%s: unknown rope kind %u", fn, rope);
    if (rope == YHIP_ROPE_MROPE && (n_rot == 0 || n_rot % 2 || n_rot > head_dim))
        return fail(YHIP_EINVAL, "%s: n_rot %u must be even and at most head_dim", fn, n_rot);
    if (q_out && !valid_dtype(q_out_dtype)) return fail(YHIP_EINVAL, "%s: bad q_out dtype", fn);
    const uint64_t kv_dim = (uint64_t)n_kv_heads * head_dim, qd = (uint64_t)n_heads * head_dim;
    if (k_stride < kv_dim || v_stride < kv_dim || (q_out && (q_stride < qd || q_out_stride < qd)))
        return fail(YHIP_EINVAL, "%s: strides must cover the heads", fn);
    if ((uint64_t)pos_start + B > kv_stride)
        return fail(YHIP_EINVAL, "%s: rows %u..%u exceed kv_stride %u", fn, pos_start, pos_start + B, kv_stride);
    // pairs of adjacent elements move as one 8-byte (f32) or 4-byte (f16/bf16) access
    const uint32_t qo_align = q_out_dtype == YHIP_F32 ? 8u : 4u;
    if ((uintptr_t)k % 8 || (uintptr_t)v % 8 || (uintptr_t)kcache % 4 || k_stride % 2 || v_stride % 2 ||
        (q_out && ((uintptr_t)q % 8 || (uintptr_t)q_out % qo_align || q_stride % 2 || q_out_stride % 2)))
        return fail(YHIP_EINVAL, "%s: q/k/v must be 8-byte aligned with even strides", fn);
    if (B == 0) return done(hipSuccess, "");
    yhip::RopeArgs a = {};
    a.q_out = q_out;
    a.q = q;
    a.k = k;
    a.v = v;
    a.kc = kcache;
    a.vc = vcache;
    a.q_out_dtype = q_out_dtype;
    a.q_out_stride = q_out_stride;
    a.q_stride = q_stride;
    a.k_stride = k_stride;
    a.v_stride = v_stride;
    a.pos_start = pos_start;
    a.B = B;
    a.n_heads = n_heads;
    a.n_kv = n_kv_heads;
    a.D = head_dim;
    a.kv_stride = kv_stride;
    a.kind = rope;
    a.n_rot = rope == YHIP_ROPE_MROPE ? n_rot : head_dim;
    rope_freqs(a.freq, rope, a.n_rot, theta);
    return done(yhip::launch_rope_kv(a, (hipStream_t)stream), fn);
}

size_t yhip_o_proj_workspace(uint32_t B, uint32_t hidden, uint32_t qdim, uint32_t w_dtype, uint32_t att_dtype)
{
    return yhip::oproj_workspace(B, qdim, w_dtype == YHIP_F16, att_dtype == YHIP_F16, hidden);
}

int yhip_o_proj(float* x, uint32_t x_stride, const void* att, uint32_t att_dtype, uint32_t att_stride,
                const void* w, uint32_t w_dtype, uint32_t B, uint32_t hidden, uint32_t qdim, void* workspace,
                size_t workspace_bytes, void* stream)
{
    const char* fn = "yhip_o_proj";
    if (!x || !att || !w) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (w_dtype != YHIP_F16 && w_dtype != YHIP_F32)
        return fail(YHIP_EINVAL, "%s: w_dtype must be YHIP_F16 or YHIP_F32", fn);
    if (att_dtype != YHIP_F32 && !(att_dtype == YHIP_F16 && w_dtype == YHIP_F16))
        return fail(YHIP_EINVAL, "%s: att_dtype must be YHIP_F32, or YHIP_F16 with f16 weights", fn);
    if (hidden == 0 || qdim == 0 || qdim % 8) return fail(YHIP_EINVAL, "%s: qdim %u must be a positive multiple of 8", fn, qdim);
    if (x_stride < hidden || att_stride < qdim || att_stride % 8 || x_stride >= (1u << 27))
        return fail(YHIP_EINVAL, "%s: strides must cover the rows (att_stride a multiple of 8, x_stride < 2^27)", fn);
    if ((uintptr_t)w % 16 || (uintptr_t)att % 16 || (uintptr_t)x % 4)
        return fail(YHIP_EINVAL, "%s: w and att must be 16-byte aligned", fn);
    // the GEMM addresses the weights with 32-bit byte offsets (f16 parts)
    if ((uint64_t)B * qdim > 0x7fffffffull || (uint64_t)hidden * qdim >= (1ull << 30))
        return fail(YHIP_EINVAL, "%s: too many elements", fn);
    if (B == 0) return done(hipSuccess, "");
    const size_t need = yhip::oproj_workspace(B, qdim, w_dtype == YHIP_F16, att_dtype == YHIP_F16, hidden);
    if (need && (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256))
        return fail(YHIP_ENOSPC, "%s: workspace of %zu bytes (256-byte aligned) needed, %zu given", fn, need,
                    workspace_bytes);
    if (need && ((const char*)workspace < (const char*)x + (size_t)B * x_stride * 4 &&
                 (const char*)x < (const char*)workspace + need))
        return fail(YHIP_EINVAL, "%s: workspace overlaps x", fn);
    yhip::OProjArgs a = {};
    a.x = x;
    a.att = att;
    a.w = w;
    a.x_stride = x_stride;
    a.att_stride = att_stride;
    a.B = B;
    a.hidden = hidden;
    a.qdim = qdim;
    a.w_f16 = w_dtype == YHIP_F16;
    a.att_f16 = att_dtype == YHIP_F16;
    const char* msg = yhip::launch_oproj(a, workspace, workspace_bytes, (hipStream_t)stream);
    if (msg) return fail(YHIP_EDEVICE, "%s: %s", fn, msg);
    return done(hipSuccess, "");
}

int yhip_gdn_decode(float* S, float* S_out, const float* conv_in, float* conv_out, float* y, const float* qkv,
                    const float* z,
                    const float* alpha, const float* beta_raw, const float* conv_w, const float* dt_bias,
                    const float* ssm_a, const void* norm_w, uint32_t norm_w_dtype, uint32_t n_k_heads,
                    uint32_t n_v_heads, uint32_t head_dim, uint32_t kwidth, float l2_eps, float norm_eps,
                    void* stream)
{
    const char* fn = "yhip_gdn_decode";
    if (!S || !conv_in || !conv_out || !y || !qkv || !z || !alpha || !beta_raw || !conv_w || !dt_bias || !ssm_a ||
        !norm_w)
        return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (head_dim != 64 && head_dim != 128) return fail(YHIP_EINVAL, "%s: head_dim %u not 64 or 128", fn, head_dim);
    if (n_k_heads == 0 || n_v_heads < n_k_heads)
        return fail(YHIP_EINVAL, "%s: need 1 <= n_k_heads (%u) <= n_v_heads (%u)", fn, n_k_heads, n_v_heads);
    if (kwidth < 1 || kwidth > 8) return fail(YHIP_EINVAL, "%s: kwidth %u not in 1..8", fn, kwidth);
    if (norm_w_dtype != YHIP_F32 && norm_w_dtype != YHIP_F16) return fail(YHIP_EINVAL, "%s: bad norm_w dtype", fn);
    if ((uintptr_t)S % 16) return fail(YHIP_EINVAL, "%s: S must be 16-byte aligned", fn);
    if (int rc = state_out_ok(fn, S, S_out, (size_t)n_v_heads * head_dim * head_dim)) return rc;
    const uint64_t conv_dim = (uint64_t)(2 * n_k_heads + n_v_heads) * head_dim;
    if (conv_dim * kwidth > 0x7fffffffull) return fail(YHIP_EINVAL, "%s: too many channels", fn);
    const size_t line = (size_t)conv_dim * kwidth * sizeof(float);
    if ((const char*)conv_out < (const char*)conv_in + line && (const char*)conv_in < (const char*)conv_out + line)
        return fail(YHIP_EINVAL, "%s: conv_out overlaps conv_in", fn);
    yhip::GdnDecodeArgs a = {};
    a.S = S;
    a.S_out = S_out;
    a.conv_in = conv_in;
    a.conv_out = conv_out;
    a.qkv = qkv;
    a.z = z;
    a.alpha = alpha;
    a.beta_raw = beta_raw;
    a.conv_w = conv_w;
    a.dt_bias = dt_bias;
    a.ssm_a = ssm_a;
    a.norm_w = norm_w;
    a.y = y;
    a.n_k = n_k_heads;
    a.n_v = n_v_heads;
    a.D = head_dim;
    a.kwidth = kwidth;
    a.conv_dim = (uint32_t)conv_dim;
    a.norm_w_f16 = norm_w_dtype == YHIP_F16;
    a.l2_eps = l2_eps;
    a.norm_eps = norm_eps;
    return done(yhip::launch_gdn_decode(a, (hipStream_t)stream), fn);
}

int yhip_gdn_conv(float* out, uint32_t out_stride, const float* x, uint32_t x_stride, float* conv_state,
                  float* conv_state_out, const float* conv_w, uint32_t T, uint32_t dim, uint32_t kwidth, int silu,
                  void* stream)
{
    const char* fn = "yhip_gdn_conv";
    if (!out || !x || !conv_state || !conv_w) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (dim == 0 || kwidth == 0 || kwidth > 8) return fail(YHIP_EINVAL, "%s: need dim >= 1 and kwidth in 1..8", fn);
    if (x_stride < dim || out_stride < dim) return fail(YHIP_EINVAL, "%s: strides must cover dim channels", fn);
    if ((uint64_t)T * (x_stride > out_stride ? x_stride : out_stride) > 0xffffffffull)
        return fail(YHIP_EINVAL, "%s: too many elements", fn);
    const size_t line_bytes = (size_t)kwidth * dim * sizeof(float);
    if (!conv_state_out) conv_state_out = conv_state;
    if (conv_state_out != conv_state && (const char*)conv_state_out < (const char*)conv_state + line_bytes &&
        (const char*)conv_state < (const char*)conv_state_out + line_bytes)
        return fail(YHIP_EINVAL, "%s: conv_state_out overlaps conv_state without being it", fn);
    if (T == 0)  // no token: the delay line after the call is the one before it
        return done(conv_state_out == conv_state ? hipSuccess
                                                  : hipMemcpyAsync(conv_state_out, conv_state, line_bytes,
                                                                   hipMemcpyDeviceToDevice, (hipStream_t)stream),
                    fn);
    {
        const uintptr_t o0 = (uintptr_t)out, o1 = o0 + ((size_t)(T - 1) * out_stride + dim) * sizeof(float);
        const uintptr_t x0 = (uintptr_t)x, x1 = x0 + ((size_t)(T - 1) * x_stride + dim) * sizeof(float);
        if (o0 < x1 && x0 < o1) return fail(YHIP_EINVAL, "%s: out must not overlap x", fn);
    }
    yhip::GdnConvArgs a = {};
    a.out = out;
    a.x = x;
    a.state = conv_state;
    a.state_out = conv_state_out;
    a.w = conv_w;
    a.out_stride = out_stride;
    a.x_stride = x_stride;
    a.T = T;
    a.dim = dim;
    a.kwidth = kwidth;
    a.silu = silu != 0;
    return done(yhip::launch_gdn_conv(a, (hipStream_t)stream), fn);
}

int yhip_gdn_gated_norm(float* y, uint32_t y_stride, const float* x, uint32_t x_stride, const float* z,
                        uint32_t z_stride, const void* w, uint32_t w_dtype, uint32_t T, uint32_t n_heads,
                        uint32_t head_dim, float eps, void* stream)
{
    const char* fn = "yhip_gdn_gated_norm";
    if (!y || !x || !z || !w) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (head_dim == 0 || head_dim % 64 || head_dim > 256)
        return fail(YHIP_EINVAL, "%s: head_dim %u must be 64, 128, 192 or 256", fn, head_dim);
    if (w_dtype != YHIP_F32 && w_dtype != YHIP_F16) return fail(YHIP_EINVAL, "%s: w_dtype must be F32 or F16", fn);
    if (n_heads == 0) return fail(YHIP_EINVAL, "%s: n_heads must be >= 1", fn);
    const uint64_t row = (uint64_t)n_heads * head_dim;
    if (x_stride < row || z_stride < row || y_stride < row)
        return fail(YHIP_EINVAL, "%s: strides must cover n_heads*head_dim", fn);
    if ((uint64_t)T * n_heads > 0x7fffffffull) return fail(YHIP_EINVAL, "%s: too many rows", fn);
    if (T == 0) return done(hipSuccess, "");
    yhip::GdnNormArgs a = {};
    a.y = y;
    a.x = x;
    a.z = z;
    a.w = w;
    a.y_stride = y_stride;
    a.x_stride = x_stride;
    a.z_stride = z_stride;
    a.T = T;
    a.n_heads = n_heads;
    a.head_dim = head_dim;
    a.w_f16 = w_dtype == YHIP_F16;
    a.eps = eps;
    return done(yhip::launch_gdn_gated_norm(a, (hipStream_t)stream), fn);
}

int yhip_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt_bias, const float* ssm_a,
                   uint32_t T, uint32_t n_v_heads, void* stream)
{
    const char* fn = "yhip_gdn_gates";
    if (!beta || !gate || !alpha || !dt_bias || !ssm_a) return fail(YHIP_EINVAL, "%s: null pointer", fn);
    if (n_v_heads == 0) return fail(YHIP_EINVAL, "%s: n_v_heads must be >= 1", fn);
    if ((uint64_t)T * n_v_heads > 0x7fffffffull) return fail(YHIP_EINVAL, "%s: too many elements", fn);
    if (T == 0) return done(hipSuccess, "");
    return done(yhip::launch_gdn_gates(beta, gate, alpha, dt_bias, ssm_a, T, n_v_heads, (hipStream_t)stream), fn);
}

}  // extern "C"
