/* device_hip.c -- yllm device backend for MI355X (gfx950): the attention of
 * every block runs on the GPU, the rest of the block on the engine's CPU
 * operators.
 *
 * Drop-in for the Device plugin interface (inference/include/device.h:37-50,
 * factory pattern of inference/device/device_cpu.c:82-110).  load_weights
 * installs fwd_block / fwd_block_batch (yllm.h:115-116) in place of the CPU
 * ones (engine_attach_cpu_fwd, engine.c:1111-1120).  The contract of those
 * (engine.c:1156-1158, 652, 1404, 1460): the block input is e->x (decode) or
 * e->pb rows (batch), the output replaces it in place, the layer's KV row for
 * each position is written before attention, the return is 0 or -1.
 *
 * Per block this backend computes exactly the reference block
 * (engine_fwd_block_at, engine.c:992-1109; forward_block_batch_default,
 * engine.c:435-590) with the engine's own exported operators -- rmsnorm,
 * matmul / matmul_batch, rope_inplace(_qwen), swiglu, f32_to_f16 -- in the
 * same order, and replaces only the attention loop: q, k, v go to HBM, the
 * K/V rows are stored into the head-major HBM cache (yhip_kv_store), and
 * yhip_attn_decode / yhip_attn_prefill produce the attention output, which
 * comes back for o_proj.  The f16 K/V rows are also written to the engine's
 * host array e->kv, so host KV is always current: a CPU fallback, session
 * save (cache.c:174-247) and the CPU path of any layer stay valid.
 *
 * ARCH_QWEN35 (fwd_block_qwen35, engine.c:736-982) is covered too.  Its
 * Gated-DeltaNet layers run the whole mixer after the projections on the
 * GPU -- gates, conv1d + silu, l2norm, the recurrence and the gated RMSNorm
 * (yhip_gdn_gates, yhip_gdn_conv, yhip_gdn_chunk, yhip_gdn_gated_norm; a
 * decode token in one yhip_gdn_decode launch) -- with the recurrent state
 * and the conv delay line resident in HBM; the projections and the FFN stay
 * on the engine's operators.  e->ssm_state / e->ssm_conv are brought up to
 * date only when the host needs them.  Its gated attention layers (d = 256,
 * QK-norm, M-RoPE on 64 dims, sigmoid gate) use the same KV store and
 * decode / prefill entry points with the gate fused.  The reference's batch
 * forward for qwen35 runs token by token (engine.c:723-734); here a batch is
 * one GPU call per layer.
 *
 * Failure handling: any HIP error in a block marks the backend failed; that
 * block is recomputed with the saved CPU forward (e->x is untouched until
 * the attention output is back) and -1 is returned; every later block runs
 * on the CPU.  device_mode stays DEV_MODE_CPU: the host holds x and a valid
 * KV copy at every block boundary, so every CPU branch of the engine is
 * correct with this backend bound.  The GDN state and delay line live in two
 * HBM buffers each: a block reads one and writes the other, and only a
 * block that succeeded makes its output current, so after a failure --
 * before, during or after the kernels -- HBM still holds the state from
 * before the block, which the fallback copies to the host.  If that copy
 * fails too (a device that is gone), the host state is stale: the block
 * reports the loss on stderr, fills its output rows with NaN so the caller
 * sees it in the logits, and returns -2 instead of continuing on wrong
 * state.
 */
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "llf.h"
#include "matvec.h"
#include "yllm.h"
#include "yllm_device_hip.h"
#include "yllm_hip.h"

/* ABI pins: this file reads these fields of the reference structs; the
 * offsets are those of the reference headers on x86-64 (gcc). */
_Static_assert(sizeof(Device) == 48, "Device layout differs from device.h:37-50");
_Static_assert(sizeof(Engine) == 576, "Engine layout differs from yllm.h");
_Static_assert(offsetof(Engine, kv) == 264, "Engine.kv");
_Static_assert(offsetof(Engine, kv_dim) == 272, "Engine.kv_dim");
_Static_assert(offsetof(Engine, max_seq) == 276, "Engine.max_seq");
_Static_assert(offsetof(Engine, fwd_block) == 288, "Engine.fwd_block");
_Static_assert(offsetof(Engine, fwd_block_batch) == 296, "Engine.fwd_block_batch");
_Static_assert(offsetof(Engine, layer_begin) == 304, "Engine.layer_begin");
_Static_assert(offsetof(Engine, x) == 312, "Engine.x");
_Static_assert(offsetof(Engine, hb) == 320, "Engine.hb");
_Static_assert(offsetof(Engine, hb2) == 328, "Engine.hb2");
_Static_assert(offsetof(Engine, ffn) == 336, "Engine.ffn");
_Static_assert(offsetof(Engine, pb) == 384, "Engine.pb");
_Static_assert(offsetof(Engine, pb2) == 392, "Engine.pb2");
_Static_assert(offsetof(Engine, pbq) == 400, "Engine.pbq");
_Static_assert(offsetof(Engine, pb_cap) == 448, "Engine.pb_cap");
_Static_assert(offsetof(Engine, ssm_state) == 360, "Engine.ssm_state");
_Static_assert(offsetof(Engine, ssm_conv) == 368, "Engine.ssm_conv");
_Static_assert(offsetof(Engine, pbg) == 424, "Engine.pbg");
_Static_assert(offsetof(Engine, pbu) == 432, "Engine.pbu");
_Static_assert(offsetof(Engine, dev) == 528, "Engine.dev");
_Static_assert(offsetof(Engine, d_kv) == 536, "Engine.d_kv");
_Static_assert(offsetof(Engine, w_dev) == 544, "Engine.w_dev");
_Static_assert(offsetof(Engine, weights_ready) == 552, "Engine.weights_ready");
_Static_assert(offsetof(Engine, device_mode) == 556, "Engine.device_mode");

/* DeviceKind has no HIP entry in the reference enum (device.h:15-19); an
 * integrated build adds DEV_HIP there and compiles this file with
 * -DYLLM_DEV_HIP_KIND=DEV_HIP.  Standalone, the kind is the next free value. */
#ifndef YLLM_DEV_HIP_KIND
#define YLLM_DEV_HIP_KIND 3
#endif

typedef int (*FwdFn)(Engine*, uint32_t, uint32_t);
typedef int (*FwdBatchFn)(Engine*, uint32_t, uint32_t, uint32_t);

typedef struct {
    int device_id;
    hipStream_t stream;
    /* model shape; qdim = n_heads * head_dim (== hidden except for qwen35) */
    uint32_t arch, hidden, n_heads, n_kv, head_dim, qdim, kv_dim, n_blocks, max_seq;
    /* HBM KV: one slot per attention layer of first..last, K then V */
    uint32_t first, last, kv_stride, n_kv_slots;
    uint64_t layer_elems;
    uint16_t* d_cache;
    int32_t* kv_slot;   /* per layer first..last: its KV slot, -1 for a GDN layer */
    uint32_t* dev_len;  /* per KV slot: rows 0..dev_len-1 are in HBM */
    /* Gated-DeltaNet layers (qwen35): per layer first..last its state slot
     * (-1 for an attention layer) and its index among the model's GDN layers
     * (gdn_index_of, engine.c:711-720: the slot of e->ssm_state / ssm_conv) */
    int32_t* gdn_slot;
    uint32_t* gdn_ord;
    /* per state slot, where the current GDN state is: STATE_HOST (e->ssm_state;
     * HBM stale), STATE_BOTH, STATE_DEV (HBM; e->ssm_state stale until
     * sync_state_to_host) */
    uint8_t* state_loc;
    uint32_t n_gdn_slots, conv_chan, kwidth, n_v, n_k, hvd, value_dim;
    /* per state slot two HBM states [n_v][hvd][hvd] and two delay lines
     * [kwidth][conv_chan]: a block reads the current one (state_cur /
     * conv_cur) and writes the other, which becomes current only when the
     * block succeeded; conv_loc is where the current line is (STATE_*) */
    float* d_state;
    uint8_t* state_cur;
    float* d_conv;
    uint8_t *conv_loc, *conv_cur;
    float* d_gb;        /* gate [cap][n_v], then beta [cap][n_v] */
    float* d_xc;        /* the conv + silu output rows [cap][conv_chan] */
    float* d_z;         /* the z rows [cap][value_dim] */
    void* d_gws;        /* chunked-form workspace for cap tokens */
    size_t gws_bytes;
    uint16_t* d_kvstage; /* engine-layout rows on their way to the host (kv_to_host) */
    uint32_t kvstage_rows;
    /* per slot the layer's conv weights, dt_bias, ssm_a and norm weights
     * (gdnw_n floats, the norm weights f32 or f16 per norm_dt); a decode
     * token runs the whole GDN mixer in one launch (yhip_gdn_decode) when
     * fused_decode is set (n_v >= n_k) */
    float* d_gdnw;
    uint8_t* norm_dt;
    float* d_dec;       /* the token's qkv | z | alpha | beta_raw */
    float* h_raw;       /* a decode token's q | k before RoPE */
    uint32_t gdnw_n;
    int fused_decode;
    /* staging for one call: q (or a GDN qkv row), k, v, gate, output */
    uint32_t cap, q_w, o_w;
    float *d_q, *d_k, *d_v, *d_g, *d_out;
    uint16_t* d_rows;  /* host f16 rows on their way into HBM (catch-up) */
    void* d_ws;
    size_t ws_bytes;
    void* d_pws;        /* prefill key-split partials for up to cap tokens per call */
    size_t pws_bytes;
    /* host rows of a qwen35 block: normed input, q or qkv, gate or z,
     * k, v, alpha / beta / gate, GPU output, projection output */
    float *h_n, *h_q, *h_z, *h_k, *h_v, *h_ab, *h_o, *h_x;
    /* fallback */
    FwdFn cpu_fwd;
    FwdBatchFn cpu_fwd_batch;
    int failed;
    /* test hook (device_hip_fail_after / device_hip_fail_mode): calls left
     * before the simulated failure, where it strikes (FAIL_*), a pending
     * failure for the block being computed, and a device whose copies fail */
    int fail_after, fail_mode, fail_pending, dead;
} HipCtx;

static HipCtx* ctx_of(const Engine* e)
{
    return e && e->dev ? (HipCtx*)e->dev->handle : NULL;
}

enum { STATE_HOST = 0, STATE_BOTH = 1, STATE_DEV = 2 };

/* where the test hook strikes (device_hip_fail_mode) */
enum { FAIL_BEFORE = 0, FAIL_AFTER = 1, FAIL_LOST = 2 };

static size_t state_elems(const HipCtx* c)
{
    return (size_t)c->n_v * c->hvd * c->hvd;
}

static size_t conv_elems(const HipCtx* c)
{
    return (size_t)c->kwidth * c->conv_chan;
}

/* HBM state / delay line `which` (0 or 1) of a state slot */
static float* state_buf(const HipCtx* c, int32_t slot, int which)
{
    return c->d_state + ((size_t)slot * 2 + (size_t)which) * state_elems(c);
}

static float* conv_buf(const HipCtx* c, int32_t slot, int which)
{
    return c->d_conv + ((size_t)slot * 2 + (size_t)which) * conv_elems(c);
}

/* device -> host copy of n bytes, then wait; -1 when it fails (or the test
 * hook has taken the device away) */
static int copy_back(HipCtx* c, void* dst, const void* src, size_t n)
{
    if (c->dead) return -1;
    if (hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return -1;
    return 0;
}

/* Make e->ssm_conv of GDN layer `layer` current when HBM holds its current
 * delay line.  Returns 0, or -1 when the copy fails. */
static int sync_conv_to_host(Engine* e, HipCtx* c, uint32_t layer)
{
    const uint32_t li = layer - c->first;
    const int32_t slot = c->gdn_slot[li];
    if (slot < 0 || !c->conv_loc || c->conv_loc[slot] != STATE_DEV) return 0;
    if (copy_back(c, e->ssm_conv + (size_t)c->gdn_ord[li] * conv_elems(c), conv_buf(c, slot, c->conv_cur[slot]),
                  conv_elems(c) * 4) != 0)
        return -1;
    c->conv_loc[slot] = STATE_BOTH;
    return 0;
}

/* Make e->ssm_state (and e->ssm_conv) of GDN layer `layer` current when HBM
 * holds its current state: one synchronous copy each.  Returns 0, or -1 when
 * a copy fails: the host then keeps the state of its last copy, which is
 * stale by every GPU update since. */
static int sync_state_to_host(Engine* e, HipCtx* c, uint32_t layer)
{
    const uint32_t li = layer - c->first;
    const int32_t slot = c->gdn_slot[li];
    if (sync_conv_to_host(e, c, layer) != 0) return -1;
    if (slot < 0 || c->state_loc[slot] != STATE_DEV) return 0;
    if (copy_back(c, e->ssm_state + (size_t)c->gdn_ord[li] * state_elems(c), state_buf(c, slot, c->state_cur[slot]),
                  state_elems(c) * 4) != 0)
        return -1;
    c->state_loc[slot] = STATE_BOTH;
    return 0;
}

static int sync_states_to_host(Engine* e, HipCtx* c)
{
    uint32_t l;
    int rc = 0;
    if (!c->state_loc || !c->gdn_slot) return 0;
    if (c->stream && hipStreamSynchronize(c->stream) != hipSuccess) rc = -1;
    for (l = c->first; l <= c->last; l++)
        if (sync_state_to_host(e, c, l) != 0) rc = -1;
    return rc;
}

static int say(char* err, size_t errlen, const char* what, const char* detail)
{
    if (err && errlen) snprintf(err, errlen, "hip: %s%s%s", what, detail ? ": " : "", detail ? detail : "");
    return -1;
}

static int hip_ok(hipError_t rc, char* err, size_t errlen, const char* what)
{
    return rc == hipSuccess ? 0 : say(err, errlen, what, hipGetErrorString(rc));
}

static uint16_t* layer_k(const HipCtx* c, uint32_t layer)
{
    return c->d_cache + (size_t)c->kv_slot[layer - c->first] * 2 * c->layer_elems;
}

static uint16_t* layer_v(const HipCtx* c, uint32_t layer)
{
    return layer_k(c, layer) + c->layer_elems;
}

static void dfree(void* p)
{
    if (p) hipFree(p);
}

static void free_staging(HipCtx* c)
{
    dfree(c->d_pws);
    c->d_pws = NULL;
    c->pws_bytes = 0;
    dfree(c->d_q);
    dfree(c->d_k);
    dfree(c->d_v);
    dfree(c->d_g);
    dfree(c->d_out);
    dfree(c->d_rows);
    dfree(c->d_gb);
    dfree(c->d_xc);
    dfree(c->d_z);
    dfree(c->d_gws);
    free(c->h_n);
    free(c->h_q);
    free(c->h_z);
    free(c->h_k);
    free(c->h_v);
    free(c->h_ab);
    free(c->h_o);
    free(c->h_x);
    c->d_q = c->d_k = c->d_v = c->d_g = c->d_out = c->d_gb = c->d_xc = c->d_z = NULL;
    c->d_rows = NULL;
    c->d_gws = NULL;
    c->h_n = c->h_q = c->h_z = c->h_k = c->h_v = c->h_ab = c->h_o = c->h_x = NULL;
    c->gws_bytes = 0;
    c->cap = 0;
}

static void release(HipCtx* c)
{
    if (!c) return;
    free_staging(c);
    dfree(c->d_cache);
    dfree(c->d_state);
    dfree(c->d_ws);
    if (c->stream) hipStreamDestroy(c->stream);
    free(c->dev_len);
    free(c->kv_slot);
    free(c->gdn_slot);
    free(c->gdn_ord);
    free(c->state_loc);
    free(c->state_cur);
    dfree(c->d_kvstage);
    dfree(c->d_conv);
    dfree(c->d_gdnw);
    dfree(c->d_dec);
    free(c->conv_loc);
    free(c->conv_cur);
    free(c->norm_dt);
    free(c->h_raw);
    {
        int id = c->device_id;
        memset(c, 0, sizeof(*c));
        c->device_id = id;
        c->fail_after = -1;
    }
}

/* staging for up to `rows` tokens of one call */
static int ensure_cap(HipCtx* c, uint32_t rows)
{
    int q35 = c->arch == ARCH_QWEN35;
    if (rows <= c->cap) return 0;
    free_staging(c);
    if (hipMalloc((void**)&c->d_q, (size_t)rows * c->q_w * 4) != hipSuccess ||
        hipMalloc((void**)&c->d_out, (size_t)rows * c->o_w * 4) != hipSuccess ||
        hipMalloc((void**)&c->d_k, (size_t)rows * c->kv_dim * 4) != hipSuccess ||
        hipMalloc((void**)&c->d_v, (size_t)rows * c->kv_dim * 4) != hipSuccess ||
        hipMalloc((void**)&c->d_rows, (size_t)rows * c->kv_dim * 2 * 2) != hipSuccess)
        return -1;
    if (q35) {
        size_t wide = c->q_w > c->o_w ? c->q_w : c->o_w;
        if (hipMalloc((void**)&c->d_g, (size_t)rows * c->qdim * 4) != hipSuccess) return -1;
        c->h_n = (float*)malloc((size_t)rows * c->hidden * 4);
        c->h_q = (float*)malloc((size_t)rows * c->q_w * 4);
        c->h_z = (float*)malloc((size_t)rows * wide * 4);
        c->h_k = (float*)malloc((size_t)rows * c->kv_dim * 4);
        c->h_v = (float*)malloc((size_t)rows * c->kv_dim * 4);
        c->h_o = (float*)malloc((size_t)rows * c->o_w * 4);
        c->h_x = (float*)malloc((size_t)rows * c->hidden * 4);
        if (!c->h_n || !c->h_q || !c->h_z || !c->h_k || !c->h_v || !c->h_o || !c->h_x) return -1;
        if (c->n_gdn_slots) {
            c->h_ab = (float*)malloc((size_t)rows * 2 * c->n_v * 4);
            if (!c->h_ab || hipMalloc((void**)&c->d_gb, (size_t)rows * 2 * c->n_v * 4) != hipSuccess ||
                hipMalloc((void**)&c->d_xc, (size_t)rows * c->conv_chan * 4) != hipSuccess ||
                hipMalloc((void**)&c->d_z, (size_t)rows * c->value_dim * 4) != hipSuccess)
                return -1;
            c->gws_bytes = yhip_gdn_chunk_workspace(rows, c->n_v, c->hvd);
            if (c->gws_bytes && hipMalloc(&c->d_gws, c->gws_bytes) != hipSuccess) return -1;
        }
    }
    /* the prefill's key-split partials, for every call of up to `rows`
     * tokens ending at or before max_seq */
    for (uint32_t b = 1; b <= rows; ++b) {
        size_t n = yhip_attn_prefill_workspace(b, c->max_seq, c->n_heads, c->n_kv, c->head_dim);
        if (n > c->pws_bytes) c->pws_bytes = n;
    }
    if (c->pws_bytes && hipMalloc(&c->d_pws, c->pws_bytes) != hipSuccess) return -1;
    c->cap = rows;
    return 0;
}

/* Rows dev_len..upto-1 of a layer exist only in host KV (written by a CPU
 * block or restored from a session): bring them into HBM, in chunks of the
 * staging capacity.  Host rows are f16 bits already; yhip_kv_store copies
 * f16 sources bit for bit. */
static int catch_up(HipCtx* c, Engine* e, uint32_t layer, uint32_t upto)
{
    uint32_t* have = &c->dev_len[c->kv_slot[layer - c->first]];
    const uint16_t* hk = e->kv + (size_t)layer * e->max_seq * c->kv_dim;
    const uint16_t* hv = e->kv + (size_t)(c->n_blocks + layer) * e->max_seq * c->kv_dim;
    while (*have < upto) {
        uint32_t n = upto - *have;
        size_t off = (size_t)*have * c->kv_dim, bytes;
        if (n > c->cap) n = c->cap;
        bytes = (size_t)n * c->kv_dim * 2;
        if (hipMemcpyAsync(c->d_rows, hk + off, bytes, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
            hipMemcpyAsync(c->d_rows + (size_t)n * c->kv_dim, hv + off, bytes, hipMemcpyHostToDevice,
                           c->stream) != hipSuccess)
            return -1;
        if (yhip_kv_store(layer_k(c, layer), layer_v(c, layer), c->d_rows, c->d_rows + (size_t)n * c->kv_dim,
                          YHIP_F16, *have, n, c->n_kv, c->head_dim, c->kv_stride, c->stream) != YHIP_OK)
            return -1;
        *have += n;
    }
    return 0;
}

/* Whether this block call may use the GPU.  Returns 1 (yes), 0 (no: the
 * layer is outside the resident range, or the backend failed earlier) or -1
 * (the GPU fails at this call before any GPU work: the test hook's count ran
 * out in FAIL_BEFORE mode).  In the other modes the block runs its GPU work
 * and then fails at gpu_after (fail_pending). */
static int gpu_turn(HipCtx* c, uint32_t layer, uint32_t pos_end)
{
    if (layer < c->first || layer > c->last || pos_end > c->max_seq || c->failed) return 0;
    if (c->fail_after == 0) {
        c->fail_after = -1;
        if (c->fail_mode == FAIL_BEFORE) {
            c->failed = 1;
            return -1;
        }
        c->fail_pending = 1;
        return 1;
    }
    if (c->fail_after > 0) c->fail_after--;
    return 1;
}

/* The point of a block after its kernels ran and its output came back: 0,
 * or -1 when the test hook fails the block here (as a lost result copy
 * would; FAIL_LOST also takes the device away for every later copy). */
static int gpu_after(HipCtx* c)
{
    if (!c->fail_pending) return 0;
    c->fail_pending = 0;
    hipStreamSynchronize(c->stream);
    if (c->fail_mode == FAIL_LOST) c->dead = 1;
    return -1;
}

static const uint8_t* layer_base(const Engine* e, uint32_t layer)
{
    return (const uint8_t*)e->ws.map.base + e->ws.model.dir[layer].offset;
}

static void rope_heads(uint32_t arch, float* v, uint32_t n, uint32_t d, uint32_t pos, float theta)
{
    uint32_t i;
    for (i = 0; i < n; i++) {
        if (arch == ARCH_QWEN)
            rope_inplace_qwen(v + (size_t)i * d, d, pos, theta);
        else
            rope_inplace(v + (size_t)i * d, d, pos, theta);
    }
}

static void add_bias(float* y, const LlfTensorMeta* t, const uint8_t* base, uint32_t n)
{
    if (t->size > 0) {
        const float* b = (const float*)(base + t->offset);
        uint32_t j;
        for (j = 0; j < n; j++) y[j] += b[j];
    }
}

static void head_norm(float* v, const LlfTensorMeta* t, const uint8_t* base, uint32_t n, uint32_t d, float eps)
{
    if (t->size > 0) {
        uint32_t i;
        for (i = 0; i < n; i++) rmsnorm(v + (size_t)i * d, v + (size_t)i * d, base + t->offset, d, eps, t->dtype);
    }
}

/* q, k, v of one token after bias, QK-norm and RoPE; the f16 K/V row goes to
 * host KV (engine.c:1015-1072) */
static void token_qkv(Engine* e, const HipCtx* c, uint32_t layer, uint32_t pos, const uint8_t* base,
                      const LlfTensorMeta* mt, float eps, float theta, float* q, float* k, float* v, float* raw)
{
    uint16_t* hk = e->kv + (size_t)layer * e->max_seq * c->kv_dim + (size_t)pos * c->kv_dim;
    uint16_t* hv = e->kv + (size_t)(c->n_blocks + layer) * e->max_seq * c->kv_dim + (size_t)pos * c->kv_dim;
    uint32_t j;
    add_bias(q, &mt[SLOT_QBIAS], base, c->hidden);
    add_bias(k, &mt[SLOT_KBIAS], base, c->kv_dim);
    add_bias(v, &mt[SLOT_VBIAS], base, c->kv_dim);
    head_norm(q, &mt[SLOT_QNORM], base, c->n_heads, c->head_dim, eps);
    head_norm(k, &mt[SLOT_KNORM], base, c->n_kv, c->head_dim, eps);
    if (raw) {  /* q | k before RoPE, for a kernel that rotates them itself */
        memcpy(raw, q, (size_t)c->hidden * 4);
        memcpy(raw + c->hidden, k, (size_t)c->kv_dim * 4);
    }
    rope_heads(c->arch, q, c->n_heads, c->head_dim, pos, theta);
    rope_heads(c->arch, k, c->n_kv, c->head_dim, pos, theta);
    for (j = 0; j < c->kv_dim; j++) {
        hk[j] = f32_to_f16(k[j]);
        hv[j] = f32_to_f16(v[j]);
    }
}

static void scalars(const Engine* e, float* eps, float* theta)
{
    memcpy(eps, &e->ws.model.h.norm_eps_bits, 4);
    memcpy(theta, &e->ws.model.h.rope_theta_bits, 4);
}

/* decode attention on the GPU: the token's q | k before RoPE (raw) and v ->
 * att_out.  One launch rotates q and k with the reference's angles (the host
 * rotated the same rows, bit for bit, into e->kv), stores the token's key and
 * value and attends (yhip_attn_decode_rope). */
static int gpu_decode(HipCtx* c, Engine* e, uint32_t layer, uint32_t pos, const float* raw, const float* v,
                      float theta, float* att_out)
{
    uint16_t *kc = layer_k(c, layer), *vc = layer_v(c, layer);
    size_t nq = c->hidden, nkv = c->kv_dim;
    const uint32_t rope = c->arch == ARCH_QWEN ? YHIP_ROPE_HALF : YHIP_ROPE_PAIRS;
    if (ensure_cap(c, 1) != 0) return -1;
    if (catch_up(c, e, layer, pos) != 0) return -1;
    if (hipMemcpyAsync(c->d_q, raw, nq * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        hipMemcpyAsync(c->d_k, raw + nq, nkv * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        hipMemcpyAsync(c->d_v, v, nkv * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess)
        return -1;
    if (yhip_attn_decode_rope(c->d_out, c->d_q, c->d_k, c->d_v, kc, vc, pos, c->n_heads, c->n_kv, c->head_dim,
                              c->kv_stride, rope, 0, theta, NULL, c->d_ws, c->ws_bytes, c->stream) != YHIP_OK)
        return -1;
    c->dev_len[c->kv_slot[layer - c->first]] = pos + 1;
    if (hipMemcpyAsync(att_out, c->d_out, nq * 4, hipMemcpyDeviceToHost, c->stream) != hipSuccess) return -1;
    if (hipStreamSynchronize(c->stream) != hipSuccess) return -1;
    return gpu_after(c);
}

/* ---- ARCH_QWEN35 blocks (fwd_block_qwen35, engine.c:736-982) ---------- */

/* y[B][out] = x[B][in] . W^T: the engine's matmul for one row (as its
 * per-token forward), matmul_batch for a batch */
static void proj(float* y, const float* x, const uint8_t* base, const LlfTensorMeta* t, uint32_t out, uint32_t in,
                 uint32_t B)
{
    if (B == 1)
        matmul(y, x, base + t->offset, out, in, t->dtype);
    else
        matmul_batch(y, x, base + t->offset, out, in, t->dtype, B);
}

/* GDN layer, engine.c:764-850 up to the output projection: c->h_n (normed
 * rows) -> c->h_x (ssm_out rows).  The projections run on the host; the
 * mixer after them on the GPU, from the HBM state and delay line current
 * before the call into the other buffer of each pair.  Only when the
 * output is back do those buffers become current, so a failed call leaves
 * the state from before it.  Returns 0 or -1. */
static int q35_gdn(Engine* e, HipCtx* c, uint32_t layer, uint32_t B, const uint8_t* base, const LlfTensorMeta* mt,
                   float eps)
{
    const uint32_t hidden = c->hidden, cc = c->conv_chan, vd = c->value_dim, nv = c->n_v, hvd = c->hvd;
    const uint32_t kd = c->n_k * hvd, li = layer - c->first;
    const size_t state_n = state_elems(c), conv_n = conv_elems(c);
    const int32_t slot = c->gdn_slot[li];
    const int scur = c->state_cur[slot], ccur = c->conv_cur[slot];
    float *S_in = state_buf(c, slot, scur), *S_out = state_buf(c, slot, 1 - scur);
    float *line_in = conv_buf(c, slot, ccur), *line_out = conv_buf(c, slot, 1 - ccur);
    const float* w = c->d_gdnw + (size_t)slot * c->gdnw_n;  /* conv_w | dt_bias | ssm_a | norm_w */
    const uint32_t ndt = c->norm_dt[slot];
    float *qkv = c->h_q, *z = c->h_z, *alpha = c->h_ab, *beta = alpha + (size_t)B * nv;
    int ok;

    proj(qkv, c->h_n, base, &mt[SLOT_QKV], cc, hidden, B);
    proj(z, c->h_n, base, &mt[SLOT_GATE_ATTN], vd, hidden, B);
    proj(alpha, c->h_n, base, &mt[SLOT_SSM_ALPHA], nv, hidden, B);
    proj(beta, c->h_n, base, &mt[SLOT_SSM_BETA], nv, hidden, B);
    /* the state and the delay line go up only when the host holds the
     * current ones (first call, after a CPU block or a restore) */
    ok = (c->state_loc[slot] != STATE_HOST ||
          hipMemcpyAsync(S_in, e->ssm_state + (size_t)c->gdn_ord[li] * state_n, state_n * 4, hipMemcpyHostToDevice,
                         c->stream) == hipSuccess) &&
         (c->conv_loc[slot] != STATE_HOST ||
          hipMemcpyAsync(line_in, e->ssm_conv + (size_t)c->gdn_ord[li] * conv_n, conv_n * 4, hipMemcpyHostToDevice,
                         c->stream) == hipSuccess);
    if (!ok) return -1;
    if (B == 1 && c->fused_decode) {
        /* one launch: gates, conv1d_update + silu, l2 norms, the state update
         * and rmsnorm_gated (engine.c:788-847); beta follows alpha in h_ab */
        float* d_z = c->d_dec + cc;
        float* d_ab = d_z + vd;
        ok = hipMemcpyAsync(c->d_dec, qkv, (size_t)cc * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
             hipMemcpyAsync(d_z, z, (size_t)vd * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
             hipMemcpyAsync(d_ab, alpha, (size_t)2 * nv * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
             yhip_gdn_decode(S_in, S_out, line_in, line_out, c->d_out, c->d_dec, d_z, d_ab, d_ab + nv, w, w + conv_n,
                             w + conv_n + nv, w + conv_n + 2 * nv, ndt, c->n_k, nv, hvd, c->kwidth, eps, eps,
                             c->stream) == YHIP_OK;
    } else {
        /* the batch (or a decode token when n_v < n_k): the gates in place
         * (alpha's rows become the log-decay gate, beta's the sigmoid,
         * engine.c:788-793), conv1d + silu of every row (805-812), the
         * recurrence over the rows in order with l2norm (826-831, chunked
         * from 64 rows), rmsnorm_gated per v head (840-850) */
        float *d_gate = c->d_gb, *d_beta = c->d_gb + (size_t)B * nv;
        ok = hipMemcpyAsync(c->d_q, qkv, (size_t)B * cc * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
             hipMemcpyAsync(c->d_z, z, (size_t)B * vd * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
             hipMemcpyAsync(d_gate, alpha, (size_t)2 * B * nv * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
             yhip_gdn_gates(d_beta, d_gate, d_gate, w + conv_n, w + conv_n + nv, B, nv, c->stream) == YHIP_OK &&
             yhip_gdn_conv(c->d_xc, cc, c->d_q, cc, line_in, line_out, w, B, cc, c->kwidth, 1, c->stream) ==
                 YHIP_OK &&
             yhip_gdn_chunk(S_in, S_out, c->d_out, vd, c->d_xc, c->d_xc + kd, cc, c->d_xc + 2 * kd, cc, d_gate,
                            d_beta, B, c->n_k, nv, hvd, eps, c->d_gws, c->gws_bytes, c->stream) == YHIP_OK &&
             yhip_gdn_gated_norm(c->d_out, vd, c->d_out, vd, c->d_z, vd, w + conv_n + 2 * nv, ndt, B, nv, hvd, eps,
                                 c->stream) == YHIP_OK;
    }
    ok = ok &&
         hipMemcpyAsync(c->h_o, c->d_out, (size_t)B * vd * 4, hipMemcpyDeviceToHost, c->stream) == hipSuccess &&
         hipStreamSynchronize(c->stream) == hipSuccess && gpu_after(c) == 0;
    if (!ok) return -1;
    c->state_cur[slot] = (uint8_t)(1 - scur);
    c->conv_cur[slot] = (uint8_t)(1 - ccur);
    c->state_loc[slot] = STATE_DEV;
    c->conv_loc[slot] = STATE_DEV;
    proj(c->h_x, c->h_o, base, &mt[SLOT_SSM_OUT], hidden, vd, B);
    return 0;
}

/* gated attention layer, engine.c:886-966 up to o_proj: c->h_n -> c->h_x */
static int q35_attn(Engine* e, HipCtx* c, uint32_t layer, uint32_t pos0, uint32_t B, const uint8_t* base,
                    const LlfTensorMeta* mt, float eps, float theta)
{
    const uint32_t hidden = c->hidden, qd = c->qdim, kvd = c->kv_dim, hd = c->head_dim;
    uint16_t *kc = layer_k(c, layer), *vc = layer_v(c, layer);
    uint32_t b, h, j;
    int ok;

    proj(c->h_q, c->h_n, base, &mt[SLOT_Q], qd, hidden, B);
    proj(c->h_z, c->h_n, base, &mt[SLOT_QGATE], qd, hidden, B);
    proj(c->h_k, c->h_n, base, &mt[SLOT_K], kvd, hidden, B);
    proj(c->h_v, c->h_n, base, &mt[SLOT_V], kvd, hidden, B);
    for (b = 0; b < B; b++) {
        float* q = c->h_q + (size_t)b * qd;
        float* k = c->h_k + (size_t)b * kvd;
        const float* v = c->h_v + (size_t)b * kvd;
        uint32_t pos = pos0 + b;
        uint16_t* hk = e->kv + (size_t)layer * e->max_seq * kvd + (size_t)pos * kvd;
        uint16_t* hv = e->kv + (size_t)(c->n_blocks + layer) * e->max_seq * kvd + (size_t)pos * kvd;
        head_norm(q, &mt[SLOT_QNORM], base, c->n_heads, hd, eps);
        head_norm(k, &mt[SLOT_KNORM], base, c->n_kv, hd, eps);
        if (B == 1) {  /* q | k before RoPE: the decode launch rotates them */
            memcpy(c->h_raw, q, (size_t)qd * 4);
            memcpy(c->h_raw + qd, k, (size_t)kvd * 4);
        }
        for (h = 0; h < c->n_heads; h++) rope_inplace_mrope(q + (size_t)h * hd, hd, 64, pos, theta);
        for (h = 0; h < c->n_kv; h++) rope_inplace_mrope(k + (size_t)h * hd, hd, 64, pos, theta);
        for (j = 0; j < kvd; j++) {
            hk[j] = f32_to_f16(k[j]);
            hv[j] = f32_to_f16(v[j]);
        }
    }

    /* a decode token: M-RoPE over 64 dims, the KV store and the gated
     * attention in one launch, from the unrotated q and k */
    const float* qs = B == 1 ? c->h_raw : c->h_q;
    const float* ks = B == 1 ? c->h_raw + qd : c->h_k;
    ok = catch_up(c, e, layer, pos0) == 0 &&
         hipMemcpyAsync(c->d_q, qs, (size_t)B * qd * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
         hipMemcpyAsync(c->d_g, c->h_z, (size_t)B * qd * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
         hipMemcpyAsync(c->d_k, ks, (size_t)B * kvd * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
         hipMemcpyAsync(c->d_v, c->h_v, (size_t)B * kvd * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
         (B == 1 ||
          yhip_kv_store(kc, vc, c->d_k, c->d_v, YHIP_F32, pos0, B, c->n_kv, hd, c->kv_stride, c->stream) == YHIP_OK);
    if (!ok) return -1;
    if (B == 1)
        ok = yhip_attn_decode_rope(c->d_out, c->d_q, c->d_k, c->d_v, kc, vc, pos0, c->n_heads, c->n_kv, hd,
                                   c->kv_stride, YHIP_ROPE_MROPE, 64, theta, c->d_g, c->d_ws, c->ws_bytes,
                                   c->stream) == YHIP_OK;
    else
        ok = yhip_attn_prefill(c->d_out, YHIP_F32, qd, c->d_q, YHIP_F32, qd, kc, vc, pos0, B, c->n_heads, c->n_kv, hd,
                               c->kv_stride, c->d_g, qd, c->d_pws, c->pws_bytes, c->stream) == YHIP_OK;
    if (!ok) return -1;
    c->dev_len[c->kv_slot[layer - c->first]] = pos0 + B;
    ok = ok &&
         hipMemcpyAsync(c->h_o, c->d_out, (size_t)B * qd * 4, hipMemcpyDeviceToHost, c->stream) == hipSuccess &&
         hipStreamSynchronize(c->stream) == hipSuccess && gpu_after(c) == 0;
    if (!ok) return -1;
    proj(c->h_x, c->h_o, base, &mt[SLOT_O], hidden, qd, B);
    return 0;
}

/* One qwen35 block over B rows X[B][hidden] at positions pos0..pos0+B-1:
 * norm1, the layer's mixer (GDN or gated attention), residual, norm2,
 * SwiGLU FFN, residual.  X is written only after the GPU part succeeded. */
static int q35_block(Engine* e, HipCtx* c, uint32_t layer, uint32_t pos0, uint32_t B, float* X)
{
    const uint8_t* base = layer_base(e, layer);
    const LlfTensorMeta* mt = &e->ws.model.metas[e->ws.model.base_idx[layer]];
    const uint32_t hidden = c->hidden;
    const uint32_t inter = mt[SLOT_GATE].shape[0] * mt[SLOT_GATE].shape[1] / hidden;
    float eps, theta, *fg, *fu;
    uint32_t b, j;
    int rc;
    scalars(e, &eps, &theta);
    for (b = 0; b < B; b++)
        rmsnorm(c->h_n + (size_t)b * hidden, X + (size_t)b * hidden, base + mt[SLOT_NORM1].offset, hidden, eps,
                mt[SLOT_NORM1].dtype);
    if (c->gdn_slot[layer - c->first] >= 0)
        rc = q35_gdn(e, c, layer, B, base, mt, eps);
    else
        rc = q35_attn(e, c, layer, pos0, B, base, mt, eps, theta);
    if (rc != 0) return -1;

    for (b = 0; b < B; b++) {
        float* xb = X + (size_t)b * hidden;
        const float* ob = c->h_x + (size_t)b * hidden;
        for (j = 0; j < hidden; j++) xb[j] += ob[j];
        rmsnorm(c->h_n + (size_t)b * hidden, xb, base + mt[SLOT_NORM2].offset, hidden, eps, mt[SLOT_NORM2].dtype);
    }
    fg = B == 1 ? e->ffn : e->pbg;
    fu = B == 1 ? e->ffn + inter : e->pbu;
    proj(fg, c->h_n, base, &mt[SLOT_GATE], inter, hidden, B);
    proj(fu, c->h_n, base, &mt[SLOT_UP], inter, hidden, B);
    for (b = 0; b < B; b++)
        swiglu(fg + (size_t)b * inter, fg + (size_t)b * inter, fu + (size_t)b * inter, inter);
    proj(c->h_x, fg, base, &mt[SLOT_DOWN], hidden, inter, B);
    for (b = 0; b < B; b++) {
        float* xb = X + (size_t)b * hidden;
        const float* db = c->h_x + (size_t)b * hidden;
        for (j = 0; j < hidden; j++) xb[j] += db[j];
    }
    return 0;
}

/* fwd_block / fwd_block_batch for qwen35.  A GDN block computed on the CPU
 * first takes the current state and delay line from HBM (when HBM holds
 * them; after a failed GPU block these are the ones from before it) and
 * leaves the HBM copies stale; they are re-sent before the layer's next GPU
 * call.  When that copy fails the host state is stale: the block output
 * becomes NaN (the loss shows in the logits instead of as wrong tokens), a
 * message goes to stderr and the block returns -2. */
static int q35_fwd(Engine* e, HipCtx* c, uint32_t layer, uint32_t pos0, uint32_t B, int batch)
{
    float* X = batch ? e->pb : e->x;
    int turn = B > c->cap ? 0 : gpu_turn(c, layer, pos0 + B);
    if (turn > 0 && q35_block(e, c, layer, pos0, B, X) == 0) return 0;
    if (turn > 0) {
        c->failed = 1;
        c->fail_pending = 0;
        turn = -1;
    }
    if (layer >= c->first && layer <= c->last && c->gdn_slot[layer - c->first] >= 0) {
        const int32_t slot = c->gdn_slot[layer - c->first];
        if (sync_state_to_host(e, c, layer) != 0) {
            const size_t n = (size_t)B * c->hidden;
            size_t i;
            fprintf(stderr,
                    "hip: the recurrent state of layer %u is lost (HBM held it and the device no longer answers);"
                    " the block output is NaN\n",
                    layer);
            for (i = 0; i < n; i++) X[i] = NAN;
            return -2;
        }
        c->state_loc[slot] = STATE_HOST;
        c->conv_loc[slot] = STATE_HOST;
    }
    if (batch)
        c->cpu_fwd_batch(e, layer, pos0, B);
    else
        c->cpu_fwd(e, layer, pos0);
    return turn;
}

/* fwd_block: engine_fwd_block_at (engine.c:992-1109) with the attention
 * loop (1074-1096) on the GPU */
static int hip_fwd_block(Engine* e, uint32_t layer, uint32_t pos)
{
    HipCtx* c = ctx_of(e);
    const uint8_t* base;
    const LlfTensorMeta* mt;
    float eps, theta, *x, *x2, *q, *k, *v, *att_out, *fg, *fu;
    uint32_t hidden, kv_dim, inter, j;
    int turn;
    if (!c) return -1;
    if (c->arch == ARCH_QWEN35) return q35_fwd(e, c, layer, pos, 1, 0);
    turn = gpu_turn(c, layer, pos + 1);
    if (turn <= 0) {
        c->cpu_fwd(e, layer, pos);
        return turn;
    }
    base = layer_base(e, layer);
    mt = &e->ws.model.metas[e->ws.model.base_idx[layer]];
    hidden = c->hidden;
    kv_dim = c->kv_dim;
    inter = mt[SLOT_GATE].shape[0] * mt[SLOT_GATE].shape[1] / hidden;
    scalars(e, &eps, &theta);
    x = e->x;
    x2 = e->hb;
    q = e->hb2;
    k = q + hidden;
    v = k + kv_dim;
    att_out = v + kv_dim;

    rmsnorm(x2, x, base + mt[SLOT_NORM1].offset, hidden, eps, mt[SLOT_NORM1].dtype);
    matmul(q, x2, base + mt[SLOT_Q].offset, hidden, hidden, mt[SLOT_Q].dtype);
    matmul(k, x2, base + mt[SLOT_K].offset, kv_dim, hidden, mt[SLOT_K].dtype);
    matmul(v, x2, base + mt[SLOT_V].offset, kv_dim, hidden, mt[SLOT_V].dtype);
    token_qkv(e, c, layer, pos, base, mt, eps, theta, q, k, v, c->h_raw);

    if (gpu_decode(c, e, layer, pos, c->h_raw, v, theta, att_out) != 0) {
        c->failed = 1;
        c->cpu_fwd(e, layer, pos);  /* x is still the block input */
        return -1;
    }

    /* o_proj, residual, norm2, SwiGLU FFN, residual (engine.c:1097-1108) */
    memcpy(x2, att_out, (size_t)hidden * 4);
    matmul(att_out, x2, base + mt[SLOT_O].offset, hidden, hidden, mt[SLOT_O].dtype);
    for (j = 0; j < hidden; j++) x[j] += att_out[j];
    rmsnorm(x2, x, base + mt[SLOT_NORM2].offset, hidden, eps, mt[SLOT_NORM2].dtype);
    fg = e->ffn;
    fu = e->ffn + inter;
    matmul(fg, x2, base + mt[SLOT_GATE].offset, inter, hidden, mt[SLOT_GATE].dtype);
    matmul(fu, x2, base + mt[SLOT_UP].offset, inter, hidden, mt[SLOT_UP].dtype);
    swiglu(x2, fg, fu, inter);
    matmul(att_out, x2, base + mt[SLOT_DOWN].offset, hidden, inter, mt[SLOT_DOWN].dtype);
    for (j = 0; j < hidden; j++) x[j] += att_out[j];
    return 0;
}

/* causal attention of B tokens at pos_start.. on the GPU: e->pbq, pbk, pbv
 * -> e->pb2 */
static int gpu_prefill(HipCtx* c, Engine* e, uint32_t layer, uint32_t pos_start, uint32_t B)
{
    uint16_t *kc = layer_k(c, layer), *vc = layer_v(c, layer);
    size_t nq = (size_t)B * c->hidden, nkv = (size_t)B * c->kv_dim;
    if (ensure_cap(c, B) != 0) return -1;
    if (catch_up(c, e, layer, pos_start) != 0) return -1;
    if (hipMemcpyAsync(c->d_q, e->pbq, nq * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        hipMemcpyAsync(c->d_k, e->pbk, nkv * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        hipMemcpyAsync(c->d_v, e->pbv, nkv * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess)
        return -1;
    if (yhip_kv_store(kc, vc, c->d_k, c->d_v, YHIP_F32, pos_start, B, c->n_kv, c->head_dim, c->kv_stride,
                      c->stream) != YHIP_OK)
        return -1;
    c->dev_len[c->kv_slot[layer - c->first]] = pos_start + B;
    if (yhip_attn_prefill(c->d_out, YHIP_F32, c->hidden, c->d_q, YHIP_F32, c->hidden, kc, vc, pos_start, B,
                          c->n_heads, c->n_kv, c->head_dim, c->kv_stride, NULL, 0, c->d_pws, c->pws_bytes,
                          c->stream) != YHIP_OK)
        return -1;
    if (hipMemcpyAsync(e->pb2, c->d_out, nq * 4, hipMemcpyDeviceToHost, c->stream) != hipSuccess) return -1;
    if (hipStreamSynchronize(c->stream) != hipSuccess) return -1;
    return gpu_after(c);
}

/* fwd_block_batch: forward_block_batch_default (engine.c:435-590) with the
 * attention loop (532-563) on the GPU */
static int hip_fwd_block_batch(Engine* e, uint32_t layer, uint32_t pos_start, uint32_t B)
{
    HipCtx* c = ctx_of(e);
    const uint8_t* base;
    const LlfTensorMeta* mt;
    float eps, theta;
    uint32_t hidden, kv_dim, inter, b, j;
    int turn;
    if (!c) return -1;
    if (B == 0) return 0;
    if (c->arch == ARCH_QWEN35) return q35_fwd(e, c, layer, pos_start, B, 1);
    turn = gpu_turn(c, layer, pos_start + B);
    if (turn <= 0) {
        c->cpu_fwd_batch(e, layer, pos_start, B);
        return turn;
    }
    base = layer_base(e, layer);
    mt = &e->ws.model.metas[e->ws.model.base_idx[layer]];
    hidden = c->hidden;
    kv_dim = c->kv_dim;
    inter = mt[SLOT_GATE].shape[0] * mt[SLOT_GATE].shape[1] / hidden;
    scalars(e, &eps, &theta);

    for (b = 0; b < B; b++)
        rmsnorm(e->pb2 + (size_t)b * hidden, e->pb + (size_t)b * hidden, base + mt[SLOT_NORM1].offset, hidden,
                eps, mt[SLOT_NORM1].dtype);
    matmul_batch(e->pbq, e->pb2, base + mt[SLOT_Q].offset, hidden, hidden, mt[SLOT_Q].dtype, B);
    matmul_batch(e->pbk, e->pb2, base + mt[SLOT_K].offset, kv_dim, hidden, mt[SLOT_K].dtype, B);
    matmul_batch(e->pbv, e->pb2, base + mt[SLOT_V].offset, kv_dim, hidden, mt[SLOT_V].dtype, B);
    for (b = 0; b < B; b++)
        token_qkv(e, c, layer, pos_start + b, base, mt, eps, theta, e->pbq + (size_t)b * hidden,
                  e->pbk + (size_t)b * kv_dim, e->pbv + (size_t)b * kv_dim, NULL);

    if (gpu_prefill(c, e, layer, pos_start, B) != 0) {
        c->failed = 1;
        c->cpu_fwd_batch(e, layer, pos_start, B);  /* e->pb is still the block input */
        return -1;
    }

    /* o_proj, residual, norm2, SwiGLU FFN, residual (engine.c:565-589) */
    matmul_batch(e->pbq, e->pb2, base + mt[SLOT_O].offset, hidden, hidden, mt[SLOT_O].dtype, B);
    for (b = 0; b < B; b++) {
        float* xb = e->pb + (size_t)b * hidden;
        const float* ob = e->pbq + (size_t)b * hidden;
        for (j = 0; j < hidden; j++) xb[j] += ob[j];
        rmsnorm(e->pb2 + (size_t)b * hidden, xb, base + mt[SLOT_NORM2].offset, hidden, eps, mt[SLOT_NORM2].dtype);
    }
    matmul_batch(e->pbg, e->pb2, base + mt[SLOT_GATE].offset, inter, hidden, mt[SLOT_GATE].dtype, B);
    matmul_batch(e->pbu, e->pb2, base + mt[SLOT_UP].offset, inter, hidden, mt[SLOT_UP].dtype, B);
    for (b = 0; b < B; b++)
        swiglu(e->pbg + (size_t)b * inter, e->pbg + (size_t)b * inter, e->pbu + (size_t)b * inter, inter);
    matmul_batch(e->pbq, e->pbg, base + mt[SLOT_DOWN].offset, hidden, inter, mt[SLOT_DOWN].dtype, B);
    for (b = 0; b < B; b++) {
        float* xb = e->pb + (size_t)b * hidden;
        const float* db = e->pbq + (size_t)b * hidden;
        for (j = 0; j < hidden; j++) xb[j] += db[j];
    }
    return 0;
}

/* Layer map of [first, last]: KV slots for attention layers, state slots
 * and GDN ordinals for qwen35's Gated-DeltaNet layers (a layer is GDN when
 * it has a conv1d tensor, as engine_init and gdn_index_of decide,
 * engine.c:283-305, 711-720), and the GDN shape of fwd_block_qwen35
 * (engine.c:766-772).  Returns 0 or -1 with err set. */
static int plan_layers(Engine* e, HipCtx* c, char* err, size_t errlen)
{
    const LlModel* m = &e->ws.model;
    uint32_t nl = c->last - c->first + 1, l, ord = 0;
    c->kv_slot = (int32_t*)calloc(nl, sizeof(int32_t));
    c->gdn_slot = (int32_t*)calloc(nl, sizeof(int32_t));
    c->gdn_ord = (uint32_t*)calloc(nl, sizeof(uint32_t));
    if (!c->kv_slot || !c->gdn_slot || !c->gdn_ord) return say(err, errlen, "out of host memory", NULL);
    for (l = 1; l <= c->last; l++) {
        const LlfTensorMeta* mt = &m->metas[m->base_idx[l]];
        int gdn = c->arch == ARCH_QWEN35 && mt[SLOT_SSM_CONV1D].size > 0;
        if (gdn) {
            uint32_t cc = mt[SLOT_SSM_CONV1D].shape[1], kw = mt[SLOT_SSM_CONV1D].shape[0];
            uint32_t nv = mt[SLOT_SSM_A].shape[0], hvd = mt[SLOT_SSM_NORM].shape[0];
            if (c->conv_chan == 0) {
                if (hvd != 64 && hvd != 128) return say(err, errlen, "GDN head dim must be 64 or 128", NULL);
                if (nv == 0 || kw == 0 || cc <= nv * hvd || (cc - nv * hvd) % (2 * hvd))
                    return say(err, errlen, "GDN conv channels do not split into q, k, v heads", NULL);
                if (mt[SLOT_SSM_CONV1D].dtype != DT_F32 || mt[SLOT_SSM_A].dtype != DT_F32 ||
                    mt[SLOT_SSM_DT].dtype != DT_F32)
                    return say(err, errlen, "GDN conv1d, ssm_a and ssm_dt must be f32", NULL);
                if (!e->ssm_state || !e->ssm_conv) return say(err, errlen, "engine has no GDN state", NULL);
                c->conv_chan = cc;
                c->kwidth = kw;
                c->n_v = nv;
                c->hvd = hvd;
                c->value_dim = nv * hvd;
                c->n_k = (cc - nv * hvd) / (2 * hvd);
            } else if (cc != c->conv_chan || kw != c->kwidth || nv != c->n_v || hvd != c->hvd) {
                return say(err, errlen, "GDN layers differ in shape", NULL);
            }
        }
        if (l >= c->first) {
            c->kv_slot[l - c->first] = gdn ? -1 : (int32_t)c->n_kv_slots++;
            c->gdn_slot[l - c->first] = gdn ? (int32_t)c->n_gdn_slots++ : -1;
            c->gdn_ord[l - c->first] = gdn ? ord : 0;
        }
        if (gdn) ord++;
    }
    return 0;
}

/* HBM for the GDN layers: two states and two delay lines per state slot
 * (state_cur / conv_cur name the current ones), and per slot the layer's
 * conv weights, dt_bias, ssm_a and gated-norm weights.  The norm weights are
 * f32 or, like the engine reads every other type, f16 bits
 * (engine.c:838-850).  A decode token is one yhip_gdn_decode launch when
 * n_v >= n_k (fused_decode); otherwise it takes the batch path. */
static int setup_gdn(Engine* e, HipCtx* c, char* err, size_t errlen)
{
    const size_t conv_n = conv_elems(c), state_n = state_elems(c);
    const size_t dec_n = (size_t)c->conv_chan + c->value_dim + 2 * (size_t)c->n_v;
    uint32_t l;
    if (c->kwidth > 8) return say(err, errlen, "GDN conv width above 8 is not supported", NULL);
    c->fused_decode = c->n_v >= c->n_k;
    c->gdnw_n = (uint32_t)((conv_n + 2 * c->n_v + c->hvd + 3) / 4 * 4);
    c->state_loc = (uint8_t*)calloc(c->n_gdn_slots, 1); /* STATE_HOST */
    c->state_cur = (uint8_t*)calloc(c->n_gdn_slots, 1);
    c->conv_loc = (uint8_t*)calloc(c->n_gdn_slots, 1);
    c->conv_cur = (uint8_t*)calloc(c->n_gdn_slots, 1);
    c->norm_dt = (uint8_t*)calloc(c->n_gdn_slots, 1);
    if (!c->state_loc || !c->state_cur || !c->conv_loc || !c->conv_cur || !c->norm_dt)
        return say(err, errlen, "out of host memory", NULL);
    /* the HBM state is loaded from e->ssm_state by each layer's first call */
    if (hip_ok(hipMalloc((void**)&c->d_state, (size_t)c->n_gdn_slots * 2 * state_n * 4), err, errlen,
               "GDN state allocation") ||
        hip_ok(hipMalloc((void**)&c->d_conv, (size_t)c->n_gdn_slots * 2 * conv_n * 4), err, errlen,
               "GDN delay lines") ||
        hip_ok(hipMalloc((void**)&c->d_gdnw, (size_t)c->n_gdn_slots * c->gdnw_n * 4), err, errlen, "GDN weights") ||
        hip_ok(hipMalloc((void**)&c->d_dec, dec_n * 4), err, errlen, "GDN decode staging"))
        return -1;
    for (l = c->first; l <= c->last; l++) {
        const int32_t slot = c->gdn_slot[l - c->first];
        const uint8_t* base = layer_base(e, l);
        const LlfTensorMeta* mt = &e->ws.model.metas[e->ws.model.base_idx[l]];
        uint32_t ndt;
        float* w;
        if (slot < 0) continue;
        ndt = mt[SLOT_SSM_NORM].dtype == DT_F32 ? YHIP_F32 : YHIP_F16;
        c->norm_dt[slot] = (uint8_t)ndt;
        w = c->d_gdnw + (size_t)slot * c->gdnw_n;
        if (hip_ok(hipMemcpy(w, base + mt[SLOT_SSM_CONV1D].offset, conv_n * 4, hipMemcpyHostToDevice), err, errlen,
                   "GDN conv weights") ||
            hip_ok(hipMemcpy(w + conv_n, base + mt[SLOT_SSM_DT].offset, (size_t)c->n_v * 4, hipMemcpyHostToDevice),
                   err, errlen, "GDN dt_bias") ||
            hip_ok(hipMemcpy(w + conv_n + c->n_v, base + mt[SLOT_SSM_A].offset, (size_t)c->n_v * 4,
                             hipMemcpyHostToDevice),
                   err, errlen, "GDN ssm_a") ||
            hip_ok(hipMemcpy(w + conv_n + 2 * c->n_v, base + mt[SLOT_SSM_NORM].offset,
                             (size_t)c->hvd * (ndt == YHIP_F32 ? 4 : 2), hipMemcpyHostToDevice),
                   err, errlen, "GDN norm weights"))
            return -1;
    }
    return 0;
}

static int hip_load_weights(Engine* e, char* err, size_t errlen)
{
    HipCtx* c = ctx_of(e);
    const LlfHeader* h;
    uint32_t first, last;
    size_t cache_bytes;
    if (!c) return say(err, errlen, "no backend state", NULL);
    h = &e->ws.model.h;
    release(c);
    if (h->arch != ARCH_QWEN35 && h->n_heads * h->head_dim != h->hidden)
        return say(err, errlen, "n_heads*head_dim != hidden is not supported", NULL);
    if (h->head_dim != 64 && h->head_dim != 128 && h->head_dim != 256)
        return say(err, errlen, "head_dim must be 64, 128 or 256", NULL);
    if (h->n_kv_heads == 0 || h->n_heads % h->n_kv_heads || h->n_heads / h->n_kv_heads > 16)
        return say(err, errlen, "need n_kv_heads | n_heads and at most 16 query heads per kv head", NULL);
    if (e->kv_dim != h->n_kv_heads * h->head_dim) return say(err, errlen, "engine kv_dim mismatch", NULL);

    /* block layers of this engine's range: [layer_begin, layer_end) ∩ [1, n_blocks] */
    first = e->layer_begin > 1 ? e->layer_begin : 1;
    last = e->layer_end > 0 && e->layer_end - 1 < h->n_blocks ? e->layer_end - 1 : h->n_blocks;
    if (first > last) first = last = 1;

    c->arch = h->arch;
    c->hidden = h->hidden;
    c->n_heads = h->n_heads;
    c->n_kv = h->n_kv_heads;
    c->head_dim = h->head_dim;
    c->qdim = h->n_heads * h->head_dim;
    c->kv_dim = e->kv_dim;
    c->n_blocks = h->n_blocks;
    c->max_seq = e->max_seq;
    c->first = first;
    c->last = last;
    if (plan_layers(e, c, err, errlen) != 0) return -1;
    c->q_w = c->qdim > c->conv_chan ? c->qdim : c->conv_chan;
    c->o_w = c->qdim > c->value_dim ? c->qdim : c->value_dim;

    if (hip_ok(hipSetDevice(c->device_id), err, errlen, "hipSetDevice") ||
        hip_ok(hipStreamCreate(&c->stream), err, errlen, "hipStreamCreate"))
        return -1;
    c->kv_stride = (e->max_seq + 63) / 64 * 64;
    c->layer_elems = yhip_kv_layer_elems(c->n_kv, c->head_dim, c->kv_stride);
    cache_bytes = (size_t)c->n_kv_slots * 2 * c->layer_elems * 2;
    if (cache_bytes &&
        (hip_ok(hipMalloc((void**)&c->d_cache, cache_bytes), err, errlen, "KV cache allocation") ||
         hip_ok(hipMemsetAsync(c->d_cache, 0, cache_bytes, c->stream), err, errlen, "KV cache clear")))
        return -1;
    c->dev_len = (uint32_t*)calloc(c->n_kv_slots + 1, sizeof(uint32_t));
    if (!c->dev_len) return say(err, errlen, "out of host memory", NULL);
    if (c->n_gdn_slots && setup_gdn(e, c, err, errlen) != 0) return -1;
    if (ensure_cap(c, e->pb_cap > 0 ? e->pb_cap : 64) != 0) return say(err, errlen, "staging allocation", NULL);
    c->h_raw = (float*)malloc(((size_t)(c->qdim > c->hidden ? c->qdim : c->hidden) + c->kv_dim) * 4);
    if (!c->h_raw) return say(err, errlen, "out of host memory", NULL);
    c->ws_bytes = yhip_attn_decode_workspace(1, c->max_seq, c->max_seq, c->n_heads, c->n_kv, c->head_dim);
    if (c->ws_bytes && hip_ok(hipMalloc(&c->d_ws, c->ws_bytes), err, errlen, "decode workspace")) return -1;
    if (hip_ok(hipStreamSynchronize(c->stream), err, errlen, "set-up")) return -1;
    /* dev_len starts at 0: rows already in host KV (a CPU prefill before the
     * bind, a restored session) are uploaded by the first block call that
     * reads them */

    engine_attach_cpu_fwd(e);
    c->cpu_fwd = e->fwd_block;
    c->cpu_fwd_batch = e->fwd_block_batch;
    c->failed = 0;
    e->fwd_block = hip_fwd_block;
    e->fwd_block_batch = hip_fwd_block_batch;
    e->w_dev = NULL;  /* weights stay in host memory */
    e->d_kv = c->d_cache;
    e->weights_ready = 1;
    e->device_mode = DEV_MODE_CPU;
    return 0;
}

static void hip_free_dev(Engine* e)
{
    HipCtx* c = ctx_of(e);
    if (c) {
        if (c->stream) hipStreamSynchronize(c->stream);
        /* the engine continues on the CPU with e->ssm_state */
        if (sync_states_to_host(e, c) != 0)
            fprintf(stderr, "hip: free_dev could not copy the recurrent state back; e->ssm_state is stale\n");
        release(c);
    }
    if (e->fwd_block == hip_fwd_block) engine_attach_cpu_fwd(e);
    e->w_dev = NULL;
    e->d_kv = NULL;
    e->weights_ready = 0;
    e->device_mode = DEV_MODE_CPU;
}

Device* device_create_hip(int device_id, char* err, size_t errlen)
{
    int n = 0;
    hipDeviceProp_t prop;
    Device* d;
    HipCtx* c;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        say(err, errlen, "no HIP device", NULL);
        return NULL;
    }
    if (device_id < 0 || device_id >= n) {
        say(err, errlen, "device id out of range", NULL);
        return NULL;
    }
    if (hipGetDeviceProperties(&prop, device_id) != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        say(err, errlen, "device is not gfx950 (the kernels are built for MI355X only)", prop.gcnArchName);
        return NULL;
    }
    d = (Device*)calloc(1, sizeof(Device));
    c = (HipCtx*)calloc(1, sizeof(HipCtx));
    if (!d || !c) {
        free(d);
        free(c);
        say(err, errlen, "out of host memory", NULL);
        return NULL;
    }
    c->device_id = device_id;
    c->fail_after = -1;
    d->kind = (DeviceKind)YLLM_DEV_HIP_KIND;
    d->id = device_id;
    d->handle = c;
    d->load_weights = hip_load_weights;
    d->free_dev = hip_free_dev;
    d->prefetch_layer = NULL;
    d->release_layer = NULL;
    return d;
}

static int move_kv(Engine* e, uint32_t n_pos, int to_host)
{
    HipCtx* c = ctx_of(e);
    uint32_t l;
    if (!c || !c->stream || c->failed) return -1;
    if (n_pos > c->max_seq) n_pos = c->max_seq;
    if (!to_host && c->state_loc) memset(c->state_loc, STATE_HOST, c->n_gdn_slots);
    if (!to_host && c->conv_loc) memset(c->conv_loc, STATE_HOST, c->n_gdn_slots);
    if (c->dead) return -1;
    if (to_host && sync_states_to_host(e, c) != 0) return -1;
    for (l = c->first; l <= c->last && n_pos > 0; l++) {
        uint16_t* hk = e->kv + (size_t)l * e->max_seq * c->kv_dim;
        uint16_t* hv = e->kv + (size_t)(c->n_blocks + l) * e->max_seq * c->kv_dim;
        if (c->kv_slot[l - c->first] < 0) continue;
        if (to_host) {
            /* rows p0.. of the head-major cache, converted in pieces through one
             * staging buffer (allocated at the first call and kept): the K rows
             * of piece p0 start p0 rows into every head, its V tiles p0/32
             * tiles in (p0 is a multiple of 64) */
            uint32_t p0;
            if (!c->d_kvstage) {
                c->kvstage_rows = c->max_seq < 4096 ? (c->max_seq + 63) / 64 * 64 : 4096;
                if (hipMalloc((void**)&c->d_kvstage, (size_t)c->kvstage_rows * c->kv_dim * 2 * 2) != hipSuccess) {
                    c->d_kvstage = NULL;
                    return -1;
                }
            }
            for (p0 = 0; p0 < n_pos; p0 += c->kvstage_rows) {
                const uint32_t n = n_pos - p0 < c->kvstage_rows ? n_pos - p0 : c->kvstage_rows;
                const size_t bytes = (size_t)n * c->kv_dim * 2, off = (size_t)p0 * c->kv_dim;
                uint16_t* dk = c->d_kvstage;
                uint16_t* dv = dk + (size_t)c->kvstage_rows * c->kv_dim;
                if (yhip_kv_to_engine(dk, dv, layer_k(c, l) + (size_t)p0 * c->head_dim,
                                      layer_v(c, l) + (size_t)(p0 / 32) * c->head_dim * 32, n, c->n_kv, c->head_dim,
                                      c->kv_stride, c->stream) != YHIP_OK ||
                    hipMemcpyAsync(hk + off, dk, bytes, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
                    hipMemcpyAsync(hv + off, dv, bytes, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
                    hipStreamSynchronize(c->stream) != hipSuccess)
                    return -1;
            }
        } else {
            c->dev_len[c->kv_slot[l - c->first]] = 0;
            if (catch_up(c, e, l, n_pos) != 0) return -1;
        }
    }
    return hipStreamSynchronize(c->stream) == hipSuccess ? 0 : -1;
}

int device_hip_kv_from_host(Engine* e, uint32_t n_pos)
{
    return move_kv(e, n_pos, 0);
}

int device_hip_kv_to_host(Engine* e, uint32_t n_pos)
{
    return move_kv(e, n_pos, 1);
}

void device_hip_fail_after(Engine* e, int n_calls)
{
    HipCtx* c = ctx_of(e);
    if (c) c->fail_after = n_calls < 0 ? -1 : n_calls;
}

void device_hip_fail_mode(Engine* e, int mode)
{
    HipCtx* c = ctx_of(e);
    if (c) c->fail_mode = mode == FAIL_AFTER || mode == FAIL_LOST ? mode : FAIL_BEFORE;
}
