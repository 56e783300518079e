/* e2e_driver.c -- end-to-end check of the HIP device backend inside the
 * reference engine (TEST INFRASTRUCTURE).
 *
 * Compiled only into oracle/_ref/libyref_e2e.so (oracle/Makefile, target
 * `e2e`) together with the reference's own engine sources under
 * /root/reference and yllm_amd/device/device_hip.c, linked with
 * libyllm_hip.so.  A synthetic model is written with the reference's own LLF
 * writer (llf_emit, convert.c:31; its convert_dummy at convert.c:174 writes
 * nine metas per layer where the engine reads 28, llf.c:36, so the engine
 * cannot load its output); the same prompt then runs through
 * the engine bound to the CPU device and bound to the HIP backend, and the
 * tests compare the logits and the greedy tokens.
 *
 * Routing of decode blocks.  The reference engine sends a decode block to
 * e->fwd_block only in its accelerator modes (forward_layer, engine.c:1155-1158);
 * in DEV_MODE_CPU it calls engine_fwd_block_at directly (1159-1165).  The
 * integration changes that one line so the CPU branch calls e->fwd_block
 * (INTEGRATION.md); this library is built with that change (oracle/Makefile,
 * target e2e, rewrites engine.c:1164 on its way into the compiler), so
 * decode steps here are plain engine_forward calls in DEV_MODE_CPU.  For the
 * CPU device e->fwd_block is the engine's own block (engine_fwd_block_at for
 * llama / qwen, fwd_block_qwen35 for qwen35); batched prefill goes through
 * e->fwd_block_batch in DEV_MODE_CPU without any change (engine.c:652).
 */
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <math.h>

#include "cache.h"
#include "convert.h"
#include "yllm.h"
#include "yllm_device_hip.h"

/* splitmix64 draws -> uniform in [-a, a) */
static uint64_t mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static void fill(float* w, size_t n, float a, uint64_t seed)
{
    size_t i;
    for (i = 0; i < n; i++) {
        double u = ((double)(mix(seed + (i + 1) * 0x9e3779b97f4a7c15ull) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        w[i] = (float)((2.0 * u - 1.0) * a);
    }
}

/* The tensors of a synthetic model on their way to llf_emit. */
typedef struct {
    ConvItem* items;
    void** bufs;
    int n, cap;
    uint32_t seed;
} Items;

/* one tensor of ROWS x COLS (COLS 0 or 1: a vector), uniform in
 * center +- amp, stored f16 or f32 */
static int add(Items* t, uint32_t layer, uint32_t slot, const char* name, uint32_t rows, uint32_t cols, int f16,
               float amp, float center)
{
    size_t n = (size_t)rows * (cols > 1 ? cols : 1), j;
    float* w;
    ConvItem* it;
    if (t->n >= t->cap) return -1;
    w = (float*)malloc(n * 4);
    if (!w) return -1;
    it = &t->items[t->n];
    fill(w, n, amp, (uint64_t)t->seed * 1000003u + (uint64_t)t->n * 7919u);
    if (center != 0.0f)
        for (j = 0; j < n; j++) w[j] += center;
    it->layer = layer;
    it->slot = slot;
    it->ndim = cols > 1 ? 2 : 1;
    it->shape[0] = rows;
    it->shape[1] = cols > 1 ? cols : 0;
    snprintf(it->name, sizeof it->name, "%s", name);
    if (f16) {
        uint16_t* h = (uint16_t*)malloc(n * 2);
        if (!h) {
            free(w);
            return -1;
        }
        f32_to_f16_buf(w, h, n);
        free(w);
        t->bufs[t->n] = h;
        it->dtype = DT_F16;
        it->nbytes = n * 2;
    } else {
        t->bufs[t->n] = w;
        it->dtype = DT_F32;
        it->nbytes = n * 4;
    }
    it->src = (const uint8_t*)t->bufs[t->n];
    t->n++;
    return 0;
}

static int items_open(Items* t, int cap, uint32_t seed, char* err, size_t errlen)
{
    t->items = (ConvItem*)calloc((size_t)cap, sizeof(ConvItem));
    t->bufs = (void**)calloc((size_t)cap, sizeof(void*));
    t->n = 0;
    t->cap = cap;
    t->seed = seed;
    if (t->items && t->bufs) return 0;
    free(t->items);
    free(t->bufs);
    snprintf(err, errlen, "out of memory");
    return -1;
}

static int items_emit(Items* t, const char* path, const LlfHeader* h, int add_failed, char* err, size_t errlen)
{
    int rc, i;
    if (add_failed) {
        snprintf(err, errlen, "out of memory building the model");
        rc = -1;
    } else {
        rc = llf_emit(path, h, t->items, t->n, err, errlen);
    }
    for (i = 0; i < t->n; i++) free(t->bufs[i]);
    free(t->bufs);
    free(t->items);
    return rc;
}

static void header(LlfHeader* h, uint32_t arch, uint32_t blocks, uint32_t hidden, uint32_t heads, uint32_t kv_heads,
                   uint32_t head_dim, uint32_t vocab, uint32_t seq)
{
    float eps = 1e-5f, theta = 10000.0f;
    memset(h, 0, sizeof *h);
    memcpy(h->magic, YLLM_MAGIC, 8);
    h->version = YLLM_VERSION;
    h->arch = arch;
    h->n_blocks = blocks;
    h->vocab = vocab;
    h->hidden = hidden;
    h->n_heads = heads;
    h->n_kv_heads = kv_heads;
    h->head_dim = head_dim;
    h->max_seq = seq;
    h->dtype = DT_F16;
    memcpy(&h->norm_eps_bits, &eps, 4);
    memcpy(&h->rope_theta_bits, &theta, 4);
}

/* A synthetic model in the LLF format, written by the reference's own
 * llf_emit (convert.c:31-140) as its converters do: layer 0 the f16
 * embedding, layers 1..blocks the nine block tensors (f32 norms near 1, f16
 * projections uniform in +-sqrt(3/in), so activations keep unit scale),
 * plus q/k/v biases for ARCH_QWEN, then the final norm and the f16 output
 * matrix.  Returns 0 or -1 with err set. */
int ye_make_model(const char* path, uint32_t arch, uint32_t blocks, uint32_t hidden, uint32_t heads,
                  uint32_t kv_heads, uint32_t vocab, uint32_t seq, uint32_t seed, uint32_t ffn, char* err,
                  size_t errlen)
{
    /* ffn: the FFN width, 0 for the usual 8/3 hidden (a narrow FFN keeps the
     * CPU side of long-prompt runs short; the FFN is not on the path) */
    const uint32_t hd = hidden / heads, kv_dim = kv_heads * hd;
    const uint32_t inter = ffn ? ffn : ((hidden * 8 / 3 + 63) / 64) * 64;
    Items t;
    LlfHeader h;
    uint32_t b;
    int bad = 0;
    if (items_open(&t, 3 + (int)blocks * 12, seed, err, errlen) != 0) return -1;
    header(&h, arch, blocks, hidden, heads, kv_heads, hd, vocab, seq);
    bad |= add(&t, 0, SLOT_EMBED, "embed", vocab, hidden, 1, 1.0f, 0.0f);
    for (b = 1; b <= blocks; b++) {
        bad |= add(&t, b, SLOT_NORM1, "norm1", hidden, 1, 0, 0.1f, 1.0f);
        bad |= add(&t, b, SLOT_Q, "q", hidden, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_K, "k", kv_dim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_V, "v", kv_dim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_O, "o", hidden, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_NORM2, "norm2", hidden, 1, 0, 0.1f, 1.0f);
        bad |= add(&t, b, SLOT_GATE, "gate", inter, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_UP, "up", inter, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_DOWN, "down", hidden, inter, 1, sqrtf(3.0f / inter), 0.0f);
        if (arch == ARCH_QWEN) {
            bad |= add(&t, b, SLOT_QBIAS, "q_bias", hidden, 1, 0, 0.5f, 0.0f);
            bad |= add(&t, b, SLOT_KBIAS, "k_bias", kv_dim, 1, 0, 0.5f, 0.0f);
            bad |= add(&t, b, SLOT_VBIAS, "v_bias", kv_dim, 1, 0, 0.5f, 0.0f);
        }
    }
    bad |= add(&t, blocks + 1, 0, "final_norm", hidden, 1, 0, 0.1f, 1.0f);
    bad |= add(&t, blocks + 2, 0, "output", vocab, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
    return items_emit(&t, path, &h, bad, err, errlen);
}

/* A synthetic qwen35 hybrid model (ARCH_QWEN35), in the tensor slots
 * fwd_block_qwen35 reads (engine.c:736-982): block b is a gated attention
 * layer when b % 4 == 0 (heads x head_dim query and gate projections,
 * kv_heads x head_dim K/V, per-head QK-norm) and a Gated-DeltaNet layer
 * otherwise (qkv projection of 2*n_k*hvd + n_v*hvd conv channels, z gate,
 * f32 conv1d of width 4, ssm_a in [-1.5, -0.5], dt bias, alpha / beta
 * projections, gated-norm weight and ssm_out).  Every block has the SwiGLU
 * FFN, ffn wide (0: the usual 8/3 hidden).  Returns 0 or -1 with err set. */
int ye_make_model_q35(const char* path, uint32_t blocks, uint32_t hidden, uint32_t heads, uint32_t kv_heads,
                      uint32_t head_dim, uint32_t n_k, uint32_t n_v, uint32_t hvd, uint32_t vocab, uint32_t seq,
                      uint32_t seed, uint32_t ffn, char* err, size_t errlen)
{
    const uint32_t qdim = heads * head_dim, kv_dim = kv_heads * head_dim;
    const uint32_t vdim = n_v * hvd, conv = 2 * n_k * hvd + vdim, kwidth = 4;
    const uint32_t inter = ffn ? ffn : ((hidden * 8 / 3 + 63) / 64) * 64;
    Items t;
    LlfHeader h;
    uint32_t b;
    int bad = 0;
    if (items_open(&t, 3 + (int)blocks * 16, seed, err, errlen) != 0) return -1;
    header(&h, ARCH_QWEN35, blocks, hidden, heads, kv_heads, head_dim, vocab, seq);
    bad |= add(&t, 0, SLOT_EMBED, "embed", vocab, hidden, 1, 1.0f, 0.0f);
    for (b = 1; b <= blocks; b++) {
        bad |= add(&t, b, SLOT_NORM1, "norm1", hidden, 1, 0, 0.1f, 1.0f);
        if (b % 4 == 0) {
            bad |= add(&t, b, SLOT_Q, "q", qdim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_QGATE, "q_gate", qdim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_K, "k", kv_dim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_V, "v", kv_dim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_O, "o", hidden, qdim, 1, sqrtf(3.0f / qdim), 0.0f);
            bad |= add(&t, b, SLOT_QNORM, "q_norm", head_dim, 1, 0, 0.1f, 1.0f);
            bad |= add(&t, b, SLOT_KNORM, "k_norm", head_dim, 1, 0, 0.1f, 1.0f);
        } else {
            bad |= add(&t, b, SLOT_QKV, "qkv", conv, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_GATE_ATTN, "z", vdim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_SSM_CONV1D, "conv1d", kwidth, conv, 0, sqrtf(3.0f / kwidth), 0.0f);
            bad |= add(&t, b, SLOT_SSM_A, "ssm_a", n_v, 1, 0, 0.5f, -1.0f);
            bad |= add(&t, b, SLOT_SSM_DT, "ssm_dt", n_v, 1, 0, 0.5f, 0.0f);
            bad |= add(&t, b, SLOT_SSM_ALPHA, "alpha", n_v, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_SSM_BETA, "beta", n_v, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
            bad |= add(&t, b, SLOT_SSM_NORM, "ssm_norm", hvd, 1, 0, 0.1f, 1.0f);
            bad |= add(&t, b, SLOT_SSM_OUT, "ssm_out", hidden, vdim, 1, sqrtf(3.0f / vdim), 0.0f);
        }
        bad |= add(&t, b, SLOT_NORM2, "norm2", hidden, 1, 0, 0.1f, 1.0f);
        bad |= add(&t, b, SLOT_GATE, "gate", inter, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_UP, "up", inter, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        bad |= add(&t, b, SLOT_DOWN, "down", hidden, inter, 1, sqrtf(3.0f / inter), 0.0f);
    }
    bad |= add(&t, blocks + 1, 0, "final_norm", hidden, 1, 0, 0.1f, 1.0f);
    bad |= add(&t, blocks + 2, 0, "output", vocab, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
    return items_emit(&t, path, &h, bad, err, errlen);
}

/* engine_bind_device (engine.c:354-384) with the HIP factory in place of
 * device_create; when it fails the caller rebinds the CPU device, as main.c
 * does on a failed bind.  Returns 0 if HIP is bound, -1 if the CPU is. */
static int bind_hip(Engine* e, int device_id, char* err, size_t errlen)
{
    if (e->dev) {
        if (e->dev->free_dev) e->dev->free_dev(e);
        device_destroy(e->dev);
        e->dev = NULL;
    }
    e->weights_ready = 0;
    e->device_mode = DEV_MODE_CPU;
    e->w_dev = NULL;
    e->d_kv = NULL;
    e->dev = device_create_hip(device_id, err, errlen);
    if (e->dev && e->dev->load_weights(e, err, errlen) == 0) return 0;
    if (e->dev) {
        if (e->dev->free_dev) e->dev->free_dev(e);
        device_destroy(e->dev);
        e->dev = NULL;
    }
    {
        char err2[256];
        if (engine_bind_device(e, DEV_CPU, 0, err2, sizeof err2) != 0) return -2;
    }
    return -1;
}

static uint32_t argmax(const float* v, uint32_t n)
{
    uint32_t i, best = 0;
    for (i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* Run prompt[0..n_prompt) as a batched prefill, then n_decode greedy decode
 * steps.  logits: [(n_decode+1)][vocab] (after the prefill, after each
 * step); tokens: [n_decode] chosen tokens.  use_hip: 0 = CPU device, 1 = HIP
 * backend.  fail_after >= 0 arms the backend's failure hook, fail_mode says
 * where it strikes (device_hip_fail_mode).  status[0] = bind result (0 HIP,
 * -1 fell back to CPU), status[1] = KV rows (all layers, K and V) whose HBM
 * copy differs from host KV at the end (HIP without the hook only, else -1).
 * gdn_out (may be NULL): the engine's GDN delay lines then recurrent states
 * at the end (e->ssm_conv, e->ssm_state; for HIP after device_hip_kv_to_host
 * brought them to the host), up to gdn_cap floats; status[2] = the floats
 * they hold.  Returns 0 or -1 with err set. */
int ye_run(const char* path, int use_hip, int device_id, int fail_after, int fail_mode, const uint32_t* prompt,
           int n_prompt, int n_decode, float* logits, uint32_t* tokens, int* status, float* gdn_out,
           size_t gdn_cap, char* err, size_t errlen)
{
    Engine e;
    uint32_t vocab, pos;
    int i;
    memset(&e, 0, sizeof e);
    status[0] = 0;
    status[1] = -1;
    status[2] = 0;
    if (engine_init(&e, path, 0, 0, err, errlen) != 0) return -1;
    vocab = e.ws.model.h.vocab;
    if (use_hip) {
        status[0] = bind_hip(&e, device_id, err, errlen);
        if (status[0] == -2) {
            engine_free(&e);
            return -1;
        }
        if (status[0] == 0 && fail_after >= 0) {
            device_hip_fail_mode(&e, fail_mode);
            device_hip_fail_after(&e, fail_after);
        }
    }
    if (engine_forward_prefill(&e, prompt, n_prompt, 0) != 0) {
        snprintf(err, errlen, "prefill failed");
        engine_free(&e);
        return -1;
    }
    memcpy(logits, e.logits, (size_t)vocab * 4);
    pos = (uint32_t)n_prompt;
    for (i = 0; i < n_decode; i++, pos++) {
        uint32_t tok = argmax(logits + (size_t)i * vocab, vocab);
        tokens[i] = tok;
        engine_forward(&e, tok, pos);
        memcpy(logits + (size_t)(i + 1) * vocab, e.logits, (size_t)vocab * 4);
    }
    if (use_hip && status[0] == 0 && fail_after < 0) {
        /* the HBM cache, converted back to the engine layout, must equal the
         * host KV that the backend mirrored row by row */
        size_t slot = (size_t)e.max_seq * e.kv_dim;
        uint32_t nb = e.ws.model.h.n_blocks, l;
        uint16_t* keep = (uint16_t*)malloc((size_t)(2 * nb + 1) * slot * 2);
        int diff = 0;
        if (!keep) {
            engine_free(&e);
            return -1;
        }
        memcpy(keep, e.kv, (size_t)(2 * nb + 1) * slot * 2);
        memset(e.kv, 0xff, (size_t)(2 * nb + 1) * slot * 2);
        if (device_hip_kv_to_host(&e, pos) != 0) {
            snprintf(err, errlen, "device_hip_kv_to_host failed");
            free(keep);
            engine_free(&e);
            return -1;
        }
        for (l = 1; l <= nb; l++) {
            const LlfTensorMeta* mt = &e.ws.model.metas[e.ws.model.base_idx[l]];
            size_t r;
            if (e.ws.model.h.arch == ARCH_QWEN35 && mt[SLOT_SSM_CONV1D].size > 0) continue; /* no KV */
            for (r = 0; r < (size_t)pos; r++) {
                if (memcmp(e.kv + l * slot + r * e.kv_dim, keep + l * slot + r * e.kv_dim, e.kv_dim * 2)) diff++;
                if (memcmp(e.kv + (nb + l) * slot + r * e.kv_dim, keep + (nb + l) * slot + r * e.kv_dim,
                           e.kv_dim * 2))
                    diff++;
            }
        }
        status[1] = diff;
        free(keep);
    }
    if (gdn_out && e.ssm_state && e.ssm_conv) {
        /* the shapes engine_init sized the two arrays with (engine.c:283-305) */
        const LlModel* m = &e.ws.model;
        size_t n_gdn = 0, conv_n = 0, state_n = 0, got;
        uint32_t l;
        for (l = 1; l <= m->h.n_blocks; l++) {
            const LlfTensorMeta* mt = &m->metas[m->base_idx[l]];
            if (mt[SLOT_SSM_CONV1D].size == 0) continue;
            if (n_gdn++ == 0) {
                conv_n = (size_t)mt[SLOT_SSM_CONV1D].shape[0] * mt[SLOT_SSM_CONV1D].shape[1];
                state_n = (size_t)mt[SLOT_SSM_A].shape[0] * mt[SLOT_SSM_NORM].shape[0] * mt[SLOT_SSM_NORM].shape[0];
            }
        }
        got = n_gdn * (conv_n + state_n);
        if (got <= gdn_cap) {
            memcpy(gdn_out, e.ssm_conv, n_gdn * conv_n * 4);
            memcpy(gdn_out + n_gdn * conv_n, e.ssm_state, n_gdn * state_n * 4);
            status[2] = (int)got;
        }
    }
    engine_free(&e);
    return 0;
}

/* One greedy decode step (through e->fwd_block, see the file comment). */
static void decode_step(Engine* e, uint32_t tok, uint32_t pos)
{
    engine_forward(e, tok, pos);
}

static int open_bound(Engine* e, const char* path, int use_hip, int device_id, int* bound, char* err,
                      size_t errlen)
{
    memset(e, 0, sizeof *e);
    *bound = -1;
    if (engine_init(e, path, 0, 0, err, errlen) != 0) return -1;
    if (use_hip) {
        *bound = bind_hip(e, device_id, err, errlen);
        if (*bound == -2) {
            engine_free(e);
            return -1;
        }
    }
    return 0;
}

/* Session save and resume through the reference's YLLMSKV01 format
 * (sess_kv_save / sess_kv_load, cache.c:174-247).  Engine A runs the prompt
 * as a batched prefill and n_before greedy decode steps, then saves its KV
 * (pos = n_prompt + n_before rows) to sess_path and is freed.  Engine B, a
 * fresh engine bound the same way, loads the file and, for the HIP backend,
 * sends the loaded rows to HBM with device_hip_kv_from_host; it then decodes
 * n_after steps from A's next greedy token.  logits: [n_after][vocab] of B's
 * steps; tokens: [n_before + n_after] all chosen tokens.  status[0] = bind
 * result of B (0 HIP, -1 CPU), status[1] = the position sess_kv_load gave.
 * Returns 0 or -1 with err set. */
int ye_resume(const char* path, int use_hip, int device_id, const uint32_t* prompt, int n_prompt, int n_before,
              int n_after, const char* sess_path, float* logits, uint32_t* tokens, int* status, char* err,
              size_t errlen)
{
    Engine e;
    uint32_t vocab, pos, next, loaded = 0;
    int i, bound;
    float* last;
    status[0] = status[1] = -1;
    if (open_bound(&e, path, use_hip, device_id, &bound, err, errlen) != 0) return -1;
    vocab = e.ws.model.h.vocab;
    if (engine_forward_prefill(&e, prompt, n_prompt, 0) != 0) {
        snprintf(err, errlen, "prefill failed");
        engine_free(&e);
        return -1;
    }
    last = (float*)malloc((size_t)vocab * 4);
    if (!last) {
        engine_free(&e);
        return -1;
    }
    memcpy(last, e.logits, (size_t)vocab * 4);
    pos = (uint32_t)n_prompt;
    for (i = 0; i < n_before; i++, pos++) {
        tokens[i] = argmax(last, vocab);
        decode_step(&e, tokens[i], pos);
        memcpy(last, e.logits, (size_t)vocab * 4);
    }
    next = argmax(last, vocab);
    free(last);
    if (sess_kv_save(&e, pos, sess_path) != 0) {
        snprintf(err, errlen, "sess_kv_save failed");
        engine_free(&e);
        return -1;
    }
    engine_free(&e);

    if (open_bound(&e, path, use_hip, device_id, &bound, err, errlen) != 0) return -1;
    status[0] = bound;
    if (sess_kv_load(&e, sess_path, &loaded) != 0) {
        snprintf(err, errlen, "sess_kv_load failed");
        engine_free(&e);
        return -1;
    }
    status[1] = (int)loaded;
    if (bound == 0 && device_hip_kv_from_host(&e, loaded) != 0) {
        snprintf(err, errlen, "device_hip_kv_from_host failed");
        engine_free(&e);
        return -1;
    }
    pos = loaded;
    for (i = 0; i < n_after; i++, pos++) {
        tokens[n_before + i] = next;
        decode_step(&e, next, pos);
        memcpy(logits + (size_t)i * vocab, e.logits, (size_t)vocab * 4);
        next = argmax(e.logits, vocab);
    }
    engine_free(&e);
    return 0;
}
