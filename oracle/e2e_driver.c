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
 * integration adds one line that makes the CPU branch call e->fwd_block
 * (which is engine_fwd_block_at for the CPU device).  This unmodified build
 * gets the same routing by running each decode step with device_mode set
 * to DEV_MODE_VULKAN: in a build without Vulkan every Vulkan hook is the
 * CPU stub of device_cpu.c:175-202 (returns -1 or does nothing), so the step
 * is the CPU step except that blocks go through e->fwd_block.  Batched
 * prefill already goes through e->fwd_block_batch in DEV_MODE_CPU
 * (engine.c:652).
 */
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <math.h>

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

/* A synthetic model in the LLF format, written by the reference's own
 * llf_emit (convert.c:31-140) as its converters do: layer 0 the f16
 * embedding, layers 1..blocks the nine block tensors (f32 norms near 1, f16
 * projections uniform in +-sqrt(3/in), so activations keep unit scale),
 * plus q/k/v biases for ARCH_QWEN, then the final norm and the f16 output
 * matrix.  Returns 0 or -1 with err set. */
int ye_make_model(const char* path, uint32_t arch, uint32_t blocks, uint32_t hidden, uint32_t heads,
                  uint32_t kv_heads, uint32_t vocab, uint32_t seq, uint32_t seed, char* err, size_t errlen)
{
    const uint32_t hd = hidden / heads, kv_dim = kv_heads * hd;
    const uint32_t inter = ((hidden * 8 / 3 + 63) / 64) * 64;
    const uint32_t per_block = arch == ARCH_QWEN ? 12 : 9;
    const int n_items = 1 + (int)(blocks * per_block) + 2;
    ConvItem* items = (ConvItem*)calloc((size_t)n_items, sizeof(ConvItem));
    void** bufs = (void**)calloc((size_t)n_items, sizeof(void*));
    LlfHeader h;
    int k = 0, rc, i;
    uint32_t b;
    float eps = 1e-5f, theta = 10000.0f;
    if (!items || !bufs) {
        free(items);
        free(bufs);
        snprintf(err, errlen, "out of memory");
        return -1;
    }
    memset(&h, 0, sizeof h);
    memcpy(h.magic, YLLM_MAGIC, 8);
    h.version = YLLM_VERSION;
    h.arch = arch;
    h.n_blocks = blocks;
    h.vocab = vocab;
    h.hidden = hidden;
    h.n_heads = heads;
    h.n_kv_heads = kv_heads;
    h.head_dim = hd;
    h.max_seq = seq;
    h.dtype = DT_F16;
    memcpy(&h.norm_eps_bits, &eps, 4);
    memcpy(&h.rope_theta_bits, &theta, 4);

#define ADD(LAYER, SLOT, NAME, ROWS, COLS, F16, AMP, CENTER)                                         \
    do {                                                                                          \
        size_t n_ = (size_t)(ROWS) * (COLS);                                                      \
        float* w_ = (float*)malloc(n_ * 4);                                                       \
        ConvItem* it_ = &items[k];                                                                \
        fill(w_, n_, (AMP), (uint64_t)seed * 1000003u + (uint64_t)k * 7919u);                     \
        if ((CENTER) != 0.0f) {                                                                   \
            size_t j_;                                                                            \
            for (j_ = 0; j_ < n_; j_++) w_[j_] += (CENTER);                                       \
        }                                                                                         \
        it_->layer = (LAYER);                                                                     \
        it_->slot = (SLOT);                                                                       \
        it_->ndim = (COLS) > 1 ? 2 : 1;                                                           \
        it_->shape[0] = (ROWS);                                                                   \
        it_->shape[1] = (COLS) > 1 ? (COLS) : 0;                                                  \
        snprintf(it_->name, sizeof it_->name, "%s", (NAME));                                      \
        if (F16) {                                                                                \
            uint16_t* h_ = (uint16_t*)malloc(n_ * 2);                                             \
            f32_to_f16_buf(w_, h_, n_);                                                           \
            free(w_);                                                                             \
            bufs[k] = h_;                                                                         \
            it_->dtype = DT_F16;                                                                  \
            it_->nbytes = n_ * 2;                                                                 \
        } else {                                                                                  \
            bufs[k] = w_;                                                                         \
            it_->dtype = DT_F32;                                                                  \
            it_->nbytes = n_ * 4;                                                                 \
        }                                                                                         \
        it_->src = (const uint8_t*)bufs[k];                                                       \
        k++;                                                                                      \
    } while (0)

    ADD(0, SLOT_EMBED, "embed", vocab, hidden, 1, 1.0f, 0.0f);
    for (b = 1; b <= blocks; b++) {
        ADD(b, SLOT_NORM1, "norm1", hidden, 1, 0, 0.1f, 1.0f);
        ADD(b, SLOT_Q, "q", hidden, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        ADD(b, SLOT_K, "k", kv_dim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        ADD(b, SLOT_V, "v", kv_dim, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        ADD(b, SLOT_O, "o", hidden, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        ADD(b, SLOT_NORM2, "norm2", hidden, 1, 0, 0.1f, 1.0f);
        ADD(b, SLOT_GATE, "gate", inter, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        ADD(b, SLOT_UP, "up", inter, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
        ADD(b, SLOT_DOWN, "down", hidden, inter, 1, sqrtf(3.0f / inter), 0.0f);
        if (arch == ARCH_QWEN) {
            ADD(b, SLOT_QBIAS, "q_bias", hidden, 1, 0, 0.5f, 0.0f);
            ADD(b, SLOT_KBIAS, "k_bias", kv_dim, 1, 0, 0.5f, 0.0f);
            ADD(b, SLOT_VBIAS, "v_bias", kv_dim, 1, 0, 0.5f, 0.0f);
        }
    }
    ADD(blocks + 1, 0, "final_norm", hidden, 1, 0, 0.1f, 1.0f);
    ADD(blocks + 2, 0, "output", vocab, hidden, 1, sqrtf(3.0f / hidden), 0.0f);
#undef ADD
    rc = llf_emit(path, &h, items, k, err, errlen);
    for (i = 0; i < k; i++) free(bufs[i]);
    free(bufs);
    free(items);
    return rc;
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
 * backend.  fail_after >= 0 arms the backend's failure hook.  status[0] =
 * bind result (0 HIP, -1 fell back to CPU), status[1] = KV rows (all
 * layers, K and V) whose HBM copy differs from host KV at the end (HIP
 * without the hook only, else -1).  Returns 0 or -1 with err set. */
int ye_run(const char* path, int use_hip, int device_id, int fail_after, const uint32_t* prompt, int n_prompt,
           int n_decode, float* logits, uint32_t* tokens, int* status, char* err, size_t errlen)
{
    Engine e;
    uint32_t vocab, pos;
    int i;
    memset(&e, 0, sizeof e);
    status[0] = 0;
    status[1] = -1;
    if (engine_init(&e, path, 0, 0, err, errlen) != 0) return -1;
    vocab = e.ws.model.h.vocab;
    if (use_hip) {
        status[0] = bind_hip(&e, device_id, err, errlen);
        if (status[0] == -2) {
            engine_free(&e);
            return -1;
        }
        if (status[0] == 0 && fail_after >= 0) device_hip_fail_after(&e, fail_after);
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
        if (use_hip && status[0] == 0) {
            DeviceMode saved = e.device_mode;
            e.device_mode = DEV_MODE_VULKAN;  /* see the file comment */
            engine_forward(&e, tok, pos);
            e.device_mode = saved;
        } else {
            engine_forward(&e, tok, pos);
        }
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
            size_t r;
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
    engine_free(&e);
    return 0;
}
