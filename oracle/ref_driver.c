/* ref_driver.c -- drives the reference engine's own CPU layer forward on a
 * synthetic one-block model (TEST INFRASTRUCTURE).
 *
 * Compiled only into oracle/_ref/libyref.so together with the reference
 * sources under /root/reference (oracle/Makefile, target `ref`), against the
 * reference's own headers.  It lets tests read the exact outputs of the
 * attention loops that are inline in the reference (engine.c:1074-1096,
 * 532-563, 935-960) and of the GDN gate maths (engine.c:788-793), which no
 * reference function returns on its own.
 *
 * How the attention output is recovered exactly.  The layer's weights are
 * f32; NORM1/NORM2 are ones, O is the identity, GATE/UP/DOWN are zero, so the
 * block returns x + attn (the FFN adds exact zeros).  The input x has a single
 * non-zero coordinate c, so every projection is one product s*W[:,c] (s = the
 * rmsnorm output at c) and the residual leaves attn[i] untouched for i != c.
 * Columns c and c+1 of Q/K/V are equal and the layer is run twice, with c and
 * then c+1, which recovers every coordinate.  The query actually used (after
 * RoPE / QK-norm) is read back, or rebuilt with the reference's own exported
 * rmsnorm/rope functions where the engine overwrites it.
 */
#include "yllm.h"
#include "matvec.h"
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <stdio.h>

#define NL 4u  /* embed, block 1, final norm, output */

typedef struct {
    Engine e;
    LlfTensorMeta* metas;
    LlfLayerDir dir[NL];
    uint32_t base_idx[NL];
    float* blob;
    size_t blob_floats;
    size_t used;
} Rig;

static float bits_to_f(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

static float* rig_tensor(Rig* r, uint32_t slot, uint32_t s0, uint32_t s1)
{
    size_t n = (size_t)s0 * (s1 ? s1 : 1);
    LlfTensorMeta* tm = &r->metas[r->base_idx[1] + slot];
    memset(tm, 0, sizeof(*tm));
    tm->dtype = DT_F32;
    tm->ndim = s1 ? 2 : 1;
    tm->shape[0] = s0;
    tm->shape[1] = s1;
    tm->offset = (uint64_t)r->used * 4;
    tm->size = (uint64_t)n * 4;
    size_t padded = (n + 15) & ~(size_t)15;
    if (r->used + padded > r->blob_floats) {
        fprintf(stderr, "ref_driver: weight blob too small (%zu + %zu > %zu floats)\n", r->used, padded,
                r->blob_floats);
        abort();
    }
    float* p = r->blob + r->used;
    r->used += padded;
    return p;
}

static int rig_init(Rig* r, uint32_t arch, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                    uint32_t hidden, uint32_t max_seq, size_t blob_floats, uint32_t pb_cap)
{
    memset(r, 0, sizeof(*r));
    r->metas = (LlfTensorMeta*)calloc((size_t)NL * BLOCK_TENSORS_MTP, sizeof(LlfTensorMeta));
    r->blob = (float*)calloc(blob_floats, 4);
    if (!r->metas || !r->blob) return -1;
    r->blob_floats = blob_floats;
    uint32_t i;
    for (i = 0; i < NL; i++) r->base_idx[i] = i * BLOCK_TENSORS_MTP;
    Engine* e = &r->e;
    LlfHeader* h = &e->ws.model.h;
    h->arch = arch;
    h->n_blocks = 1;
    h->vocab = 8;
    h->hidden = hidden;
    h->n_heads = n_heads;
    h->n_kv_heads = n_kv;
    h->head_dim = hd;
    h->max_seq = max_seq;
    h->dtype = DT_F32;
    h->norm_eps_bits = f_to_bits(1e-6f);
    h->rope_theta_bits = f_to_bits(10000.0f);
    e->ws.model.n_layers = NL;
    e->ws.model.dir = r->dir;
    e->ws.model.metas = r->metas;
    e->ws.model.base_idx = r->base_idx;
    e->ws.map.base = r->blob;
    e->ws.map.size = blob_floats * 4;
    r->dir[1].offset = 0;
    r->dir[1].size = blob_floats * 4;
    e->arch = arch;
    e->kv_dim = n_kv * hd;
    e->max_seq = max_seq;
    e->kv = (uint16_t*)calloc((size_t)3 * max_seq * e->kv_dim, 2);
    e->x = (float*)calloc(hidden, 4);
    e->hb = (float*)calloc((size_t)hidden * 9, 4);
    e->hb2 = (float*)calloc((size_t)hidden * 9, 4);
    e->att = (float*)calloc((size_t)max_seq * n_heads, 4);
    e->scratch = (float*)calloc(65536, 4);
    e->pb_cap = pb_cap;
    e->pb = (float*)calloc((size_t)pb_cap * hidden, 4);
    e->pb2 = (float*)calloc((size_t)pb_cap * hidden, 4);
    e->pbq = (float*)calloc((size_t)pb_cap * hidden, 4);
    e->pbk = (float*)calloc((size_t)pb_cap * e->kv_dim, 4);
    e->pbv = (float*)calloc((size_t)pb_cap * e->kv_dim, 4);
    e->pba = (float*)calloc((size_t)pb_cap * n_heads * max_seq, 4);
    if (!e->kv || !e->x || !e->hb || !e->hb2 || !e->att || !e->scratch || !e->pb || !e->pb2 ||
        !e->pbq || !e->pbk || !e->pbv || !e->pba)
        return -1;
    return 0;
}

/* FFN of the block: NORM2 ones, GATE/UP/DOWN zero, inter = 16 */
static int rig_ffn(Rig* r, uint32_t hidden)
{
    uint32_t inter = 16, i;
    float* n2 = rig_tensor(r, SLOT_NORM2, hidden, 0);
    for (i = 0; i < hidden; i++) n2[i] = 1.0f;
    rig_tensor(r, SLOT_GATE, hidden, inter);
    rig_tensor(r, SLOT_UP, hidden, inter);
    rig_tensor(r, SLOT_DOWN, inter, hidden);
    Engine* e = &r->e;
    e->inter = inter;
    e->ffn = (float*)calloc((size_t)2 * inter, 4);
    e->pbg = (float*)calloc((size_t)e->pb_cap * inter, 4);
    e->pbu = (float*)calloc((size_t)e->pb_cap * inter, 4);
    return (e->ffn && e->pbg && e->pbu) ? 0 : -1;
}

static void rig_free(Rig* r)
{
    Engine* e = &r->e;
    free(e->kv); free(e->x); free(e->hb); free(e->hb2); free(e->att); free(e->scratch);
    free(e->ffn); free(e->pb); free(e->pb2); free(e->pbq); free(e->pbk); free(e->pbv);
    free(e->pbg); free(e->pbu); free(e->pba); free(e->ssm_state); free(e->ssm_conv);
    free(r->metas); free(r->blob);
}

static void set_col(float* w, uint32_t rows, uint32_t cols, uint32_t c, const float* colv)
{
    uint32_t i;
    for (i = 0; i < rows; i++) w[(size_t)i * cols + c] = colv[i];
}

static void set_identity(float* w, uint32_t n)
{
    uint32_t i;
    for (i = 0; i < n; i++) w[(size_t)i * n + i] = 1.0f;
}

static void load_prev_kv(Rig* r, const uint16_t* kprev, const uint16_t* vprev, uint32_t n_rows)
{
    Engine* e = &r->e;
    size_t row = e->kv_dim;
    uint16_t* kc = e->kv + (size_t)1 * e->max_seq * row;
    uint16_t* vc = e->kv + (size_t)2 * e->max_seq * row;
    if (n_rows) {
        memcpy(kc, kprev, (size_t)n_rows * row * 2);
        memcpy(vc, vprev, (size_t)n_rows * row * 2);
    }
}

static void read_kv(Rig* r, uint16_t* krows, uint16_t* vrows, uint32_t n_rows)
{
    Engine* e = &r->e;
    size_t row = e->kv_dim;
    memcpy(krows, e->kv + (size_t)1 * e->max_seq * row, (size_t)n_rows * row * 2);
    memcpy(vrows, e->kv + (size_t)2 * e->max_seq * row, (size_t)n_rows * row * 2);
}

/* engine.c:992-1109 (decode attention at 1074-1096) for a llama (arch 0) or
 * qwen (arch 1) block.  kprev/vprev: rows 0..pos-1 [pos][n_kv*hd] f16 bits.
 * wq [n_heads*hd], wk/wv [n_kv*hd]: the projection column.  Outputs: q_used
 * (after RoPE), krows/vrows (rows 0..pos), att [n_heads*hd]. */
int yr_decode(uint32_t arch, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t pos,
              const uint16_t* kprev, const uint16_t* vprev, const float* wq, const float* wk,
              const float* wv, float xval, float* q_used, uint16_t* krows, uint16_t* vrows,
              float* att)
{
    uint32_t hidden = n_heads * hd, kv_dim = n_kv * hd, i, run;
    uint32_t max_seq = pos + 1;
    size_t need = (size_t)hidden * hidden * 2 + (size_t)kv_dim * hidden * 2 + (size_t)hidden * 64 + 4096;
    Rig r;
    if (hidden < 2 || rig_init(&r, arch, n_heads, n_kv, hd, hidden, max_seq, need, 1) != 0) return -1;
    float* n1 = rig_tensor(&r, SLOT_NORM1, hidden, 0);
    for (i = 0; i < hidden; i++) n1[i] = 1.0f;
    float* Wq = rig_tensor(&r, SLOT_Q, hidden, hidden);
    float* Wk = rig_tensor(&r, SLOT_K, hidden, kv_dim);
    float* Wv = rig_tensor(&r, SLOT_V, hidden, kv_dim);
    float* Wo = rig_tensor(&r, SLOT_O, hidden, hidden);
    if (rig_ffn(&r, hidden) != 0) { rig_free(&r); return -1; }
    set_col(Wq, hidden, hidden, 0, wq); set_col(Wq, hidden, hidden, 1, wq);
    set_col(Wk, kv_dim, hidden, 0, wk); set_col(Wk, kv_dim, hidden, 1, wk);
    set_col(Wv, kv_dim, hidden, 0, wv); set_col(Wv, kv_dim, hidden, 1, wv);
    set_identity(Wo, hidden);
    load_prev_kv(&r, kprev, vprev, pos);
    for (run = 0; run < 2; run++) {
        memset(r.e.x, 0, (size_t)hidden * 4);
        r.e.x[run] = xval;
        if (engine_fwd_block_at(&r.e, 1, pos, (const uint8_t*)r.blob, r.e.kv) != 0) { rig_free(&r); return -1; }
        if (run == 0) {
            memcpy(att, r.e.x, (size_t)hidden * 4);
            memcpy(q_used, r.e.hb2, (size_t)hidden * 4);
        } else {
            att[0] = r.e.x[0];
            if (memcmp(q_used, r.e.hb2, (size_t)hidden * 4) != 0) { rig_free(&r); return -2; }
        }
    }
    read_kv(&r, krows, vrows, pos + 1);
    rig_free(&r);
    return 0;
}

/* engine.c:435-587 (attention at 532-563): B tokens from pos_start.  Token b
 * uses input coordinate 2b (run 0) / 2b+1 (run 1), so hidden >= 2B.
 * wq: [B][n_heads*hd], wk/wv: [B][n_kv*hd].  Outputs q_used [B][hidden]
 * (rebuilt with the reference rmsnorm/rope, the engine overwrites it),
 * krows/vrows rows 0..pos_start+B-1, att [B][hidden]. */
int yr_prefill(uint32_t arch, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t pos_start,
               uint32_t B, const uint16_t* kprev, const uint16_t* vprev, const float* wq,
               const float* wk, const float* wv, float xval, float* q_used, uint16_t* krows,
               uint16_t* vrows, float* att)
{
    uint32_t hidden = n_heads * hd, kv_dim = n_kv * hd, i, b, run;
    uint32_t max_seq = pos_start + B;
    size_t need = (size_t)hidden * hidden * 2 + (size_t)kv_dim * hidden * 2 + (size_t)hidden * 64 + 4096;
    Rig r;
    if (B == 0 || hidden < 2 * B) return -1;
    if (rig_init(&r, arch, n_heads, n_kv, hd, hidden, max_seq, need, B) != 0) return -1;
    float* n1 = rig_tensor(&r, SLOT_NORM1, hidden, 0);
    for (i = 0; i < hidden; i++) n1[i] = 1.0f;
    float* Wq = rig_tensor(&r, SLOT_Q, hidden, hidden);
    float* Wk = rig_tensor(&r, SLOT_K, hidden, kv_dim);
    float* Wv = rig_tensor(&r, SLOT_V, hidden, kv_dim);
    float* Wo = rig_tensor(&r, SLOT_O, hidden, hidden);
    if (rig_ffn(&r, hidden) != 0) { rig_free(&r); return -1; }
    for (b = 0; b < B; b++) {
        set_col(Wq, hidden, hidden, 2 * b, wq + (size_t)b * hidden);
        set_col(Wq, hidden, hidden, 2 * b + 1, wq + (size_t)b * hidden);
        set_col(Wk, kv_dim, hidden, 2 * b, wk + (size_t)b * kv_dim);
        set_col(Wk, kv_dim, hidden, 2 * b + 1, wk + (size_t)b * kv_dim);
        set_col(Wv, kv_dim, hidden, 2 * b, wv + (size_t)b * kv_dim);
        set_col(Wv, kv_dim, hidden, 2 * b + 1, wv + (size_t)b * kv_dim);
    }
    set_identity(Wo, hidden);
    engine_attach_cpu_fwd(&r.e);
    load_prev_kv(&r, kprev, vprev, pos_start);
    for (run = 0; run < 2; run++) {
        memset(r.e.pb, 0, (size_t)B * hidden * 4);
        for (b = 0; b < B; b++) r.e.pb[(size_t)b * hidden + 2 * b + run] = xval;
        if (r.e.fwd_block_batch(&r.e, 1, pos_start, B) != 0) { rig_free(&r); return -1; }
        for (b = 0; b < B; b++) {
            float* dst = att + (size_t)b * hidden;
            const float* src = r.e.pb + (size_t)b * hidden;
            if (run == 0) memcpy(dst, src, (size_t)hidden * 4);
            else dst[2 * b] = src[2 * b];
        }
    }
    /* the query the attention loop saw: rmsnorm -> single-column projection -> RoPE */
    {
        float theta = bits_to_f(r.e.ws.model.h.rope_theta_bits);
        float eps = bits_to_f(r.e.ws.model.h.norm_eps_bits);
        float* xr = (float*)calloc(hidden, 4);
        float* x2 = (float*)calloc(hidden, 4);
        for (b = 0; b < B; b++) {
            float* qb = q_used + (size_t)b * hidden;
            memset(xr, 0, (size_t)hidden * 4);
            xr[2 * b] = xval;
            rmsnorm(x2, xr, (const uint8_t*)n1, hidden, eps, DT_F32);
            for (i = 0; i < hidden; i++) qb[i] = 0.0f + x2[2 * b] * wq[(size_t)b * hidden + i];
            for (i = 0; i < n_heads; i++) {
                if (arch == ARCH_QWEN) rope_inplace_qwen(qb + (size_t)i * hd, hd, pos_start + b, theta);
                else rope_inplace(qb + (size_t)i * hd, hd, pos_start + b, theta);
            }
        }
        free(xr); free(x2);
    }
    read_kv(&r, krows, vrows, pos_start + B);
    rig_free(&r);
    return 0;
}

/* engine.c:886-982 (attention 935-957, gate 959-960): qwen35 gated-attention
 * block.  wq/wg [n_heads*hd], wk/wv [n_kv*hd].  Outputs q_used (after QK-norm
 * and M-RoPE), gate_used, krows/vrows rows 0..pos, att (after the sigmoid gate). */
int yr_gated(uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t pos,
             const uint16_t* kprev, const uint16_t* vprev, const float* wq, const float* wg,
             const float* wk, const float* wv, float xval, float* q_used, float* gate_used,
             uint16_t* krows, uint16_t* vrows, float* att)
{
    uint32_t hidden = n_heads * hd, kv_dim = n_kv * hd, i, run;
    uint32_t max_seq = pos + 1;
    size_t need = (size_t)hidden * hidden * 3 + (size_t)kv_dim * hidden * 2 + (size_t)hidden * 64 + 4096;
    Rig r;
    if (hd < 64 || 2 * hidden + 2 * kv_dim > 65536) return -1;
    if (rig_init(&r, ARCH_QWEN35, n_heads, n_kv, hd, hidden, max_seq, need, 1) != 0) return -1;
    float* n1 = rig_tensor(&r, SLOT_NORM1, hidden, 0);
    for (i = 0; i < hidden; i++) n1[i] = 1.0f;
    float* Wq = rig_tensor(&r, SLOT_Q, hidden, hidden);
    float* Wk = rig_tensor(&r, SLOT_K, hidden, kv_dim);
    float* Wv = rig_tensor(&r, SLOT_V, hidden, kv_dim);
    float* Wo = rig_tensor(&r, SLOT_O, hidden, hidden);
    float* Wg = rig_tensor(&r, SLOT_QGATE, hidden, hidden);
    float* qn = rig_tensor(&r, SLOT_QNORM, hd, 0);
    float* kn = rig_tensor(&r, SLOT_KNORM, hd, 0);
    for (i = 0; i < hd; i++) { qn[i] = 1.0f; kn[i] = 1.0f; }
    if (rig_ffn(&r, hidden) != 0) { rig_free(&r); return -1; }
    set_col(Wq, hidden, hidden, 0, wq); set_col(Wq, hidden, hidden, 1, wq);
    set_col(Wg, hidden, hidden, 0, wg); set_col(Wg, hidden, hidden, 1, wg);
    set_col(Wk, kv_dim, hidden, 0, wk); set_col(Wk, kv_dim, hidden, 1, wk);
    set_col(Wv, kv_dim, hidden, 0, wv); set_col(Wv, kv_dim, hidden, 1, wv);
    set_identity(Wo, hidden);
    engine_attach_cpu_fwd(&r.e);
    load_prev_kv(&r, kprev, vprev, pos);
    for (run = 0; run < 2; run++) {
        memset(r.e.x, 0, (size_t)hidden * 4);
        r.e.x[run] = xval;
        if (r.e.fwd_block(&r.e, 1, pos) != 0) { rig_free(&r); return -1; }
        if (run == 0) {
            memcpy(att, r.e.x, (size_t)hidden * 4);
            memcpy(q_used, r.e.scratch, (size_t)hidden * 4);
            memcpy(gate_used, r.e.scratch + hidden, (size_t)hidden * 4);
        } else {
            att[0] = r.e.x[0];
        }
    }
    read_kv(&r, krows, vrows, pos + 1);
    rig_free(&r);
    return 0;
}

/* engine.c:760-883 (gates 786-793, l2norm 826-827, recurrence 831): one GDN
 * step of a qwen35 block with n_k key heads and n_v value heads of size hd.
 * wqkv [2*n_k*hd + n_v*hd], walpha/wbeta [n_v]: projection columns; dt, a
 * [n_v]; S [n_v*hd*hd] in/out.  Outputs: q_used/k_used [n_k*hd] (after conv,
 * silu, l2norm), v_used [n_v*hd], alpha_raw/beta_raw [n_v] (the projections,
 * rebuilt with the reference rmsnorm), beta/gate [n_v] as computed by the
 * block. */
int yr_gdn(uint32_t n_k, uint32_t n_v, uint32_t hd, const float* wqkv, const float* walpha,
           const float* wbeta, const float* dt, const float* a, float xval, float* S,
           float* q_used, float* k_used, float* v_used, float* alpha_raw, float* beta_raw,
           float* beta, float* gate)
{
    uint32_t key_dim = n_k * hd, value_dim = n_v * hd, conv = 2 * key_dim + value_dim;
    uint32_t kwidth = 4, hidden = 64, i;
    size_t need = (size_t)conv * hidden + (size_t)value_dim * hidden * 2 + (size_t)n_v * hidden * 2 +
                  (size_t)conv * kwidth + (size_t)hidden * 64 + 8192;
    Rig r;
    if (conv > 16384 || value_dim > 7000 || n_v > 48) return -1;
    if (rig_init(&r, ARCH_QWEN35, 2, 1, hidden / 2, hidden, 4, need, 1) != 0) return -1;
    float* n1 = rig_tensor(&r, SLOT_NORM1, hidden, 0);
    for (i = 0; i < hidden; i++) n1[i] = 1.0f;
    float* Wqkv = rig_tensor(&r, SLOT_QKV, hidden, conv);
    rig_tensor(&r, SLOT_GATE_ATTN, hidden, value_dim);
    float* Wc = rig_tensor(&r, SLOT_SSM_CONV1D, kwidth, conv);
    float* A = rig_tensor(&r, SLOT_SSM_A, n_v, 0);
    float* D = rig_tensor(&r, SLOT_SSM_DT, n_v, 0);
    float* Wa = rig_tensor(&r, SLOT_SSM_ALPHA, hidden, n_v);
    float* Wb = rig_tensor(&r, SLOT_SSM_BETA, hidden, n_v);
    float* sn = rig_tensor(&r, SLOT_SSM_NORM, hd, 0);
    rig_tensor(&r, SLOT_SSM_OUT, value_dim, hidden);
    if (rig_ffn(&r, hidden) != 0) { rig_free(&r); return -1; }
    for (i = 0; i < hd; i++) sn[i] = 1.0f;
    set_col(Wqkv, conv, hidden, 0, wqkv);
    set_col(Wa, n_v, hidden, 0, walpha);
    set_col(Wb, n_v, hidden, 0, wbeta);
    memcpy(A, a, (size_t)n_v * 4);
    memcpy(D, dt, (size_t)n_v * 4);
    /* conv taps: the current input passes through with weight 1 */
    for (i = 0; i < conv; i++) Wc[(size_t)i * kwidth + (kwidth - 1)] = 1.0f;
    r.e.ssm_state = (float*)malloc((size_t)n_v * hd * hd * 4);
    r.e.ssm_conv = (float*)calloc((size_t)kwidth * conv, 4);
    if (!r.e.ssm_state || !r.e.ssm_conv) { rig_free(&r); return -1; }
    memcpy(r.e.ssm_state, S, (size_t)n_v * hd * hd * 4);
    engine_attach_cpu_fwd(&r.e);
    r.e.x[0] = xval;
    if (r.e.fwd_block(&r.e, 1, 0) != 0) { rig_free(&r); return -1; }
    memcpy(S, r.e.ssm_state, (size_t)n_v * hd * hd * 4);
    memcpy(q_used, r.e.scratch, (size_t)key_dim * 4);
    memcpy(k_used, r.e.scratch + key_dim, (size_t)key_dim * 4);
    memcpy(v_used, r.e.scratch + 2 * key_dim, (size_t)value_dim * 4);
    memcpy(beta, r.e.scratch + 32816, (size_t)n_v * 4);
    memcpy(gate, r.e.scratch + 32864, (size_t)n_v * 4);
    {
        float eps = bits_to_f(r.e.ws.model.h.norm_eps_bits);
        float* xr = (float*)calloc(hidden, 4);
        float* x2 = (float*)calloc(hidden, 4);
        xr[0] = xval;
        rmsnorm(x2, xr, (const uint8_t*)n1, hidden, eps, DT_F32);
        for (i = 0; i < n_v; i++) {
            alpha_raw[i] = 0.0f + x2[0] * walpha[i];
            beta_raw[i] = 0.0f + x2[0] * wbeta[i];
        }
        free(xr); free(x2);
    }
    rig_free(&r);
    return 0;
}
