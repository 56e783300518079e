/* attn_ref.c -- CPU oracle for the attention hot path (TEST INFRASTRUCTURE).
 *
 * Restates, in the reference's arithmetic order, the CPU loops of
 * evilbinary/yllm that the HIP kernels replace.  Used only by tests/ as the
 * checker and by bench.py as the timed CPU baseline.  See yref.h for the
 * pinning of each function.
 */
#include "yref.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int yo_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* matvec.c:1023-1031: max, exp(x - max) with a running sum, divide */
void yo_softmax(float* v, uint32_t n)
{
    float mx = v[0];
    float sum = 0.0f;
    uint32_t i;
    for (i = 1; i < n; i++)
        if (v[i] > mx) mx = v[i];
    for (i = 0; i < n; i++) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    for (i = 0; i < n; i++) v[i] /= sum;
}

/* matvec.c:942-949: x / max(||x||, eps) */
void yo_l2norm(float* v, uint32_t n, float eps)
{
    float ss = 0.0f;
    uint32_t i;
    for (i = 0; i < n; i++) ss += v[i] * v[i];
    float r = 1.0f / fmaxf(sqrtf(ss), eps);
    for (i = 0; i < n; i++) v[i] *= r;
}

/* engine.c:1068-1072 / 518-529 / 928-934 */
void yo_kv_store(uint16_t* kcache, uint16_t* vcache, const float* k, const float* v,
                 uint32_t pos_start, uint32_t B, uint32_t kv_dim)
{
    uint32_t b, j;
    for (b = 0; b < B; b++) {
        uint16_t* kr = kcache + (size_t)(pos_start + b) * kv_dim;
        uint16_t* vr = vcache + (size_t)(pos_start + b) * kv_dim;
        const float* ks = k + (size_t)b * kv_dim;
        const float* vs = v + (size_t)b * kv_dim;
        for (j = 0; j < kv_dim; j++) {
            kr[j] = yo_f32_to_f16(ks[j]);
            vr[j] = yo_f32_to_f16(vs[j]);
        }
    }
}

/* One query head against keys 0..n_keys-1 of one kv head, in the order of
 * engine.c:1082-1095: scores acc=0, += q*k in dimension order, times
 * 1/sqrtf(d); softmax over the n_keys scores; out = sum_s a_s * v_s in key
 * order, dimension by dimension.  kh/vh point at the head's first element of
 * row 0; rows are row_stride u16 apart.  att: n_keys floats of scratch. */
static void attend_one_head(float* out, const float* qh, const uint16_t* kh, const uint16_t* vh,
                            size_t row_stride, uint32_t n_keys, uint32_t hd, float inv_d, float* att)
{
    uint32_t s, j;
    for (s = 0; s < n_keys; s++) {
        const uint16_t* kr = kh + (size_t)s * row_stride;
        float acc = 0.0f;
        for (j = 0; j < hd; j++) acc += qh[j] * yo_f16_to_f32(kr[j]);
        att[s] = acc * inv_d;
    }
    yo_softmax(att, n_keys);
    memset(out, 0, (size_t)hd * sizeof(float));
    for (s = 0; s < n_keys; s++) {
        const uint16_t* vr = vh + (size_t)s * row_stride;
        float a = att[s];
        for (j = 0; j < hd; j++) out[j] += a * yo_f16_to_f32(vr[j]);
    }
}

/* engine.c:1074-1096 */
void yo_attn_decode(float* out, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                    uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim)
{
    size_t kv_dim = (size_t)n_kv_heads * head_dim;
    uint32_t n_keys = pos + 1;
    float inv_d = 1.0f / sqrtf((float)head_dim);
    float* att = (float*)malloc((size_t)n_heads * n_keys * sizeof(float));
    int hh;
    if (!att) return;
#pragma omp parallel for schedule(static)
    for (hh = 0; hh < (int)n_heads; hh++) {
        uint32_t kvh = (uint32_t)hh * n_kv_heads / n_heads;      /* engine.c:1079 */
        attend_one_head(out + (size_t)hh * head_dim, q + (size_t)hh * head_dim,
                        kcache + (size_t)kvh * head_dim, vcache + (size_t)kvh * head_dim,
                        kv_dim, n_keys, head_dim, inv_d, att + (size_t)hh * n_keys);
    }
    free(att);
}

/* engine.c:532-563 */
void yo_attn_prefill(float* out, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                     uint32_t pos_start, uint32_t B, uint32_t n_heads, uint32_t n_kv_heads,
                     uint32_t head_dim, uint32_t q_stride)
{
    size_t kv_dim = (size_t)n_kv_heads * head_dim;
    uint32_t max_keys = pos_start + B;
    float inv_d = 1.0f / sqrtf((float)head_dim);
    float* att = (float*)malloc((size_t)n_heads * max_keys * sizeof(float));
    int hh;
    if (!att) return;
#pragma omp parallel for schedule(static)
    for (hh = 0; hh < (int)n_heads; hh++) {
        uint32_t kvh = (uint32_t)hh * n_kv_heads / n_heads;      /* engine.c:537 */
        uint32_t bb;
        for (bb = 0; bb < B; bb++) {
            attend_one_head(out + (size_t)bb * q_stride + (size_t)hh * head_dim,
                            q + (size_t)bb * q_stride + (size_t)hh * head_dim,
                            kcache + (size_t)kvh * head_dim, vcache + (size_t)kvh * head_dim,
                            kv_dim, pos_start + bb + 1, head_dim, inv_d,
                            att + (size_t)hh * max_keys);
        }
    }
    free(att);
}

/* engine.c:959-960 */
void yo_gate_sigmoid(float* x, const float* gate, uint32_t n)
{
    uint32_t i;
    for (i = 0; i < n; i++) x[i] *= 1.0f / (1.0f + expf(-gate[i]));
}

/* engine.c:788-793 */
void yo_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt,
                  const float* a, uint32_t n_vheads)
{
    uint32_t h;
    for (h = 0; h < n_vheads; h++) {
        beta[h] = 1.0f / (1.0f + expf(-beta[h]));
        float z = alpha[h] + dt[h];
        float softplus = log1pf(expf(z));
        gate[h] = softplus * a[h];
    }
}

/* matvec.c:975-1004.  Column j of head h (length hk, contiguous) is decayed
 * by g = expf(gate[h]) while its dot with k accumulates; delta_j =
 * (v_j - dot) * beta; the column gains k * delta_j; after all columns are
 * updated, o_j = (column_j . q) * (1/sqrtf(hv)). */
void yo_gdn_state_update(float* S, float* out, const float* q, const float* k, const float* v,
                         const float* gate, const float* beta, uint32_t num_k_heads, uint32_t hk,
                         uint32_t n_vheads, uint32_t hv)
{
    const float scale = 1.0f / sqrtf((float)hv);
    uint32_t h, j, i;
    for (h = 0; h < n_vheads; h++) {
        uint32_t kh = h % num_k_heads;                           /* matvec.c:983 */
        const float* qh = q + (size_t)kh * hk;
        const float* kv = k + (size_t)kh * hk;
        const float* vh = v + (size_t)h * hv;
        float* Sh = S + (size_t)h * hk * hv;
        float* oh = out + (size_t)h * hv;
        float g = expf(gate[h]);
        float bt = beta[h];
        for (j = 0; j < hv; j++) {
            float* col = Sh + (size_t)j * hv;
            float dot = 0.0f;
            float delta;
            for (i = 0; i < hk; i++) {
                col[i] *= g;
                dot += col[i] * kv[i];
            }
            delta = (vh[j] - dot) * bt;
            for (i = 0; i < hk; i++) col[i] += kv[i] * delta;
        }
        for (j = 0; j < hv; j++) {
            const float* col = Sh + (size_t)j * hv;
            float dot = 0.0f;
            for (i = 0; i < hk; i++) dot += col[i] * qh[i];
            oh[j] = dot * scale;
        }
    }
}

/* engine.c:826-831 per token, T tokens in order */
void yo_gdn_sequence(float* S, float* out, float* q, float* k, const float* v,
                     const float* gate, const float* beta, uint32_t T, uint32_t num_k_heads,
                     uint32_t hk, uint32_t n_vheads, uint32_t hv, float eps)
{
    uint32_t t, i;
    size_t qk_dim = (size_t)num_k_heads * hk;
    size_t v_dim = (size_t)n_vheads * hv;
    for (t = 0; t < T; t++) {
        float* qt = q + t * qk_dim;
        float* kt = k + t * qk_dim;
        for (i = 0; i < num_k_heads; i++) yo_l2norm(qt + (size_t)i * hk, hk, eps);
        for (i = 0; i < num_k_heads; i++) yo_l2norm(kt + (size_t)i * hk, hk, eps);
        yo_gdn_state_update(S, out + t * v_dim, qt, kt, v + t * v_dim,
                            gate + (size_t)t * n_vheads, beta + (size_t)t * n_vheads,
                            num_k_heads, hk, n_vheads, hv);
    }
}

/* matvec.c:956-968.  Products and sums are separate roundings (the reference
 * is compiled in ISO C mode without FMA contraction). */
void yo_conv1d_update(float* state, float* x, const float* w, uint32_t dim, uint32_t kwidth)
{
    uint32_t ch, i;
    memmove(state, state + dim, (size_t)(kwidth - 1) * dim * sizeof(float));
    memcpy(state + (size_t)(kwidth - 1) * dim, x, (size_t)dim * sizeof(float));
    for (ch = 0; ch < dim; ch++) {
        float acc = 0.0f;
        for (i = 0; i < kwidth; i++) acc += state[(size_t)i * dim + ch] * w[(size_t)ch * kwidth + i];
        x[ch] = acc;
    }
}

/* engine.c:809-812 */
void yo_conv_silu_sequence(float* state, float* x, const float* w, uint32_t T, uint32_t dim, uint32_t kwidth)
{
    uint32_t t, ch;
    for (t = 0; t < T; t++) {
        float* row = x + (size_t)t * dim;
        yo_conv1d_update(state, row, w, dim, kwidth);
        for (ch = 0; ch < dim; ch++) row[ch] = row[ch] / (1.0f + expf(-row[ch]));
    }
}

/* matvec.c:1007-1021 */
void yo_rmsnorm_gated(float* y, const float* x, const void* w, int w_f16, const float* z, uint32_t n, float eps)
{
    float s = 0.0f;
    uint32_t i;
    for (i = 0; i < n; i++) s += x[i] * x[i];
    {
        const float inv = 1.0f / sqrtf(s / (float)n + eps);
        for (i = 0; i < n; i++) {
            const float wgt = w_f16 ? yo_f16_to_f32(((const uint16_t*)w)[i]) : ((const float*)w)[i];
            const float zg = z[i];
            y[i] = x[i] * wgt * inv * (zg / (1.0f + expf(-zg)));
        }
    }
}

/* matvec.c:890-939: rope_inplace (kind 1, pairs (2j, 2j+1)), rope_inplace_qwen
 * (kind 2, pairs (j, j+d/2)) and rope_inplace_mrope (kind 3, pairs
 * (j, j+n_rot/2) for j < n_rot/2, other dims unchanged); kind 0 leaves v.
 * Products and differences are separate roundings. */
void yo_rope(float* v, uint32_t d, uint32_t pos, float theta, int kind, uint32_t n_rot)
{
    uint32_t n_pairs, span, j;
    if (kind == 0) return;
    span = kind == 3 ? n_rot : d;
    n_pairs = span / 2;
    for (j = 0; j < n_pairs; j++) {
        const uint32_t i0 = kind == 1 ? 2 * j : j;
        const uint32_t i1 = kind == 1 ? 2 * j + 1 : j + n_pairs;
        const float freq = powf(theta, -2.0f * (float)j / (float)span);
        const float ang = freq * (float)pos;
        const float c = cosf(ang), s = sinf(ang);
        const float a = v[i0], b = v[i1];
        v[i0] = a * c - b * s;
        v[i1] = a * s + b * c;
    }
}

/* engine.c:1054-1072 (and 532-550 batched): per token, RoPE on every q and
 * k head, then k and v rounded into the engine-layout caches at row pos. */
void yo_rope_kv_store(float* q, float* k, const float* v, uint16_t* kcache, uint16_t* vcache, uint32_t pos_start,
                      uint32_t B, uint32_t n_heads, uint32_t n_kv, uint32_t d, int kind, uint32_t n_rot,
                      float theta)
{
    const size_t qd = (size_t)n_heads * d, kvd = (size_t)n_kv * d;
    uint32_t b, h;
    size_t j;
    for (b = 0; b < B; b++) {
        const uint32_t pos = pos_start + b;
        float* qb = q + b * qd;
        float* kb = k + b * kvd;
        const float* vb = v + b * kvd;
        for (h = 0; h < n_heads; h++) yo_rope(qb + (size_t)h * d, d, pos, theta, kind, n_rot);
        for (h = 0; h < n_kv; h++) yo_rope(kb + (size_t)h * d, d, pos, theta, kind, n_rot);
        for (j = 0; j < kvd; j++) {
            kcache[(size_t)pos * kvd + j] = yo_f32_to_f16(kb[j]);
            vcache[(size_t)pos * kvd + j] = yo_f32_to_f16(vb[j]);
        }
    }
}

/* matvec.c:98-122 (matmul_f32 / matmul_f16): y[o] = sum_i x[i] * w[o*in + i]
 * in i order from 0, w f32 (w_f16 == 0) or f16 bits. */
void yo_matmul(float* y, const float* x, const void* w, int w_f16, uint32_t out, uint32_t in)
{
    uint32_t o, i;
    for (o = 0; o < out; o++) {
        float acc = 0.0f;
        if (w_f16) {
            const uint16_t* wr = (const uint16_t*)w + (size_t)o * in;
            for (i = 0; i < in; i++) acc += x[i] * yo_f16_to_f32(wr[i]);
        } else {
            const float* wr = (const float*)w + (size_t)o * in;
            for (i = 0; i < in; i++) acc += x[i] * wr[i];
        }
        y[o] = acc;
    }
}

/* engine.c:969-973 per token: y = matmul(att_out, W_o), then x += y.
 * x [B][hidden], att [B][qdim], in place on x. */
void yo_o_proj(float* x, const float* att, const void* w, int w_f16, uint32_t B, uint32_t hidden, uint32_t qdim)
{
    float* y = (float*)malloc((size_t)hidden * sizeof(float));
    uint32_t b, j;
    if (!y) return;
    for (b = 0; b < B; b++) {
        yo_matmul(y, att + (size_t)b * qdim, w, w_f16, hidden, qdim);
        for (j = 0; j < hidden; j++) x[(size_t)b * hidden + j] += y[j];
    }
    free(y);
}
