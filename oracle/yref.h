/* yref.h -- CPU oracle for the yllm attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a clean-room C99 restatement of the
 * reference engine's CPU attention, KV-store, softmax and Gated-DeltaNet loops
 * (evilbinary/yllm).  It is the checker for the HIP kernels and the CPU
 * baseline timed by bench.py; nothing in the product library links it.
 *
 * Numerics follow the reference bit for bit when built with the reference's
 * flags (Makefile:122,165: -O2 -std=c99 -fopenmp -mavx2 -mfma -mf16c, no
 * -ffast-math; ISO C mode keeps GCC from contracting a*b+c into FMA):
 * same loop order, fp32 scalar accumulation, out-of-line f16 decode, libm
 * expf/sqrtf/log1pf.  Each function names the reference lines it restates.
 *
 * Pinning (tests/test_oracle.py): every function is compared bit-exactly with
 * the reference compiled from its own sources (oracle/_ref, when buildable)
 * and with committed golden vectors produced from it (tests/golden/), and is
 * additionally checked against closed forms (single key -> V row, equal keys
 * -> mean of V, softmax shift invariance, causality, GDN beta=0 decay and
 * orthonormal-key retrieval).  No function here is "parity unpinned".
 *
 * KV layout here is the ENGINE layout (yllm.h:109, engine.c:261): per layer
 * K and V are u16 f16 bit arrays [max_seq][n_kv*head_dim], row = position.
 */
#ifndef YLLM_ORACLE_YREF_H
#define YLLM_ORACLE_YREF_H

#include <stdint.h>
#include <stddef.h>

/* platform.c:316-338 -- exact IEEE half -> float, subnormals included */
float yo_f16_to_f32(uint16_t h);
/* platform.c:340-379 -- float -> half, round half away from zero on the
 * magnitude (mant += 0x1000), f32 subnormals -> signed zero, overflow -> inf */
uint16_t yo_f32_to_f16(float f);
/* platform.c:381-391 -- bf16 -> half by exponent rebias, f16-subnormal range
 * flushed to signed zero, mantissa truncated (exact: bf16 has 7 bits) */
uint16_t yo_bf16_to_f16(uint16_t b);
/* bf16 bits -> float (exact) */
float yo_bf16_to_f32(uint16_t b);
void yo_f32_to_f16_buf(const float* src, uint16_t* dst, size_t n);

/* OpenMP threads a parallel loop here would use (1 without OpenMP) */
int yo_threads(void);

/* matvec.c:1023-1031 */
void yo_softmax(float* v, uint32_t n);
/* matvec.c:942-949 */
void yo_l2norm(float* v, uint32_t n, float eps);

/* engine.c:1068-1072 (decode) / 518-529 (batch) / 928-934 (qwen35):
 * rows pos_start..pos_start+B-1 of one layer's K and V caches.
 * k, v: [B][kv_dim] fp32. */
void yo_kv_store(uint16_t* kcache, uint16_t* vcache, const float* k, const float* v,
                 uint32_t pos_start, uint32_t B, uint32_t kv_dim);

/* engine.c:1074-1096: one query token at position pos attends to keys
 * 0..pos.  q: [n_heads*head_dim] fp32; out: [n_heads*head_dim] fp32.
 * OpenMP static over heads as the reference. */
void yo_attn_decode(float* out, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                    uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim);

/* engine.c:532-563: B query tokens at positions pos_start+b, each causal over
 * keys 0..pos_start+b.  q/out rows are q_stride floats apart, head h at h*head_dim.
 * The reference runs prefill in chunks of <=64 tokens (engine.c:622-652) and
 * routes chunks of <16 tokens through the decode path (628); per token the
 * arithmetic is identical, so one call covers any chunking. */
void yo_attn_prefill(float* out, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                     uint32_t pos_start, uint32_t B, uint32_t n_heads, uint32_t n_kv_heads,
                     uint32_t head_dim, uint32_t q_stride);

/* engine.c:959-960: x[i] *= 1/(1+expf(-gate[i])) */
void yo_gate_sigmoid(float* x, const float* gate, uint32_t n);

/* engine.c:788-793: beta <- sigmoid(beta_raw); gate <- softplus(alpha+dt)*a
 * (softplus computed as log1pf(expf(.)) like the reference). */
void yo_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt,
                  const float* a, uint32_t n_vheads);

/* matvec.c:975-1004: one recurrent step for all v-heads.
 * S: [n_vheads][hv][hk] (column j of head h, the state is stored transposed),
 * q,k: [num_k_heads*hk] (v-head h uses k-head h % num_k_heads),
 * v: [n_vheads*hv], gate: [n_vheads] log-decay, beta: [n_vheads].
 * out: [n_vheads*hv]. */
void yo_gdn_state_update(float* S, float* out, const float* q, const float* k, const float* v,
                         const float* gate, const float* beta, uint32_t num_k_heads, uint32_t hk,
                         uint32_t n_vheads, uint32_t hv);

/* engine.c:826-831 for T consecutive tokens: per token l2-normalise q and k
 * per k-head (eps), then one gdn_state_update.  q,k: [T][num_k_heads*hk]
 * (normalised in place), v: [T][n_vheads*hv], gate/beta: [T][n_vheads],
 * out: [T][n_vheads*hv].  S is updated in place. */
void yo_gdn_sequence(float* S, float* out, float* q, float* k, const float* v,
                     const float* gate, const float* beta, uint32_t T, uint32_t num_k_heads,
                     uint32_t hk, uint32_t n_vheads, uint32_t hv, float eps);

/* matvec.c:956-968 (conv1d_update): the delay line state [kwidth][dim]
 * shifts up one row, x becomes its last row, and
 * x[ch] = sum_i state[i][ch] * w[ch*kwidth + i] (in i order), in place. */
void yo_conv1d_update(float* state, float* x, const float* w, uint32_t dim, uint32_t kwidth);

/* engine.c:809-812 for T consecutive tokens: conv1d_update then silu
 * x / (1 + expf(-x)) per channel.  x: [T][dim] in place. */
void yo_conv_silu_sequence(float* state, float* x, const float* w, uint32_t T, uint32_t dim, uint32_t kwidth);

/* matvec.c:1007-1021 (rmsnorm_gated): inv = 1/sqrtf(sum x^2 / n + eps);
 * y[i] = x[i] * w[i] * inv * (z[i] / (1 + expf(-z[i]))); w f32 (w_f16 == 0)
 * or f16 bits. */
void yo_rmsnorm_gated(float* y, const float* x, const void* w, int w_f16, const float* z, uint32_t n, float eps);

/* matvec.c:890-939 (rope_inplace / rope_inplace_qwen / rope_inplace_mrope):
 * kind 1 rotates pairs (2j, 2j+1), kind 2 pairs (j, j+d/2), kind 3 pairs
 * (j, j+n_rot/2) of the first n_rot dims only, kind 0 nothing; freq =
 * powf(theta, -2j/span) with span = d (n_rot for kind 3), angle = freq*pos,
 * (a, b) -> (a cos - b sin, a sin + b cos).  One head of d floats, in place. */
void yo_rope(float* v, uint32_t d, uint32_t pos, float theta, int kind, uint32_t n_rot);

/* engine.c:1054-1072: for each of B tokens at pos_start.., yo_rope on the
 * n_heads q heads and n_kv k heads (q [B][n_heads*d], k [B][n_kv*d] in
 * place), then k and v [B][n_kv*d] rounded (yo_f32_to_f16) into the
 * engine-layout caches at row pos (kcache, vcache [rows][n_kv*d]). */
/* matvec.c:98-122 (matmul_f32 / matmul_f16): y[o] = sum_i x[i] * w[o*in + i],
 * summed in i order from 0; w f32 (w_f16 == 0) or f16 bits, rows of `in`. */
void yo_matmul(float* y, const float* x, const void* w, int w_f16, uint32_t out, uint32_t in);

/* engine.c:969-973 for B tokens: x[b] += matmul(att[b], W_o) (hidden outputs
 * of qdim inputs); x [B][hidden] updated in place. */
void yo_o_proj(float* x, const float* att, const void* w, int w_f16, uint32_t B, uint32_t hidden, uint32_t qdim);

void yo_rope_kv_store(float* q, float* k, const float* v, uint16_t* kcache, uint16_t* vcache, uint32_t pos_start,
                      uint32_t B, uint32_t n_heads, uint32_t n_kv, uint32_t d, int kind, uint32_t n_rot,
                      float theta);

#endif
