/* yllm_hip.h -- C ABI of the MI355X (gfx950) attention backend for yllm.
 *
 * Kernel-level entry points that an engine device layer calls per layer.
 * They replace the attention part of the reference's CUDA kernel ABI
 * (inference/cuda/cuda_kernels.h:50-63: cuda_k_store_kv, cuda_k_store_kv_batch,
 * cuda_k_attn_decode, cuda_k_attn_prefill) and the CPU loops it mirrors
 * (inference/core/engine.c:1068-1096, 518-563, 928-960, 786-831;
 * matvec.c:942-1004).
 *
 * Conventions (all entry points):
 *   - extern "C", plain pointers and sizes, fixed-width integers;
 *   - every pointer argument is DEVICE memory unless its comment says host;
 *   - `stream` is a hipStream_t (NULL = the default stream); work is queued
 *     asynchronously on it and nothing synchronises;
 *   - return 0 on success, a negative YHIP_E* code otherwise, with a message
 *     available from yhip_last_error() (per host thread).  Unlike the
 *     reference (void, silent no-op for head_dim > 256), bad shapes are
 *     reported, never ignored.
 *
 * KV cache layout in HBM (per sequence, per layer), designed for coalesced
 * per-head streaming and for the MFMA operand shapes of the kernels:
 *   K : u16 f16 bits [n_kv_heads][kv_stride][head_dim]   (row = position)
 *   V : u16 f16 bits [n_kv_heads][kv_stride/32][head_dim][32]
 *       (tiles of 32 positions; within a tile, row = dimension, so one
 *       16-byte load holds 8 consecutive positions of one dimension)
 * kv_stride is the position capacity, a multiple of 64 (>= the engine's
 * max_seq).  The reference's engine layout ([max_seq][n_kv*head_dim] per
 * layer, yllm.h:109 / engine.c:261) converts with yhip_kv_from_engine /
 * yhip_kv_to_engine.  Values are stored with the reference CPU rounding
 * (platform.c:340-379: ties away from zero, f32 subnormals to zero), not RNE.
 *
 * Grouped-query mapping is the reference's: query head h reads kv head
 * h*n_kv_heads/n_heads (engine.c:537,940,1079).  head_dim is 64, 128 or 256.
 */
#ifndef YLLM_HIP_H
#define YLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types: the LLF codes DT_F16 / DT_F32 / DT_BF16 (llf.h:15-17) */
#define YHIP_F16 0u
#define YHIP_F32 1u
#define YHIP_BF16 2u

#define YHIP_OK 0
#define YHIP_EINVAL (-22)   /* bad shape, stride, dtype or null pointer */
#define YHIP_ENOSPC (-28)   /* workspace too small */
#define YHIP_EDEVICE (-5)   /* HIP runtime error (launch, copy, device) */

/* Message for the last non-zero return on this host thread ("" if none). */
const char* yhip_last_error(void);

/* Library version string and the gfx target it was built for. */
const char* yhip_version(void);

/* Elements (u16) of one layer's K (or V) cache for one sequence. */
uint64_t yhip_kv_layer_elems(uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride);

/* ---- KV store ------------------------------------------------------------
 * Replaces cuda_k_store_kv / cuda_k_store_kv_batch (cuda_kernels.h:50-53),
 * semantics of engine.c:1068-1072 / 518-529 / 928-934: rows pos_start ..
 * pos_start+B-1 of K and V, from k, v [B][n_kv_heads*head_dim] of element
 * type src_dtype (YHIP_F32 as the engine, or YHIP_F16 / YHIP_BF16).  The
 * rows must fit: pos_start + B <= kv_stride. */
int yhip_kv_store(uint16_t* kcache, uint16_t* vcache, const void* k, const void* v,
                  uint32_t src_dtype, uint32_t pos_start, uint32_t B, uint32_t n_kv_heads,
                  uint32_t head_dim, uint32_t kv_stride, void* stream);

/* Engine layout <-> head-major layout for n_rows positions of one layer
 * (session save / restore, cache.c:174-247; host-written KV,
 * device_cuda.c:534-549).  eng_k/eng_v: [n_rows][n_kv_heads*head_dim]. */
int yhip_kv_from_engine(uint16_t* kcache, uint16_t* vcache, const uint16_t* eng_k,
                        const uint16_t* eng_v, uint32_t n_rows, uint32_t n_kv_heads,
                        uint32_t head_dim, uint32_t kv_stride, void* stream);
int yhip_kv_to_engine(uint16_t* eng_k, uint16_t* eng_v, const uint16_t* kcache,
                      const uint16_t* vcache, uint32_t n_rows, uint32_t n_kv_heads,
                      uint32_t head_dim, uint32_t kv_stride, void* stream);

/* ---- Decode (split-K flash decoding) -------------------------------------
 * Replaces cuda_k_attn_decode (cuda_kernels.h:55-58); semantics of
 * engine.c:1074-1096: one query token per head at position pos attends to
 * keys 0..pos.  q, att_out: [n_heads*head_dim] fp32.  gate: NULL, or
 * [n_heads*head_dim] fp32 and att_out is multiplied by sigmoid(gate) (the
 * qwen35 gated attention, engine.c:959-960).  Needs
 * yhip_attn_decode_workspace(1, pos+1, pos+1, ...) bytes of workspace. */
int yhip_attn_decode(float* att_out, const float* q, const uint16_t* kcache,
                     const uint16_t* vcache, uint32_t pos, uint32_t n_heads,
                     uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride,
                     const float* gate, void* workspace, size_t workspace_bytes, void* stream);

/* The decode step with its RoPE and KV store fused into one launch: what
 * yhip_rope_kv_store (one token at pos, q_out fp32) followed by
 * yhip_attn_decode computes (engine.c:1054-1096; qwen35 910-960).  q, k, v are the token's raw
 * (unrotated) fp32 rows, [n_heads*head_dim] and [n_kv_heads*head_dim]; q is
 * not modified.  The key and value of position pos are rotated, rounded with
 * the reference f32->f16 rounding and stored into kcache / vcache (row pos is
 * overwritten and need not be initialised; the attention uses the new bits,
 * never what the row held).  rope, n_rot and theta as yhip_rope_kv_store
 * (n_rot a multiple of 8); gate and workspace as yhip_attn_decode.  q and
 * att_out 16-byte aligned.  The cosines and sines are the host's cosf / sinf
 * of the reference's angles, so q and the stored key are rotated exactly as
 * the reference rotates them (yhip_rope_kv_store uses the device's, an ulp
 * or two apart).  It saves the separate RoPE launch of every decode token:
 * the workgroup whose key range holds pos rotates the token's key and uses it
 * directly, the others rotate only the query. */
int yhip_attn_decode_rope(float* att_out, const float* q, const float* k, const float* v, uint16_t* kcache,
                          uint16_t* vcache, uint32_t pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t kv_stride, uint32_t rope, uint32_t n_rot, float theta, const float* gate,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Ragged batch of independent sequences (one query token each).  No
 * reference counterpart beyond calling the decode once per engine; it is the
 * multi-sequence form of the same computation.
 *   kcaches/vcaches: device arrays [n_seq] of device pointers, each one
 *                    sequence's layer cache in the layout above;
 *   lens:            device [n_seq], keys per sequence (a sequence with 0
 *                    keys gets a zero output row);
 *   max_len, total_len: host values, the maximum and the sum of lens (they
 *                    size the split; max_len must bound every lens[i]);
 *   q/att_out rows:  q_stride / out_stride floats apart per sequence;
 *   gate:            NULL or rows gate_stride floats apart. */
int yhip_attn_decode_batch(float* att_out, uint32_t out_stride, const float* q,
                           uint32_t q_stride, const uint16_t* const* kcaches,
                           const uint16_t* const* vcaches, const uint32_t* lens,
                           uint32_t n_seq, uint32_t max_len, uint64_t total_len,
                           uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                           uint32_t kv_stride, const float* gate, uint32_t gate_stride,
                           void* workspace, size_t workspace_bytes, void* stream);

/* yhip_attn_decode_batch without a workspace: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that forbid hipMalloc): the split-K partials
 * go to a fixed scratch array of YHIP_DECODE_SCRATCH_BYTES that the library
 * holds on each GPU it runs on until the process ends, and the call itself
 * allocates nothing.  Arguments, checks and results are those of
 * yhip_attn_decode_batch; shapes whose partials exceed the scratch return
 * YHIP_ENOSPC (use yhip_attn_decode_batch with a workspace for them).  All
 * calls on one GPU share its scratch: calls that overlap on one GPU (two
 * streams, two host threads) race; serialise them.  The first call on each
 * device resolves the scratch's address there. */
#define YHIP_DECODE_SCRATCH_BYTES (16u << 20)
int yhip_attn_decode_batch_noalloc(float* att_out, uint32_t out_stride, const float* q, uint32_t q_stride,
                                   const uint16_t* const* kcaches, const uint16_t* const* vcaches,
                                   const uint32_t* lens, uint32_t n_seq, uint32_t max_len, uint64_t total_len,
                                   uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride,
                                   const float* gate, uint32_t gate_stride, void* stream);

/* Workspace bytes for the decode entry points (0 when the context is short
 * enough for one split).  It holds the per-split partial results and needs
 * no initialisation.  For n_seq = 1 the size serves yhip_attn_decode at
 * every pos < max_len (and the batch form with one sequence of at most
 * max_len keys), so one workspace sized for the engine's max_seq lasts a
 * whole generation.  For n_seq > 1 it is what a batch call with exactly
 * these n_seq, max_len and total_len needs (the split plan depends on all
 * three; a call checks its own need and returns YHIP_ENOSPC when the
 * workspace is short).  Calls that share a workspace must not run
 * concurrently (e.g. on two streams). */
size_t yhip_attn_decode_workspace(uint32_t n_seq, uint32_t max_len, uint64_t total_len,
                                  uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim);

/* ---- Prefill (causal GQA, MFMA) ------------------------------------------
 * Replaces cuda_k_attn_prefill (cuda_kernels.h:59-63); semantics of
 * engine.c:532-563 (and 935-960 with gate): B query tokens at positions
 * pos_start+b, b < B, each attending causally to keys 0..pos_start+b, all of
 * which must already be stored.  q rows are q_stride elements of q_dtype
 * apart (head h at h*head_dim), out rows out_stride elements of out_dtype;
 * dtypes YHIP_F32 / YHIP_F16 / YHIP_BF16.  gate: NULL or fp32 rows
 * gate_stride apart.  Computes QK^T and PV on f16 MFMA with fp32
 * accumulation and an fp32 online softmax.
 *
 * A launch with fewer (128-query block, head) items than CUs -- the
 * engine's prefill issues at most 64 tokens per call (engine.c:270-272,
 * 622-653) -- packs each kv head's query heads into full blocks and splits
 * the keys over workgroups so the GPU fills; the splits' partial results
 * need yhip_attn_prefill_workspace bytes of workspace (16-byte aligned, no
 * initialisation; 0 when the launch does not split).  With workspace NULL
 * such a launch runs unsplit (correct, slower for long prefixes). */
int yhip_attn_prefill(void* att_out, uint32_t out_dtype, uint32_t out_stride, const void* q,
                      uint32_t q_dtype, uint32_t q_stride, const uint16_t* kcache,
                      const uint16_t* vcache, uint32_t pos_start, uint32_t B, uint32_t n_heads,
                      uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride,
                      const float* gate, uint32_t gate_stride, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Workspace bytes that serve every yhip_attn_prefill call of B tokens with
 * pos_start + B <= max_end (an engine sizes one for its chunk size and
 * max_seq).  Calls sharing a workspace must not run concurrently. */
size_t yhip_attn_prefill_workspace(uint32_t B, uint32_t max_end, uint32_t n_heads, uint32_t n_kv_heads,
                                   uint32_t head_dim);

/* ---- RoPE + KV store (the step before attention) ---------------------------
 * rope: YHIP_ROPE_PAIRS = rope_inplace, (v[2j], v[2j+1]) (matvec.c:890-904,
 * llama); YHIP_ROPE_HALF = rope_inplace_qwen, (v[j], v[j+d/2]) (907-921,
 * qwen); YHIP_ROPE_MROPE = rope_inplace_mrope, (v[j], v[j+n_rot/2]) over the
 * first n_rot dims only (924-939, qwen35 with n_rot = 64); YHIP_ROPE_NONE
 * leaves q and k as they are.  freq = powf(theta, -2j/dn) (dn = head_dim, or
 * n_rot), angle = freq * pos, in float like the reference (the device
 * powf/cosf/sinf differ from the host library by an ulp or two). */
#define YHIP_ROPE_NONE 0u
#define YHIP_ROPE_PAIRS 1u
#define YHIP_ROPE_HALF 2u
#define YHIP_ROPE_MROPE 3u

/* Fused RoPE + KV store for B tokens at positions pos_start.. (engine.c:
 * 1054-1072; qwen35 910-934): q and k fp32 rows (post-projection, post
 * QK-norm) are rotated; q goes to q_out (YHIP_F32 / F16 / BF16, rows
 * q_out_stride apart; q_out may be q itself with F32 and the same stride;
 * q_out NULL skips q); k is stored into the head-major K cache and v (fp32
 * rows v_stride apart) into the V tiles, both with the reference f32->f16
 * rounding, as yhip_kv_store does.  Strides are in elements, so q, k, v may
 * be slices of one fused projection row; q, k, v (and an f32 q_out) must be
 * 8-byte aligned, an f16/bf16 q_out 4-byte aligned, every stride even.
 * One launch. */
int yhip_rope_kv_store(void* q_out, uint32_t q_out_dtype, uint32_t q_out_stride, const float* q, uint32_t q_stride,
                       const float* k, uint32_t k_stride, const float* v, uint32_t v_stride, uint16_t* kcache,
                       uint16_t* vcache, uint32_t pos_start, uint32_t B, uint32_t n_heads, uint32_t n_kv_heads,
                       uint32_t head_dim, uint32_t kv_stride, uint32_t rope, uint32_t n_rot, float theta,
                       void* stream);

/* ---- o_proj (the step after attention) -------------------------------------
 * x[b] += W_o . att[b] for B tokens: matmul(att_out, x2, SLOT_O) then the
 * residual add (engine.c:969-973; qwen35 after its gate, 958-973), with
 * matmul_f16 / matmul_f32 (matvec.c:98-122, dispatch 785-795); replaces the
 * reference CUDA backend's cublasGemmEx call for this product
 * (cuda_kernels.cu:104-112).  w: W_o [hidden][qdim] row-major, YHIP_F16 or
 * YHIP_F32 (the reference's matmul reads DT_BF16 slots as f16 bits,
 * matvec.c:793, so BF16 is refused; the quantised slot types stay on the
 * engine's CPU matmul).  att [B][qdim] is YHIP_F32 (the engine's att_out) or
 * YHIP_F16 (an attention output written as f16; needs f16 weights); x
 * [B][hidden] f32; rows att_stride / x_stride elements apart; x is updated
 * in place.  Up to 8 tokens: one pass over the weights, products and sums in
 * f32 (no workspace).  More: an f16 MFMA GEMM with f32 accumulation and the
 * residual add fused (f32 att, and f32 weights, enter as f16 hi + lo parts
 * whose products accumulate together: about 22 bits of each operand); the
 * parts take yhip_o_proj_workspace bytes (0 for f16 att).  qdim must be a
 * multiple of 8; w and att 16-byte aligned with att_stride a multiple of 8
 * elements; hidden * qdim below 2^30. */
size_t yhip_o_proj_workspace(uint32_t B, uint32_t hidden, uint32_t qdim, uint32_t w_dtype, uint32_t att_dtype);
int yhip_o_proj(float* x, uint32_t x_stride, const void* att, uint32_t att_dtype, uint32_t att_stride,
                const void* w, uint32_t w_dtype, uint32_t B, uint32_t hidden, uint32_t qdim, void* workspace,
                size_t workspace_bytes, void* stream);

/* ---- Gated DeltaNet (qwen35 linear attention) ------------------------------
 * State S: fp32 [n_v_heads][head_dim][head_dim], S[h][j][i] = column j of
 * v-head h (the reference's transposed storage, matvec.c:972-973); v-head h
 * reads k-head h % n_k_heads (matvec.c:983).  gate is the log-decay
 * (softplus(alpha+dt)*a, so g = exp(gate)) and beta the sigmoid, one per
 * v-head and token, as yhip_gdn_gates produces them.  When l2_eps > 0, q and
 * k are first L2-normalised per k-head with x / max(|x|, l2_eps)
 * (l2norm_inplace, matvec.c:942-949, as engine.c:826-827 calls it); with
 * l2_eps <= 0 they are used as given.  Arithmetic is fp32.  head_dim (d_k =
 * d_v) is 64 or 128; S, q, k, v must be 16-byte aligned.
 *
 * One token: replaces gdn_state_update (matvec.c:975-1004) plus the l2norm
 * before it.  q, k: [n_k_heads*head_dim]; v, out: [n_v_heads*head_dim];
 * gate, beta: [n_v_heads]. */
int yhip_gdn_step(float* S, float* out, const float* q, const float* k, const float* v, const float* gate,
                  const float* beta, uint32_t n_k_heads, uint32_t n_v_heads, uint32_t head_dim, float l2_eps,
                  void* stream);

/* T consecutive tokens (the per-token loop of the qwen35 batch forward,
 * engine.c:723-734, for the recurrence part): rows of q/k are qk_stride
 * floats apart, v rows v_stride, out rows out_stride (multiples of 4); gate
 * and beta are [T][n_v_heads].  The state after token T-1 goes to S_out:
 * NULL (or S) updates S in place; another buffer (16-byte aligned, not
 * overlapping S) receives it and S keeps the state before the call, so a
 * caller that alternates two buffers still holds the previous state when a
 * later step of its own fails.  out row t is the output of token t.
 *
 * With a workspace of yhip_gdn_chunk_workspace(T, n_v_heads, head_dim)
 * bytes (16-byte aligned, no initialisation) and T >= 64, the chunked form
 * runs: 64-token chunks are reduced in parallel to matrix products (MFMA)
 * and only the chunk-to-chunk state hand-over is sequential.  Out of place
 * (S_out another buffer) that sequential part runs on two workgroups per 16
 * state rows when they fit the GPU (faster; the same bits as in place).
 * With workspace NULL (or T < 64) the recurrence runs token by token. */
int yhip_gdn_chunk(float* S, float* S_out, float* out, uint32_t out_stride, const float* q, const float* k,
                   uint32_t qk_stride, const float* v, uint32_t v_stride, const float* gate, const float* beta,
                   uint32_t T, uint32_t n_k_heads, uint32_t n_v_heads, uint32_t head_dim, float l2_eps,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of the chunked form for T tokens (0 when T < 64). */
size_t yhip_gdn_chunk_workspace(uint32_t T, uint32_t n_v_heads, uint32_t head_dim);

/* One decode token of a Gated DeltaNet layer in one launch (engine.c:786-847
 * after the projections): the gates of alpha / beta_raw (788-793),
 * conv1d_update + silu of the projected row qkv (805-812, the conv bit for bit
 * the reference's), l2norm of q and k with l2_eps (826-827), the state update
 * (gdn_state_update, matvec.c:975-1004) and rmsnorm_gated of each v head with
 * z, norm_w and norm_eps (845-847) into y.  qkv is [2*n_k*head_dim +
 * n_v*head_dim] (q | k | v), z and y [n_v*head_dim], alpha, beta_raw,
 * dt_bias, ssm_a [n_v]; conv_w [conv_dim][kwidth] f32; norm_w [head_dim]
 * YHIP_F32 or YHIP_F16.  The delay line [kwidth][conv_dim] (row kwidth-1 the
 * newest input, as yhip_gdn_conv keeps it) is read from conv_in and written
 * to conv_out, which must not overlap it: swap the two every token.  S
 * (16-byte aligned) holds the state before the token; the state after it
 * goes to S_out as for yhip_gdn_chunk (NULL: in place).  head_dim 64 or
 * 128, n_v_heads >= n_k_heads, kwidth 1..8. */
int yhip_gdn_decode(float* S, float* S_out, const float* conv_in, float* conv_out, float* y, const float* qkv,
                    const float* z, const float* alpha, const float* beta_raw, const float* conv_w,
                    const float* dt_bias, const float* ssm_a, const void* norm_w, uint32_t norm_w_dtype,
                    uint32_t n_k_heads, uint32_t n_v_heads, uint32_t head_dim, uint32_t kwidth, float l2_eps,
                    float norm_eps, void* stream);

/* The GDN gates of T tokens (engine.c:788-793), in place like the engine:
 * beta[t][h] <- 1/(1+exp(-beta[t][h])), gate[t][h] <- log1p(exp(alpha[t][h]
 * + dt_bias[h])) * ssm_a[h]. */
int yhip_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt_bias, const float* ssm_a,
                   uint32_t T, uint32_t n_v_heads, void* stream);

/* The causal conv1d + silu ahead of the recurrence for T tokens in order:
 * conv1d_update (matvec.c:956-968) then silu (engine.c:809-812) per token.
 * conv_state: the delay line, fp32 [kwidth][dim] (row kwidth-1 newest, the
 * engine's e->ssm_conv slot, engine.c:802) before the call; the line after
 * it goes to conv_state_out (NULL or conv_state: in place; else a buffer not
 * overlapping conv_state, which then keeps the line before the call); conv_w: fp32
 * [dim][kwidth] (the gguf layout the reference reads, w[ch*kwidth + i]).
 * x: T rows of dim channels x_stride floats apart (the qkv projection
 * rows); out: T rows out_stride apart, not overlapping x (a token's
 * window reads the kwidth-1 inputs before it).  silu = 0 stores the
 * conv values themselves (bit for bit the reference's; with silu the
 * device expf adds its own rounding).  kwidth 1..8. */
int yhip_gdn_conv(float* out, uint32_t out_stride, const float* x, uint32_t x_stride, float* conv_state,
                  float* conv_state_out, const float* conv_w, uint32_t T, uint32_t dim, uint32_t kwidth, int silu,
                  void* stream);

/* Gated RMSNorm after the recurrence (rmsnorm_gated, matvec.c:1007-1021,
 * applied per v-head at engine.c:845-847): for token t and head h,
 * y = x * w * (1/sqrtf(mean(x^2) + eps)) * (z / (1 + expf(-z))) over the
 * head's head_dim values.  x, z, y: T rows of n_heads*head_dim with their
 * own strides (y may alias x); w: [head_dim] fp32 (w_dtype YHIP_F32) or f16
 * bits (YHIP_F16).  head_dim a multiple of 64, at most 256. */
int yhip_gdn_gated_norm(float* y, uint32_t y_stride, const float* x, uint32_t x_stride, const float* z,
                        uint32_t z_stride, const void* w, uint32_t w_dtype, uint32_t T, uint32_t n_heads,
                        uint32_t head_dim, float eps, void* stream);

/* ---- Synthetic inputs (host) ----------------------------------------------
 * Seeded generator shared by the tests and the benchmark so that the CPU
 * oracle and the GPU see identical bits: splitmix64 as the reference's yrng
 * (platform.c:405-417), uniforms u = ((r>>40)+0.5)*2^-24, Box-Muller in
 * double, value = (float)(sigma*z).  Draw i of a stream uses generator state
 * seed + (i+1)*0x9e3779b97f4a7c15, so chunks can be generated independently. */
void yhip_synth_normal(uint64_t seed, uint64_t first, float sigma, float* out, uint64_t n);
/* Round in place to f16-representable values with the reference rounding
 * (platform.c:340-379), or to bf16 with round-to-nearest-even. */
void yhip_synth_round_f16(float* x, uint64_t n);
void yhip_synth_round_bf16(float* x, uint64_t n);
/* Host conversions used to prepare inputs: reference f32->f16 rounding,
 * exact f16->f32, f32->bf16 RNE bits. */
void yhip_host_f32_to_f16(const float* src, uint16_t* dst, uint64_t n);
void yhip_host_f16_to_f32(const uint16_t* src, float* dst, uint64_t n);
void yhip_host_f32_to_bf16(const float* src, uint16_t* dst, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* YLLM_HIP_H */
