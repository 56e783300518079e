// internal.hpp -- launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace yhip {

// ---- kv_store.hip ----
hipError_t launch_kv_store(uint16_t* kc, uint16_t* vc, const void* k, const void* v, uint32_t dt,
                           uint32_t pos_start, uint32_t B, uint32_t n_kv, uint32_t D,
                           uint32_t kv_stride, hipStream_t st);
hipError_t launch_kv_from_engine(uint16_t* kc, uint16_t* vc, const uint16_t* ek, const uint16_t* ev,
                                 uint32_t rows, uint32_t n_kv, uint32_t D, uint32_t kv_stride,
                                 hipStream_t st);
hipError_t launch_kv_to_engine(uint16_t* ek, uint16_t* ev, const uint16_t* kc, const uint16_t* vc,
                               uint32_t rows, uint32_t n_kv, uint32_t D, uint32_t kv_stride,
                               hipStream_t st);

// ---- attn_decode.hip ----
struct DecodeArgs {
    const float* q;                 // rows q_stride apart per sequence
    const uint16_t* const* kptrs;   // per-sequence K bases (device array) or null
    const uint16_t* const* vptrs;
    const uint16_t* k0;             // single-sequence K/V when kptrs is null
    const uint16_t* v0;
    const uint32_t* lens;           // per-sequence key counts (device) or null
    uint32_t len0;                  // key count when lens is null
    float* out;
    const float* gate;
    float* part_ml;                 // [n_seq][n_kv][n_splits][gmax][2]
    float* part_o;                  // [n_seq][n_kv][n_splits][gmax][D]
    uint32_t n_seq, n_heads, n_kv, D, kv_stride;
    uint32_t q_stride, out_stride, gate_stride;
    uint32_t split_keys, n_splits, gmax;
    float c;                        // log2(e)/sqrt(D)
};
constexpr uint32_t kMaxSplits = 256;
// Split plan for the shapes; returns the workspace bytes (0 without splits).
size_t decode_plan(uint32_t n_seq, uint32_t max_len, uint64_t total_len, uint32_t n_heads,
                   uint32_t n_kv, uint32_t D, uint32_t* split_keys, uint32_t* n_splits);
// Workspace bytes that serve the shapes: for one sequence, every call with
// len <= max_len (the split count is not monotone in len); for a batch, the
// call's own plan.
size_t decode_workspace_bound(uint32_t n_seq, uint32_t max_len, uint64_t total_len, uint32_t n_heads,
                              uint32_t n_kv, uint32_t D);
// carve the workspace into part_ml / part_o for a plan
void decode_bind_workspace(DecodeArgs& a, void* workspace);
hipError_t launch_decode(const DecodeArgs& a, hipStream_t st);
// RoPE and the KV store of the token at position len0 - 1 fused into a
// single-sequence decode: q is the raw (unrotated) query row; k, v the raw
// key and value rows of the token (fp32, n_kv * D each)
struct DecodeRope {
    const float* k;
    const float* v;
    uint16_t* kc;        // the K cache and V tiles the token is stored into
    uint16_t* vc;
    uint32_t kind, n_rot;
    float cs[2][128];    // cos, sin of pair j's angle at the token's position, host cosf / sinf
};
hipError_t launch_decode_rope(const DecodeArgs& a, const DecodeRope& r, hipStream_t st);

// ---- api.hip ----
// The checks, plan and launches of yhip_attn_decode_batch with the partials
// in `workspace` of workspace_bytes (ws_name names it in the error message).
int decode_batch_common(const char* fn, float* att_out, uint32_t out_stride, const float* q, uint32_t q_stride,
                        const uint16_t* const* kcaches, const uint16_t* const* vcaches, const uint32_t* lens,
                        uint32_t n_seq, uint32_t max_len, uint64_t total_len, uint32_t n_heads,
                        uint32_t n_kv_heads, uint32_t head_dim, uint32_t kv_stride, const float* gate,
                        uint32_t gate_stride, void* workspace, size_t workspace_bytes, const char* ws_name,
                        void* stream);
// sets the per-thread message of yhip_last_error and returns code
int api_fail(int code, const char* msg);

// ---- attn_prefill.hip ----
struct PrefillArgs {
    const void* q;
    uint32_t q_dtype, q_stride;
    const uint16_t* kc;
    const uint16_t* vc;
    uint32_t kv_stride;
    void* out;
    uint32_t out_dtype, out_stride;
    const float* gate;
    uint32_t gate_stride;
    uint32_t pos_start, B, n_heads, n_kv, D;
    float c;
    // set by the launcher: the (query block, head) items are grouped by kv
    // head per XCD (xcd_map) and dealt to gridDim.x resident workgroups in
    // snake order, heaviest first
    uint32_t xcd_map;
    // Split mode (set by prefill_plan for launches with fewer work items
    // than CUs, e.g. the engine's 64-token chunks over a long prefix): an
    // item is (row block, kv head, key split).  With pack, the rows of a kv
    // head are its query heads' B queries each (head-major, G*B rows), so
    // 128 rows fill a workgroup even when B < 128; otherwise rows are the B
    // queries of one head.  Split s covers key tiles [s*split_tiles,
    // (s+1)*split_tiles); with n_split > 1 the workgroups write (max, sum,
    // unnormalised O) partials and a merge kernel forms the output.
    uint32_t split_mode, pack, n_split, split_tiles, n_rb, gmax;
    float* part_ml;  // [n_split][n_heads][B][2]
    float* part_o;   // [n_split][n_heads][B][D]
};
// Work plan of a prefill launch: fills the split-mode fields of a and
// returns the workspace bytes it needs (0 without partials).
size_t prefill_plan(PrefillArgs& a);
// Workspace bytes that serve every launch of B query tokens with pos_start +
// B <= max_end (the split count does not grow with pos_start beyond a bound).
size_t prefill_workspace_bound(uint32_t B, uint32_t max_end, uint32_t n_heads, uint32_t n_kv, uint32_t D);
void prefill_bind_workspace(PrefillArgs& a, void* workspace);
// keys per tile of the prefill kernels at head_dim D (the unit of split_tiles)
uint32_t prefill_tile_keys(uint32_t D);
hipError_t launch_prefill(const PrefillArgs& a, hipStream_t st);

// ---- rope.hip ----
struct RopeArgs {
    void* q_out;            // rows q_out_stride apart, dtype q_out_dtype (null: no q)
    const float* q;         // rows q_stride apart
    const float* k;         // rows k_stride apart
    const float* v;         // rows v_stride apart
    uint16_t* kc;           // head-major K cache
    uint16_t* vc;           // V tiles
    uint32_t q_out_dtype, q_out_stride, q_stride, k_stride, v_stride;
    uint32_t pos_start, B, n_heads, n_kv, D, kv_stride, kind, n_rot;
    // set by the launcher: waves per token, heads per wave, workgroups of each role
    uint32_t groups, heads_per_wave, rope_blocks, v_blocks;
    // freq[j] = powf(theta, -2j/span) for the rotated pairs j < span/2,
    // computed on the host with the C library's powf, as the reference does
    float freq[128];
};
hipError_t launch_rope_kv(RopeArgs a, hipStream_t st);

// ---- o_proj.hip ----
struct OProjArgs {
    float* x;               // [B] rows x_stride apart, residual in / out
    const void* att;        // [B] rows att_stride apart, f16 when att_f16 else f32
    const void* w;          // [hidden][qdim], f16 when w_f16 else f32
    uint32_t x_stride, att_stride, B, hidden, qdim, w_f16, att_f16;
};
constexpr uint32_t kGemvRows = 8;  // up to this many tokens: one pass over the weights
size_t oproj_workspace(uint32_t B, uint32_t qdim, uint32_t w_f16, uint32_t att_f16, uint32_t hidden);
// null on success, else a message
const char* launch_oproj(const OProjArgs& a, void* ws, size_t ws_bytes, hipStream_t st);

// ---- gdn_conv.hip ----
struct GdnConvArgs {
    float* out;             // [T] rows out_stride apart (not overlapping x)
    const float* x;         // [T] rows x_stride apart
    float* state;           // delay line [kwidth][dim] before the call
    float* state_out;       // after the call: state itself (in place) or a buffer not overlapping it
    const float* w;         // [dim][kwidth]
    uint32_t out_stride, x_stride, T, dim, kwidth;
    int silu;
};
hipError_t launch_gdn_conv(const GdnConvArgs& a, hipStream_t st);
struct GdnNormArgs {
    float* y;               // may alias x
    const float* x;
    const float* z;
    const void* w;          // [head_dim] f32, or f16 when w_f16
    uint32_t y_stride, x_stride, z_stride, T, n_heads, head_dim, w_f16;
    float eps;
};
hipError_t launch_gdn_gated_norm(const GdnNormArgs& a, hipStream_t st);

// ---- gdn_decode.hip ----
struct GdnDecodeArgs {
    const float* S;         // [n_v][D][D] state before the token
    float* S_out;           // the state after it (S itself, or a buffer not overlapping it)
    const float* conv_in;   // delay line [kwidth][conv_dim] before the token
    float* conv_out;        // delay line after the token (not overlapping conv_in)
    const float* qkv;       // [conv_dim] projected row: q | k | v
    const float* z;         // [n_v * D]
    const float* alpha;     // [n_v]
    const float* beta_raw;  // [n_v]
    const float* conv_w;    // [conv_dim][kwidth]
    const float* dt_bias;   // [n_v]
    const float* ssm_a;     // [n_v]
    const void* norm_w;     // [D] f32, or f16 when norm_w_f16
    float* y;               // [n_v * D]
    uint32_t n_k, n_v, D, kwidth, conv_dim, norm_w_f16;
    float l2_eps, norm_eps;
    float l2_inv_eps;  // 1 / l2_eps, set by launch_gdn_decode
};
hipError_t launch_gdn_decode(const GdnDecodeArgs& a, hipStream_t st);

// ---- gdn.hip ----
struct GdnArgs {
    const float* S;                  // [n_v][D][D] state before the call, S[h][j][i]
    float* S_out;                    // the state after the call (S itself, or a buffer not overlapping it)
    float* out;                      // [T][out_stride], head h at h*D
    const float* q;                  // [T][qk_stride], k-head at kh*D
    const float* k;
    const float* v;                  // [T][v_stride], v-head h at h*D
    const float* gate;               // [T][n_v] log-decay
    const float* beta;               // [T][n_v]
    uint32_t T, n_k, n_v, D;
    uint32_t qk_stride, v_stride, out_stride;
    float eps;                       // <= 0: q, k are already normalised
    float* ws;                       // chunked form: per (v-head, chunk) intermediates, or null
    uint32_t n_chunks;
};
hipError_t launch_gdn(const GdnArgs& a, hipStream_t st);
// compute units of the current device (queried once; 256 if the query fails)
int n_cus();
// bytes of the chunked form's workspace, and its chunk length in tokens
size_t gdn_chunk_workspace(uint32_t T, uint32_t n_v, uint32_t D);
uint32_t gdn_chunk_tokens();
hipError_t launch_gdn_gates(float* beta, float* gate, const float* alpha, const float* dt, const float* ssm_a,
                            uint32_t T, uint32_t n_v, hipStream_t st);

}  // namespace yhip
