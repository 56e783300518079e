/* yllm_device_hip.h -- yllm device backend for MI355X (gfx950).
 *
 * The engine-side half of the boundary: a Device (inference/include/device.h:
 * 37-50) whose load_weights installs per-layer forward functions that run the
 * attention of each block (KV store, decode, causal prefill; for qwen35 also
 * the Gated-DeltaNet recurrence and the gated attention) on the GPU through
 * libyllm_hip.so and keep the rest of the block on the engine's own CPU
 * operators.  Built inside the reference tree (device_hip.c includes
 * yllm.h / device.h / llf.h / matvec.h) and linked with libyllm_hip.so and
 * libamdhip64.
 *
 * Engine and Device are the reference's types; they are only forward
 * declared here so this header does not depend on the reference headers.
 */
#ifndef YLLM_DEVICE_HIP_H
#define YLLM_DEVICE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct Engine;
struct Device;

/* Factory, the HIP counterpart of device_create_cuda (forward-declared at
 * inference/device/device_cpu.c:89, called by device_create at 82-110).
 * Returns a calloc'ed Device (freed by device_destroy after free_dev,
 * engine.c:360-364) or NULL with a message in err when no usable gfx950
 * device `device_id` exists.  load_weights (bound by engine_bind_device,
 * engine.c:354-384) allocates the HBM KV cache for the engine's layer range
 * (attention layers) and the HBM recurrent state (qwen35 GDN layers) and
 * installs fwd_block / fwd_block_batch (yllm.h:115-116); it fails with -1 and
 * a message for shapes the kernels do not take (head_dim not 64, 128 or 256;
 * more than 16 query heads per kv head; GDN head dim not 64 or 128, conv
 * width above 8), so the caller can rebind the CPU device.  The GDN state
 * and conv delay line stay in HBM between calls: e->ssm_state / ssm_conv
 * are brought up to date when the host needs them -- before a GDN block
 * runs on the CPU (fallback), in device_hip_kv_to_host and in free_dev --
 * not after every update (1 MiB per layer and token for 16 heads of 128).
 * A GDN block reads one of two HBM copies and writes the other, so a block
 * that fails leaves the state from before it for the CPU fallback.  When
 * the device cannot give that state back either, the block returns -2,
 * writes NaN to its output rows (every later logit is NaN) and says so on
 * stderr, instead of continuing on a stale host state. */
struct Device* device_create_hip(int device_id, char* err, size_t errlen);

/* KV-cache interface (device.h:58-63 cuda_after_prefill; cache.c:174-247).
 * The backend writes every KV row to the engine's host array e->kv as well,
 * so host KV is always current after a forward; these two move rows
 * 0..n_pos-1 of every layer of the engine's range between e->kv (engine
 * layout) and the head-major HBM cache.  Call device_hip_kv_from_host after
 * KV was written on the host (sess_kv_load); it also marks every HBM GDN
 * state stale, so each is re-sent from e->ssm_state by its layer's next
 * call.  device_hip_kv_to_host rebuilds a host KV copy from HBM and brings
 * e->ssm_state up to date (call it before reading the host state, e.g. for
 * a session save).  Return 0 or -1. */
int device_hip_kv_from_host(struct Engine* e, uint32_t n_pos);
int device_hip_kv_to_host(struct Engine* e, uint32_t n_pos);

/* Test hooks for the fallback path.  device_hip_fail_after: after `n_calls`
 * more GPU block forwards the backend behaves as if the GPU had failed.  A
 * failed block returns -1 after computing the block with the engine's CPU
 * forward from the host KV (and, for a GDN layer, the state copied back from
 * HBM), and every later block stays on the CPU.  n_calls < 0 disables the
 * hook.  device_hip_fail_mode sets where the failure strikes: 0 (the
 * default) before the block issues any GPU work; 1 after its kernels ran and
 * its output came back (as a failed result copy: the HBM state has moved on
 * in the buffer the block wrote); 2 as 1 with every later device copy
 * failing too (a device that is gone: a GDN state held only in HBM is then
 * lost and reported, see device_create_hip). */
void device_hip_fail_after(struct Engine* e, int n_calls);
void device_hip_fail_mode(struct Engine* e, int mode);

#ifdef __cplusplus
}
#endif

#endif /* YLLM_DEVICE_HIP_H */
