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
 * more than 16 query heads per kv head; GDN head dim not 64 or 128), so the
 * caller can rebind the CPU device.  The GDN state stays in HBM between
 * calls: e->ssm_state is brought up to date when the host needs it -- before
 * a GDN block runs on the CPU (fallback), in device_hip_kv_to_host and in
 * free_dev -- not after every update (1 MiB per layer and token at the
 * fifth configuration's shape).  After a GPU failure, a layer updated on the
 * GPU since its last copy keeps its last host state when that copy fails. */
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

/* Test hook for the fallback path: after `n_calls` more GPU block forwards
 * the backend behaves as if the GPU had failed (no GPU work is issued for
 * that call).  A failed block returns -1 after computing the block with the
 * engine's CPU forward from the host KV, and every later block stays on
 * the CPU.  n_calls < 0 disables the hook. */
void device_hip_fail_after(struct Engine* e, int n_calls);

#ifdef __cplusplus
}
#endif

#endif /* YLLM_DEVICE_HIP_H */
