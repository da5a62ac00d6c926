/* ggml-helix-hip.h -- HELIX interception point for GGML_OP_SSM_SCAN in ggml's
 * HIP backend (ggml-cuda built for ROCm).
 *
 * Counterpart of the reference's integration/ggml/ggml-helix.h:1-24 (the
 * ggml-metal hook). One call site, behind an #ifdef at the top of the HIP
 * backend's SSM_SCAN op; every entry point returns false for anything HELIX
 * does not serve, having enqueued nothing, and the caller then runs its own
 * kernel unchanged.
 *
 * Runtime switches (same names and meaning as the reference bridge):
 *   GGML_HELIX_DISABLE=1     never intercept
 *   GGML_HELIX_MPP=1         allow the bf16 path (default: fp32, which meets
 *                            ggml's own op tolerance)
 *   GGML_HELIX_MIN_TOKENS=n  decline sequences shorter than n (default 64)
 */
#ifndef GGML_HELIX_HIP_H
#define GGML_HELIX_HIP_H

#include <stdbool.h>
#include <stddef.h>

#include "helix/helix.h"

#ifdef __cplusplus
extern "C" {
#endif

struct ggml_tensor;

/* True when HELIX will serve SSM_SCAN `op` on HIP device `device`;
 * *scratch_bytes is then the device scratch the encode needs (0 when none).
 * Lets the caller take the scratch from its own pool (ggml_cuda_pool). */
bool ggml_hip_ssm_scan_helix_plan(int device, const struct ggml_tensor * op, size_t * scratch_bytes);

/* Enqueues SSM_SCAN `op` on `stream` (a hipStream_t) of device `device`.
 * `scratch` is device memory of at least the planned size, or NULL to use a
 * per-thread, per-device buffer the bridge grows on demand (hipMalloc: not
 * for use under stream capture). Returns false, with nothing enqueued, when
 * HELIX does not serve the op. */
bool ggml_hip_op_ssm_scan_helix(void * stream, int device, const struct ggml_tensor * op, void * scratch,
                                size_t scratch_bytes);

/* The descriptor the bridge builds for `op`, without a device: false when the
 * bridge's own gates decline it (K != 1, a non-f32 operand, fewer than
 * GGML_HELIX_MIN_TOKENS tokens, an A shape that is neither {1, H} nor
 * {d_state, H}, a state that is not dense, strides that are not whole
 * elements). helix_scan_supported() still applies on top. */
bool helix_ggml_build_desc(const struct ggml_tensor * op, helix_scan_desc * d);

#ifdef __cplusplus
}
#endif

#endif /* GGML_HELIX_HIP_H */
