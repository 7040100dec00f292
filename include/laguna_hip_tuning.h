/*
 * laguna_hip_tuning.h -- launch-shape hooks of liblaguna_hip.so for sweeps.
 *
 * Not part of the drop-in boundary (laguna_hip.h): the reference's Vulkan shaders
 * have fixed workgroup counts, and these hooks have no counterpart there.  Each
 * sets a process-wide value (an atomic, read at every launch); 0 restores the
 * automatic choice.  Every setting meets the same parity bound, and results are
 * repeatable for a fixed setting.
 */
#ifndef LAGUNA_HIP_TUNING_H
#define LAGUNA_HIP_TUNING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Upper bound on workgroups of the M = 1 quantized projections. */
int lg_set_m1_grid_cap(uint32_t cap);
/* Number of k slices of the Q4_K M = 1 matrix-core kernel (the fused SiLU down
 * projection). */
int lg_set_m1_split(uint32_t slices);
/* Small-M products (lg_dispatch_proj_quant_batch, the draft forward): ch chunks of
 * 256 elements per k slice (1, 2; 4 for Q4_K with m <= 16) and rt 16-row tiles per
 * wavefront (1, 2, 4; clamped to the kernel's register budget).  A captured
 * draft-forward graph keeps the workspace it was sized with: set this before
 * lg_dflash_graph_create. */
int lg_set_batch_shape(uint32_t ch, uint32_t rt);

#ifdef __cplusplus
}
#endif
#endif /* LAGUNA_HIP_TUNING_H */
