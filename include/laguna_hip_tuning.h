/*
 * laguna_hip_tuning.h -- launch-shape hooks and ceiling kernels of
 * liblaguna_hip.so, for sweeps and measurement.
 *
 * Not part of the drop-in boundary (laguna_hip.h), and without counterparts in the
 * reference, whose Vulkan shaders have fixed workgroup counts.
 */
#ifndef LAGUNA_HIP_TUNING_H
#define LAGUNA_HIP_TUNING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- launch-shape hooks.  Each sets a process-wide value (an atomic, read at
 * every launch); 0 restores the automatic choice.  Every setting meets the same
 * parity bound, and results are repeatable for a fixed setting. */

/* Upper bound on workgroups of the M = 1 quantized projections. */
int lg_set_m1_grid_cap(uint32_t cap);
/* Number of k slices of the Q4_K M = 1 matrix-core kernel (the fused SiLU down
 * projection). */
int lg_set_m1_split(uint32_t slices);
/* Kernel family of the Q4_K M = 1 projections: 1 = vector ALU / integer dot
 * products, 2 = int8 matrix cores (k <= 16384; other k keep family 1).  Any other
 * value is LG_EINVAL. */
int lg_set_m1_kernel(uint32_t kind);
/* Small-M products (lg_dispatch_proj_quant_batch, the draft forward): ch chunks of
 * 256 elements per k slice (1, 2; 4 for Q4_K with m <= 16) and rt 16-row tiles per
 * wavefront (1, 2, 4; clamped to the kernel's register budget).  A captured
 * draft-forward graph keeps the workspace it was sized with: set this before
 * lg_dflash_graph_create. */
int lg_set_batch_shape(uint32_t ch, uint32_t rt);
/* The forwards' RMSNorms: 1 (the default) folds them into the projections around
 * them wherever the model allows it, 0 runs each as its own launch.  The draft
 * forward folds its attention and FFN norms when every projection is on the
 * matrix-core path (n_embd a multiple of 4 up to 8192, 16-byte aligned norm weights
 * and tokens); the target forward folds each layer's residual adds and norms into
 * its Q4_K input projections when they are on the M = 1 integer-dot path (n_embd a
 * multiple of 256 up to 4096, 16-byte aligned operands).  Unlike the hooks above, 0
 * is not the automatic choice.  Set it before lg_dflash_graph_create: a captured
 * graph keeps the launches it recorded. */
int lg_set_fold_norms(uint32_t folded);

/* ---- ceiling kernels: what one launch, and one read of a buffer, cost. */

/* An empty kernel of `workgroups` x 256 threads on `stream`. */
int lg_bench_empty(uint32_t workgroups, void *stream);
/* Reads `bytes` (a positive multiple of 16) of device memory at `buf` (16-byte
 * aligned) once: each workgroup streams a contiguous 32 KiB run, every load issued
 * up front. */
int lg_bench_read(const void *buf, uint64_t bytes, void *stream);
/* The same read in other shapes, for finding the fastest read of a byte count:
 * `threads` per workgroup (256, 512, 1024), `loads` 16-byte loads per thread issued
 * at once per chunk (2, 4, 8, 16), a one-shot grid of one chunk per workgroup
 * (per_cu = 0) or a persistent grid of per_cu (1..8) workgroups per compute unit
 * looping over the chunks, and plain or nontemporal loads.  lg_bench_read is
 * (256, 8, 0, 0). */
int lg_bench_read_shape(const void *buf, uint64_t bytes, uint32_t threads, uint32_t loads, uint32_t per_cu,
                        uint32_t nontemporal, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LAGUNA_HIP_TUNING_H */
