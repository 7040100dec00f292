/*
 * laguna_hip.h -- C ABI of the MI355X (gfx950) quantized-projection library.
 *
 * This is the drop-in boundary for laguna-raw's projection path.  It replaces
 * the reference's Vulkan runtime (src/vulkan.rs) and the projection shaders
 * (kernels/proj_q4k.comp, proj_q8_0.comp, proj.comp, activation.comp,
 * dequant_q4k.comp, matmul.comp) with HIP kernels for gfx950, behind entry
 * points whose names and argument order follow the reference's dispatch_*
 * functions minus the shader handles.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Device pointers come from lg_buf_alloc
 *     (or any other hipMalloc'd memory); `stream` is a hipStream_t passed as
 *     void* (NULL = the null stream).
 *   - Weight tensors follow GGUF: a [k, n] tensor has ne0 = k contiguous, so
 *     output row i is linear elements i*k .. i*k+k-1 (kernels/proj_q4k.comp:67,
 *     kernels/proj.comp:29).  Quantized tensors are the raw GGUF blocks, uploaded
 *     byte for byte (src/model.rs:174-184).
 *   - Every call returns an lg_status.  Nothing aborts or throws across the
 *     ABI; the text of the last failure on the calling thread is returned by
 *     lg_last_error().  Launches are asynchronous on `stream`; lg_sync()
 *     waits.  The reference blocks after every dispatch
 *     (src/vulkan.rs:326-334); lg_set_blocking(1) restores that behaviour.
 *   - When a pointer was returned by lg_buf_alloc, the library checks that the
 *     extent the call reads or writes lies inside that allocation and returns
 *     LG_EINVAL otherwise (the reference binds whole buffers and never checks).
 *   - A library instance is not thread-safe per device; callers serialise.
 */
#ifndef LAGUNA_HIP_H
#define LAGUNA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids, as TensorType::from_u32 (src/gguf.rs:46-84) and
 * WeightType (src/target.rs:7-22) use them. */
typedef enum {
    LG_F32 = 0,
    LG_F16 = 1,
    LG_Q8_0 = 8,
    LG_Q4_K = 12,
    LG_BF16 = 30
} lg_dtype;

typedef enum {
    LG_OK = 0,
    LG_EINVAL = 1,      /* bad argument: null pointer, size, dtype, extent */
    LG_EHIP = 2,        /* a HIP runtime call failed (text in lg_last_error) */
    LG_ENOMEM = 3,      /* device allocation failed */
    LG_EUNSUPPORTED = 4,/* valid request this build does not implement */
    LG_EIO = 5,         /* file I/O or format error (GGUF) */
    LG_ENODEV = 6       /* no HIP device */
} lg_status;

/* ---- runtime (replaces VulkanContext / GpuBuffer, src/vulkan.rs:16-452) ---- */

/* Thread-local text of the last failure ("" if none). */
const char *lg_last_error(void);
/* Library version string. */
const char *lg_version(void);
/* Number of HIP devices (0 on a host without a GPU; never an error). */
int lg_device_count(int *count);
/* Select the device for this thread and create its per-device state
 * (VulkanContext::init, src/vulkan.rs:16-100, which takes pdevices[0]). */
int lg_init(int device);
/* 1 = every launch is followed by a stream synchronise (the reference's
 * fence wait, src/vulkan.rs:326-334); 0 = asynchronous (default). */
int lg_set_blocking(int blocking);

/* Device buffers (GpuBuffer::new / upload / read_f32, src/vulkan.rs:350-452).
 * HBM via hipMalloc; the caller owns and frees them. */
int lg_buf_alloc(void **dptr, uint64_t bytes);
int lg_buf_free(void *dptr);
int lg_buf_upload(void *dst, const void *src, uint64_t bytes, void *stream);
int lg_buf_download(void *dst, const void *src, uint64_t bytes, void *stream);
int lg_buf_memset(void *dst, int value, uint64_t bytes, void *stream);
/* Device-to-device copy (no counterpart in the reference, whose buffers are
 * host-visible and copied through the host); asynchronous on `stream`. */
int lg_buf_copy(void *dst, const void *src, uint64_t bytes, void *stream);
int lg_stream_create(void **stream);
int lg_stream_destroy(void *stream);
int lg_sync(void *stream);

/* ---- dequantization ---- */

/* dequant_to_f32 (src/dflash.rs:331-465) on the device: `n_elements` values
 * from the raw tensor bytes `data` (`data_len` bytes) into `out`.
 *   LG_Q8_0   value = float(int8 q) * d (src/dflash.rs:379-397), bit-exact.
 *   LG_Q4_K   ggml Q4_K, value = (d*sc)*q - dmin*m, the decode every
 *             quantized projection applies (kernels/proj_q4k.comp:28-87);
 *             the reference's Rust Q4_K branch (src/dflash.rs:398-436) is a
 *             different, non-ggml format and is not reproduced.
 *   LG_F32, LG_F16, LG_BF16  as the reference's branches (:333-378, :437-462;
 *             its "BF16" branch decodes IEEE f16 and is reproduced as such).
 *   other     zeros, as the reference's fallback arm (:463).
 * A block that would run past data_len ends decoding; the remaining outputs
 * are 0, as the reference's `break` (:385, :403).
 * Replaces kernels/dequant_q4k.comp, which is never dispatched. */
int lg_dequant_to_f32(const void *data, uint64_t data_len, int dtype, uint64_t n_elements,
                      float *out, void *stream);

/* ---- projections (M = 1) ---- */

/* dispatch_proj_quant (src/target.rs:1086-1099): c[i] = sum_j x[j] * W[i,j]
 * for i < n, j < k; W is raw Q8_0 / Q4_K blocks, or f32 (then proj.comp
 * semantics, row_major = 0).  x: f32[k], c: f32[n]. */
int lg_dispatch_proj_quant(const float *x, const void *w, float *c, uint32_t k, uint32_t n,
                           int dtype, void *stream);

/* dispatch_proj_quant_expert (src/target.rs:1101-1162): as above with W[i,j]
 * taken at linear element expert_offset + i*k + j (kernels/proj_q4k.comp:67).
 * As in the reference, expert_offset applies to Q4_K only: the Q8_0 and F32
 * arms ignore it (src/target.rs:1115-1138). */
int lg_dispatch_proj_quant_expert(const float *x, const void *w, float *c, uint32_t k,
                                  uint32_t n, int dtype, uint32_t expert_offset,
                                  void *stream);

/* dispatch_proj / dispatch_proj_row (src/dflash.rs:1009-1051), f32 weights,
 * kernels/proj.comp:23-33: c[i] = sum_j x[j] * w[row_major ? j*n+i : i*k+j]. */
int lg_dispatch_proj(const float *x, const float *w, float *c, uint32_t k, uint32_t n,
                     void *stream);
int lg_dispatch_proj_row(const float *x, const float *w, float *c, uint32_t k, uint32_t n,
                         uint32_t row_major, void *stream);

/* dispatch_proj_read (src/dflash.rs:1054-1090): f32 projection whose result
 * is copied to host memory `out` (n floats); synchronous. */
int lg_dispatch_proj_read(const float *x, const float *w, uint32_t k, uint32_t n, float *out,
                          void *stream);

/* dispatch_activation (src/dflash.rs:1305-1327), kernels/activation.comp:
 * h[i] = silu(gate[i]) * up[i], silu(x) = x * (1/(1+exp(-x))). */
int lg_dispatch_activation(const float *gate, const float *up, float *h, uint32_t n,
                           void *stream);

/* Fused dispatch_activation + dispatch_proj_quant for the FFN down
 * projection (src/dflash.rs:967-968): c = W * (silu(gate) * up), with
 * gate, up: f32[k].  The activation is computed inside the projection kernel
 * and never written to memory. */
int lg_dispatch_silu_mul_proj_quant(const float *gate, const float *up, const void *w,
                                    float *c, uint32_t k, uint32_t n, int dtype,
                                    void *stream);

/* ---- small-M products (replaces kernels/matmul.comp) ---- */

/* Block-verify product: c[r][i] = sum_j x[r][j] * W[i,j] for r < m, i < n.
 * x is row-major [m][k] of x_dtype LG_F32 or LG_BF16 (raw bf16 bits); c is
 * f32 [m][n]; W is Q4_K or Q8_0 raw blocks or f32.  1 <= m <= 64; m = 1 is the
 * same product as lg_dispatch_proj_quant. */
int lg_dispatch_proj_quant_batch(const void *x, int x_dtype, const void *w, float *c,
                                 uint32_t k, uint32_t n, uint32_t m, int w_dtype,
                                 void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LAGUNA_HIP_H */
