/*
 * CPU oracle for the GGUF Q4_K / Q8_0 quantized-projection path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * the smoke test and the benchmark's CPU-baseline leg compare against.  No
 * product code links, loads or calls it; the product path is the HIP library
 * and fails loudly when that library is missing.
 *
 * Every function restates reference code line by line, in the same f32
 * operation order (built with -ffp-contract=off, no fast-math), and cites
 * the reference file:line it follows.  Paths are relative to the reference
 * repository root (laguna-raw).
 *
 * Pinning (how each function is checked beyond "retyping the formula"):
 *   orc_half_to_f32       reference unit tests src/dflash.rs:1334-1344
 *                         (0x3C00 -> 1.0, 0x3E00 -> 1.5), exhaustive 65536-code
 *                         comparison against numpy's IEEE decoder on every
 *                         normal/zero/inf code, closed-form subnormal quirk.
 *   orc_dequant_to_f32    reference unit tests src/dflash.rs:1347-1373
 *                         (Q8_0 d=1,q=1 -> 1.0; f32 passthrough; unsupported
 *                         -> zeros), exact-product closed forms, and an
 *                         independent vectorised numpy restatement
 *                         (tests/golden/make_golden.py) on random tensors.
 *   orc_q4k_value /
 *   orc_dequant_q4k       closed forms that isolate nibble order, the j<4 and
 *                         j>=4 scale/min packing and both high-bit fields;
 *                         independent numpy restatement on random blocks.
 *   orc_proj_*            layout known answer src/lib.rs:120-165 (k=8, n=3),
 *                         one-hot and all-ones inputs (exact column / row
 *                         sums), linearity, and the f64 accumulation bound.
 *   orc_silu_mul_*        closed forms silu(0)=0, silu(x)->x, silu(-x) ->0
 *                         and the identity silu(x)-silu(-x)=x.
 *   orc_legacy_q4k        (the non-ggml Q4_K branch of dequant_to_f32) closed
 *                         forms only; it is recorded, not a product target.
 *   orc_argmax_f32        numpy's last-occurrence argmax on NaN-free rows, and
 *                         closed forms for ties, signed zeros, infinities, empty
 *                         input and NaN positions (start, middle, end, all).
 */
#ifndef LAGUNA_ORACLE_H
#define LAGUNA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (src/gguf.rs:46-84). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_BF16 = 30 };

/* The reference's half decoder, src/dflash.rs:314-329 (named bf16_to_f32 there
 * but it decodes IEEE binary16; subnormals decode as 2^-14*(1+m/1024)). */
float orc_half_to_f32(uint16_t h);

/* dequant_to_f32, src/dflash.rs:331-465, including its Q4_K branch, which is
 * NOT ggml Q4_K (the legacy record-sum decode of :398-436). */
void orc_dequant_to_f32(const uint8_t *data, size_t len, uint32_t dtype,
                        size_t n_elements, float *out);

/* ggml Q4_K element at linear index lin, kernels/proj_q4k.comp:46-87. */
float orc_q4k_value(const uint8_t *data, uint64_t lin);
/* Q8_0 element at linear index lin, kernels/proj_q8_0.comp:59-63. */
float orc_q8_0_value(const uint8_t *data, uint64_t lin);

/* Whole-tensor ggml Q4_K dequant (the decode proj_q4k.comp applies), bounded
 * by the data length the way the Q8_0 branch of dequant_to_f32 is
 * (src/dflash.rs:379-397): a block that would run past `len` ends the loop
 * and the remaining outputs stay 0. */
void orc_dequant_q4k(const uint8_t *data, size_t len, size_t n_elements, float *out);

/* kernels/proj.comp:23-33: c[i] = sum_j x[j] * w[row_major ? j*n+i : i*k+j]. */
void orc_proj_f32(const float *x, const float *w, float *c, uint32_t k, uint32_t n,
                  uint32_t row_major);
/* kernels/proj_q8_0.comp:47-66. */
/* Multi-threaded forms (OpenMP, for the benchmark's CPU baseline); the same values
 * as orc_dequant_to_f32 (Q8_0) and orc_proj_f32. */
void orc_dequant_q8_0_mt(const uint8_t *data, size_t len, size_t n, float *out, int threads);
void orc_proj_f32_mt(const float *x, const float *w, float *c, uint32_t k, uint32_t n, uint32_t row_major,
                     int threads);
void orc_proj_q8_0(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n);
/* kernels/proj_q4k.comp:60-92 (uint32 linear index, as the shader). */
void orc_proj_q4k(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n,
                  uint32_t expert_offset);
/* Same loops split over `threads` OpenMP threads by output row (CPU baseline). */
void orc_proj_q4k_mt(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n,
                     int threads);
void orc_proj_q8_0_mt(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n,
                      int threads);

/* f64 accumulation of the exactly dequantized weights (the parity yardstick):
 * y[r*n+i] = sum_j x[r*k+j] * W[i,j] in double, absdot[r*n+i] = sum_j |x W|,
 * for rows r < m of a row-major [m][k] activation.  W[i,j] is element
 * elem_offset + i*k + j of the tensor (dtype Q4_K, Q8_0 or F32). */
void orc_proj_quant_f64(const float *x, uint32_t m, const uint8_t *w, uint32_t dtype,
                        uint32_t k, uint32_t n, uint64_t elem_offset, double *y,
                        double *absdot);

/* As orc_proj_quant_f64 for a single f64 activation vector x[k] (the f64
 * restatement of the fused silu(gate)*up input). */
void orc_proj_quant_f64x(const double *x, const uint8_t *w, uint32_t dtype, uint32_t k,
                         uint32_t n, double *y, double *absdot);

/* kernels/activation.comp:21-28: h = silu(g) * up, silu(x) = x * (1/(1+exp(-x))). */
void orc_silu_mul_f32(const float *g, const float *up, float *h, uint32_t n);
void orc_silu_mul_f64(const float *g, const float *up, double *h, uint32_t n);

/* src/lib.rs:456-464: the reference's argmax over n logits (0 when n = 0). */
size_t orc_argmax_f32(const float *v, size_t n);

#ifdef __cplusplus
}
#endif

#endif
