/*
 * CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h for the pinning of each
 * function).  Built with -O2 -ffp-contract=off and no fast-math so every f32
 * expression rounds exactly where the reference's source text rounds.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/dflash.rs:314-329 */
float orc_half_to_f32(uint16_t h_bits) {
    uint32_t sign = ((uint32_t)h_bits & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h_bits >> 10) & 0x1Fu;
    uint32_t mant = ((uint32_t)h_bits & 0x3FFu) << 13;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign);
        return bits_f32(sign | (113u << 23) | mant);
    } else if (exp == 31) {
        return bits_f32(sign | 0x7F800000u | mant);
    }
    return bits_f32(sign | ((exp + 112u) << 23) | mant);
}

/* Legacy Q4_K branch of dequant_to_f32, src/dflash.rs:398-436: bf16 d/k4/signs
 * (bits << 16) from bytes 0-5, 3-bit codes from bytes 6.., q*d + s*k4. */
static void legacy_q4k(const uint8_t *data, size_t len, size_t n, float *out) {
    size_t n_blocks = (n + 255) / 256;
    for (size_t b = 0; b < n_blocks; b++) {
        size_t base = b * 144;
        if (base + 144 > len) break;
        float d = bits_f32((uint32_t)rd16(data + base) << 16);
        float k4 = bits_f32((uint32_t)rd16(data + base + 2) << 16);
        float signs = bits_f32((uint32_t)rd16(data + base + 4) << 16);
        size_t start = b * 256;
        size_t end = start + 256 < n ? start + 256 : n;
        for (size_t i = 0; i < end - start; i++) {
            size_t byte_idx = base + 6 + i / 2;
            if (byte_idx >= base + 144) break;
            uint8_t byte = data[byte_idx];
            uint8_t q = (i % 2 == 0) ? ((byte >> 4) & 0x07) : (byte & 0x07);
            float s = signs < 0.0f ? -1.0f : 1.0f;
            float qd = (float)q * d;
            float sk = s * k4;
            out[start + i] = qd + sk;
        }
    }
}

/* src/dflash.rs:331-465 */
void orc_dequant_to_f32(const uint8_t *data, size_t len, uint32_t dtype, size_t n,
                        float *out) {
    memset(out, 0, n * sizeof(float));
    switch (dtype) {
    case ORC_F32: /* :333-350 */
        for (size_t i = 0; i < n; i++) {
            size_t off = i * 4;
            if (off + 4 <= len) {
                uint32_t u = (uint32_t)data[off] | ((uint32_t)data[off + 1] << 8) |
                             ((uint32_t)data[off + 2] << 16) | ((uint32_t)data[off + 3] << 24);
                out[i] = bits_f32(u);
            }
        }
        break;
    case ORC_BF16: /* :351-378 (decodes IEEE f16, with the subnormal quirk) */
        for (size_t i = 0; i < n; i++) {
            size_t off = i * 2;
            if (off + 2 <= len) out[i] = orc_half_to_f32(rd16(data + off));
        }
        break;
    case ORC_Q8_0: /* :379-397 */
    {
        size_t n_blocks = (n + 31) / 32;
        for (size_t b = 0; b < n_blocks; b++) {
            size_t off = b * 34;
            if (off + 34 > len) break;
            float d = orc_half_to_f32(rd16(data + off));
            size_t start = b * 32;
            size_t end = start + 32 < n ? start + 32 : n;
            for (size_t i = 0; i < end - start; i++) {
                float q = (float)(int8_t)data[off + 2 + i];
                out[start + i] = q * d;
            }
        }
        break;
    }
    case ORC_Q4_K: /* :398-436 */
        legacy_q4k(data, len, n, out);
        break;
    case ORC_F16: /* :437-462 (IEEE subnormals, canonical NaN) */
        for (size_t i = 0; i < n; i++) {
            size_t off = i * 2;
            if (off + 2 > len) continue;
            uint16_t h = rd16(data + off);
            float sign = (h & 0x8000) ? -1.0f : 1.0f;
            int exp = (h >> 10) & 0x1F;
            float mant = (float)(h & 0x3FF);
            if (exp == 0) {
                if (mant == 0.0f) out[i] = sign * 0.0f;
                else out[i] = sign * ldexpf(1.0f, -14) * (mant / 1024.0f);
            } else if (exp == 31) {
                out[i] = mant == 0.0f ? sign * INFINITY : bits_f32(0x7FC00000u);
            } else {
                out[i] = sign * ldexpf(1.0f, exp - 15) * (1.0f + mant / 1024.0f);
            }
        }
        break;
    default: /* :463 unsupported -> zeros */
        break;
    }
}

/* kernels/proj_q4k.comp:46-58 */
static void get_scale_min_k4(uint32_t j, const uint8_t *s, uint32_t *d, uint32_t *m) {
    uint32_t b0 = s[j];
    uint32_t b4 = s[4 + (j & 3)];
    uint32_t bp = s[8 + (j & 3)];
    if (j < 4) {
        *d = b0 & 63u;
        *m = b4 & 63u;
    } else {
        uint32_t d_hi = s[j - 4];
        *d = (bp & 15u) | ((d_hi >> 6) << 4);
        *m = (bp >> 4) | ((b4 >> 6) << 4);
    }
}

/* kernels/proj_q4k.comp:67-87 for one linear element index. */
float orc_q4k_value(const uint8_t *data, uint64_t lin) {
    uint64_t blk = lin / 256, elm = lin % 256;
    const uint8_t *b = data + blk * 144;
    float d = orc_half_to_f32(rd16(b));
    float dmin = orc_half_to_f32(rd16(b + 2));
    uint32_t sb = (uint32_t)(elm / 32), group64 = (uint32_t)(elm / 64), within64 = (uint32_t)(elm % 64);
    uint32_t q_byte = b[16 + group64 * 32 + (within64 % 32)];
    float q = (float)((within64 < 32) ? (q_byte & 0xFu) : ((q_byte >> 4) & 0xFu));
    uint32_t sc, mn;
    get_scale_min_k4(sb, b + 4, &sc, &mn);
    /* :87  float w = d * float(d_sc) * q - dmin_f * float(m_sc);  (left to right) */
    float t1 = d * (float)sc;
    float t2 = t1 * q;
    float t3 = dmin * (float)mn;
    return t2 - t3;
}

/* kernels/proj_q8_0.comp:59-63 for one linear element index. */
float orc_q8_0_value(const uint8_t *data, uint64_t lin) {
    uint64_t blk = lin / 32, elm = lin % 32;
    const uint8_t *b = data + blk * 34;
    float d = orc_half_to_f32(rd16(b));
    int q = (int)(int8_t)b[2 + elm];
    return (float)q * d;
}

void orc_dequant_q4k(const uint8_t *data, size_t len, size_t n, float *out) {
    memset(out, 0, n * sizeof(float));
    size_t n_blocks = (n + 255) / 256;
    for (size_t b = 0; b < n_blocks; b++) {
        if (b * 144 + 144 > len) break;
        size_t start = b * 256, end = start + 256 < n ? start + 256 : n;
        for (size_t i = start; i < end; i++) out[i] = orc_q4k_value(data, i);
    }
}

/* The Q8_0 arm of orc_dequant_to_f32 (src/dflash.rs:379-397) on `threads` OpenMP
 * threads: block b is decoded alone, and the serial loop's `break` at the first
 * block that runs past len becomes the bound b < len / 34.  Same values. */
void orc_dequant_q8_0_mt(const uint8_t *data, size_t len, size_t n, float *out, int threads) {
    memset(out, 0, n * sizeof(float));
    size_t n_blocks = (n + 31) / 32, whole = len / 34;
    if (n_blocks > whole) n_blocks = whole;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (size_t b = 0; b < n_blocks; b++) {
        size_t off = b * 34;
        float d = orc_half_to_f32(rd16(data + off));
        size_t start = b * 32;
        size_t end = start + 32 < n ? start + 32 : n;
        for (size_t i = 0; i < end - start; i++) {
            float q = (float)(int8_t)data[off + 2 + i];
            out[start + i] = q * d;
        }
    }
}

/* kernels/proj.comp:23-33 */
void orc_proj_f32(const float *x, const float *w, float *c, uint32_t k, uint32_t n,
                  uint32_t row_major) {
    for (uint32_t i = 0; i < n; i++) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < k; j++) {
            uint32_t idx = row_major ? (j * n + i) : (j + i * k);
            float p = x[j] * w[idx];
            acc += p;
        }
        c[i] = acc;
    }
}

/* orc_proj_f32 with its rows on `threads` OpenMP threads (each row's sum in the
 * shader's order, so the same values). */
void orc_proj_f32_mt(const float *x, const float *w, float *c, uint32_t k, uint32_t n, uint32_t row_major,
                     int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (uint32_t i = 0; i < n; i++) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < k; j++) {
            uint32_t idx = row_major ? (j * n + i) : (j + i * k);
            float p = x[j] * w[idx];
            acc += p;
        }
        c[i] = acc;
    }
}

static float q8_row(const float *x, const uint8_t *w, uint32_t k, uint32_t i) {
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; j++) {
        uint32_t lin = i * k + j; /* uint arithmetic as in the shader */
        float wv = orc_q8_0_value(w, lin);
        float p = x[j] * wv;
        acc += p;
    }
    return acc;
}

static float q4k_row(const float *x, const uint8_t *w, uint32_t k, uint32_t i, uint32_t off) {
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; j++) {
        uint32_t lin = off + i * k + j;
        float wv = orc_q4k_value(w, lin);
        float p = x[j] * wv;
        acc += p;
    }
    return acc;
}

/* kernels/proj_q8_0.comp:47-66 */
void orc_proj_q8_0(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) c[i] = q8_row(x, w, k, i);
}

/* kernels/proj_q4k.comp:60-92 */
void orc_proj_q4k(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n,
                  uint32_t expert_offset) {
    for (uint32_t i = 0; i < n; i++) c[i] = q4k_row(x, w, k, i, expert_offset);
}

void orc_proj_q4k_mt(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n,
                     int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (uint32_t i = 0; i < n; i++) c[i] = q4k_row(x, w, k, i, 0);
}

void orc_proj_q8_0_mt(const float *x, const uint8_t *w, float *c, uint32_t k, uint32_t n,
                      int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (uint32_t i = 0; i < n; i++) c[i] = q8_row(x, w, k, i);
}

void orc_proj_quant_f64(const float *x, uint32_t m, const uint8_t *w, uint32_t dtype,
                        uint32_t k, uint32_t n, uint64_t elem_offset, double *y,
                        double *absdot) {
    for (uint32_t i = 0; i < n; i++) {
        for (uint32_t r = 0; r < m; r++) {
            y[(size_t)r * n + i] = 0.0;
            absdot[(size_t)r * n + i] = 0.0;
        }
        for (uint32_t j = 0; j < k; j++) {
            uint64_t lin = elem_offset + (uint64_t)i * k + j;
            float wv;
            if (dtype == ORC_Q4_K) wv = orc_q4k_value(w, lin);
            else if (dtype == ORC_Q8_0) wv = orc_q8_0_value(w, lin);
            else memcpy(&wv, w + lin * 4, 4);
            for (uint32_t r = 0; r < m; r++) {
                double p = (double)x[(size_t)r * k + j] * (double)wv;
                y[(size_t)r * n + i] += p;
                absdot[(size_t)r * n + i] += fabs(p);
            }
        }
    }
}

void orc_proj_quant_f64x(const double *x, const uint8_t *w, uint32_t dtype, uint32_t k,
                         uint32_t n, double *y, double *absdot) {
    for (uint32_t i = 0; i < n; i++) {
        double acc = 0.0, a = 0.0;
        for (uint32_t j = 0; j < k; j++) {
            uint64_t lin = (uint64_t)i * k + j;
            float wv;
            if (dtype == ORC_Q4_K) wv = orc_q4k_value(w, lin);
            else if (dtype == ORC_Q8_0) wv = orc_q8_0_value(w, lin);
            else memcpy(&wv, w + lin * 4, 4);
            double p = x[j] * (double)wv;
            acc += p;
            a += fabs(p);
        }
        y[i] = acc;
        absdot[i] = a;
    }
}

/* kernels/activation.comp:21-28 */
void orc_silu_mul_f32(const float *g, const float *up, float *h, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        float e = expf(-g[i]);
        float den = 1.0f + e;
        float r = 1.0f / den;
        float s = g[i] * r;
        h[i] = s * up[i];
    }
}

void orc_silu_mul_f64(const float *g, const float *up, double *h, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        double x = g[i];
        h[i] = x * (1.0 / (1.0 + exp(-x))) * (double)up[i];
    }
}

/* src/lib.rs:456-464: logits.iter().copied().enumerate().max_by(|a, b|
 * a.1.partial_cmp(&b.1).unwrap_or(Equal)).map(|(i, _)| i).unwrap_or(0).
 * Iterator::max_by keeps the running best only when compare(best, next) is
 * Greater; Less, Equal and unordered (NaN, mapped to Equal) take the next. */
size_t orc_argmax_f32(const float *v, size_t n) {
    if (n == 0) return 0;
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (!(v[best] > v[i])) best = i;
    return best;
}
