// Whole-tensor dequantization on the device: lg_dequant_to_f32.
//
// Reference: dequant_to_f32 (src/dflash.rs:331-465), a serial CPU loop run at
// model load.  Q8_0 follows its branch (:379-397); Q4_K follows the ggml decode
// of kernels/proj_q4k.comp:28-87 (the Rust Q4_K branch is a different format).
// Both products are exact in f32 (f16 d has 11 significant bits, sc <= 63,
// q <= 15, |int8| <= 128), so `(d*sc)*q - dmin*m` rounds once, at the
// subtraction, and the result is bit-identical to the reference for every
// non-NaN input; __fmul_rn/__fsub_rn keep the compiler from reassociating.
#include "lg_common.hpp"

namespace {

using namespace lg;

// One thread per 16-byte quant chunk: 8 threads per 144-byte super-block, each
// producing 32 values (16 low nibbles of sub-block 2g, 16 high nibbles of 2g+1).
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t *__restrict__ data,
                                                     uint64_t blocks_avail, uint64_t n,
                                                     float *__restrict__ out, int vec_out) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t b = gid >> 3;
    const uint32_t c = gid & 7u, g = c >> 1, h = c & 1u;
    const uint64_t base = b * QK_K + 64u * g + 16u * h;  // first low-nibble element
    if (base >= n) return;
    float lo[16], hi[16];
    if (b < blocks_avail) {
        const uint8_t *blk = data + b * Q4K_BYTES;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qs = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * g + 16 * h);
        const float d = ref_half(hd.x & 0xFFFFu), dmin = ref_half(hd.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        scale_min_k4(2 * g, hd.y, hd.z, hd.w, sc0, m0);
        scale_min_k4(2 * g + 1, hd.y, hd.z, hd.w, sc1, m1);
        const float a0 = __fmul_rn(d, (float)sc0), b0 = __fmul_rn(dmin, (float)m0);
        const float a1 = __fmul_rn(d, (float)sc1), b1 = __fmul_rn(dmin, (float)m1);
        const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
            lo[i] = __fsub_rn(__fmul_rn(a0, (float)(byte & 15u)), b0);
            hi[i] = __fsub_rn(__fmul_rn(a1, (float)(byte >> 4)), b1);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) lo[i] = hi[i] = 0.0f;
    }
    if (vec_out && base + 48 <= n) {
        float4 *o = reinterpret_cast<float4 *>(out + base);
        float4 *p = reinterpret_cast<float4 *>(out + base + 32);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[i] = make_float4(lo[4 * i], lo[4 * i + 1], lo[4 * i + 2], lo[4 * i + 3]);
            p[i] = make_float4(hi[4 * i], hi[4 * i + 1], hi[4 * i + 2], hi[4 * i + 3]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if (base + i < n) out[base + i] = lo[i];
            if (base + 32 + i < n) out[base + 32 + i] = hi[i];
        }
    }
}

// Byte-addressed variant for a tensor base that is not 16-byte aligned.
__global__ __launch_bounds__(256) void k_dequant_q4k_bytes(const uint8_t *__restrict__ data,
                                                           uint64_t blocks_avail, uint64_t n,
                                                           float *__restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t b = i / QK_K;
    if (b >= blocks_avail) {
        out[i] = 0.0f;
        return;
    }
    const uint8_t *blk = data + b * Q4K_BYTES;
    const uint32_t e = i % QK_K, j = e / 32, g = e / 64, w = e % 64;
    uint32_t s[3];
    for (int t = 0; t < 3; t++)
        s[t] = blk[4 + 4 * t] | (blk[5 + 4 * t] << 8) | (blk[6 + 4 * t] << 16) | ((uint32_t)blk[7 + 4 * t] << 24);
    uint32_t sc, mn;
    scale_min_k4(j, s[0], s[1], s[2], sc, mn);
    const float d = ref_half(blk[0] | (blk[1] << 8)), dmin = ref_half(blk[2] | (blk[3] << 8));
    const uint32_t byte = blk[16 + 32 * g + (w % 32)];
    const float q = (float)(w < 32 ? (byte & 15u) : (byte >> 4));
    out[i] = __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), q), __fmul_rn(dmin, (float)mn));
}

// One thread per 34-byte Q8_0 block (value = float(q) * d, src/dflash.rs:389-394).
__global__ __launch_bounds__(256) void k_dequant_q8_0(const uint8_t *__restrict__ data,
                                                      uint64_t blocks_avail, uint64_t n,
                                                      float *__restrict__ out, int vec_out) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t base = b * QK8_0;
    if (base >= n) return;
    float v[32];
    if (b < blocks_avail) {
        const uint8_t *blk = data + b * Q80_BYTES;
        const float d = ref_half(blk[0] | (blk[1] << 8));
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = __fmul_rn((float)(int8_t)blk[2 + i], d);
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = 0.0f;
    }
    if (vec_out && base + 32 <= n) {
        float4 *o = reinterpret_cast<float4 *>(out + base);
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
        for (int i = 0; i < 32; i++)
            if (base + i < n) out[base + i] = v[i];
    }
}

// F32 / F16 / "BF16" branches (src/dflash.rs:333-378, :437-462), element-wise,
// with the reference's per-element length check.
__global__ __launch_bounds__(256) void k_dequant_elem(const uint8_t *__restrict__ data, uint64_t len,
                                                      int dtype, uint64_t n, float *__restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float r = 0.0f;
    if (dtype == LG_F32) {
        if (i * 4 + 4 <= len)
            r = __uint_as_float(data[4 * i] | (data[4 * i + 1] << 8) | (data[4 * i + 2] << 16) |
                                ((uint32_t)data[4 * i + 3] << 24));
    } else if (i * 2 + 2 <= len) {
        const uint32_t h = data[2 * i] | (data[2 * i + 1] << 8);
        if (dtype == LG_BF16) {
            r = ref_half(h);
        } else {  // LG_F16: IEEE subnormals, canonical NaN
            const uint32_t e = (h >> 10) & 31u, m = h & 0x3FFu;
            const float sign = (h & 0x8000u) ? -1.0f : 1.0f;
            if (e == 0) r = __fmul_rn(__fmul_rn(sign, 6.103515625e-05f), __fdiv_rn((float)m, 1024.0f));
            else if (e == 31) r = m == 0 ? sign * __builtin_inff() : __uint_as_float(0x7FC00000u);
            else r = __fmul_rn(__fmul_rn(sign, ldexpf(1.0f, (int)e - 15)), __fadd_rn(1.0f, __fdiv_rn((float)m, 1024.0f)));
        }
    }
    out[i] = r;
}

inline unsigned grid_for(uint64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace

extern "C" int lg_dequant_to_f32(const void *data, uint64_t data_len, int dtype, uint64_t n,
                                 float *out, void *stream) {
    clear_error();
    if (n == 0) return LG_OK;
    LG_REQUIRE(out, "lg_dequant_to_f32: null out");
    LG_REQUIRE(data || data_len == 0, "lg_dequant_to_f32: null data with data_len %llu",
               (unsigned long long)data_len);
    LG_REQUIRE(n <= (1ull << 40), "lg_dequant_to_f32: n_elements %llu too large", (unsigned long long)n);
    LG_EXTENT(out, n * 4, "lg_dequant_to_f32 out");
    if (data_len) LG_EXTENT(data, data_len, "lg_dequant_to_f32 data");
    hipStream_t s = (hipStream_t)stream;
    const auto *d = static_cast<const uint8_t *>(data);
    const int vec_out = (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    switch (dtype) {
    case LG_Q4_K: {
        const uint64_t need = (n + QK_K - 1) / QK_K, have = data_len / Q4K_BYTES;
        const uint64_t avail = have < need ? have : need;
        if ((reinterpret_cast<uintptr_t>(d) & 15u) == 0)
            hipLaunchKernelGGL(k_dequant_q4k, dim3(grid_for(need * 8)), dim3(256), 0, s, d, avail, n, out, vec_out);
        else
            hipLaunchKernelGGL(k_dequant_q4k_bytes, dim3(grid_for(n)), dim3(256), 0, s, d, avail, n, out);
        return after_launch("dequant_q4k", s);
    }
    case LG_Q8_0: {
        const uint64_t need = (n + QK8_0 - 1) / QK8_0, have = data_len / Q80_BYTES;
        const uint64_t avail = have < need ? have : need;
        hipLaunchKernelGGL(k_dequant_q8_0, dim3(grid_for(need)), dim3(256), 0, s, d, avail, n, out, vec_out);
        return after_launch("dequant_q8_0", s);
    }
    case LG_F32:
    case LG_F16:
    case LG_BF16:
        hipLaunchKernelGGL(k_dequant_elem, dim3(grid_for(n)), dim3(256), 0, s, d, data_len, dtype, n, out);
        return after_launch("dequant_elem", s);
    default:  // src/dflash.rs:463: unsupported types decode to zeros
        LG_HIP_TRY(hipMemsetAsync(out, 0, n * 4, s));
        return after_launch("dequant_zeros", s);
    }
}
