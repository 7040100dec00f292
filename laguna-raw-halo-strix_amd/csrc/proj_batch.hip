// Small-M products (block verify, m <= 64 activation rows): lg_dispatch_proj_quant_batch.
// Replaces kernels/matmul.comp (never dispatched by the reference) with bf16 MFMA
// tiles on gfx950 (v_mfma_f32_16x16x32_bf16: D[16x16] += A[16x32] * B[32x16]).
//
//   A = activations: 16 rows (tokens) x 32 k (one 32-element sub-block).  f32
//       activations are split exactly into three bf16 parts hi + mid + lo (each the
//       nearest bf16 of what the previous parts leave: together all 24 significant
//       bits, so the products are f32-grade); bf16 activations use one part.  A prep kernel writes them once
//       per call in MFMA operand order, with the per-sub-block sums X of the
//       represented values, into a device workspace.
//   B = weight codes of 16 output rows x the same 32 k, built in registers from
//       the raw blocks:  Q4_K nibble q -> bf16 1 + q/16 (one shift and one and-or
//       per pair);  Q8_0 int8 q -> bf16 of q + 128 (exact: 8 significant bits).
//   Epilogue per sub-block j of output row i (D = sum_k x_k B_k):
//       Q4_K:  sum x w = 16 d sc (D - X) - dmin m X
//       Q8_0:  sum x w = d (D - 128 X)
//
// Operand lane layout (16x16x32): lane l supplies row l%16 of A / column l%16 of B
// at k-group l/16 (8 consecutive bf16); D row 4*(l/16)+r, column l%16 lands in
// lane l, register r.  Inside a k-group the order of the 8 values only has to
// agree between A and B; both use byte order {0,2,1,3,4,6,5,7}, which is the
// order the nibble-pair encoding produces.
#include <vector>

#include "lg_common.hpp"

namespace {

using namespace lg;

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int PERM[8] = {0, 2, 1, 3, 4, 6, 5, 7};

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u);  // inf / NaN
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Workspace layout, per 16-row tile tt and sub-block j (nsb = k/32 sub-blocks):
//   frag[((tt*nsb + j)*parts + part)*64 + lane] : 8 bf16 (16 bytes)
//   xsum[(tt*nsb + j)*16 + token]              : f32
template <int PARTS>
__global__ __launch_bounds__(64) void k_prep_x(const void *__restrict__ xv, uint32_t m, uint32_t k,
                                               uint4 *__restrict__ frag, float *__restrict__ xsum) {
    const uint32_t nsb = k / 32;
    const uint32_t j = blockIdx.x, tt = blockIdx.y, l = threadIdx.x;
    const uint32_t tok = tt * 16 + (l & 15u), kg = l >> 4;
    uint32_t pc[PARTS][8];
    float part = 0.0f;
#pragma unroll
    for (int v = 0; v < 8; v++) {
        const uint32_t e = j * 32 + 8 * kg + PERM[v];
#pragma unroll
        for (int p = 0; p < PARTS; p++) pc[p][v] = 0;
        if (tok < m) {
            if constexpr (PARTS == 1) {
                pc[0][v] = static_cast<const uint16_t *>(xv)[(uint64_t)tok * k + e];
                part += bf16_to_f32(pc[0][v]);
            } else {
                const float x = static_cast<const float *>(xv)[(uint64_t)tok * k + e];
                float r = x;
#pragma unroll
                for (int p = 0; p < PARTS; p++) {
                    pc[p][v] = f32_to_bf16_rne(r);
                    r -= bf16_to_f32(pc[p][v]);  // exact: r stays a multiple of x's last place
                }
                part += x;  // the parts sum to x exactly
            }
        }
    }
    const uint64_t base = ((uint64_t)tt * nsb + j) * PARTS;
#pragma unroll
    for (int p = 0; p < PARTS; p++)
        frag[(base + p) * 64 + l] = make_uint4(pc[p][0] | pc[p][1] << 16, pc[p][2] | pc[p][3] << 16,
                                               pc[p][4] | pc[p][5] << 16, pc[p][6] | pc[p][7] << 16);
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
    if (l < 16) xsum[((uint64_t)tt * nsb + j) * 16 + l] = part;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    uint4 u = make_uint4(a, b, c, d);
    return __builtin_bit_cast(bf16x8, u);
}

// Q4_K nibble pairs -> bf16 (1 + q/16) pairs, byte order {0,2,1,3} per dword.
__device__ __forceinline__ void q4_codes(uint32_t v0, uint32_t v1, bf16x8 &lo, bf16x8 &hi) {
    uint32_t M = 0x00780078u, C = 0x3F803F80u;
    asm volatile("" : "+v"(M), "+v"(C));  // VGPR operands: one v_and_or_b32 per pair
    lo = as_bf16x8(((v0 << 3) & M) | C, ((v0 >> 5) & M) | C, ((v1 << 3) & M) | C, ((v1 >> 5) & M) | C);
    hi = as_bf16x8(((v0 >> 1) & M) | C, ((v0 >> 9) & M) | C, ((v1 >> 1) & M) | C, ((v1 >> 9) & M) | C);
}

// int8 bytes -> bf16 of (q + 128), byte order {0,2,1,3} per dword.
__device__ __forceinline__ void q8_codes(uint32_t v, uint32_t &p02, uint32_t &p13) {
    const uint32_t u = v ^ 0x80808080u;
    const uint32_t f0 = __float_as_uint(ubyte_f<0>(u));
    const uint32_t f1 = __float_as_uint(ubyte_f<1>(u));
    const uint32_t f2 = __float_as_uint(ubyte_f<2>(u));
    const uint32_t f3 = __float_as_uint(ubyte_f<3>(u));
    p02 = (f0 >> 16) | (f2 & 0xFFFF0000u);
    p13 = (f1 >> 16) | (f3 & 0xFFFF0000u);
}

// One wavefront = 16 output rows x all of k x up to TT 16-row activation tiles.
template <int PARTS, int TT>
__global__ __launch_bounds__(256) void k_q4k_batch(const uint4 *__restrict__ frag, const float *__restrict__ xsum,
                                                   const uint8_t *__restrict__ w, float *__restrict__ c, uint32_t m,
                                                   uint32_t k, uint32_t n, uint64_t row_bytes) {
    const uint32_t l = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row = (blockIdx.x * 4 + wave) * 16 + (l & 15u), kg = l >> 4;
    const bool live = row < n;
    const uint32_t nsb = k / 32, nb = k / QK_K;
    const uint8_t *wr = w + (uint64_t)(live ? row : 0) * row_bytes;
    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;

    for (uint32_t b = 0; b < nb; b++) {
        const uint8_t *blk = wr + (uint64_t)b * Q4K_BYTES;
        uint4 hd = make_uint4(0, 0, 0, 0);
        uint2 qv[4];
        if (live) {
            hd = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
            for (int g = 0; g < 4; g++) qv[g] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * g + 8 * kg);
        } else {
#pragma unroll
            for (int g = 0; g < 4; g++) qv[g] = make_uint2(0, 0);
        }
        const float d16 = 16.0f * ref_half(hd.x & 0xFFFFu), dmin = ref_half(hd.x >> 16);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            bf16x8 blo, bhi;
            q4_codes(qv[g].x, qv[g].y, blo, bhi);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t j = 2 * g + u;
                uint32_t sc, mn;
                scale_min_k4(j, hd.y, hd.z, hd.w, sc, mn);
                const float a = d16 * (float)sc;
                const float cc = __builtin_fmaf(dmin, (float)mn, a);
                const uint32_t sb = b * 8 + j;
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const uint64_t fb = ((uint64_t)t * nsb + sb) * PARTS;
                    f32x4 D = {0.f, 0.f, 0.f, 0.f};
                    const bf16x8 a0 = __builtin_bit_cast(bf16x8, frag[fb * 64 + l]);
                    D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, u ? bhi : blo, D, 0, 0, 0);
#pragma unroll
                    for (int p = 1; p < PARTS; p++) {
                        const bf16x8 ap = __builtin_bit_cast(bf16x8, frag[(fb + p) * 64 + l]);
                        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap, u ? bhi : blo, D, 0, 0, 0);
                    }
                    const float4 X = *reinterpret_cast<const float4 *>(xsum + ((uint64_t)t * nsb + sb) * 16 + 4 * kg);
                    acc[t][0] = __builtin_fmaf(a, D[0], __builtin_fmaf(-cc, X.x, acc[t][0]));
                    acc[t][1] = __builtin_fmaf(a, D[1], __builtin_fmaf(-cc, X.y, acc[t][1]));
                    acc[t][2] = __builtin_fmaf(a, D[2], __builtin_fmaf(-cc, X.z, acc[t][2]));
                    acc[t][3] = __builtin_fmaf(a, D[3], __builtin_fmaf(-cc, X.w, acc[t][3]));
                }
            }
        }
    }
    if (live) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = t * 16 + 4 * kg + r;
                if (tok < m) c[(uint64_t)tok * n + row] = acc[t][r];
            }
    }
}

template <int PARTS, int TT>
__global__ __launch_bounds__(256) void k_q80_batch(const uint4 *__restrict__ frag, const float *__restrict__ xsum,
                                                   const uint8_t *__restrict__ w, float *__restrict__ c, uint32_t m,
                                                   uint32_t k, uint32_t n, uint64_t row_bytes) {
    const uint32_t l = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row = (blockIdx.x * 4 + wave) * 16 + (l & 15u), kg = l >> 4;
    const bool live = row < n;
    const uint32_t nsb = k / 32;
    const uint8_t *wr = w + (uint64_t)(live ? row : 0) * row_bytes;
    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;

    for (uint32_t sb = 0; sb < nsb; sb++) {
        const uint16_t *blk = reinterpret_cast<const uint16_t *>(wr + (uint64_t)sb * Q80_BYTES);  // 2-byte aligned
        uint32_t v0 = 0, v1 = 0, dbits = 0;
        if (live) {
            dbits = blk[0];
            const uint16_t *q = blk + 1 + 4 * kg;
            v0 = q[0] | ((uint32_t)q[1] << 16);
            v1 = q[2] | ((uint32_t)q[3] << 16);
        }
        const float d = ref_half(dbits);
        uint32_t a0, a1, a2, a3;
        q8_codes(v0, a0, a1);
        q8_codes(v1, a2, a3);
        const bf16x8 B = as_bf16x8(a0, a1, a2, a3);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const uint64_t fb = ((uint64_t)t * nsb + sb) * PARTS;
            f32x4 D = {0.f, 0.f, 0.f, 0.f};
            D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, frag[fb * 64 + l]), B, D, 0, 0, 0);
#pragma unroll
            for (int p = 1; p < PARTS; p++)
                D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, frag[(fb + p) * 64 + l]), B, D,
                                                            0, 0, 0);
            const float4 X = *reinterpret_cast<const float4 *>(xsum + ((uint64_t)t * nsb + sb) * 16 + 4 * kg);
            acc[t][0] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X.x, D[0]), acc[t][0]);
            acc[t][1] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X.y, D[1]), acc[t][1]);
            acc[t][2] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X.z, D[2]), acc[t][2]);
            acc[t][3] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X.w, D[3]), acc[t][3]);
        }
    }
    if (live) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = t * 16 + 4 * kg + r;
                if (tok < m) c[(uint64_t)tok * n + row] = acc[t][r];
            }
    }
}

// Fallback for shapes outside the MFMA path (f32 weights, k not a multiple of the
// block, unaligned pointers): one wavefront per output row, element-wise decode.
__global__ __launch_bounds__(256) void k_generic_batch(const void *__restrict__ xv, int x_bf16,
                                                       const void *__restrict__ wv, float *__restrict__ c, uint32_t m,
                                                       uint32_t k, uint32_t n, int dtype) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const uint8_t *w = static_cast<const uint8_t *>(wv);
    for (uint32_t t0 = 0; t0 < m; t0 += 8) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t j = lane; j < k; j += 64) {
            const uint64_t lin = (uint64_t)row * k + j;
            float wj;
            if (dtype == LG_Q4_K) {
                const uint8_t *blk = w + (lin / QK_K) * Q4K_BYTES;
                const uint32_t e = lin % QK_K, sbj = e / 32, g = e / 64, wi = e % 64;
                uint32_t s[3];
                for (int q = 0; q < 3; q++)
                    s[q] = blk[4 + 4 * q] | (blk[5 + 4 * q] << 8) | (blk[6 + 4 * q] << 16) | ((uint32_t)blk[7 + 4 * q] << 24);
                uint32_t sc, mn;
                scale_min_k4(sbj, s[0], s[1], s[2], sc, mn);
                const uint32_t byte = blk[16 + 32 * g + (wi % 32)];
                const float q = (float)(wi < 32 ? (byte & 15u) : (byte >> 4));
                wj = __fsub_rn(__fmul_rn(__fmul_rn(ref_half(blk[0] | (blk[1] << 8)), (float)sc), q),
                               __fmul_rn(ref_half(blk[2] | (blk[3] << 8)), (float)mn));
            } else if (dtype == LG_Q8_0) {
                const uint8_t *blk = w + (lin / QK8_0) * Q80_BYTES;
                wj = __fmul_rn((float)(int8_t)blk[2 + lin % QK8_0], ref_half(blk[0] | (blk[1] << 8)));
            } else {
                wj = static_cast<const float *>(wv)[lin];
            }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                if (t0 + t < m) {
                    const uint64_t xi = (uint64_t)(t0 + t) * k + j;
                    const float xj = x_bf16 ? bf16_to_f32(static_cast<const uint16_t *>(xv)[xi])
                                            : static_cast<const float *>(xv)[xi];
                    acc[t] = __builtin_fmaf(xj, wj, acc[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float s = wave_sum(acc[t]);
            if (lane == 0 && t0 + t < m) c[(uint64_t)(t0 + t) * n + row] = s;
        }
    }
}

// Per-device workspace for activation fragments; grown on demand, kept for the
// life of the process.  Calls on one device share it: calls that overlap in time
// on different streams of the same device must be serialised by the caller.
struct Workspace {
    void *ptr = nullptr;
    uint64_t bytes = 0;
};
std::vector<Workspace> g_ws;

int workspace(uint64_t need, void **out) {
    int dev = 0;
    LG_HIP_TRY(hipGetDevice(&dev));
    if ((size_t)dev >= g_ws.size()) g_ws.resize(dev + 1);
    Workspace &ws = g_ws[dev];
    if (ws.bytes < need) {
        if (ws.ptr) {
            LG_HIP_TRY(hipDeviceSynchronize());  // earlier launches may still read it
            LG_HIP_TRY(hipFree(ws.ptr));
        }
        ws.ptr = nullptr;
        ws.bytes = 0;
        const uint64_t sz = (need + (1u << 20) - 1) & ~(uint64_t)((1u << 20) - 1);
        hipError_t e = hipMalloc(&ws.ptr, sz);
        if (e != hipSuccess) return fail(LG_ENOMEM, "batch workspace (%llu bytes): %s", (unsigned long long)sz,
                                         hipGetErrorString(e));
        ws.bytes = sz;
    }
    *out = ws.ptr;
    return LG_OK;
}

template <int PARTS>
int launch_main(int dtype, const uint4 *frag, const float *xs, const uint8_t *w, float *c, uint32_t m, uint32_t k,
                uint32_t n, hipStream_t s) {
    const uint32_t tiles = (m + 15) / 16;
    const dim3 grid((n + 63) / 64), block(256);
    if (dtype == LG_Q4_K) {
        const uint64_t rb = (uint64_t)k / QK_K * Q4K_BYTES;
        switch (tiles) {
        case 1: hipLaunchKernelGGL((k_q4k_batch<PARTS, 1>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        case 2: hipLaunchKernelGGL((k_q4k_batch<PARTS, 2>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        case 3: hipLaunchKernelGGL((k_q4k_batch<PARTS, 3>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        default: hipLaunchKernelGGL((k_q4k_batch<PARTS, 4>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        }
    } else {
        const uint64_t rb = (uint64_t)k / QK8_0 * Q80_BYTES;
        switch (tiles) {
        case 1: hipLaunchKernelGGL((k_q80_batch<PARTS, 1>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        case 2: hipLaunchKernelGGL((k_q80_batch<PARTS, 2>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        case 3: hipLaunchKernelGGL((k_q80_batch<PARTS, 3>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        default: hipLaunchKernelGGL((k_q80_batch<PARTS, 4>), grid, block, 0, s, frag, xs, w, c, m, k, n, rb); break;
        }
    }
    return after_launch(dtype == LG_Q4_K ? "proj_q4k_batch" : "proj_q8_0_batch", s);
}

}  // namespace

namespace lg {

uint64_t proj_batch_ws_bytes(uint32_t k, uint32_t m, int x_dtype) {
    const uint64_t tiles = (m + 15) / 16, nsb = k / 32;
    const int parts = x_dtype == LG_BF16 ? 1 : 3;
    return tiles * nsb * parts * 64 * 16 + tiles * nsb * 16 * 4;
}

int proj_batch(const void *x, int x_dtype, const void *w, float *c, uint32_t k, uint32_t n, uint32_t m, int w_dtype,
               void *ws_given, uint64_t ws_bytes, hipStream_t s) {
    const char *name = "lg_dispatch_proj_quant_batch";
    if (n == 0 || m == 0) return LG_OK;
    LG_REQUIRE(m <= 64, "%s: m=%u exceeds 64", name, m);
    LG_REQUIRE(x && w && c, "%s: null pointer", name);
    LG_REQUIRE(x_dtype == LG_F32 || x_dtype == LG_BF16, "%s: activation dtype %d (want F32 or BF16)", name, x_dtype);
    LG_REQUIRE(w_dtype == LG_Q4_K || w_dtype == LG_Q8_0 || w_dtype == LG_F32, "%s: weight dtype %d", name, w_dtype);
    const uint64_t xbytes = (uint64_t)m * k * (x_dtype == LG_F32 ? 4 : 2);
    LG_EXTENT(c, (uint64_t)m * n * 4, name);
    if (k == 0) {
        LG_HIP_TRY(hipMemsetAsync(c, 0, (uint64_t)m * n * 4, s));
        return after_launch(name, s);
    }
    LG_EXTENT(x, xbytes, name);
    LG_EXTENT(w, tensor_bytes(w_dtype, (uint64_t)n * k), name);
    const uint32_t blk = w_dtype == LG_Q4_K ? QK_K : QK8_0;
    const bool fast = w_dtype != LG_F32 && k % blk == 0 && k % 32 == 0 &&
                      (w_dtype != LG_Q4_K || (reinterpret_cast<uintptr_t>(w) & 15u) == 0) &&
                      (reinterpret_cast<uintptr_t>(w) & 1u) == 0;
    if (!fast) {
        hipLaunchKernelGGL(k_generic_batch, dim3((n + 3) / 4), dim3(256), 0, s, x, (int)(x_dtype == LG_BF16), w, c, m,
                           k, n, w_dtype);
        return after_launch(name, s);
    }
    const uint32_t tiles = (m + 15) / 16, nsb = k / 32;
    const int parts = x_dtype == LG_BF16 ? 1 : 3;
    const uint64_t frag_bytes = (uint64_t)tiles * nsb * parts * 64 * 16;
    void *ws = ws_given;
    int st = LG_OK;
    if (ws) {
        LG_REQUIRE(ws_bytes >= proj_batch_ws_bytes(k, m, x_dtype), "%s: workspace of %llu bytes too small", name,
                   (unsigned long long)ws_bytes);
    } else {
        st = workspace(proj_batch_ws_bytes(k, m, x_dtype), &ws);
        if (st != LG_OK) return st;
    }
    uint4 *frag = static_cast<uint4 *>(ws);
    float *xs = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + frag_bytes);
    if (parts == 1)
        hipLaunchKernelGGL(k_prep_x<1>, dim3(nsb, tiles), dim3(64), 0, s, x, m, k, frag, xs);
    else
        hipLaunchKernelGGL(k_prep_x<3>, dim3(nsb, tiles), dim3(64), 0, s, x, m, k, frag, xs);
    st = after_launch("prep_x", s);
    if (st != LG_OK) return st;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    return parts == 1 ? launch_main<1>(w_dtype, frag, xs, wb, c, m, k, n, s)
                      : launch_main<3>(w_dtype, frag, xs, wb, c, m, k, n, s);
}

}  // namespace lg

extern "C" int lg_dispatch_proj_quant_batch(const void *x, int x_dtype, const void *w, float *c, uint32_t k,
                                            uint32_t n, uint32_t m, int w_dtype, void *stream) {
    clear_error();
    return lg::proj_batch(x, x_dtype, w, c, k, n, m, w_dtype, nullptr, 0, (hipStream_t)stream);
}
