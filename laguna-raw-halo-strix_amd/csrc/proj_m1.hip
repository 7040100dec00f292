// M = 1 projections: c[i] = sum_j x[j] * W[i,j] over raw GGUF blocks.
//
// Replaces kernels/proj_q4k.comp, proj_q8_0.comp, proj.comp and activation.comp
// (one invocation per output row, per-element byte decode, uncoalesced) with
// wavefront-cooperative gfx950 kernels:
//
// Q4_K (k % 256 == 0, 16-byte aligned tensor): lane p of a row team owns the
// 64-element group p of the row (super-block p/4, group p%4).  Per row it loads
// the 16-byte block header and the 32 quant bytes of its group with three
// 16-byte loads; the team's loads together cover the row's bytes exactly once.
// The lane keeps its 64 activations in registers for every row it visits.
// Nibbles are turned into f16 values 1 + q/16 with one shift and one and-or per
// pair and accumulated with v_fma_mix_f32 against the f32 activations:
//     S = sum x (1 + q/16)  =>  sum x q = 16 (S - X),  X = sum x (per lane, once)
// and the block's scale and min enter once per 32-element sub-block:
//     sum_j x_j ((d sc) q_j - dmin m) = 16 d sc (S - X) - dmin m X.
// Partial sums meet in a DPP/swizzle wavefront reduction (and LDS across the
// waves of a team when k > 4096).
//
// Q8_0: the same lane ownership (64 elements = two 34-byte blocks, 68 bytes,
// dword aligned).  Rows are staged through LDS with coalesced 16-byte loads and
// each lane reads its 17 dwords back (stride 17 dwords: no bank conflicts).
// Bytes are biased to unsigned (q + 128), converted with v_cvt_f32_ubyte and
// corrected by 128 X per block.
//
// Inputs outside these fast paths (k not a multiple of 256, unaligned pointers,
// element offsets that are not block aligned) go to a per-element kernel that
// follows the reference's linear addressing exactly (lin = offset + i*k + j).
#include "lg_common.hpp"

namespace {

using namespace lg;

uint32_t g_grid_cap = 0;  // 0 = automatic

constexpr uint32_t M1_MAX_K = 16384;  // 4 waves x 64 lanes x 64 elements

// ------------------------------------------------------------------------------------------
// activation staging

__device__ __forceinline__ float silu_mul(float g, float u) {
    // kernels/activation.comp:21-28: silu(g) * up, silu(x) = x * (1 / (1 + exp(-x)))
    return g * (1.0f / (1.0f + __expf(-g))) * u;
}

// Load this lane's 64 activations (elements 64p .. 64p+63) into registers, either
// straight from global memory or from an LDS copy of the whole vector (padded by
// 4 floats per 64 so that 16-byte LDS reads by consecutive lanes spread over banks).
template <int TEAMS, bool FUSE>
__device__ __forceinline__ void load_x(const float *__restrict__ x, const float *__restrict__ up,
                                       uint32_t k, uint32_t p, bool active, float *lds,
                                       float (&xr)[64]) {
    if constexpr (TEAMS > 1) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const float4 *u4 = reinterpret_cast<const float4 *>(up);
        for (uint32_t e4 = threadIdx.x; e4 < k / 4; e4 += blockDim.x) {
            float4 v = x4[e4];
            if constexpr (FUSE) {
                const float4 u = u4[e4];
                v = make_float4(silu_mul(v.x, u.x), silu_mul(v.y, u.y), silu_mul(v.z, u.z), silu_mul(v.w, u.w));
            }
            const uint32_t e = 4 * e4;
            *reinterpret_cast<float4 *>(lds + e + 4 * (e >> 6)) = v;
        }
        __syncthreads();
        if (active) {
            const float4 *s4 = reinterpret_cast<const float4 *>(lds + 68 * p);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4 v = s4[i];
                xr[4 * i] = v.x, xr[4 * i + 1] = v.y, xr[4 * i + 2] = v.z, xr[4 * i + 3] = v.w;
            }
        }
    } else {
        if (active) {
            const float4 *x4 = reinterpret_cast<const float4 *>(x + 64 * p);
            const float4 *u4 = reinterpret_cast<const float4 *>(up + 64 * p);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float4 v = x4[i];
                if constexpr (FUSE) {
                    const float4 u = u4[i];
                    v = make_float4(silu_mul(v.x, u.x), silu_mul(v.y, u.y), silu_mul(v.z, u.z), silu_mul(v.w, u.w));
                }
                xr[4 * i] = v.x, xr[4 * i + 1] = v.y, xr[4 * i + 2] = v.z, xr[4 * i + 3] = v.w;
            }
        }
    }
    if (!active) {
#pragma unroll
        for (int i = 0; i < 64; i++) xr[i] = 0.0f;
    }
}

__device__ __forceinline__ float h_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }
__device__ __forceinline__ float h_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// Team-wide sum of R row partials: DPP/swizzle inside each wave, LDS across the TW
// waves of a team.  The caller guarantees uniform control flow for the barriers.
template <int TW, int R>
__device__ __forceinline__ void team_store(float (&acc)[R], uint32_t row0, uint32_t n, float *__restrict__ y,
                                           float *red, uint32_t lane, uint32_t wt) {
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if constexpr (TW == 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (row0 + r < n) y[row0 + r] = acc[r];
        }
    } else {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) red[r * TW + wt] = acc[r];
        }
        __syncthreads();
        if (wt == 0 && lane < (uint32_t)R && row0 + lane < n) {
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t < TW; t++) s += red[lane * TW + t];
            y[row0 + lane] = s;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------
// Q4_K

struct Q4Lane {
    uint32_t g;          // group within the super-block (0..3): sub-blocks 2g, 2g+1
    uint32_t sa[2], sb[2], ma[2], mb[2];  // bit offsets of the 4 + 2 scale/min bits
};

__device__ __forceinline__ Q4Lane q4_lane(uint32_t g) {
    Q4Lane L;
    L.g = g;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t j = 2 * g + u;
        if (j < 4) {  // sc = s[j] & 63, m = s[j+4] & 63
            L.sa[u] = 8 * j, L.sb[u] = 8 * j + 4, L.ma[u] = 8 * j, L.mb[u] = 8 * j + 4;
        } else {      // sc = s[j+4]&15 | (s[j-4]>>6)<<4, m = s[j+4]>>4 | (s[j]>>6)<<4
            L.sa[u] = 8 * (j - 4), L.sb[u] = 8 * (j - 4) + 6, L.ma[u] = 8 * (j - 4) + 4, L.mb[u] = 8 * (j - 4) + 6;
        }
    }
    return L;
}

// One lane's contribution to one row: 64 weights of super-block header `hd`
// (d, dmin, scales) and quant bytes qa (bytes 0-15 of the group) and qb (16-31).
__device__ __forceinline__ float q4_dot(const uint4 &hd, const uint4 &qa, const uint4 &qb, const float (&xr)[64],
                                        float X0, float X1, const Q4Lane &L) {
    // Mask and bias live in VGPRs so that each pair is one shift + one v_and_or_b32
    // (a GFX9 VOP3 instruction cannot encode two literal constants).
    uint32_t M = 0x03C003C0u, C = 0x3C003C00u;
    asm volatile("" : "+v"(M), "+v"(C));
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    float s0a = 0.f, s0b = 0.f, s1a = 0.f, s1b = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const uint32_t v = q[t];
        const uint32_t p02 = ((v << 6) & M) | C;  // low nibbles of bytes 4t, 4t+2  -> sub-block 2g
        const uint32_t p13 = ((v >> 2) & M) | C;  // low nibbles of bytes 4t+1, 4t+3
        const uint32_t h02 = ((v << 2) & M) | C;  // high nibbles of bytes 4t, 4t+2 -> sub-block 2g+1
        const uint32_t h13 = ((v >> 6) & M) | C;  // high nibbles of bytes 4t+1, 4t+3
        s0a = __builtin_fmaf(xr[4 * t + 0], h_lo(p02), s0a);
        s0b = __builtin_fmaf(xr[4 * t + 1], h_lo(p13), s0b);
        s0a = __builtin_fmaf(xr[4 * t + 2], h_hi(p02), s0a);
        s0b = __builtin_fmaf(xr[4 * t + 3], h_hi(p13), s0b);
        s1a = __builtin_fmaf(xr[32 + 4 * t + 0], h_lo(h02), s1a);
        s1b = __builtin_fmaf(xr[32 + 4 * t + 1], h_lo(h13), s1b);
        s1a = __builtin_fmaf(xr[32 + 4 * t + 2], h_hi(h02), s1a);
        s1b = __builtin_fmaf(xr[32 + 4 * t + 3], h_hi(h13), s1b);
    }
    const float S0 = s0a + s0b, S1 = s1a + s1b;
    // scales and mins of sub-blocks 2g and 2g+1 (kernels/proj_q4k.comp:46-58)
    const bool lo = L.g < 2;
    const uint32_t srcA = lo ? hd.y : hd.w, srcM = lo ? hd.z : hd.w;
    const float d = ref_half(hd.x & 0xFFFFu), dmin = ref_half(hd.x >> 16);
    const float d16 = d * 16.0f;
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t sc = __builtin_amdgcn_ubfe(srcA, L.sa[u], 4) | (__builtin_amdgcn_ubfe(hd.y, L.sb[u], 2) << 4);
        const uint32_t mn = __builtin_amdgcn_ubfe(srcM, L.ma[u], 4) | (__builtin_amdgcn_ubfe(hd.z, L.mb[u], 2) << 4);
        const float a = d16 * (float)sc;                     // 16 d sc
        const float c = __builtin_fmaf(dmin, (float)mn, a);  // 16 d sc + dmin m
        const float S = u ? S1 : S0, X = u ? X1 : X0;
        acc = __builtin_fmaf(a, S, acc);
        acc = __builtin_fmaf(-c, X, acc);
    }
    return acc;
}

template <int TW, int TEAMS, int R, bool FUSE>
__global__ __launch_bounds__(TW *TEAMS * 64) void k_q4k_m1(const float *__restrict__ x, const float *__restrict__ up,
                                                            const uint8_t *__restrict__ w, float *__restrict__ y,
                                                            uint32_t k, uint32_t n, uint64_t row_bytes) {
    __shared__ __attribute__((aligned(16))) float xs[TEAMS > 1 ? 4096 + 256 : 4];
    __shared__ float red[TW > 1 ? R * TW : 1];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t team = wave / TW, wt = wave % TW;
    const uint32_t P = k >> 6;
    const uint32_t p = wt * 64 + lane;
    const bool active = p < P;
    float xr[64];
    load_x<TEAMS, FUSE>(x, up, k, p, active, xs, xr);
    float X0 = 0.f, X1 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) X0 += xr[i], X1 += xr[32 + i];
    const Q4Lane L = q4_lane(p & 3u);
    const uint64_t lane_off = (uint64_t)(p >> 2) * Q4K_BYTES;
    const uint32_t step = TEAMS * R;
    for (uint32_t r0 = blockIdx.x * step; r0 < n; r0 += gridDim.x * step) {
        const uint32_t rb = r0 + team * R;
        uint4 hd[R], qa[R], qb[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (active && rb + r < n) {
                const uint8_t *blk = w + (uint64_t)(rb + r) * row_bytes + lane_off;
                hd[r] = *reinterpret_cast<const uint4 *>(blk);
                qa[r] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * L.g);
                qb[r] = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * L.g);
            } else {
                hd[r] = qa[r] = qb[r] = make_uint4(0, 0, 0, 0);
            }
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = q4_dot(hd[r], qa[r], qb[r], xr, X0, X1, L);
        team_store<TW, R>(acc, rb, n, y, red, lane, wt);
    }
}

// ------------------------------------------------------------------------------------------
// Q8_0

template <int TW, int TEAMS, int R>
__global__ __launch_bounds__(TW *TEAMS * 64) void k_q80_m1(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                            float *__restrict__ y, uint32_t k, uint32_t n,
                                                            uint64_t row_bytes) {
    constexpr uint32_t SEG = 64 * 68;  // bytes of one wave's share of a row
    __shared__ __attribute__((aligned(16))) float xs[TEAMS > 1 ? 4096 + 256 : 4];
    __shared__ __attribute__((aligned(16))) uint32_t stage[TW * TEAMS][R][SEG / 4];
    __shared__ float red[TW > 1 ? R * TW : 1];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t team = wave / TW, wt = wave % TW;
    const uint32_t P = k >> 6;
    const uint32_t p = wt * 64 + lane;
    const bool active = p < P;
    float xr[64];
    load_x<TEAMS, false>(x, nullptr, k, p, active, xs, xr);
    float X0 = 0.f, X1 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) X0 += xr[i], X1 += xr[32 + i];
    // this wave's byte range of a row: groups wt*64 .. min(P, wt*64+64)
    const uint32_t groups = P > wt * 64 ? (P - wt * 64 < 64 ? P - wt * 64 : 64) : 0;
    const uint32_t seg16 = groups * 68 / 16;  // groups is a multiple of 4 -> whole 16-byte units
    const uint32_t step = TEAMS * R;
    for (uint32_t r0 = blockIdx.x * step; r0 < n; r0 += gridDim.x * step) {
        const uint32_t rb = r0 + team * R;
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (rb + r < n) {
                const uint4 *src = reinterpret_cast<const uint4 *>(w + (uint64_t)(rb + r) * row_bytes + (uint64_t)wt * SEG);
                uint4 *dst = reinterpret_cast<uint4 *>(stage[wave][r]);
                for (uint32_t c = lane; c < seg16; c += 64) dst[c] = src[c];
            }
        }
        __syncthreads();
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            acc[r] = 0.0f;
            if (active && rb + r < n) {
                const uint32_t *D = stage[wave][r] + 17 * lane;
                uint32_t v[17];
#pragma unroll
                for (int i = 0; i < 17; i++) v[i] = D[i];
                const float d0 = ref_half(v[0] & 0xFFFFu), d1 = ref_half(v[8] >> 16);
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    // block 0 quants start 2 bytes into the lane's 68 bytes: realign
                    const uint32_t a = __builtin_amdgcn_alignbit(v[t + 1], v[t], 16) ^ 0x80808080u;
                    const uint32_t b = v[9 + t] ^ 0x80808080u;
                    s0 = __builtin_fmaf(xr[4 * t + 0], ubyte_f<0>(a), s0);
                    s0 = __builtin_fmaf(xr[4 * t + 1], ubyte_f<1>(a), s0);
                    s0 = __builtin_fmaf(xr[4 * t + 2], ubyte_f<2>(a), s0);
                    s0 = __builtin_fmaf(xr[4 * t + 3], ubyte_f<3>(a), s0);
                    s1 = __builtin_fmaf(xr[32 + 4 * t + 0], ubyte_f<0>(b), s1);
                    s1 = __builtin_fmaf(xr[32 + 4 * t + 1], ubyte_f<1>(b), s1);
                    s1 = __builtin_fmaf(xr[32 + 4 * t + 2], ubyte_f<2>(b), s1);
                    s1 = __builtin_fmaf(xr[32 + 4 * t + 3], ubyte_f<3>(b), s1);
                }
                // sum x q = S - 128 X  (q + 128 was accumulated)
                acc[r] = d0 * __builtin_fmaf(-128.0f, X0, s0) + d1 * __builtin_fmaf(-128.0f, X1, s1);
            }
        }
        team_store<TW, R>(acc, rb, n, y, red, lane, wt);
        if constexpr (TW == 1) __syncthreads();  // stage[] is rewritten by the next iteration
    }
}

// ------------------------------------------------------------------------------------------
// Reference-semantics fallback: one wavefront per row, element-wise decode at the
// reference's linear index (kernels/proj_q4k.comp:67, proj_q8_0.comp:54).

__device__ __forceinline__ float q4k_elem(const uint8_t *__restrict__ w, uint64_t lin) {
    const uint8_t *blk = w + (lin / QK_K) * Q4K_BYTES;
    const uint32_t e = lin % QK_K, j = e / 32, g = e / 64, wi = e % 64;
    const float d = ref_half(blk[0] | (blk[1] << 8)), dmin = ref_half(blk[2] | (blk[3] << 8));
    const uint32_t b0 = blk[4 + j], b4 = blk[8 + (j & 3)], bp = blk[12 + (j & 3)];
    uint32_t sc, mn;
    if (j < 4) {
        sc = b0 & 63u, mn = b4 & 63u;
    } else {
        sc = (bp & 15u) | ((blk[4 + j - 4] >> 6) << 4);
        mn = (bp >> 4) | ((b4 >> 6) << 4);
    }
    const uint32_t byte = blk[16 + 32 * g + (wi % 32)];
    const float q = (float)(wi < 32 ? (byte & 15u) : (byte >> 4));
    return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), q), __fmul_rn(dmin, (float)mn));
}

__device__ __forceinline__ float q80_elem(const uint8_t *__restrict__ w, uint64_t lin) {
    const uint8_t *blk = w + (lin / QK8_0) * Q80_BYTES;
    return __fmul_rn((float)(int8_t)blk[2 + lin % QK8_0], ref_half(blk[0] | (blk[1] << 8)));
}

template <bool FUSE>
__global__ __launch_bounds__(256) void k_generic_m1(const float *__restrict__ x, const float *__restrict__ up,
                                                    const void *__restrict__ wv, float *__restrict__ y, uint32_t k,
                                                    uint32_t n, int dtype, uint64_t off) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const uint8_t *w = static_cast<const uint8_t *>(wv);
    float acc = 0.0f;
    for (uint32_t j = lane; j < k; j += 64) {
        const uint64_t lin = off + (uint64_t)row * k + j;
        float wj;
        if (dtype == LG_Q4_K) wj = q4k_elem(w, lin);
        else if (dtype == LG_Q8_0) wj = q80_elem(w, lin);
        else wj = static_cast<const float *>(wv)[lin];
        float xj = x[j];
        if constexpr (FUSE) xj = silu_mul(xj, up[j]);
        acc = __builtin_fmaf(xj, wj, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// ------------------------------------------------------------------------------------------
// f32 weights: kernels/proj.comp (row_major = 0: w[i*k+j]; 1: w[j*n+i])

__global__ __launch_bounds__(256) void k_f32_rows(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ y, uint32_t k, uint32_t n, int vec) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const float *wr = w + (uint64_t)row * k;
    float acc = 0.0f;
    if (vec) {
        const float4 *w4 = reinterpret_cast<const float4 *>(wr);
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (uint32_t j = lane; j < k / 4; j += 64) {
            const float4 a = w4[j], b = x4[j];
            acc = __builtin_fmaf(a.x, b.x, acc);
            acc = __builtin_fmaf(a.y, b.y, acc);
            acc = __builtin_fmaf(a.z, b.z, acc);
            acc = __builtin_fmaf(a.w, b.w, acc);
        }
    } else {
        for (uint32_t j = lane; j < k; j += 64) acc = __builtin_fmaf(wr[j], x[j], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

__global__ __launch_bounds__(256) void k_f32_cols(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ y, uint32_t k, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; j++) acc = __builtin_fmaf(x[j], w[(uint64_t)j * n + i], acc);
    y[i] = acc;
}

__global__ __launch_bounds__(256) void k_activation(const float *__restrict__ g, const float *__restrict__ u,
                                                    float *__restrict__ h, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = silu_mul(g[i], u[i]);
}

// ------------------------------------------------------------------------------------------
// host dispatch

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

uint32_t grid_for(uint32_t n, uint32_t rows_per_wg, uint32_t cap_default) {
    uint32_t g = (n + rows_per_wg - 1) / rows_per_wg;
    const uint32_t cap = g_grid_cap ? g_grid_cap : cap_default;
    return g < cap ? g : cap;
}

constexpr int R_Q4 = 2, R_Q8 = 2;

template <bool FUSE>
int launch_q4k(const float *x, const float *up, const uint8_t *w, float *y, uint32_t k, uint32_t n, hipStream_t s) {
    const uint64_t rb = (uint64_t)k / QK_K * Q4K_BYTES;
    const uint32_t P = k / 64;
    if (P <= 64) {
        hipLaunchKernelGGL((k_q4k_m1<1, 4, R_Q4, FUSE>), dim3(grid_for(n, 4 * R_Q4, 1024)), dim3(256), 0, s, x, up, w,
                           y, k, n, rb);
    } else if (P <= 128) {
        hipLaunchKernelGGL((k_q4k_m1<2, 1, R_Q4, FUSE>), dim3(grid_for(n, R_Q4, 2048)), dim3(128), 0, s, x, up, w, y,
                           k, n, rb);
    } else if (P <= 192) {
        hipLaunchKernelGGL((k_q4k_m1<3, 1, R_Q4, FUSE>), dim3(grid_for(n, R_Q4, 2048)), dim3(192), 0, s, x, up, w, y,
                           k, n, rb);
    } else {
        hipLaunchKernelGGL((k_q4k_m1<4, 1, R_Q4, FUSE>), dim3(grid_for(n, R_Q4, 2048)), dim3(256), 0, s, x, up, w, y,
                           k, n, rb);
    }
    return after_launch("proj_q4k_m1", s);
}

int launch_q80(const float *x, const uint8_t *w, float *y, uint32_t k, uint32_t n, hipStream_t s) {
    const uint64_t rb = (uint64_t)k / QK8_0 * Q80_BYTES;
    const uint32_t P = k / 64;
    if (P <= 64) {
        hipLaunchKernelGGL((k_q80_m1<1, 4, R_Q8>), dim3(grid_for(n, 4 * R_Q8, 1024)), dim3(256), 0, s, x, w, y, k, n,
                           rb);
    } else if (P <= 128) {
        hipLaunchKernelGGL((k_q80_m1<2, 1, R_Q8>), dim3(grid_for(n, R_Q8, 2048)), dim3(128), 0, s, x, w, y, k, n, rb);
    } else if (P <= 192) {
        hipLaunchKernelGGL((k_q80_m1<3, 1, R_Q8>), dim3(grid_for(n, R_Q8, 2048)), dim3(192), 0, s, x, w, y, k, n, rb);
    } else {
        hipLaunchKernelGGL((k_q80_m1<4, 1, R_Q8>), dim3(grid_for(n, R_Q8, 2048)), dim3(256), 0, s, x, w, y, k, n, rb);
    }
    return after_launch("proj_q8_0_m1", s);
}

// Shared front end of every quantized M=1 entry point.
int proj_quant(const float *x, const float *up, const void *w, float *c, uint32_t k, uint32_t n, int dtype,
               uint32_t expert_offset, void *stream, const char *name) {
    clear_error();
    if (n == 0) return LG_OK;  // the reference dispatches zero workgroups
    LG_REQUIRE(x && w && c, "%s: null pointer (x=%p w=%p c=%p)", name, (const void *)x, w, (void *)c);
    LG_REQUIRE(dtype == LG_Q4_K || dtype == LG_Q8_0 || dtype == LG_F32, "%s: unsupported weight dtype %d", name,
               dtype);
    hipStream_t s = (hipStream_t)stream;
    if (k == 0) {  // empty sum: c = 0
        LG_EXTENT(c, (uint64_t)n * 4, name);
        LG_HIP_TRY(hipMemsetAsync(c, 0, (uint64_t)n * 4, s));
        return after_launch(name, s);
    }
    const bool fuse = up != nullptr;
    if (dtype != LG_Q4_K) expert_offset = 0;  // src/target.rs:1115-1138 ignore it for Q8_0/F32
    const uint64_t elems = (uint64_t)expert_offset + (uint64_t)n * k;
    LG_EXTENT(x, (uint64_t)k * 4, name);
    if (fuse) LG_EXTENT(up, (uint64_t)k * 4, name);
    LG_EXTENT(c, (uint64_t)n * 4, name);
    LG_EXTENT(w, tensor_bytes(dtype, elems), name);

    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const bool vec_ok = aligned16(x) && (!fuse || aligned16(up)) && k % QK_K == 0 && k <= M1_MAX_K;
    if (dtype == LG_Q4_K && vec_ok && expert_offset % QK_K == 0) {
        const uint8_t *wbase = wb + (uint64_t)expert_offset / QK_K * Q4K_BYTES;
        if (aligned16(wbase))
            return fuse ? launch_q4k<true>(x, up, wbase, c, k, n, s) : launch_q4k<false>(x, nullptr, wbase, c, k, n, s);
    }
    if (dtype == LG_Q8_0 && vec_ok && !fuse && aligned16(wb)) return launch_q80(x, wb, c, k, n, s);
    if (dtype == LG_F32 && !fuse) {
        hipLaunchKernelGGL(k_f32_rows, dim3((n + 3) / 4), dim3(256), 0, s, x, reinterpret_cast<const float *>(w), c, k,
                           n, (int)(aligned16(x) && aligned16(w) && k % 4 == 0));
        return after_launch(name, s);
    }
    if (fuse)
        hipLaunchKernelGGL(k_generic_m1<true>, dim3((n + 3) / 4), dim3(256), 0, s, x, up, w, c, k, n, dtype,
                           (uint64_t)expert_offset);
    else
        hipLaunchKernelGGL(k_generic_m1<false>, dim3((n + 3) / 4), dim3(256), 0, s, x, nullptr, w, c, k, n, dtype,
                           (uint64_t)expert_offset);
    return after_launch(name, s);
}

}  // namespace

extern "C" {

int lg_dispatch_proj_quant(const float *x, const void *w, float *c, uint32_t k, uint32_t n, int dtype,
                           void *stream) {
    return proj_quant(x, nullptr, w, c, k, n, dtype, 0, stream, "lg_dispatch_proj_quant");
}

int lg_dispatch_proj_quant_expert(const float *x, const void *w, float *c, uint32_t k, uint32_t n, int dtype,
                                  uint32_t expert_offset, void *stream) {
    return proj_quant(x, nullptr, w, c, k, n, dtype, expert_offset, stream, "lg_dispatch_proj_quant_expert");
}

int lg_dispatch_silu_mul_proj_quant(const float *gate, const float *up, const void *w, float *c, uint32_t k,
                                    uint32_t n, int dtype, void *stream) {
    if (!up && n) return fail(LG_EINVAL, "lg_dispatch_silu_mul_proj_quant: null up");
    return proj_quant(gate, up, w, c, k, n, dtype, 0, stream, "lg_dispatch_silu_mul_proj_quant");
}

int lg_dispatch_proj_row(const float *x, const float *w, float *c, uint32_t k, uint32_t n, uint32_t row_major,
                         void *stream) {
    clear_error();
    if (n == 0) return LG_OK;
    LG_REQUIRE(x && w && c, "lg_dispatch_proj_row: null pointer");
    if (!row_major) return proj_quant(x, nullptr, w, c, k, n, LG_F32, 0, stream, "lg_dispatch_proj_row");
    hipStream_t s = (hipStream_t)stream;
    LG_EXTENT(x, (uint64_t)k * 4, "lg_dispatch_proj_row x");
    LG_EXTENT(w, (uint64_t)k * n * 4, "lg_dispatch_proj_row w");
    LG_EXTENT(c, (uint64_t)n * 4, "lg_dispatch_proj_row c");
    hipLaunchKernelGGL(k_f32_cols, dim3((n + 255) / 256), dim3(256), 0, s, x, w, c, k, n);
    return after_launch("lg_dispatch_proj_row", s);
}

int lg_dispatch_proj(const float *x, const float *w, float *c, uint32_t k, uint32_t n, void *stream) {
    return lg_dispatch_proj_row(x, w, c, k, n, 0, stream);
}

int lg_dispatch_proj_read(const float *x, const float *w, uint32_t k, uint32_t n, float *out, void *stream) {
    clear_error();
    if (n == 0) return LG_OK;
    LG_REQUIRE(out, "lg_dispatch_proj_read: null out");
    float *tmp = nullptr;
    LG_HIP_TRY(hipMalloc(&tmp, (uint64_t)n * 4));
    int st = lg_dispatch_proj_row(x, w, tmp, k, n, 0, stream);
    if (st == LG_OK) {
        hipError_t e = hipMemcpyAsync(out, tmp, (uint64_t)n * 4, hipMemcpyDeviceToHost, (hipStream_t)stream);
        if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
        if (e != hipSuccess) st = fail(LG_EHIP, "lg_dispatch_proj_read: %s", hipGetErrorString(e));
    }
    (void)hipFree(tmp);
    return st;
}

int lg_dispatch_activation(const float *gate, const float *up, float *h, uint32_t n, void *stream) {
    clear_error();
    if (n == 0) return LG_OK;
    LG_REQUIRE(gate && up && h, "lg_dispatch_activation: null pointer");
    LG_EXTENT(gate, (uint64_t)n * 4, "lg_dispatch_activation gate");
    LG_EXTENT(up, (uint64_t)n * 4, "lg_dispatch_activation up");
    LG_EXTENT(h, (uint64_t)n * 4, "lg_dispatch_activation h");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_activation, dim3((n + 255) / 256), dim3(256), 0, s, gate, up, h, n);
    return after_launch("lg_dispatch_activation", s);
}

// Upper bound on workgroups of the M=1 quantized kernels (0 = automatic).  A
// tuning hook for launch-shape sweeps; results do not depend on it.
int lg_set_m1_grid_cap(uint32_t cap) {
    g_grid_cap = cap;
    return LG_OK;
}

}  // extern "C"
