// Small-M products (block verify, m <= 64 activation rows): lg_dispatch_proj_quant_batch.
// Replaces kernels/matmul.comp (never dispatched by the reference) with bf16 MFMA
// tiles on gfx950 (v_mfma_f32_16x16x32_bf16: D[16x16] += A[16x32] * B[32x16]).
//
//   A = activations: 16 rows (tokens) x 32 k (one 32-element sub-block).  f32
//       activations are split exactly into three bf16 parts x = x0 + x1 + x2 (each
//       the nearest bf16 of what the previous parts leave: together all 24
//       significant bits, so the products are f32-grade); bf16 activations are one
//       part.  Each workgroup builds the fragments of its slice of k straight from
//       the activations, with the per-sub-block sums X, in LDS.
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
//
// Work split (split-K): workgroup (blockIdx.x, blockIdx.y) = 64*RT output rows (RT
// 16-row tiles per wavefront) x slice blockIdx.y of k (CH chunks of 256 elements:
// one Q4_K super-block or eight Q8_0 blocks per row and chunk).  With one slice
// the workgroup writes the result; otherwise each writes its slice's partial sums
// and the last workgroup of a row group to finish (a per-row-group arrival counter,
// reset by that workgroup) adds the slices in slice order: the result does not
// depend on which workgroup finishes last.  A single plain product of many rounds of
// workgroups (a vocab-sized head) instead has its slices only store their partial
// sums, and a second launch (k_mm_sum) adds them in the same order, so no workgroup
// waits for its arrival.
#include <mutex>
#include <vector>

#include "lg_common.hpp"

namespace {

using namespace lg;

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32): a low, b high.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// a[j] = 16 d sc_j for the 8 sub-blocks (the code term's scales).
__device__ __forceinline__ void q4k_scales_a(uint32_t s0, uint32_t s2, float d16, float (&a)[8]) {
    const uint32_t sl = s0 & 0x3F3F3F3Fu, sh = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const float scf[8] = {ubyte_f<0>(sl), ubyte_f<1>(sl), ubyte_f<2>(sl), ubyte_f<3>(sl),
                          ubyte_f<0>(sh), ubyte_f<1>(sh), ubyte_f<2>(sh), ubyte_f<3>(sh)};
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = d16 * scf[j];
}

// The X coefficients -(16 d sc_j + dmin m_j) of sub-blocks j = g and g + 4 (g < 4, a
// lane's k-group): the B operand of the f32 product that adds the min terms.
__device__ __forceinline__ void q4k_min_coef(uint32_t s0, uint32_t s1, uint32_t s2, float d16, float dmin,
                                             uint32_t g, float &c_lo, float &c_hi) {
    const uint32_t b0 = s0 >> (8 * g), b1 = s1 >> (8 * g), b2 = s2 >> (8 * g);
    const uint32_t sc_lo = b0 & 63u, m_lo = b1 & 63u;
    const uint32_t sc_hi = (b2 & 15u) | (((b0 >> 6) & 3u) << 4), m_hi = ((b2 >> 4) & 15u) | (((b1 >> 6) & 3u) << 4);
    c_lo = -__builtin_fmaf(dmin, (float)m_lo, d16 * (float)sc_lo);
    c_hi = -__builtin_fmaf(dmin, (float)m_hi, d16 * (float)sc_hi);
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

// A launch runs up to MM_JOBS products that share the activations x (and k): job
// j owns workgroup columns g0 .. g0 + ceil(n / (64 RT)) - 1 and writes out[m][n]
// (plus res, when given), using `part` for its slice partial sums.  Arrival
// counters are indexed by the global workgroup column.
//
// RMSNorm folded into the products (kernels/rmsnorm.comp:23-34), for the draft's
// residual stream:
//  * a producing job (ss != null, not GLU) also writes y = out * yw[row] (the next
//    norm's weight applied) and, per token, the sum of out^2 over each workgroup
//    column's rows: ss[token * columns + column];
//  * a consuming launch (NORM kernels) takes such a y as its activations and scales
//    the results of tokens t >= rs_tok0 by (sum_p rs_ss[(t - rs_tok0) * rs_cols + p]
//    / k + rs_eps)^-1/2, so W (x w / rms) = (W (x w)) / rms replaces the norm launch.
//    The workgroup that finishes a column computes the scales, with the slices'
//    partial sums in flight.
constexpr int MM_JOBS = 4;
constexpr uint32_t MM_SS_LOADS = 4;  // partial sums a consuming lane loads (per-token capacity 4 * 16 / TT)
struct MmJob {
    const uint8_t *w;
    float *out;
    const float *res;
    float *part;
    float *y;
    const float *yw;
    float *ss;
    uint32_t n, g0;
    const float *qkw;  // QK-norm weights (heads of 128 rows, RT = 2), or null
};
struct MmJobs {
    MmJob j[MM_JOBS];
    uint32_t count;
    uint32_t tiled;  // Q4_K weights in LG_Q4_K_T16 tiles
    const float *rs_ss;
    uint32_t rs_cols, rs_tok0;
    float rs_eps;
    const float *rope;  // the QK jobs' rotation table: [token][cos 64 | sin 64]
    float qk_eps;
};
// GLU launches pair two products of n rows each (gate: job 0, up: job 1): every
// workgroup column covers the same 32*RT rows of both, wavefronts 0-1 the gate
// rows and 2-3 the up rows, and writes only silu(gate) * up, to job 0's output.
#define MM_JOB_SELECT                                                                     \
    uint32_t J_ = 0;                                                                      \
    if constexpr (GLU) J_ = threadIdx.x >> 7;                                             \
    else _Pragma("unroll") for (int j_ = 1; j_ < MM_JOBS; j_++) if ((uint32_t)j_ < jobs.count && \
                                                              blockIdx.x >= jobs.j[j_].g0) J_ = j_; \
    const uint8_t *w = jobs.j[J_].w;                                                      \
    float *out = jobs.j[J_].out;                                                          \
    const float *res = jobs.j[J_].res;                                                    \
    float *part = jobs.j[J_].part;                                                        \
    const uint32_t n = jobs.j[J_].n, bx = blockIdx.x - jobs.j[J_].g0

__device__ __forceinline__ float silu_mul(float g, float u) {
    // kernels/activation.comp:21-28: silu(g) * up, silu(x) = x * (1 / (1 + exp(-x)))
    return g * (1.0f / (1.0f + expf(-g))) * u;
}

// The activation fragments of a slice, built in LDS by the whole workgroup.
//   lf[((t*SB + jj)*PARTS + p)*64 + lane] : part p of the A operand of token tile t,
//                                          sub-block jj of the slice
//   lx[(t*SB + jj)*16 + token]            : X, the sum of the 32 activations
// A unit is (token tile t, sub-block jj, k-group kg, token tl): 8 activations.
// load() issues the global loads (branch-free: tokens past m and sub-blocks past k
// read a valid element and are zeroed at store()), store() splits and writes.
template <int TT, int PARTS, int CH, bool FUSE = false>
struct Frags {
    static constexpr int SB = 8 * CH;
    static constexpr int PER = TT * 16 * SB * 4 / 256;  // units per thread
    float4 r[PER][2];                                    // f32 activations (FUSE: gate)
    float4 ru[FUSE ? PER : 1][2];                        // FUSE: up
    uint4 h[PER];                                        // bf16 activations
    __device__ __forceinline__ static void unit(int i, uint32_t &t, uint32_t &jj, uint32_t &kg, uint32_t &tl) {
        const uint32_t u = i * 256 + threadIdx.x;
        tl = u & 15u;
        kg = (u >> 4) & 3u;
        jj = (u >> 6) % SB;
        t = u / (64 * SB);
    }

    __device__ __forceinline__ void load(const void *__restrict__ x, const float *__restrict__ up, uint32_t m,
                                         uint32_t k, uint32_t sb0) {
        const uint32_t nsb = k / 32;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            uint32_t t, jj, kg, tl;
            unit(i, t, jj, kg, tl);
            const uint32_t tok = t * 16 + tl < m ? t * 16 + tl : m - 1;
            const uint32_t sb = sb0 + jj < nsb ? sb0 + jj : nsb - 1;
            const uint64_t e = (uint64_t)tok * k + 32 * sb + 8 * kg;
            if constexpr (PARTS == 1) {
                h[i] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + e);
            } else {
                const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + e);
                r[i][0] = p[0];
                r[i][1] = p[1];
                if constexpr (FUSE) {
                    const float4 *pu = reinterpret_cast<const float4 *>(up + e);
                    ru[i][0] = pu[0];
                    ru[i][1] = pu[1];
                }
            }
        }
    }

    __device__ __forceinline__ void store(uint4 *lf, float *lx, uint32_t m, uint32_t k, uint32_t sb0) const {
        const uint32_t nsb = k / 32;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            uint32_t t, jj, kg, tl;
            unit(i, t, jj, kg, tl);
            const bool valid = t * 16 + tl < m && sb0 + jj < nsb;
            float sum;
            uint32_t wd[PARTS][4];  // fragment slots 0..7 hold activations 0,2,1,3,4,6,5,7
            if constexpr (PARTS == 1) {
                const uint32_t raw[4] = {h[i].x, h[i].y, h[i].z, h[i].w};  // activations 0..7, two per word
                // slot pairs (0,1), (2,3), (4,5), (6,7) hold activations (0,2), (1,3), (4,6), (5,7)
                const uint32_t w0 = (raw[0] & 0xFFFFu) | (raw[1] << 16), w1 = (raw[0] >> 16) | (raw[1] & 0xFFFF0000u);
                const uint32_t w2 = (raw[2] & 0xFFFFu) | (raw[3] << 16), w3 = (raw[2] >> 16) | (raw[3] & 0xFFFF0000u);
                wd[0][0] = valid ? w0 : 0u;
                wd[0][1] = valid ? w1 : 0u;
                wd[0][2] = valid ? w2 : 0u;
                wd[0][3] = valid ? w3 : 0u;
                float v[8];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    v[2 * q] = __uint_as_float(wd[0][q] << 16);
                    v[2 * q + 1] = __uint_as_float(wd[0][q] & 0xFFFF0000u);
                }
                sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
            } else {
                float f[8] = {r[i][0].x, r[i][0].y, r[i][0].z, r[i][0].w, r[i][1].x, r[i][1].y, r[i][1].z, r[i][1].w};
                if constexpr (FUSE) {  // kernels/activation.comp:21-28
                    const float u[8] = {ru[i][0].x, ru[i][0].y, ru[i][0].z, ru[i][0].w,
                                        ru[i][1].x, ru[i][1].y, ru[i][1].z, ru[i][1].w};
#pragma unroll
                    for (int q = 0; q < 8; q++) f[q] = silu_mul(f[q], u[q]);
                }
#pragma unroll
                for (int q = 0; q < 8; q++) f[q] = valid ? f[q] : 0.0f;
                sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
                // pairs in slot order: (0,2) (1,3) (4,6) (5,7); each part is the nearest
                // bf16 of what the earlier parts leave (exact residuals)
                float lo[4] = {f[0], f[1], f[4], f[5]}, hi[4] = {f[2], f[3], f[6], f[7]};
#pragma unroll
                for (int p = 0; p < PARTS; p++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        wd[p][q] = pk_bf16(lo[q], hi[q]);
                        if (p + 1 < PARTS) {
                            lo[q] -= __uint_as_float(wd[p][q] << 16);
                            hi[q] -= __uint_as_float(wd[p][q] & 0xFFFF0000u);
                        }
                    }
            }
#pragma unroll
            for (int p = 0; p < PARTS; p++)
                lf[((t * SB + jj) * PARTS + p) * 64 + kg * 16 + tl] = make_uint4(wd[p][0], wd[p][1], wd[p][2], wd[p][3]);
            sum += __shfl_xor(sum, 16);  // the 4 k-groups of this token and sub-block
            sum += __shfl_xor(sum, 32);
            if (kg == 0) lx[(t * SB + jj) * 16 + tl] = sum;
        }
    }
};

// NORM: token threadIdx.x / LT of the launch (LT = 16 / TT lanes per token) takes its
// partial sums p = sub, sub + LT, ... (branch-free: slots past the columns and tokens
// without a scale read a valid slot, dropped in rs_store).
template <int TT>
__device__ __forceinline__ void ss_load(float (&ssv)[MM_SS_LOADS], const MmJobs &jobs, uint32_t m) {
    constexpr uint32_t LT = 16 / TT;
    const uint32_t tok = threadIdx.x / LT, sub = threadIdx.x % LT, cols = jobs.rs_cols, tok0 = jobs.rs_tok0;
    const uint32_t rows = m > tok0 ? m - tok0 : 1u;
    const uint32_t r = tok >= tok0 && tok - tok0 < rows ? tok - tok0 : 0u;
#pragma unroll
    for (uint32_t j = 0; j < MM_SS_LOADS; j++) {
        const uint32_t p = sub + LT * j;
        ssv[j] = jobs.rs_ss[(uint64_t)r * cols + (p < cols ? p : cols - 1)];
    }
}

// NORM: rsl[t] = (sum of token t's partials / k + eps)^-1/2, or 1 for tokens below
// tok0 (and past m).  The lanes of a token add their slots in slot order, then meet
// in DPP steps within their 16-lane row: xor 1, xor 2 (quad_perm), the half-row
// mirror (lane i and 7 - i of each 8) and, for 16 lanes per token, the row mirror
// (i and 15 - i).  Every lane of the token ends with the sum.
template <int TT>
__device__ __forceinline__ void rs_store(const float (&ssv)[MM_SS_LOADS], float *rsl, const MmJobs &jobs, uint32_t m,
                                         uint32_t k) {
    constexpr uint32_t LT = 16 / TT;
    const uint32_t tok = threadIdx.x / LT, sub = threadIdx.x % LT, tok0 = jobs.rs_tok0;
    float s = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < MM_SS_LOADS; j++) s += sub + LT * j < jobs.rs_cols ? ssv[j] : 0.0f;
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x141, 0xF, 0xF, false));  // row_half_mirror
    if constexpr (LT == 16)
        s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x140, 0xF, 0xF, false));  // row_mirror
    if (sub == 0) rsl[tok] = tok >= tok0 && tok < m ? 1.0f / sqrtf(s / (float)k + jobs.rs_eps) : 1.0f;
}

// The workgroup's results: the output itself (one slice), or its slice's partial
// sums and, in the last workgroup of the row group to finish, their ordered sum;
// scaled per token by rsl (NORM), and with y and the column's sums of squares when
// ssout is given (not GLU).
// QK-norm and NeoX RoPE of whole heads (kernels/qk_norm_rope.comp:23-67,
// src/dflash.rs:898-904) in the workgroup that finishes a column: with RT = 2 a
// column is 128 rows, one head, and wavefront w holds dims 32 w + 16 i + (lane & 15)
// (tile i).  Per token, the head's sum of squares meets in LDS in wavefront order,
// and the rotation partner of dim d (d + 64 or d - 64) is read through LDS from
// wavefront w ^ 2.  rope: per token, the cosines then the sines of its 64 angles.
template <int TT>
__device__ __forceinline__ void qk_head(float (&v)[2][TT][4], const float *__restrict__ w,
                                        const float *__restrict__ rope, float eps, uint32_t m, float *xch) {
    __shared__ float ssq[4][TT * 16];
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4, wave = threadIdx.x >> 6;
    float wd[2];
#pragma unroll
    for (int i = 0; i < 2; i++) wd[i] = w[32 * wave + 16 * i + (l & 15u)];
    __syncthreads();  // every wavefront is past its products: xch (the fragment LDS) is free
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float q = row16_sum(__builtin_fmaf(v[1][t][r], v[1][t][r], v[0][t][r] * v[0][t][r]));
            if ((l & 15u) == 0) ssq[wave][t * 16 + 4 * kg + r] = q;
        }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t tok = t * 16 + 4 * kg + r;
            const float tot = ((ssq[0][tok] + ssq[1][tok]) + ssq[2][tok]) + ssq[3][tok];
            const float rms = 1.0f / sqrtf(tot / 128.0f + eps);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                v[i][t][r] = v[i][t][r] * wd[i] * rms;
                xch[((wave * 2 + i) * TT + t) * 256 + r * 64 + l] = v[i][t][r];
            }
        }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t tok = t * 16 + 4 * kg + r, tc = tok < m ? tok : m - 1;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float p = xch[(((wave ^ 2u) * 2 + i) * TT + t) * 256 + r * 64 + l];
                const uint32_t dm = 32 * (wave & 1u) + 16 * i + (l & 15u);
                const float c = rope[(uint64_t)tc * 128 + dm], sn = rope[(uint64_t)tc * 128 + 64 + dm];
                v[i][t][r] = wave < 2 ? v[i][t][r] * c - p * sn : v[i][t][r] * c + p * sn;
            }
        }
}

template <int TT, int RT, bool GLU, bool NORM>
__device__ __forceinline__ void finish(const float (&acc)[RT][TT][4], float *out, const float *res, float *part,
                                       uint32_t *cnt, uint32_t rt0, uint32_t m, uint32_t n, float *xch,
                                       const MmJobs &jobs, uint32_t k, float *y, const float *yw, float *ssout,
                                       uint32_t bx, const float *qkw) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
    const uint32_t S = gridDim.y, s = blockIdx.y;
    const uint64_t mn = (uint64_t)m * n;
    if (S > 1) {
        float *ps = part + s * mn;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint32_t row = (rt0 + i) * 16 + (l & 15u);
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t tok = t * 16 + 4 * kg + r;
                    if (row < n && tok < m)
                        __hip_atomic_store(ps + (uint64_t)tok * n + row, acc[i][t][r], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
        }
        // the last workgroup of the column to arrive adds the slices
        __shared__ uint32_t last;
        if (!arrive_last(&cnt[blockIdx.x], S, &last)) return;
    }
    // NORM: the partial sums of squares behind the token scales, loaded with the
    // slices' partial sums (only the workgroup that finishes a column reads them)
    float ssv[MM_SS_LOADS];
    if constexpr (NORM) ss_load<TT>(ssv, jobs, m);
    // Slices are added in slice order (the sum does not depend on arrival order);
    // the loads of G slices for all RT row tiles are in flight together.
    constexpr uint32_t G = RT * TT >= 16 ? 1u : 16u / (RT * TT);
    float v[RT][TT][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) v[i][t][r] = S > 1 ? 0.0f : acc[i][t][r];
    for (uint32_t q0 = 0; q0 < (S > 1 ? S : 0u); q0 += G) {
        float pv[G][RT][TT][4];
#pragma unroll
        for (uint32_t g = 0; g < G; g++) {
            const uint32_t q = q0 + g < S ? q0 + g : S - 1;
#pragma unroll
            for (int i = 0; i < RT; i++) {
                const uint32_t row = (rt0 + i) * 16 + (l & 15u);
                const uint32_t rowc = row < n ? row : n - 1;
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const uint32_t tok = t * 16 + 4 * kg + r;
                        pv[g][i][t][r] = __hip_atomic_load(part + q * mn + (uint64_t)(tok < m ? tok : m - 1) * n + rowc,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
            }
        }
#pragma unroll
        for (uint32_t g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) v[i][t][r] += q0 + g < S ? pv[g][i][t][r] : 0.0f;
    }
    if constexpr (NORM) {
        __shared__ float rsl[TT * 16];
        rs_store<TT>(ssv, rsl, jobs, m, k);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) v[i][t][r] *= rsl[t * 16 + 4 * kg + r];
    }
    if constexpr (!GLU && RT == 2)
        if (qkw) qk_head<TT>(v, qkw, jobs.rope, jobs.qk_eps, m, xch);  // uniform over the workgroup
    if constexpr (GLU) {
        // wavefronts 2-3 pass their up sums through LDS (`xch`, free once every
        // wavefront is past its products) to wavefronts 0-1, which hold the gate sums
        // of the same rows and tokens (kernels/activation.comp:21-28)
        const uint32_t wave = threadIdx.x >> 6;
        __syncthreads();
        if (wave >= 2) {
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) xch[(((wave - 2) * RT + i) * TT + t) * 256 + r * 64 + l] = v[i][t][r];
        }
        __syncthreads();
        if (wave >= 2) return;
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    v[i][t][r] = silu_mul(v[i][t][r], xch[((wave * RT + i) * TT + t) * 256 + r * 64 + l]);
    }
    float sq[TT][4];  // ssout: this lane's sum of out^2 over its rows, per token
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) sq[t][r] = 0.0f;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint32_t row = (rt0 + i) * 16 + (l & 15u);
        if (row >= n) continue;
        const float wy = !GLU && ssout ? yw[row] : 0.0f;
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = t * 16 + 4 * kg + r;
                if (tok < m) {
                    const uint64_t o = (uint64_t)tok * n + row;
                    const float ov = res ? res[o] + v[i][t][r] : v[i][t][r];
                    out[o] = ov;
                    if (!GLU && ssout) {
                        y[o] = ov * wy;
                        sq[t][r] = __builtin_fmaf(ov, ov, sq[t][r]);
                    }
                }
            }
    }
    if constexpr (!GLU) {
        if (ssout) {  // uniform: every wavefront of the workgroup is here
            // the wavefront's 16 rows per tile (the lanes of a k-group) in a DPP
            // reduction, then the four wavefronts in wavefront order
            __shared__ float ssl[4][TT * 16];
            const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float rsum = row16_sum(sq[t][r]);
                    if ((l & 15u) == 0) ssl[wave][t * 16 + 4 * kg + r] = rsum;
                }
            __syncthreads();
            const uint32_t tk = threadIdx.x, cols = (n + 64 * RT - 1) / (64 * RT);
            if (tk < TT * 16 && tk < m) ssout[(uint64_t)tk * cols + bx] = (ssl[0][tk] + ssl[1][tk]) + (ssl[2][tk] + ssl[3][tk]);
        }
    }
}

// A split-k workgroup of a wide launch: slice blockIdx.y's partial sums of the
// wavefront's rows, part[slice][token][row], with plain stores; the launch after it
// (k_mm_sum) adds the slices, so the workgroup leaves as soon as they are issued.
template <int TT, int RT>
__device__ __forceinline__ void store_slice(const float (&acc)[RT][TT][4], float *part, uint32_t rt0, uint32_t m,
                                            uint32_t n) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
    float *ps = part + (uint64_t)blockIdx.y * m * n;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint32_t row = (rt0 + i) * 16 + (l & 15u);
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = t * 16 + 4 * kg + r;
                if (row < n && tok < m) ps[(uint64_t)tok * n + row] = acc[i][t][r];
            }
    }
}

// The finishing launch of a wide split-k product (one plain product: no residual, no
// epilogue).  Workgroup (c, t) covers rows 64c .. 64c+63 and tokens 16t .. 16t+15:
// thread (token threadIdx.x / 16, quad threadIdx.x % 16) adds rows 4 quad .. 4 quad + 3
// of the S slices in slice order, with the loads of SUM_MAXS slices in flight at once.
// V4: rows in float4 (n % 4 == 0 and a 16-byte aligned output).
constexpr uint32_t SUM_ROWS = 64, SUM_MAXS = 16;
// Launches of at least this many workgroups (about four rounds of the resident ones)
// finish in k_mm_sum: there every workgroup's wait for its arrival would be paid in
// each round.  Smaller ones finish in the kernel, where the last workgroups' reads of
// the partial sums overlap other columns' products (a separate finishing launch cost
// those 5-6 us per product on the draft's shapes).
constexpr uint64_t WIDE_MIN_WGS = 4096;
template <bool V4>
__global__ __launch_bounds__(256) void k_mm_sum(const float *__restrict__ part, float *__restrict__ out, uint32_t m,
                                                uint32_t n, uint32_t S) {
    const uint32_t tl = threadIdx.x >> 4, qd = threadIdx.x & 15u;
    const uint32_t tok = 16 * blockIdx.y + tl, row0 = blockIdx.x * SUM_ROWS + 4 * qd;
    const uint64_t mn = (uint64_t)m * n;
    const uint32_t tc = tok < m ? tok : m - 1;  // branch-free loads: rows and tokens past the end are clamped
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t q0 = 0; q0 < S; q0 += SUM_MAXS) {
        float4 pv[SUM_MAXS];
#pragma unroll
        for (uint32_t g = 0; g < SUM_MAXS; g++) {
            const uint32_t q = q0 + g < S ? q0 + g : S - 1;
            const float *src = part + q * mn + (uint64_t)tc * n;
            if constexpr (V4) {
                pv[g] = *reinterpret_cast<const float4 *>(src + (row0 < n ? row0 : n - 4));
            } else {
                float e4[4];
#pragma unroll
                for (int e = 0; e < 4; e++) e4[e] = src[row0 + e < n ? row0 + e : n - 1];
                pv[g] = make_float4(e4[0], e4[1], e4[2], e4[3]);
            }
        }
#pragma unroll
        for (uint32_t g = 0; g < SUM_MAXS; g++)
            if (q0 + g < S) {
                v[0] += pv[g].x;
                v[1] += pv[g].y;
                v[2] += pv[g].z;
                v[3] += pv[g].w;
            }
    }
    if (tok >= m) return;
    const uint64_t o = (uint64_t)tok * n + row0;
    if (V4 && row0 < n) {
        *reinterpret_cast<float4 *>(out + o) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (row0 + e < n) out[o + e] = v[e];
    }
}

// Q4_K.  Wavefront w owns row tiles (4*blockIdx.x + w)*RT .. +RT-1; each activation
// fragment read from LDS serves all RT tiles.  Order of work: the activation loads,
// every weight load of the slice (branch-free: rows past n and blocks past k read
// row n-1 / the last block and are never used), the fragment build while the
// weights are in flight, then the products.
template <int TT, int PARTS, int CH, int RT, bool FUSE, bool GLU, bool NORM, bool WIDE = false>
__global__ __launch_bounds__(256) void k_q4k_mm(const void *__restrict__ x, const float *__restrict__ up, MmJobs jobs,
                                                uint32_t *cnt, uint32_t m, uint32_t k, uint64_t row_bytes) {
    MM_JOB_SELECT;
    constexpr int SB = 8 * CH;
    __shared__ uint4 lf[TT * SB * PARTS * 64];
    __shared__ float lx[TT * SB * 16];
    const uint32_t l = threadIdx.x & 63u, wave = threadIdx.x >> 6, kg = l >> 4;
    const uint32_t rt0 = (GLU ? bx * 2 + (wave & 1u) : bx * 4 + wave) * RT;
    const uint32_t nb = k / QK_K, b0 = blockIdx.y * CH;
    Frags<TT, PARTS, CH, FUSE> fr;
    fr.load(x, up, m, k, 8 * b0);
    uint4 hd[RT][CH];
    uint2 qv[RT][CH][4];
    if (jobs.tiled) {  // 2304-byte tiles: each load is 512 (quants) or 256 (headers) contiguous bytes
        const uint32_t ntiles = (n + 15) / 16;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint32_t t = rt0 + i < ntiles ? rt0 + i : ntiles - 1;
#pragma unroll
            for (int cb = 0; cb < CH; cb++) {
                const uint8_t *tb = w + ((uint64_t)t * nb + (b0 + cb < nb ? b0 + cb : nb - 1)) * Q4K_TILE;
                hd[i][cb] = *reinterpret_cast<const uint4 *>(tb + 16 * (l & 15u));
#pragma unroll
                for (int g = 0; g < 4; g++) qv[i][cb][g] = *reinterpret_cast<const uint2 *>(tb + 256 + 512 * g + 8 * l);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint32_t row = (rt0 + i) * 16 + (l & 15u);
            const uint8_t *wr = w + (uint64_t)(row < n ? row : n - 1) * row_bytes;
#pragma unroll
            for (int cb = 0; cb < CH; cb++) {
                const uint8_t *blk = wr + (uint64_t)(b0 + cb < nb ? b0 + cb : nb - 1) * Q4K_BYTES;
                hd[i][cb] = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
                for (int g = 0; g < 4; g++) qv[i][cb][g] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * g + 8 * kg);
            }
        }
    }
    asm volatile("" ::: "memory");  // keep the weight loads issued ahead of the fragment build
    fr.store(lf, lx, m, k, 8 * b0);
    __syncthreads();
    float acc[RT][TT][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][t][r] = 0.0f;
#pragma unroll
    for (int cb = 0; cb < CH; cb++) {
        if (b0 + cb >= nb) continue;  // uniform: past the end of k
        // code terms a_j D_j per sub-block on the VALU; the super-block's min terms
        // -(a_j + dmin m_j) X_j as two f32 matrix products (k = the 8 sub-blocks)
        // accumulated into acc: A = X[token][sub-block], B = coefficient[sub-block][row]
        float sa[RT][8], cmin[RT][2];
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const float d16 = 16.0f * ref_half(hd[i][cb].x & 0xFFFFu), dmin = ref_half(hd[i][cb].x >> 16);
            q4k_scales_a(hd[i][cb].y, hd[i][cb].w, d16, sa[i]);
            q4k_min_coef(hd[i][cb].y, hd[i][cb].z, hd[i][cb].w, d16, dmin, kg, cmin[i][0], cmin[i][1]);
        }
#pragma unroll
        for (int g = 0; g < 4; g++) {
            bf16x8 blo[RT], bhi[RT];
#pragma unroll
            for (int i = 0; i < RT; i++) q4_codes(qv[i][cb][g].x, qv[i][cb][g].y, blo[i], bhi[i]);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t j = 2 * g + u, jj = cb * 8 + j;
                bf16x8 A[TT][PARTS];
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int p = 0; p < PARTS; p++)
                        A[t][p] = __builtin_bit_cast(bf16x8, lf[((t * SB + jj) * PARTS + p) * 64 + l]);
#pragma unroll
                for (int i = 0; i < RT; i++) {
                    const float a = sa[i][j];
#pragma unroll
                    for (int t = 0; t < TT; t++) {
                        f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int p = 0; p < PARTS; p++)
                            D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t][p], u ? bhi[i] : blo[i], D, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[i][t][r] = __builtin_fmaf(a, D[r], acc[i][t][r]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float x_lo = lx[(t * SB + cb * 8 + kg) * 16 + (l & 15u)];
            const float x_hi = lx[(t * SB + cb * 8 + kg + 4) * 16 + (l & 15u)];
#pragma unroll
            for (int i = 0; i < RT; i++) {
                f32x4 C = {acc[i][t][0], acc[i][t][1], acc[i][t][2], acc[i][t][3]};
                C = __builtin_amdgcn_mfma_f32_16x16x4f32(x_lo, cmin[i][0], C, 0, 0, 0);
                C = __builtin_amdgcn_mfma_f32_16x16x4f32(x_hi, cmin[i][1], C, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[i][t][r] = C[r];
            }
        }
    }
    static_assert(!GLU || 2 * RT * TT * 256 * 4 <= sizeof(lf), "GLU exchange fits in the fragment LDS");
    static_assert(RT != 2 || 8 * TT * 256 * 4 <= sizeof(lf), "the head exchange fits in the fragment LDS");
    if constexpr (WIDE) {  // the slices' sums are added by k_mm_sum
        store_slice<TT, RT>(acc, part, rt0, m, n);
        return;
    }
    finish<TT, RT, GLU, NORM>(acc, out, res, part, cnt, rt0, m, n, reinterpret_cast<float *>(lf), jobs, k,
                              jobs.j[J_].y, jobs.j[J_].yw, jobs.j[J_].ss, bx, jobs.j[J_].qkw);
}

// Q8_0: a chunk is 8 blocks of 34 bytes (2-byte aligned).  Raw rows are staged through
// LDS with 16-byte loads where they fit (see STAGE), else read as 16-bit words.
template <int TT, int PARTS, int CH, int RT, bool FUSE, bool GLU, bool NORM, bool WIDE = false>
__global__ __launch_bounds__(256) void k_q80_mm(const void *__restrict__ x, const float *__restrict__ up, MmJobs jobs,
                                                uint32_t *cnt, uint32_t m, uint32_t k, uint64_t row_bytes) {
    MM_JOB_SELECT;
    constexpr int SB = 8 * CH;
    __shared__ uint4 lf[TT * SB * PARTS * 64];
    __shared__ float lx[TT * SB * 16];
    const uint32_t l = threadIdx.x & 63u, wave = threadIdx.x >> 6, kg = l >> 4;
    const uint32_t rt0 = (GLU ? bx * 2 + (wave & 1u) : bx * 4 + wave) * RT;
    const uint32_t nsb = k / 32, sb0 = blockIdx.y * SB;
    // raw rows can be staged through the fragment LDS when the wavefronts' rows fit (not
    // for a gate/up pair, whose halves read different weights: the staging's barrier
    // must be reached by the whole workgroup on one condition)
    constexpr bool STAGE = !GLU && 64u * RT * SB * Q80_BYTES <= sizeof(lf);
    Frags<TT, PARTS, CH, FUSE> fr;
    fr.load(x, up, m, k, sb0);
    uint32_t dq[RT][SB], v0[RT][SB], v1[RT][SB];
    if (jobs.tiled) {  // 4352-byte tiles: one 16-byte load for a row's 8 scales, 512 contiguous bytes per quant load
        const uint32_t ntiles = (n + 15) / 16, nc = k / 256;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint32_t t = rt0 + i < ntiles ? rt0 + i : ntiles - 1;
#pragma unroll
            for (int cc = 0; cc < CH; cc++) {
                const uint32_t c = blockIdx.y * CH + cc;
                const uint8_t *tb = w + ((uint64_t)t * nc + (c < nc ? c : nc - 1)) * Q80_TILE;
                const uint4 sc = *reinterpret_cast<const uint4 *>(tb + 16 * (l & 15u));
                const uint32_t sw[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const uint2 q = *reinterpret_cast<const uint2 *>(tb + 256 + 512 * jj + 8 * l);
                    dq[i][8 * cc + jj] = (sw[jj >> 1] >> (16 * (jj & 1))) & 0xFFFFu;
                    v0[i][8 * cc + jj] = q.x;
                    v1[i][8 * cc + jj] = q.y;
                }
            }
        }
    } else if (STAGE && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 && row_bytes % 16 == 0) {  // uniform
        // Raw rows staged through the fragment LDS (free until the fragments are built):
        // each wavefront reads its 16 RT rows' SB*34 bytes of the slice with 16-byte loads
        // (RP pieces per row), then every lane picks its blocks' scale and quants out of
        // LDS as 16-bit words.  Pieces past the end of a row re-read its last piece.
        constexpr uint32_t RP = SB * Q80_BYTES / 16, NP = 16 * RT * RP, NL = (NP + 63) / 64;
        uint4 *st = lf + wave * NP;
        const uint64_t c0 = (uint64_t)sb0 * Q80_BYTES;
        uint4 pc[NL];
#pragma unroll
        for (uint32_t i = 0; i < NL; i++) {
            const uint32_t e = l + 64 * i < NP ? l + 64 * i : NP - 1;
            const uint32_t r = e / RP, row = rt0 * 16 + r;
            const uint64_t o = c0 + 16 * (e % RP);
            pc[i] = *reinterpret_cast<const uint4 *>(w + (uint64_t)(row < n ? row : n - 1) * row_bytes +
                                                     (o + 16 <= row_bytes ? o : row_bytes - 16));
        }
#pragma unroll
        for (uint32_t i = 0; i < NL; i++)
            if (l + 64 * i < NP) st[l + 64 * i] = pc[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint16_t *sw = reinterpret_cast<const uint16_t *>(st);
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint16_t *sr = sw + (i * 16 + (l & 15u)) * RP * 8;
#pragma unroll
            for (int j = 0; j < SB; j++) {
                const uint16_t *blk = sr + j * (Q80_BYTES / 2);
                const uint16_t *q = blk + 1 + 4 * kg;
                dq[i][j] = blk[0];
                v0[i][j] = q[0] | ((uint32_t)q[1] << 16);
                v1[i][j] = q[2] | ((uint32_t)q[3] << 16);
            }
        }
        __syncthreads();  // every wavefront has its weights: the LDS is free for the fragments
    } else {
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint32_t row = (rt0 + i) * 16 + (l & 15u);
            const uint8_t *wr = w + (uint64_t)(row < n ? row : n - 1) * row_bytes;
#pragma unroll
            for (int j = 0; j < SB; j++) {
                const uint16_t *blk =
                    reinterpret_cast<const uint16_t *>(wr + (uint64_t)(sb0 + j < nsb ? sb0 + j : nsb - 1) * Q80_BYTES);
                const uint16_t *q = blk + 1 + 4 * kg;
                dq[i][j] = blk[0];
                v0[i][j] = q[0] | ((uint32_t)q[1] << 16);
                v1[i][j] = q[2] | ((uint32_t)q[3] << 16);
            }
        }
    }
    asm volatile("" ::: "memory");  // keep the weight loads issued ahead of the fragment build
    fr.store(lf, lx, m, k, sb0);
    __syncthreads();
    float acc[RT][TT][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][t][r] = 0.0f;
#pragma unroll
    for (int j = 0; j < SB; j++) {
        if (sb0 + j >= nsb) continue;  // uniform: past the end of k
        bf16x8 A[TT][PARTS];
        float4 X[TT];
#pragma unroll
        for (int t = 0; t < TT; t++) {
#pragma unroll
            for (int p = 0; p < PARTS; p++)
                A[t][p] = __builtin_bit_cast(bf16x8, lf[((t * SB + j) * PARTS + p) * 64 + l]);
            X[t] = *reinterpret_cast<const float4 *>(lx + (t * SB + j) * 16 + 4 * kg);
        }
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const float d = ref_half(dq[i][j]);
            uint32_t a0, a1, a2, a3;
            q8_codes(v0[i][j], a0, a1);
            q8_codes(v1[i][j], a2, a3);
            const bf16x8 B = as_bf16x8(a0, a1, a2, a3);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int p = 0; p < PARTS; p++) D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t][p], B, D, 0, 0, 0);
                acc[i][t][0] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X[t].x, D[0]), acc[i][t][0]);
                acc[i][t][1] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X[t].y, D[1]), acc[i][t][1]);
                acc[i][t][2] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X[t].z, D[2]), acc[i][t][2]);
                acc[i][t][3] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, X[t].w, D[3]), acc[i][t][3]);
            }
        }
    }
    static_assert(!GLU || 2 * RT * TT * 256 * 4 <= sizeof(lf), "GLU exchange fits in the fragment LDS");
    static_assert(RT != 2 || 8 * TT * 256 * 4 <= sizeof(lf), "the head exchange fits in the fragment LDS");
    if constexpr (WIDE) {  // the slices' sums are added by k_mm_sum
        store_slice<TT, RT>(acc, part, rt0, m, n);
        return;
    }
    finish<TT, RT, GLU, NORM>(acc, out, res, part, cnt, rt0, m, n, reinterpret_cast<float *>(lf), jobs, k,
                              jobs.j[J_].y, jobs.j[J_].yw, jobs.j[J_].ss, bx, jobs.j[J_].qkw);
}

// Fallback for shapes outside the MFMA path (f32 weights, k not a multiple of the
// block, unaligned pointers, k = 0): one wavefront per output row, element-wise
// decode.  c = res + W x when res is given; x = silu(x) * up when up is given.
__global__ __launch_bounds__(256) void k_generic_batch(const void *__restrict__ xv, int x_bf16,
                                                       const float *__restrict__ up, const void *__restrict__ wv,
                                                       float *c, const float *res, uint32_t m, uint32_t k, uint32_t n,
                                                       int dtype) {
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
                    float xj = x_bf16 ? bf16_to_f32(static_cast<const uint16_t *>(xv)[xi])
                                      : static_cast<const float *>(xv)[xi];
                    if (up) xj = silu_mul(xj, up[xi]);
                    acc[t] = __builtin_fmaf(xj, wj, acc[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float s = wave_sum(acc[t]);
            if (lane == 0 && t0 + t < m) {
                const uint64_t o = (uint64_t)(t0 + t) * n + row;
                c[o] = res ? res[o] + s : s;
            }
        }
    }
}

// Launch shape: CH chunks per slice (the slice's fragments fill LDS: 48 KB for f32
// activations), one slice per workgroup column, RT row tiles per wavefront: the
// most that still gives 256 workgroups (n is the jobs' total rows).
struct MmShape {
    uint32_t ch, slices, tiles, rt;
};

std::atomic<uint32_t> g_mm_ch{0}, g_mm_rt{0};  // launch-shape overrides (0 = automatic)

MmShape mm_shape(int dtype, uint32_t k, uint32_t n, uint32_t m) {
    const uint32_t tiles = (m + 15) / 16 > 2 ? 2 : (m + 15) / 16;  // per launch; larger m runs in pairs of tiles
    uint32_t ch = dtype == LG_Q4_K ? (tiles == 1 ? 2 : 1) : 1;
    // chunks of 8 sub-blocks per slice: 1, 2 or (one token tile only) 4
    const uint32_t och = g_mm_ch.load(std::memory_order_relaxed), ort = g_mm_rt.load(std::memory_order_relaxed);
    if (och) ch = och >= 4 && tiles == 1 ? 4 : och >= 2 ? 2 : 1;
    if (dtype != LG_Q4_K && ch > 2) ch = 2;
    const uint32_t chunks = (k + 255) / 256, slices = (chunks + ch - 1) / ch;
    // the most rows per wavefront that still give about three workgroups per CU per
    // token tile (fewer, larger workgroups measured slower on every shape tried);
    // four (two waves per SIMD) only when two already give twelve per CU
    uint32_t rt = (n + 127) / 128 * slices >= 3072 * tiles ? 4 : 2;
    while (rt > 1 && (n + 64 * rt - 1) / (64 * rt) * slices < 768 * tiles) rt /= 2;
    if (ort) rt = ort >= 4 ? 4 : ort >= 2 ? 2 : 1;
    while (rt * ch > (dtype == LG_Q4_K ? 8u : 4u)) rt /= 2;  // register budget
    return {ch, slices, tiles, rt};
}

template <int TT, int PARTS, int CH, bool FUSE, bool GLU, bool NORM, bool WIDE>
void launch_rt(int dtype, uint32_t rt, dim3 grid, const void *x, const float *up, const MmJobs &jobs, uint32_t *cnt,
               uint32_t m, uint32_t k, uint64_t rb, hipStream_t s) {
#define LG_MM(K, R) \
    hipLaunchKernelGGL((K<TT, PARTS, CH, R, FUSE, GLU, NORM, WIDE>), grid, dim3(256), 0, s, x, up, jobs, cnt, m, k, rb)
    // mm_shape keeps rt * ch within each kernel's register budget
    if (dtype == LG_Q4_K) {
        if constexpr (4 * CH <= 8)
            if (rt == 4) {
                LG_MM(k_q4k_mm, 4);
                return;
            }
        if constexpr (2 * CH <= 8)
            if (rt == 2) {
                LG_MM(k_q4k_mm, 2);
                return;
            }
        LG_MM(k_q4k_mm, 1);
    } else {
        if constexpr (4 * CH <= 4)
            if (rt == 4) {
                LG_MM(k_q80_mm, 4);
                return;
            }
        if constexpr (2 * CH <= 4)
            if (rt == 2) {
                LG_MM(k_q80_mm, 2);
                return;
            }
        if constexpr (CH <= 2) LG_MM(k_q80_mm, 1);
    }
#undef LG_MM
}

template <int PARTS, bool FUSE, bool GLU = false, bool NORM = false, bool WIDE = false>
int launch_mm(int dtype, const MmShape &sh, uint32_t groups, const void *x, const float *up, const MmJobs &jobs,
              uint32_t *cnt, uint32_t m, uint32_t k, hipStream_t s) {
    const dim3 grid(groups, sh.slices);
    const uint64_t rb = dtype == LG_Q4_K ? (uint64_t)k / QK_K * Q4K_BYTES : (uint64_t)k / QK8_0 * Q80_BYTES;
    if (sh.tiles == 1) {
        if (sh.ch == 4) launch_rt<1, PARTS, 4, FUSE, GLU, NORM, WIDE>(dtype, sh.rt, grid, x, up, jobs, cnt, m, k, rb, s);
        else if (sh.ch == 2) launch_rt<1, PARTS, 2, FUSE, GLU, NORM, WIDE>(dtype, sh.rt, grid, x, up, jobs, cnt, m, k, rb, s);
        else launch_rt<1, PARTS, 1, FUSE, GLU, NORM, WIDE>(dtype, sh.rt, grid, x, up, jobs, cnt, m, k, rb, s);
    } else {
        if (sh.ch == 2) launch_rt<2, PARTS, 2, FUSE, GLU, NORM, WIDE>(dtype, sh.rt, grid, x, up, jobs, cnt, m, k, rb, s);
        else launch_rt<2, PARTS, 1, FUSE, GLU, NORM, WIDE>(dtype, sh.rt, grid, x, up, jobs, cnt, m, k, rb, s);
    }
    return after_launch(dtype == LG_Q4_K ? "proj_q4k_mm" : "proj_q8_0_mm", s);
}

uint64_t align256(uint64_t b) { return (b + 255) & ~(uint64_t)255; }

// Workspace layout: the arrival counters at a fixed place (offset 0, one per
// workgroup column, CNT_MAX of them) so that every call finds them zero, then the
// partial sums, job after job.
constexpr uint64_t CNT_BYTES = PROJ_WS_COUNTERS;
constexpr uint32_t CNT_MAX = CNT_BYTES / 4;

}  // namespace

namespace lg {

uint64_t proj_batch_multi_ws_bytes(uint32_t k, const uint32_t *n, uint32_t jobs, uint32_t m, int w_dtype) {
    if (w_dtype == LG_Q4_K_T16) w_dtype = LG_Q4_K;
    if (w_dtype == LG_Q8_0_T16) w_dtype = LG_Q8_0;
    if (w_dtype != LG_Q4_K && w_dtype != LG_Q8_0) return 0;
    uint64_t ntot = 0;
    for (uint32_t j = 0; j < jobs; j++) ntot += n[j];
    const uint32_t ml = m < 32 ? m : 32;
    const MmShape sh = mm_shape(w_dtype, k, (uint32_t)ntot, ml);
    if (sh.slices <= 1) return 0;
    uint64_t b = CNT_BYTES;
    for (uint32_t j = 0; j < jobs; j++) b += align256((uint64_t)sh.slices * ml * n[j] * 4);
    return b;
}

uint64_t proj_batch_ws_bytes(uint32_t k, uint32_t n, uint32_t m, int x_dtype, int w_dtype) {
    (void)x_dtype;
    return proj_batch_multi_ws_bytes(k, &n, 1, m, w_dtype);
}

uint32_t proj_batch_norm_cols(int w_dtype, uint32_t k, uint32_t n, uint32_t m) {
    if (w_dtype == LG_Q4_K_T16) w_dtype = LG_Q4_K;
    if (w_dtype == LG_Q8_0_T16) w_dtype = LG_Q8_0;
    const MmShape sh = mm_shape(w_dtype, k, n, m < 32 ? m : 32);
    return (n + 64 * sh.rt - 1) / (64 * sh.rt);
}

uint32_t proj_batch_rs_cols_max(uint32_t m) { return MM_SS_LOADS * (m > 16 ? 8u : 16u); }

bool proj_batch_mfma_ok(int w_dtype, uint32_t k, const void *w) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    if (w_dtype == LG_Q4_K_T16 || w_dtype == LG_Q8_0_T16) return k && k % QK_K == 0 && (a & 15u) == 0;
    if (w_dtype == LG_Q4_K) return k && k % QK_K == 0 && (a & 15u) == 0;
    if (w_dtype == LG_Q8_0) return k && k % QK8_0 == 0 && (a & 1u) == 0;
    return false;
}

int proj_batch_multi(const void *x, int x_dtype, const float *up, const BatchJob *jb, uint32_t njobs, uint32_t k,
                     uint32_t m, int w_dtype, void *ws_given, uint64_t ws_bytes, hipStream_t s, bool glu,
                     const RowScale *rs, const QkRope *qk) {
    const char *name = "lg_dispatch_proj_quant_batch";
    LG_REQUIRE(njobs >= 1 && njobs <= (uint32_t)MM_JOBS, "%s: %u jobs (1..%d)", name, njobs, MM_JOBS);
    LG_REQUIRE(!glu || (njobs == 2 && jb[0].n == jb[1].n && !up && x_dtype == LG_F32 && !jb[0].res && !jb[1].res),
               "%s: a gate/up pair takes two products of equal n over f32 activations, without residuals", name);
    if (m == 0) return LG_OK;
    const bool norm = rs && rs->ss && rs->tok0 < m;
    bool epi = false;
    for (uint32_t j = 0; j < njobs; j++) epi = epi || jb[j].ss;
    LG_REQUIRE(!norm || (x_dtype == LG_F32 && !up && rs->cols >= 1 && rs->cols <= proj_batch_rs_cols_max(m)),
               "%s: a folded RMSNorm takes f32 activations without up and 1..%u partial sums per row (got %u)", name,
               proj_batch_rs_cols_max(m), norm ? rs->cols : 0u);
    LG_REQUIRE(!epi || (njobs == 1 && !glu && m <= 32 && x_dtype == LG_F32 && jb[0].y && jb[0].yw),
               "%s: the RMSNorm epilogue takes one job over at most 32 f32 rows, with y and yw", name);
    LG_REQUIRE(m <= 64, "%s: m=%u exceeds 64", name, m);
    LG_REQUIRE(x, "%s: null activations", name);
    bool qkn = false;  // QK-normed jobs: whole heads of 128 rows per workgroup column (RT = 2)
    for (uint32_t j = 0; j < njobs; j++) {
        if (!jb[j].qkw) continue;
        qkn = true;
        LG_REQUIRE(qk && qk->table && jb[j].n % 128 == 0 && !jb[j].res && !jb[j].ss,
                   "%s: a QK-normed job takes the rotation table and heads of 128 rows, without residual or epilogue",
                   name);
    }
    LG_REQUIRE(!qkn || (!glu && !up && m <= 32), "%s: QK-normed jobs take plain products over at most 32 rows", name);
    LG_REQUIRE(x_dtype == LG_F32 || x_dtype == LG_BF16, "%s: activation dtype %d (want F32 or BF16)", name, x_dtype);
    LG_REQUIRE(!up || x_dtype == LG_F32, "%s: the fused SiLU(gate)*up takes f32 activations", name);
    LG_REQUIRE(w_dtype == LG_Q4_K || w_dtype == LG_Q8_0 || w_dtype == LG_F32 || w_dtype == LG_Q4_K_T16 ||
                   w_dtype == LG_Q8_0_T16,
               "%s: weight dtype %d", name, w_dtype);
    const bool tiled = w_dtype == LG_Q4_K_T16 || w_dtype == LG_Q8_0_T16;
    LG_REQUIRE(!tiled || (k % QK_K == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                          (!up || (reinterpret_cast<uintptr_t>(up) & 15u) == 0)),
               "%s: tiled weights take k a multiple of 256 (k=%u) and 16-byte aligned activations", name, k);
    const uint64_t xbytes = (uint64_t)m * k * (x_dtype == LG_F32 ? 4 : 2);
    if (k) {
        LG_EXTENT(x, xbytes, name);
        if (up) LG_EXTENT(up, xbytes, name);
    }
    uint64_t ntot = 0;
    uint32_t nv[MM_JOBS];
    for (uint32_t j = 0; j < njobs; j++) {
        const BatchJob &b = jb[j];
        nv[j] = b.n;
        ntot += b.n;
        if (b.n == 0) continue;
        LG_REQUIRE(b.w && b.c, "%s: null pointer in job %u", name, j);
        LG_EXTENT(b.c, (uint64_t)m * b.n * 4, name);
        if (b.res) LG_EXTENT(b.res, (uint64_t)m * b.n * 4, name);
        if (b.ss) {
            LG_EXTENT(b.y, (uint64_t)m * b.n * 4, name);
            LG_EXTENT(b.yw, (uint64_t)b.n * 4, name);
            LG_EXTENT(b.ss, (uint64_t)m * proj_batch_norm_cols(w_dtype, k, b.n, m) * 4, name);
        }
        if (k) LG_EXTENT(b.w, tiled ? tiled_bytes(w_dtype, k, b.n) : tensor_bytes(w_dtype, (uint64_t)b.n * k), name);
        LG_REQUIRE(!tiled || (reinterpret_cast<uintptr_t>(b.w) & 15u) == 0, "%s: unaligned tiled weights", name);
    }
    if (ntot == 0) return LG_OK;
    if (norm) LG_EXTENT(rs->ss, (uint64_t)(m - rs->tok0) * rs->cols * 4, name);
    if (tiled) w_dtype = w_dtype == LG_Q4_K_T16 ? LG_Q4_K : LG_Q8_0;  // the same kernels, reading tiles
    const uint32_t blk = w_dtype == LG_Q4_K ? QK_K : QK8_0;
    bool fast = k && w_dtype != LG_F32 && k % blk == 0 && k % 32 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                (!up || (reinterpret_cast<uintptr_t>(up) & 15u) == 0);
    for (uint32_t j = 0; j < njobs; j++)
        fast = fast && (w_dtype != LG_Q4_K || (reinterpret_cast<uintptr_t>(jb[j].w) & 15u) == 0) &&
               (reinterpret_cast<uintptr_t>(jb[j].w) & 1u) == 0;
    LG_REQUIRE(fast || !(norm || epi || qkn), "%s: a folded RMSNorm or QK-norm needs the matrix-core path (k a "
               "multiple of the block, aligned operands)", name);
    if (!fast) {
        for (uint32_t j = 0; j < njobs; j++) {
            if (jb[j].n == 0) continue;
            hipLaunchKernelGGL(k_generic_batch, dim3((jb[j].n + 3) / 4), dim3(256), 0, s, x, (int)(x_dtype == LG_BF16),
                               up, jb[j].w, jb[j].c, jb[j].res, m, k, jb[j].n, w_dtype);
            LG_TRY(after_launch(name, s));
        }
        if (glu) LG_TRY(lg_dispatch_activation(jb[0].c, jb[1].c, jb[0].c, m * jb[0].n, s));
        return LG_OK;
    }
    const uint64_t need = proj_batch_multi_ws_bytes(k, nv, njobs, m, w_dtype);
    void *ws = ws_given;
    if (need) {
        if (ws) {
            LG_REQUIRE(ws_bytes >= need, "%s: workspace of %llu bytes too small", name, (unsigned long long)ws_bytes);
        } else {
            LG_TRY(stream_workspace(s, need, &ws));
        }
    }
    const uint32_t tiles = (m + 15) / 16;
    const uint64_t xsz = x_dtype == LG_F32 ? 4 : 2;
    for (uint32_t t0 = 0; t0 < tiles; t0 += 2) {  // pairs of 16-token tiles
        const uint32_t ml = m - 16 * t0 < 32 ? m - 16 * t0 : 32;
        MmShape sh = mm_shape(w_dtype, k, (uint32_t)ntot, ml);
        if (qkn) sh.rt = 2;  // within every budget: mm_shape keeps ch <= 4 (Q4_K) and <= 2 (Q8_0)
        uint32_t *cnt = static_cast<uint32_t *>(ws);
        uint8_t *pb = ws ? static_cast<uint8_t *>(ws) + CNT_BYTES : nullptr;
        if (sh.slices > 1) LG_REQUIRE(ws, "%s: no workspace for %u slices", name, sh.slices);
        MmJobs jobs{};
        uint32_t groups = 0;
        for (uint32_t j = 0; j < njobs; j++) {
            const uint64_t off = (uint64_t)16 * t0 * jb[j].n;
            jobs.j[j] = {static_cast<const uint8_t *>(jb[j].w), jb[j].c + off, jb[j].res ? jb[j].res + off : nullptr,
                         reinterpret_cast<float *>(pb), jb[j].y, jb[j].yw, jb[j].ss, jb[j].n, groups, jb[j].qkw};
            if (pb) pb += align256((uint64_t)sh.slices * ml * jb[j].n * 4);
            groups += (jb[j].n + 64 * sh.rt - 1) / (64 * sh.rt);
        }
        if (glu) {  // both products in every workgroup column
            groups = (jb[0].n + 32 * sh.rt - 1) / (32 * sh.rt);
            jobs.j[1].g0 = 0;
        }
        jobs.count = njobs;
        jobs.tiled = tiled ? 1u : 0u;
        if (qkn) {
            jobs.rope = qk->table + (uint64_t)16 * t0 * 128;
            jobs.qk_eps = qk->eps;
        }
        // the folded norm's scaled rows in this pair of tiles (rows 16 t0 .. 16 t0 + ml - 1)
        const bool pnorm = norm && 16 * t0 + ml > rs->tok0;
        if (pnorm) {
            jobs.rs_tok0 = rs->tok0 > 16 * t0 ? rs->tok0 - 16 * t0 : 0u;
            jobs.rs_ss = rs->ss + (uint64_t)(16 * t0 > rs->tok0 ? 16 * t0 - rs->tok0 : 0u) * rs->cols;
            jobs.rs_cols = rs->cols;
            jobs.rs_eps = rs->eps;
        }
        // one plain product split over k in many rounds of workgroups: the slices only
        // store their partial sums and k_mm_sum adds them
        const bool wide = njobs == 1 && !qkn && !glu && !up && !pnorm && !jb[0].res && !jb[0].ss && sh.slices > 1 &&
                          (uint64_t)groups * sh.slices >= WIDE_MIN_WGS;
        LG_REQUIRE(groups <= CNT_MAX, "%s: %u workgroup columns exceed %u", name, groups, CNT_MAX);
        const void *xt = static_cast<const uint8_t *>(x) + (uint64_t)16 * t0 * k * xsz;
        const float *ut = up ? up + (uint64_t)16 * t0 * k : nullptr;
        if (wide && x_dtype == LG_BF16)
            LG_TRY((launch_mm<1, false, false, false, true>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        else if (wide) LG_TRY((launch_mm<3, false, false, false, true>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        else if (x_dtype == LG_BF16) LG_TRY((launch_mm<1, false>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        else if (up) LG_TRY((launch_mm<3, true>(w_dtype, sh, groups, xt, ut, jobs, cnt, ml, k, s)));
        else if (glu && pnorm) LG_TRY((launch_mm<3, false, true, true>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        else if (glu) LG_TRY((launch_mm<3, false, true>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        else if (pnorm) LG_TRY((launch_mm<3, false, false, true>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        else LG_TRY((launch_mm<3, false>(w_dtype, sh, groups, xt, nullptr, jobs, cnt, ml, k, s)));
        if (wide) {
            const MmJob &j0 = jobs.j[0];
            const dim3 sg((j0.n + SUM_ROWS - 1) / SUM_ROWS, (ml + 15) / 16);
            if (j0.n % 4 == 0 && (reinterpret_cast<uintptr_t>(j0.out) & 15u) == 0)
                hipLaunchKernelGGL(k_mm_sum<true>, sg, dim3(256), 0, s, j0.part, j0.out, ml, j0.n, sh.slices);
            else
                hipLaunchKernelGGL(k_mm_sum<false>, sg, dim3(256), 0, s, j0.part, j0.out, ml, j0.n, sh.slices);
            LG_TRY(after_launch(name, s));
        }
    }
    return LG_OK;
}

int proj_batch(const void *x, int x_dtype, const void *w, float *c, uint32_t k, uint32_t n, uint32_t m, int w_dtype,
               void *ws_given, uint64_t ws_bytes, hipStream_t s, const float *res) {
    if (n == 0 || m == 0) return LG_OK;
    LG_REQUIRE(n <= 64u * CNT_MAX, "lg_dispatch_proj_quant_batch: n=%u exceeds %u", n, 64u * CNT_MAX);
    LG_REQUIRE(x && w && c, "lg_dispatch_proj_quant_batch: null pointer");
    const BatchJob j{w, c, res, n};
    return proj_batch_multi(x, x_dtype, nullptr, &j, 1, k, m, w_dtype, ws_given, ws_bytes, s);
}

}  // namespace lg

// Launch shape of the small-M products (0 = automatic): ch chunks of 8 sub-blocks
// per k slice (1, 2, or 4 for Q4_K with one 16-token tile) and rt 16-row tiles per
// wavefront (1, 2 or 4, clamped to the register budget).  A tuning hook for
// launch-shape sweeps; results meet the same parity bound for every value.
// Workspaces sized before a change may be too small afterwards (the call then fails).
extern "C" int lg_set_batch_shape(uint32_t ch, uint32_t rt) {
    g_mm_ch.store(ch, std::memory_order_relaxed);
    g_mm_rt.store(rt, std::memory_order_relaxed);
    return LG_OK;
}

namespace {

// LG_Q4_K_T16 repack: workgroup (b, t) writes tile (t, b).  Thread p moves quant
// piece p = 64g + 16q + r (row r's bytes 32g + 8q .. +7, 8 bytes) to 256 + 8p;
// threads 0-15 also move row p's 16-byte header.  Rows past n become zero blocks.
__global__ __launch_bounds__(256) void k_repack_q4k_t16(const uint8_t *__restrict__ w, uint8_t *__restrict__ out,
                                                         uint32_t nb, uint32_t n) {
    const uint32_t b = blockIdx.x, t = blockIdx.y, p = threadIdx.x;
    const uint32_t g = p >> 6, q = (p >> 4) & 3u, r = p & 15u, row = 16 * t + r;
    uint8_t *tile = out + ((uint64_t)t * nb + b) * Q4K_TILE;
    const bool live = row < n;
    const uint8_t *blk = w + ((uint64_t)(live ? row : n - 1) * nb + b) * Q4K_BYTES;  // in bounds either way
    const uint2 qv = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * g + 8 * q);
    *reinterpret_cast<uint2 *>(tile + 256 + 8 * p) = live ? qv : make_uint2(0u, 0u);
    if (p < 16) {
        const bool hlive = 16 * t + p < n;
        const uint8_t *hb = w + ((uint64_t)(hlive ? 16 * t + p : n - 1) * nb + b) * Q4K_BYTES;
        const uint4 hv = *reinterpret_cast<const uint4 *>(hb);
        *reinterpret_cast<uint4 *>(tile + 16 * p) = hlive ? hv : make_uint4(0u, 0u, 0u, 0u);
    }
}

// LG_Q8_0_T16 repack: workgroup (c, t) writes tile (t, c) -- rows 16t..16t+15,
// blocks 8c..8c+7.  Thread p moves quant pieces p and p + 256 (piece
// 64j + 16q + r: row r's bytes 2 + 8q .. 9 + 8q of block j, read as 16-bit
// words since blocks are 2-byte aligned) and, for p < 128, the scale of row p/8,
// block p%8.  Rows past n become zero blocks.
__global__ __launch_bounds__(256) void k_repack_q80_t16(const uint8_t *__restrict__ w, uint8_t *__restrict__ out,
                                                         uint32_t nc, uint32_t n) {
    const uint32_t c = blockIdx.x, t = blockIdx.y;
    uint8_t *tile = out + ((uint64_t)t * nc + c) * Q80_TILE;
    const uint64_t rowb = (uint64_t)nc * 8 * Q80_BYTES;
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        const uint32_t p = threadIdx.x + 256 * h, j = p >> 6, q = (p >> 4) & 3u, r = p & 15u, row = 16 * t + r;
        const bool live = row < n;
        const uint16_t *src = reinterpret_cast<const uint16_t *>(w + (uint64_t)(live ? row : n - 1) * rowb +
                                                                 (uint64_t)(8 * c + j) * Q80_BYTES + 2 + 8 * q);
        const uint2 v = make_uint2(src[0] | ((uint32_t)src[1] << 16), src[2] | ((uint32_t)src[3] << 16));
        *reinterpret_cast<uint2 *>(tile + 256 + 8 * p) = live ? v : make_uint2(0u, 0u);
    }
    if (threadIdx.x < 128) {
        const uint32_t r = threadIdx.x >> 3, j = threadIdx.x & 7u, row = 16 * t + r;
        const bool live = row < n;
        const uint16_t d = *reinterpret_cast<const uint16_t *>(w + (uint64_t)(live ? row : n - 1) * rowb +
                                                               (uint64_t)(8 * c + j) * Q80_BYTES);
        *reinterpret_cast<uint16_t *>(tile + 2 * threadIdx.x) = live ? d : (uint16_t)0;
    }
}

}  // namespace

extern "C" uint64_t lg_tiled_bytes(int dtype, uint32_t k, uint32_t n) {
    return (dtype == LG_Q4_K || dtype == LG_Q8_0) && k % QK_K == 0 ? tiled_bytes(dtype, k, n) : 0;
}

extern "C" int lg_repack_tiled(const void *w, int dtype, uint32_t k, uint32_t n, void *out, void *stream) {
    clear_error();
    const char *name = "lg_repack_tiled";
    LG_REQUIRE(dtype == LG_Q4_K || dtype == LG_Q8_0, "%s: dtype %d (Q4_K and Q8_0 are tiled)", name, dtype);
    LG_REQUIRE(k % QK_K == 0, "%s: k=%u is not a multiple of 256", name, k);
    if (k == 0 || n == 0) return LG_OK;
    LG_REQUIRE(w && out, "%s: null pointer", name);
    LG_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(w) & (dtype == LG_Q4_K ? 15u : 1u)) == 0,
               "%s: misaligned pointer (out 16 bytes, w 16 for Q4_K and 2 for Q8_0)", name);
    LG_REQUIRE((n + 15) / 16 <= 65535u, "%s: n=%u exceeds %u rows", name, n, 65535u * 16);
    LG_EXTENT(w, tensor_bytes(dtype, (uint64_t)k * n), name);
    LG_EXTENT(out, tiled_bytes(dtype, k, n), name);
    hipStream_t s = (hipStream_t)stream;
    if (dtype == LG_Q4_K)
        hipLaunchKernelGGL(k_repack_q4k_t16, dim3(k / QK_K, (n + 15) / 16), dim3(256), 0, s,
                           static_cast<const uint8_t *>(w), static_cast<uint8_t *>(out), k / QK_K, n);
    else
        hipLaunchKernelGGL(k_repack_q80_t16, dim3(k / 256, (n + 15) / 16), dim3(256), 0, s,
                           static_cast<const uint8_t *>(w), static_cast<uint8_t *>(out), k / 256, n);
    return after_launch(name, s);
}

extern "C" int lg_dispatch_proj_quant_batch(const void *x, int x_dtype, const void *w, float *c, uint32_t k,
                                            uint32_t n, uint32_t m, int w_dtype, void *stream) {
    clear_error();
    return lg::proj_batch(x, x_dtype, w, c, k, n, m, w_dtype, nullptr, 0, (hipStream_t)stream);
}

// ---- allocation-free small-M product
//
// lg_dispatch_proj_quant_batch_static runs the same kernels with their arrival
// counters and partial sums in `scratch`, a file-scope device array that every GPU
// holds for the life of the process, so the call makes no allocation (for code
// under HIP graph capture, serving loops and callers that may not allocate).  Host
// code uses the address hipGetSymbolAddress returns for the current device, never
// the array's name.  Calls on one GPU share the array: calls that overlap in time on
// that GPU, on any stream, race.
constexpr uint64_t STATIC_SCRATCH_BYTES = PROJ_WS_COUNTERS + (16ull << 20);
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {

constexpr int STATIC_MAX_DEVICES = 64;
std::mutex g_static_mu;
void *g_static_ptr[STATIC_MAX_DEVICES] = {};

__global__ __launch_bounds__(256) void k_zero_words(uint32_t *p, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// The scratch address on device `dev` (current), set up once: its arrival counters
// are cleared on stream s with a kernel (the set-up may happen inside a capture,
// where a memset node must not be recorded).
int static_scratch(int dev, hipStream_t s, bool wait, void **out) {
    LG_REQUIRE(dev >= 0 && dev < STATIC_MAX_DEVICES, "static scratch: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (!g_static_ptr[dev]) {
        void *p = nullptr;
        LG_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        LG_REQUIRE(p, "static scratch: no address on device %d", dev);
        const uint32_t words = (uint32_t)(PROJ_WS_COUNTERS / 4);
        hipLaunchKernelGGL(k_zero_words, dim3((words + 255) / 256), dim3(256), 0, s, static_cast<uint32_t *>(p), words);
        LG_HIP_TRY(hipGetLastError());
        if (wait) LG_HIP_TRY(hipStreamSynchronize(s));
        g_static_ptr[dev] = p;
    }
    *out = g_static_ptr[dev];
    return LG_OK;
}

}  // namespace

namespace lg {

int static_scratch_setup(int dev) {
    void *p = nullptr;
    return static_scratch(dev, nullptr, true, &p);
}

}  // namespace lg

extern "C" int lg_dispatch_proj_quant_batch_static(const void *x, int x_dtype, const void *w, float *c, uint32_t k,
                                                   uint32_t n, uint32_t m, int w_dtype, void *stream) {
    clear_error();
    const char *name = "lg_dispatch_proj_quant_batch_static";
    if (n == 0 || m == 0) return LG_OK;
    const uint64_t need = lg::proj_batch_ws_bytes(k, n, m < 32 ? m : 32, x_dtype, w_dtype);
    LG_REQUIRE(need <= STATIC_SCRATCH_BYTES,
               "%s: k=%u n=%u m=%u needs %llu bytes of scratch, more than the %llu this entry point has", name, k, n,
               m, (unsigned long long)need, (unsigned long long)STATIC_SCRATCH_BYTES);
    int dev = 0;
    LG_HIP_TRY(hipGetDevice(&dev));
    void *ws = nullptr;
    LG_TRY(static_scratch(dev, (hipStream_t)stream, false, &ws));
    return lg::proj_batch(x, x_dtype, w, c, k, n, m, w_dtype, ws, STATIC_SCRATCH_BYTES, (hipStream_t)stream);
}

extern "C" int lg_dispatch_silu_gate_up_batch(const float *x, const void *w_gate, const void *w_up, float *h,
                                              float *u_scratch, uint32_t k, uint32_t n, uint32_t m, int w_dtype,
                                              void *stream) {
    clear_error();
    if (n == 0 || m == 0) return LG_OK;
    LG_REQUIRE(n <= 32u * CNT_MAX, "lg_dispatch_silu_gate_up_batch: n=%u exceeds %u", n, 32u * CNT_MAX);
    LG_REQUIRE(x && w_gate && w_up && h && u_scratch, "lg_dispatch_silu_gate_up_batch: null pointer");
    const lg::BatchJob jb[2] = {{w_gate, h, nullptr, n}, {w_up, u_scratch, nullptr, n}};
    return lg::proj_batch_multi(x, LG_F32, nullptr, jb, 2, k, m, w_dtype, nullptr, 0, (hipStream_t)stream, true);
}
