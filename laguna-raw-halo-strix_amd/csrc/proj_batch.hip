// Small-M products (block verify, m <= 64 activation rows): lg_dispatch_proj_quant_batch.
// Replaces kernels/matmul.comp (never dispatched by the reference) with f16 MFMA
// tiles on gfx950 (v_mfma_f32_16x16x32_f16: D[16x16] += A[16x32] * B[32x16]).
//
//   A = activations, converted by each workgroup into a "fragment record" per 16-token
//       tile and 256-element chunk of k, in LDS: each token's chunk is scaled by a
//       power of two 2^e that puts its largest magnitude in [2^14, 2^15), and every
//       scaled value v is split into two f16 parts, hi = f16(v) and lo = f16(v - hi)
//       (22 significant bits, down to the f16 subnormal step 2^-24 of the scaled
//       chunk), laid out as the MFMA's lane fragments; with them the sums X of each
//       32-element sub-block of the scaled values, and 2^-e.
//   B = weight codes of 16 output rows x 32 k, built in registers from the raw blocks
//       as f16 subnormals (gfx950's MFMA keeps f16 denormals), so the code of a nibble
//       is the nibble itself:
//         Q4_K  low nibble q -> q 2^-24 (one and per pair), high nibble -> 16 q 2^-24;
//         Q8_0  int8 q -> (q + 128) 2^-24 (xor, and per pair).
//   Per sub-block j of output row i (D_j = sum_k A_k B_k, over both parts):
//         Q4_K  sum x w = 2^24 d sc_j D_j (2^20 for high nibbles) - dmin m_j X_j
//         Q8_0  sum x w = 2^24 d_j D_j - 128 d_j X_j
//       the X terms as f32 matrix products (k = the chunk's 8 sub-blocks), and the
//       chunk's sum scaled by 2^-e per token.
//
// Operand lane layout (16x16x32): lane l supplies row l%16 of A / column l%16 of B
// at k-group l/16 (8 consecutive values); D row 4*(l/16)+r, column l%16 lands in
// lane l, register r.  Inside a k-group the order of the 8 values only has to
// agree between A and B; both use byte order {0,2,1,3,4,6,5,7}, which is the
// order the masks produce.
//
// Work split: workgroup (blockIdx.x, blockIdx.y) = 64*RT output rows (RT 16-row
// tiles per wavefront, four wavefronts) x slice blockIdx.y of k: `ch` chunks walked
// in order, the next chunk's activations and the weights two chunks ahead in flight
// while the current one is multiplied (the record double-buffered in LDS, one
// barrier per chunk).  With one slice the workgroup writes the result; otherwise each
// writes its slice's partial sums and the last workgroup of a row group to finish (a
// per-row-group arrival counter, reset by that workgroup) adds the slices in slice
// order: the result does not depend on which workgroup finishes last.
#include <mutex>
#include <vector>

#include "lg_common.hpp"

namespace {

using namespace lg;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// ref_half (the reference's binary16 decoder, src/dflash.rs:314-329) through the
// hardware conversion: IEEE for normals, zeros and inf; an exponent-0 code with a
// nonzero mantissa decodes as 2^-14 (1 + m/1024) = IEEE's m 2^-24 plus 2^-14, with
// the code's sign.  (A NaN code stays a NaN; its payload is not kept.)
__device__ __forceinline__ float ref_half_hw(uint32_t h) {
    const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    const uint32_t t = h & 0x7FFFu;
    const float q = __uint_as_float(((h & 0x8000u) << 16) | 0x38800000u);  // +-2^-14
    return t - 1u < 0x3FFu ? f + q : f;
}

__device__ __forceinline__ f16x8 as_f16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(f16x8, make_uint4(a, b, c, d));
}

// Fragment record of one (16-token tile, 256-element chunk) in LDS, FR_U4 16-byte words:
//   [0, 1024)     word (j*2 + p)*64 + (l ^ (2j + l/32)): part p (0 = hi, 1 = lo) of
//                 sub-block j's A operand, lane l: token l%16, elements
//                 32j + 8(l/16) + {0,2,1,3,4,6,5,7}.  The XOR spreads over all LDS banks
//                 the 16 threads of one token that store a word together (thread q of
//                 the token stores lane slots 16(2(q%2) + h) + token, XOR q)
//   [1024, 1056)  float2 per lane l: (X[l%16][l/16], X[l%16][l/16 + 4]), X the sums of
//                 the scaled values over each sub-block
//   [1056, 1060)  the 16 tokens' 2^-e
constexpr uint32_t FR_X = 1024, FR_S = 1056, FR_U4 = 1060;

// 2^-24 scaled codes: Q4_K nibbles in place (low nibbles of bytes 0 and 2 / 1 and 3
// of a dword: `& LO4`, high nibbles `& HI4`), Q8_0 bytes biased to unsigned.
constexpr uint32_t LO4 = 0x000F000Fu, HI4 = 0x00F000F0u, LO8 = 0x00FF00FFu;

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
constexpr uint32_t MM_SS_LOADS = 8;  // partial sums a consuming lane loads (per-token capacity 8 * 16 / TT)
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
    uint32_t tlo;      // 1: only the second token tile of a two-tile launch is needed
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
#define MM_JOB_INDEX                                                                      \
    uint32_t J_ = 0;                                                                      \
    if constexpr (GLU) J_ = __builtin_amdgcn_readfirstlane(threadIdx.x >> 7);             \
    else _Pragma("unroll") for (int j_ = 1; j_ < MM_JOBS; j_++) if ((uint32_t)j_ < jobs.count && \
                                                              blockIdx.x >= jobs.j[j_].g0) J_ = j_
#define MM_JOB_FIELDS                                                                     \
    const uint8_t *w = jobs.j[J_].w;                                                      \
    float *out = jobs.j[J_].out;                                                          \
    const float *res = jobs.j[J_].res;                                                    \
    float *part = jobs.j[J_].part;                                                        \
    const uint32_t n = jobs.j[J_].n, bx = blockIdx.x - jobs.j[J_].g0

__device__ __forceinline__ float silu_mul(float g, float u) {
    // kernels/activation.comp:21-28: silu(g) * up, silu(x) = x * (1 / (1 + exp(-x)))
    return g * (1.0f / (1.0f + expf(-g))) * u;
}

// ---- fragment records

// Maximum over each 16-lane row: DPP xor 1, xor 2 (quad_perm), then row_ror 4 and 8.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));   // quad_perm 1,0,3,2
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));   // quad_perm 2,3,0,1
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));  // row_ror 4
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));  // row_ror 8
    return v;
}


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
    // the norm weights and every rotation angle first: their loads overlap the exchanges
    float wd[2], rc[TT][4][2], rs[TT][4][2];
#pragma unroll
    for (int i = 0; i < 2; i++) wd[i] = w[32 * wave + 16 * i + (l & 15u)];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t tok = t * 16 + 4 * kg + r, tc = tok < m ? tok : m - 1;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t dm = 32 * (wave & 1u) + 16 * i + (l & 15u);
                rc[t][r][i] = rope[(uint64_t)tc * 128 + dm];
                rs[t][r][i] = rope[(uint64_t)tc * 128 + 64 + dm];
            }
        }
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
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float p = xch[(((wave ^ 2u) * 2 + i) * TT + t) * 256 + r * 64 + l];
                const float c = rc[t][r][i], sn = rs[t][r][i];
                v[i][t][r] = wave < 2 ? v[i][t][r] * c - p * sn : v[i][t][r] * c + p * sn;
            }
}

template <int TT, int RT, bool GLU, bool NORM>
__device__ __forceinline__ void finish(const float (&acc)[RT][TT][4], float *out, const float *res, float *part,
                                       uint32_t *cnt, uint32_t rt0, uint32_t m, uint32_t n, float *xch,
                                       const MmJobs &jobs, uint32_t k, float *y, const float *yw, float *ssout,
                                       uint32_t bx, const float *qkw) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
    const uint32_t S = gridDim.y, s = blockIdx.y;
    // split k: the column's partials, [slice][wavefront][RT][TT][lane] float4 (the lane's
    // four tokens of one row), each wavefront's as it holds them, in device-coherent
    // 16-byte stores and loads (mm_part_floats)
    constexpr uint32_t WB = RT * TT * 256;  // floats of one wavefront's partial
    const uint32_t pw = threadIdx.x >> 6;
    const __amdgpu_buffer_rsrc_t rp = dev_rsrc(part + (uint64_t)bx * S * 4 * WB);
    auto poff = [&](uint32_t q, int i, int t) { return 4u * ((q * 4 + pw) * WB + (i * TT + t) * 256 + 4 * l); };
    if (S > 1) {
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int t = 0; t < TT; t++)
                dev_st4(rp, poff(s, i, t), make_float4(acc[i][t][0], acc[i][t][1], acc[i][t][2], acc[i][t][3]));
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
    constexpr uint32_t G = RT * TT >= 4 ? 32u / (RT * TT) : 8u;
    float v[RT][TT][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) v[i][t][r] = S > 1 ? 0.0f : acc[i][t][r];
    for (uint32_t q0 = 0; q0 < (S > 1 ? S : 0u); q0 += G) {
        float4 pv[G][RT][TT];
#pragma unroll
        for (uint32_t g = 0; g < G; g++) {
            const uint32_t q = q0 + g < S ? q0 + g : S - 1;
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int t = 0; t < TT; t++) pv[g][i][t] = dev_ld4(rp, poff(q, i, t));
        }
#pragma unroll
        for (uint32_t g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int t = 0; t < TT; t++)
                    if (q0 + g < S) {
                        v[i][t][0] += pv[g][i][t].x;
                        v[i][t][1] += pv[g][i][t].y;
                        v[i][t][2] += pv[g][i][t].z;
                        v[i][t][3] += pv[g][i][t].w;
                    }
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

// ---- products over fragment records
//
// The weights of one chunk (256 elements of k) for a wavefront's RT row tiles: lane l
// holds row l%16's pieces of k-group l/16.
//   Q4_K: the super-block header (16 bytes) and, for each 64-element group g, the 8
//         quant bytes 32g + 8(l/16) .. +7 (low nibbles: sub-block 2g, high: 2g + 1).
//   Q8_0: per block j of the chunk, its f16 scale and quant bytes 8(l/16) .. +7.
template <int RT>
struct Q4kChunk {
    uint4 hd[RT];
    uint2 qv[RT][4];
};
template <int RT>
struct Q80Chunk {
    uint32_t sc[RT][4];  // the 8 scales, two per word
    uint2 qv[RT][8];
};

// The tiles' quant bytes, 512 contiguous bytes per load, each read once per launch:
// nontemporal loads (the draft block 582.1 -> 566.3 us, the 16-row-tile products 2-3 %
// faster; the raw paths' loads and the tiles' headers, which lanes share, measured
// slower with them).
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld_nt8(const uint8_t *p) {
    const nt_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x2 *>(p));
    return make_uint2(v.x, v.y);
}

// Rows past n (and their tiles) read row n-1 / the last tile: loads stay in bounds and
// the results are never stored.
template <int RT, bool TILED>
__device__ __forceinline__ void load_q4k(Q4kChunk<RT> &W, const uint8_t *__restrict__ w, uint32_t n, uint32_t rt0,
                                         uint32_t nb, uint32_t cb, uint64_t row_bytes) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        if constexpr (TILED) {  // 2304-byte tiles: each load reads 256 (headers) or 512 contiguous bytes
            const uint32_t ntiles = (n + 15) / 16, t = rt0 + i < ntiles ? rt0 + i : ntiles - 1;
            const uint8_t *tb = w + ((uint64_t)t * nb + cb) * Q4K_TILE;
            W.hd[i] = *reinterpret_cast<const uint4 *>(tb + 16 * (l & 15u));
#pragma unroll
            for (int g = 0; g < 4; g++) W.qv[i][g] = ld_nt8(tb + 256 + 512 * g + 8 * l);
        } else {
            // the tile's first row (scalar; tiles past n read the last tile) plus the
            // lane's row within it (clamped to n - 1)
            const uint32_t rlast = (n - 1) & ~15u, r0 = (rt0 + i) * 16 < rlast ? (rt0 + i) * 16 : rlast;
            const uint32_t rl = r0 + (l & 15u) < n ? (l & 15u) : n - 1 - r0;
            const uint8_t *blk = w + (uint64_t)r0 * row_bytes + (uint64_t)cb * Q4K_BYTES;
            const uint32_t lo = rl * (uint32_t)row_bytes;
            W.hd[i] = *reinterpret_cast<const uint4 *>(blk + lo);
#pragma unroll
            for (int g = 0; g < 4; g++) W.qv[i][g] = *reinterpret_cast<const uint2 *>(blk + lo + 16 + 32 * g + 8 * kg);
        }
    }
}

// Q8_0 over 16-row tiles (4352-byte tiles): a row's 8 scales in one 16-byte load, 512
// contiguous bytes per quant load.  Tiles past the last read the last tile.
template <int RT>
__device__ __forceinline__ void load_q80_tiled(Q80Chunk<RT> &W, const uint8_t *__restrict__ w, uint32_t n,
                                               uint32_t rt0, uint32_t nb, uint32_t cb) {
    const uint32_t l = threadIdx.x & 63u;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint32_t ntiles = (n + 15) / 16, t = rt0 + i < ntiles ? rt0 + i : ntiles - 1;
        const uint8_t *tb = w + ((uint64_t)t * nb + cb) * Q80_TILE;
        const uint4 s = *reinterpret_cast<const uint4 *>(tb + 16 * (l & 15u));
        W.sc[i][0] = s.x;
        W.sc[i][1] = s.y;
        W.sc[i][2] = s.z;
        W.sc[i][3] = s.w;
#pragma unroll
        for (int j = 0; j < 8; j++) W.qv[i][j] = ld_nt8(tb + 256 + 512 * j + 8 * l);
    }
}

// Raw Q8_0 blocks are only 2-byte aligned, so the raw path loads a chunk's rows whole:
// a 16-row tile's chunk is 16 rows x 272 bytes (8 blocks of 34), 272 aligned 16-byte
// pieces (k % 256 == 0 and a 16-byte aligned base keep them aligned), piece e of the
// tile (row e / 17, bytes 16 (e % 17) ..) in lane e % 64, round e / 64.  Before the
// chunk's products the wavefront writes them to its own LDS region, where the row's
// bytes lie as in memory, and each lane reads back its blocks' scales and quants
// (stage_q80).
constexpr uint32_t Q80_PIECES = 8 * Q80_BYTES / 16;  // 17 per row and chunk
template <int RT>
struct Q80RawChunk {
    lg_u32x4 v[RT][5];  // a vector type: HIP's uint4 struct keeps arrays of it out of registers
};

template <int RT>
__device__ __forceinline__ void load_q80_raw(Q80RawChunk<RT> &W, const uint8_t *__restrict__ w, uint32_t n,
                                             uint32_t rt0, uint32_t cb, uint64_t row_bytes) {
    const uint32_t l = threadIdx.x & 63u;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint32_t rlast = (n - 1) & ~15u, r0 = (rt0 + i) * 16 < rlast ? (rt0 + i) * 16 : rlast;
#pragma unroll
        for (int rd = 0; rd < 5; rd++) {
            const uint32_t e0 = l + 64u * rd, e = e0 < 16 * Q80_PIECES ? e0 : 16 * Q80_PIECES - 1;  // past: a repeat
            const uint32_t rr = e / Q80_PIECES, row = r0 + rr < n ? r0 + rr : n - 1;
            W.v[i][rd] = *reinterpret_cast<const lg_u32x4 *>(w + (uint64_t)row * row_bytes +
                                                             (uint64_t)cb * 8 * Q80_BYTES + 16 * (e % Q80_PIECES));
        }
    }
}

// The raw pieces through the wavefront's LDS region (RT x 4352 bytes) into the lane's
// scales and quants, as load_q80_tiled reads them from 16-row tiles.
template <int RT>
__device__ __forceinline__ void stage_q80(const Q80RawChunk<RT> &R, Q80Chunk<RT> &W, lg_u32x4 *st) {
    const uint32_t l = threadIdx.x & 63u, rr = l & 15u, kg = l >> 4;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the previous chunk's reads are done
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int rd = 0; rd < 5; rd++) {
            const uint32_t e0 = l + 64u * rd, e = e0 < 16 * Q80_PIECES ? e0 : 16 * Q80_PIECES - 1;
            st[i * 16 * Q80_PIECES + e] = R.v[i][rd];  // lanes past the tile rewrite the last piece
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint8_t *row = reinterpret_cast<const uint8_t *>(st + i * 16 * Q80_PIECES) + rr * 8 * Q80_BYTES;
        uint32_t d[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint8_t *b = row + j * Q80_BYTES;  // 4-byte aligned for even j, 2-byte for odd j
            d[j] = *reinterpret_cast<const uint16_t *>(b);
            if (j % 2 == 0) {  // quants at b + 2 + 8 kg: three aligned dwords from b + 8 kg
                const uint32_t *p = reinterpret_cast<const uint32_t *>(b + 8 * kg);
                const uint32_t a0 = p[0], a1 = p[1], a2 = p[2];
                W.qv[i][j] = make_uint2(__builtin_amdgcn_alignbit(a1, a0, 16), __builtin_amdgcn_alignbit(a2, a1, 16));
            } else {
                const uint32_t *p = reinterpret_cast<const uint32_t *>(b + 2 + 8 * kg);
                W.qv[i][j] = make_uint2(p[0], p[1]);
            }
        }
#pragma unroll
        for (int h = 0; h < 4; h++) W.sc[i][h] = d[2 * h] | (d[2 * h + 1] << 16);
    }
}

// Raw Q4_K rows the same way: a tile's chunk is 16 rows x 144 bytes (one super-block
// each), 144 aligned 16-byte pieces (piece e: row e / 9, bytes 16 (e % 9) ..), staged
// through the wavefront's LDS region, from which each lane reads its row's header and
// its 8-byte quant pieces as load_q4k reads them in place.
constexpr uint32_t Q4K_PIECES = Q4K_BYTES / 16;  // 9 per row and chunk
template <int RT>
struct Q4kRawChunk {
    lg_u32x4 v[RT][3];
};

template <int RT>
__device__ __forceinline__ void load_q4k_raw(Q4kRawChunk<RT> &W, const uint8_t *__restrict__ w, uint32_t n,
                                             uint32_t rt0, uint32_t cb, uint64_t row_bytes) {
    const uint32_t l = threadIdx.x & 63u;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint32_t rlast = (n - 1) & ~15u, r0 = (rt0 + i) * 16 < rlast ? (rt0 + i) * 16 : rlast;
#pragma unroll
        for (int rd = 0; rd < 3; rd++) {
            const uint32_t e0 = l + 64u * rd, e = e0 < 16 * Q4K_PIECES ? e0 : 16 * Q4K_PIECES - 1;  // past: a repeat
            const uint32_t rr = e / Q4K_PIECES, row = r0 + rr < n ? r0 + rr : n - 1;
            W.v[i][rd] = *reinterpret_cast<const lg_u32x4 *>(w + (uint64_t)row * row_bytes + (uint64_t)cb * Q4K_BYTES +
                                                             16 * (e % Q4K_PIECES));
        }
    }
}

template <int RT>
__device__ __forceinline__ void stage_q4k(const Q4kRawChunk<RT> &R, Q4kChunk<RT> &W, lg_u32x4 *st) {
    const uint32_t l = threadIdx.x & 63u, rr = l & 15u, kg = l >> 4;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the previous chunk's reads are done
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int rd = 0; rd < 3; rd++) {
            const uint32_t e0 = l + 64u * rd, e = e0 < 16 * Q4K_PIECES ? e0 : 16 * Q4K_PIECES - 1;
            st[i * 16 * Q4K_PIECES + e] = R.v[i][rd];  // lanes past the tile rewrite the last piece
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const uint8_t *blk = reinterpret_cast<const uint8_t *>(st + i * 16 * Q4K_PIECES) + rr * Q4K_BYTES;
        W.hd[i] = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
        for (int g = 0; g < 4; g++) W.qv[i][g] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * g + 8 * kg);
    }
}

// The fragment record of one chunk for TT token tiles, built by the workgroup from the
// activations: thread (token threadIdx.x / 16, q = threadIdx.x % 16) loads elements
// 16 q .. 16 q + 15 of the chunk (half of sub-block q / 2, k-groups 2 (q % 2) and
// 2 (q % 2) + 1) of each token tile, during the previous chunk's products, and stores
// their record words to LDS: the token's chunk maximum meets in DPP steps over its
// 16-lane row, and 2^e, the two f16 parts and the sub-block sums X follow as in
// the record layout.  XM: 0 = f32 activations, 1 = bf16, 2 = f32 silu(x) * up.
// Tokens past m repeat token m - 1 (each token's record is its own; their results are
// never stored).
template <int TT, int XM>
struct RecBuild {
    float v[TT][16];
    float u[XM == 2 ? TT : 1][16];
    __device__ __forceinline__ void load(const void *x, const float *up, uint32_t m, uint32_t k, uint32_t c) {
        const uint32_t tok = threadIdx.x >> 4, q = threadIdx.x & 15u;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const uint32_t tr = t * 16 + tok;
            const uint64_t e0 = (uint64_t)(tr < m ? tr : m - 1) * k + (uint64_t)QK_K * c + 16 * q;
            if constexpr (XM == 1) {
                const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + e0);
                const uint4 h0 = p[0], h1 = p[1];
                const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    v[t][2 * i] = bf16_to_f32(hw[i] & 0xFFFFu);
                    v[t][2 * i + 1] = __uint_as_float(hw[i] & 0xFFFF0000u);
                }
            } else {
                const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + e0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 f = p[i];
                    v[t][4 * i] = f.x;
                    v[t][4 * i + 1] = f.y;
                    v[t][4 * i + 2] = f.z;
                    v[t][4 * i + 3] = f.w;
                }
                if constexpr (XM == 2) {
                    const float4 *pu = reinterpret_cast<const float4 *>(up + e0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float4 f = pu[i];
                        u[t][4 * i] = f.x;
                        u[t][4 * i + 1] = f.y;
                        u[t][4 * i + 2] = f.z;
                        u[t][4 * i + 3] = f.w;
                    }
                }
            }
        }
    }
    __device__ __forceinline__ void store(uint4 *lds, uint32_t m) const {
        const uint32_t tok = threadIdx.x >> 4, q = threadIdx.x & 15u, j = q >> 1;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float w[16], amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float a = v[t][i];
                if constexpr (XM == 2) a = silu_mul(a, u[t][i]);  // kernels/activation.comp:21-28
                w[i] = a;
                amax = fmaxf(amax, fabsf(w[i]));
            }
            amax = row16_max(amax);
            // 2^e puts the chunk's largest magnitude in [2^14, 2^15); a zero or non-finite
            // chunk keeps e = 0 (non-finite values then reach the products as f16 inf / NaN)
            int e = 0;
            if (amax > 0.0f && amax <= 3.4028234664e38f) {
                e = 15 - __builtin_amdgcn_frexp_expf(amax);
                e = e < -126 ? -126 : (e > 126 ? 126 : e);
            }
            float sv[16], sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                sv[i] = __builtin_ldexpf(w[i], e);
                sum += sv[i];
            }
            // the two f16 parts of elements i, i + 2 in one word each (v_cvt_pk_f16_f32,
            // round to nearest even): hi the nearest f16, lo that of the exact remainder
            uint32_t hp[8], lp[8];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int i0 = 8 * (c >> 2) + (c & 1) + 4 * ((c >> 1) & 1), i1 = i0 + 2;
                const f16x2_t hv = __builtin_convertvector((f32x2_t){sv[i0], sv[i1]}, f16x2_t);
                const uint32_t hw = __builtin_bit_cast(uint32_t, hv);
                // sv - hi, exact, straight from the packed f16 halves (one v_fma_mix_f32 each)
                float r0, r1;
                asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r0) : "v"(hw), "v"(sv[i0]));
                asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r1) : "v"(hw), "v"(sv[i1]));
                const f16x2_t lv = __builtin_convertvector((f32x2_t){r0, r1}, f16x2_t);
                hp[c] = hw;
                lp[c] = __builtin_bit_cast(uint32_t, lv);
            }
            // the sub-block's sum: this thread's 16 and its neighbour's (q ^ 1), the same
            // float in both (addition is commutative)
            sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0xB1, 0xF, 0xF, false));
            uint4 *rec = lds + t * FR_U4;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t lane = ((q & 1u) * 2 + h) * 16 + tok;
                rec[(j * 2 + 0) * 64 + (lane ^ q)] = make_uint4(hp[4 * h], hp[4 * h + 1], hp[4 * h + 2], hp[4 * h + 3]);
                rec[(j * 2 + 1) * 64 + (lane ^ q)] = make_uint4(lp[4 * h], lp[4 * h + 1], lp[4 * h + 2], lp[4 * h + 3]);
            }
            float *rf = reinterpret_cast<float *>(rec);
            if ((q & 1u) == 0) rf[4 * FR_X + ((j & 3u) * 16 + tok) * 2 + (j >> 2)] = sum;
            if (q == 0) rf[4 * FR_S + tok] = __builtin_ldexpf(1.0f, -e);
        }
    }
};

// The chunk's min / bias terms and token scales: tmp += X (16x4) * coef (4x16) for
// sub-blocks kg and kg + 4, then acc += tmp * 2^-e per token.
template <int TT, int RT>
__device__ __forceinline__ void chunk_close(const uint4 *lds, f32x4 (&tmp)[RT][TT], const float (&cm)[RT][2],
                                            float (&acc)[RT][TT][4]) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
#pragma unroll
    for (int t = 0; t < TT; t++) {
        const float2 xv = reinterpret_cast<const float2 *>(lds + t * FR_U4 + FR_X)[l];
        const float4 sv = reinterpret_cast<const float4 *>(lds + t * FR_U4 + FR_S)[kg];
#pragma unroll
        for (int i = 0; i < RT; i++) {
            f32x4 C = tmp[i][t];
            C = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, cm[i][0], C, 0, 0, 0);
            C = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, cm[i][1], C, 0, 0, 0);
            acc[i][t][0] = __builtin_fmaf(C[0], sv.x, acc[i][t][0]);
            acc[i][t][1] = __builtin_fmaf(C[1], sv.y, acc[i][t][1]);
            acc[i][t][2] = __builtin_fmaf(C[2], sv.z, acc[i][t][2]);
            acc[i][t][3] = __builtin_fmaf(C[3], sv.w, acc[i][t][3]);
        }
    }
}

// The products of two sub-blocks (j0, j0 + 1) for every tile and token tile, each over
// both parts of A, and their scaled sum into tmp (started when `add` is false).  With
// one tile and one token tile both sub-blocks' products are issued before the scale
// multiplications (two independent chains); otherwise one sub-block at a time, whose
// RT * TT chains already overlap (and keep the register count down).
template <int TT, int RT>
__device__ __forceinline__ void mma_pair(const f16x8 (&A)[TT][2][2], const f16x8 (&B)[RT][2], const float (&a)[RT][8],
                                         int j0, bool add, f32x4 (&tmp)[RT][TT]) {
    constexpr int G = RT * TT == 1 ? 2 : 1;  // sub-blocks per group of products
#pragma unroll
    for (int u0 = 0; u0 < 2; u0 += G) {
        f32x4 D[RT][G][TT];
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int v = 0; v < G; v++)
#pragma unroll
                for (int t = 0; t < TT; t++)
                    D[i][v][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t][u0 + v][0], B[i][u0 + v],
                                                                        (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int v = 0; v < G; v++)
#pragma unroll
                for (int t = 0; t < TT; t++)
                    D[i][v][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t][u0 + v][1], B[i][u0 + v], D[i][v][t], 0,
                                                                        0, 0);
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int v = 0; v < G; v++)
#pragma unroll
                for (int t = 0; t < TT; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float aj = a[i][j0 + u0 + v];
                        tmp[i][t][r] = add || u0 + v > 0 ? __builtin_fmaf(aj, D[i][v][t][r], tmp[i][t][r])
                                                         : aj * D[i][v][t][r];
                    }
    }
}

// One Q4_K chunk: per tile the header's scales a_j = 2^24 d sc_j (2^20 for the high
// nibbles' sub-blocks) and the min coefficients -dmin m_j of sub-blocks kg, kg + 4.
// Per 64-element group g, every (tile, sub-block, token tile) product is issued before
// the scale multiplications that use them, so the matrix products overlap.
template <int TT, int RT>
__device__ __forceinline__ void q4k_chunk(const uint4 *lds, const Q4kChunk<RT> &W, float (&acc)[RT][TT][4]) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
    float a[RT][8], cm[RT][2];
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const float d = ref_half_hw(W.hd[i].x & 0xFFFFu), dmin = ref_half_hw(W.hd[i].x >> 16);
        const uint32_t s0 = W.hd[i].y, s1 = W.hd[i].z, s2 = W.hd[i].w;
        const uint32_t sl = s0 & 0x3F3F3F3Fu, sh = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
        const float d24 = d * 16777216.0f, d20 = d * 1048576.0f;
        a[i][0] = d24 * ubyte_f<0>(sl);
        a[i][1] = d20 * ubyte_f<1>(sl);
        a[i][2] = d24 * ubyte_f<2>(sl);
        a[i][3] = d20 * ubyte_f<3>(sl);
        a[i][4] = d24 * ubyte_f<0>(sh);
        a[i][5] = d20 * ubyte_f<1>(sh);
        a[i][6] = d24 * ubyte_f<2>(sh);
        a[i][7] = d20 * ubyte_f<3>(sh);
        const uint32_t sh8 = 8 * kg;
        const uint32_t m_lo = (s1 >> sh8) & 63u;
        const uint32_t m_hi = ((s2 >> (sh8 + 4)) & 15u) | (((s1 >> (sh8 + 6)) & 3u) << 4);
        cm[i][0] = -dmin * (float)m_lo;
        cm[i][1] = -dmin * (float)m_hi;
    }
    f32x4 tmp[RT][TT];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        f16x8 A[TT][2][2];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int p = 0; p < 2; p++)
                    A[t][u][p] = __builtin_bit_cast(
                        f16x8, lds[t * FR_U4 + ((2 * g + u) * 2 + p) * 64 + (l ^ (2 * (2 * g + u) + (l >> 5)))]);
        f16x8 B[RT][2];
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const uint32_t v0 = W.qv[i][g].x, v1 = W.qv[i][g].y, u0 = v0 >> 8, u1 = v1 >> 8;
            B[i][0] = as_f16x8(v0 & LO4, u0 & LO4, v1 & LO4, u1 & LO4);
            B[i][1] = as_f16x8(v0 & HI4, u0 & HI4, v1 & HI4, u1 & HI4);
        }
        mma_pair<TT, RT>(A, B, a, 2 * g, g > 0, tmp);
    }
    chunk_close<TT, RT>(lds, tmp, cm, acc);
}

// One Q8_0 chunk: a_j = 2^24 d_j, bias coefficients -128 d_j of blocks kg, kg + 4.
// Per pair of blocks, the products are issued before the scale multiplications.
template <int TT, int RT, bool BIASED>
__device__ __forceinline__ void q80_chunk(const uint4 *lds, const Q80Chunk<RT> &W, float (&acc)[RT][TT][4]) {
    const uint32_t l = threadIdx.x & 63u, kg = l >> 4;
    float a[RT][8], cm[RT][2];
#pragma unroll
    for (int i = 0; i < RT; i++) {
#pragma unroll
        for (int j = 0; j < 8; j++) a[i][j] = 16777216.0f * ref_half_hw((W.sc[i][j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
        // blocks kg and kg + 4: words kg / 2 and kg / 2 + 2, half kg % 2
        const uint32_t wl = kg < 2 ? W.sc[i][0] : W.sc[i][1], wh = kg < 2 ? W.sc[i][2] : W.sc[i][3];
        const uint32_t sh = 16 * (kg & 1u);
        cm[i][0] = -128.0f * ref_half_hw((wl >> sh) & 0xFFFFu);
        cm[i][1] = -128.0f * ref_half_hw((wh >> sh) & 0xFFFFu);
    }
    f32x4 tmp[RT][TT];
#pragma unroll
    for (int jp = 0; jp < 4; jp++) {
        f16x8 A[TT][2][2];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int p = 0; p < 2; p++)
                    A[t][u][p] = __builtin_bit_cast(
                        f16x8, lds[t * FR_U4 + ((2 * jp + u) * 2 + p) * 64 + (l ^ (2 * (2 * jp + u) + (l >> 5)))]);
        f16x8 B[RT][2];
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                // BIASED (tiles): the quants are stored as q + 128 already
                const uint32_t bias = BIASED ? 0u : 0x80808080u;
                const uint32_t v0 = W.qv[i][2 * jp + u].x ^ bias, v1 = W.qv[i][2 * jp + u].y ^ bias;
                B[i][u] = as_f16x8(v0 & LO8, (v0 >> 8) & LO8, v1 & LO8, (v1 >> 8) & LO8);
            }
        mma_pair<TT, RT>(A, B, a, 2 * jp, jp > 0, tmp);
    }
    chunk_close<TT, RT>(lds, tmp, cm, acc);
}

// The small-M product.  Wavefront w owns row tiles (4*bx + w)*RT .. +RT-1 (GLU: gate
// rows in wavefronts 0-1, up rows in 2-3) over chunks blockIdx.y*ch .. +ch-1 of k;
// x (and up) hold the launch's token tiles.  Software pipeline, per chunk c: the
// record of chunk c, built from the activations loaded during chunk c-1, is stored to
// LDS buffer c%2 and the workgroup meets at a barrier; then the activations of chunk
// c+1 and the weights of chunk c+2 (a ring of three chunks in registers) are issued,
// and chunk c is multiplied.
// Staged pieces per wavefront of the raw-block paths.
template <bool Q4, int RT>
constexpr uint32_t mm_spw() {
    return RT * 16 * (Q4 ? Q4K_PIECES : Q80_PIECES);
}

// The product of job J_ over TT token tiles; lrec holds two records of TT tiles,
// lstage (raw blocks) 4 mm_spw<Q4, RT>() pieces.
template <bool Q4, int TT, int RT, bool GLU, bool NORM, bool TILED, int XM>
__device__ __forceinline__ void mm_body(const void *x, const float *up, const MmJobs &jobs, uint32_t J_, uint32_t *cnt,
                                        uint32_t m, uint32_t k, uint64_t row_bytes, uint32_t ch, uint4 *lrec_base,
                                        lg_u32x4 *lstage) {
    MM_JOB_FIELDS;
    uint4 (*lrec)[TT * FR_U4] = reinterpret_cast<uint4 (*)[TT * FR_U4]>(lrec_base);
    // uniform over the wavefront: row-tile addresses are scalar
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rt0 = (GLU ? bx * 2 + (wave & 1u) : bx * 4 + wave) * RT;
    const uint32_t nb = k / QK_K, c0 = blockIdx.y * ch, nch = nb - c0 < ch ? nb - c0 : ch;
    // raw blocks: rows through a per-wavefront LDS region
    constexpr bool RAW8 = !Q4 && !TILED, RAW4 = Q4 && !TILED;
    constexpr uint32_t SPW = mm_spw<Q4, RT>();
    using Chunk = typename std::conditional<
        Q4, typename std::conditional<RAW4, Q4kRawChunk<RT>, Q4kChunk<RT>>::type,
        typename std::conditional<RAW8, Q80RawChunk<RT>, Q80Chunk<RT>>::type>::type;
    Chunk Wc[3];
    // chunk ci of the slice; past the slice the last chunk again (loads stay in bounds,
    // never multiplied)
    auto load_w = [&](Chunk &Wd, uint32_t ci) {
        const uint32_t c = c0 + (ci < nch ? ci : nch - 1);
        if constexpr (RAW4) load_q4k_raw<RT>(Wd, w, n, rt0, c, row_bytes);
        else if constexpr (Q4) load_q4k<RT, TILED>(Wd, w, n, rt0, nb, c, row_bytes);
        else if constexpr (RAW8) load_q80_raw<RT>(Wd, w, n, rt0, c, row_bytes);
        else load_q80_tiled<RT>(Wd, w, n, rt0, nb, c);
    };
    float acc[RT][TT][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][t][r] = 0.0f;
    RecBuild<TT, XM> rb;
    rb.load(x, up, m, k, c0);
    load_w(Wc[0], 0);
    load_w(Wc[1], 1);
    // chunk 0 ahead of the loop, so the loop is entered in the state it repeats
    rb.store(lrec[0], m);
    __syncthreads();
    rb.load(x, up, m, k, c0 + (1 < nch ? 1 : 0));
    __builtin_amdgcn_sched_barrier(0);  // issue order: the activations, then the weights
    load_w(Wc[2], 2);
    __builtin_amdgcn_sched_barrier(0);
    auto chunk = [&](const uint4 *rec, const Chunk &Wk) {
        if constexpr (RAW4) {
            Q4kChunk<RT> Ws;
            stage_q4k<RT>(Wk, Ws, lstage + wave * SPW);
            q4k_chunk<TT, RT>(rec, Ws, acc);
        } else if constexpr (Q4) {
            q4k_chunk<TT, RT>(rec, Wk, acc);
        } else if constexpr (RAW8) {
            Q80Chunk<RT> Ws;
            stage_q80<RT>(Wk, Ws, lstage + wave * SPW);
            q80_chunk<TT, RT, false>(rec, Ws, acc);
        } else {
            q80_chunk<TT, RT, TILED>(rec, Wk, acc);
        }
    };
    chunk(lrec[0], Wc[0]);
    // three chunks per iteration, so the ring's registers are named at compile time
    // (chunk c in Wc[c % 3]: ci = 1 mod 3)
    for (uint32_t ci = 1; ci < nch; ci += 3) {
#pragma unroll
        for (int h = 0; h < 3; h++) {
            const uint32_t c = ci + h;
            if (c >= nch) break;  // uniform
            rb.store(lrec[c & 1u], m);
            __syncthreads();
            rb.load(x, up, m, k, c0 + (c + 1 < nch ? c + 1 : nch - 1));
            __builtin_amdgcn_sched_barrier(0);
            load_w(Wc[h], c + 2);
            __builtin_amdgcn_sched_barrier(0);
            chunk(lrec[c & 1u], Wc[(h + 1) % 3]);
        }
    }
    static_assert(!GLU || 2 * RT * TT * 256 * 4 <= 2 * TT * FR_U4 * 16, "GLU exchange fits in the record LDS");
    static_assert(RT != 2 || 8 * TT * 256 * 4 <= 2 * TT * FR_U4 * 16, "the head exchange fits in the record LDS");
    finish<TT, RT, GLU, NORM>(acc, out, res, part, cnt, rt0, m, n, reinterpret_cast<float *>(lrec_base), jobs, k,
                              jobs.j[J_].y, jobs.j[J_].yw, jobs.j[J_].ss, bx, jobs.j[J_].qkw);
}

template <bool Q4, int TT, int RT, bool GLU, bool NORM, bool TILED, int XM>
__global__ __launch_bounds__(256) void k_mm_mf(const void *x, const float *up, MmJobs jobs, uint32_t *cnt, uint32_t m,
                                               uint32_t k, uint64_t row_bytes, uint32_t ch) {
    MM_JOB_INDEX;
    __shared__ uint4 lrec[2 * TT * FR_U4];
    __shared__ lg_u32x4 lstage[TILED ? 1 : 4 * mm_spw<Q4, RT>()];
    if constexpr (TT == 2 && !GLU && XM == 0) {
        if (jobs.j[J_].tlo) {  // uniform: this job takes token rows 16 .. m - 1 only (one tile)
            // a launch of that one job, held as job 0 (static indices: no private copy)
            MmJobs j1;
            j1.j[0] = jobs.j[J_];
            j1.j[0].out += (uint64_t)16 * j1.j[0].n;
            if (j1.j[0].res) j1.j[0].res += (uint64_t)16 * j1.j[0].n;
            j1.count = 1;
            j1.tiled = jobs.tiled;
            j1.rs_cols = jobs.rs_cols;
            j1.rs_eps = jobs.rs_eps;
            // the folded norm's rows, relative to the tile
            j1.rs_ss = jobs.rs_ss + (uint64_t)(jobs.rs_tok0 < 16 ? 16 - jobs.rs_tok0 : 0) * jobs.rs_cols;
            j1.rs_tok0 = jobs.rs_tok0 > 16 ? jobs.rs_tok0 - 16 : 0;
            j1.rope = jobs.rope ? jobs.rope + 16 * 128 : nullptr;
            j1.qk_eps = jobs.qk_eps;
            mm_body<Q4, 1, RT, GLU, NORM, TILED, XM>(static_cast<const float *>(x) + (uint64_t)16 * k, up, j1, 0u, cnt,
                                                     m - 16, k, row_bytes, ch, lrec, lstage);
            return;
        }
    }
    mm_body<Q4, TT, RT, GLU, NORM, TILED, XM>(x, up, jobs, J_, cnt, m, k, row_bytes, ch, lrec, lstage);
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

// Launch shape: RT 16-row tiles per wavefront, `ch` chunks of 256 elements per k
// slice, `slices` = ceil(nb / ch) workgroup rows.  Automatic choice: RT = 2 (RT = 1
// when that gives fewer than 256 workgroup columns... see mm_shape), and slices so
// that columns x slices is about MM_TARGET_PER_CU workgroups per compute unit.
struct MmShape {
    uint32_t ch, slices, rt;
};

std::atomic<uint32_t> g_mm_ch{0}, g_mm_rt{0};  // launch-shape overrides (0 = automatic)
constexpr uint32_t MM_TARGET_PER_CU = 2;

// n: rows per workgroup column's job span (the jobs' total rows; a gate/up pair's n);
// rows_per_wave_tile: 16.  glu: both products in every column (32 RT rows each).
// epi: the job writes a folded norm's per-column sums of squares, whose consumers read
// at most proj_batch_rs_cols_max partial sums per token: at most 64 columns.
MmShape mm_shape(int dtype, uint32_t k, uint32_t n, uint32_t m, bool glu, bool qk, bool epi = false) {
    const uint32_t nb = k / QK_K;
    const uint32_t cus = (uint32_t)device_cus(), target = MM_TARGET_PER_CU * cus;
    const uint32_t per = glu ? 32u : 64u;  // rows per column and row tile per wavefront
    uint32_t rt = 2;
    if ((n + per * 2 - 1) / (per * 2) < cus / 4) rt = 1;
    // a gate/up pair with at least one RT = 1 column per CU: no k split, so no partial
    // sums and no finishing workgroup (the draft's 14336-row pair: 448 columns of whole
    // k against 224 x 2 slices, 610.2 -> 604.9 us per block forward)
    if (glu && m <= 16 && (n + per - 1) / per >= cus) rt = 1;
    const uint32_t ort = g_mm_rt.load(std::memory_order_relaxed);
    if (ort) rt = ort >= 4 ? 4 : ort >= 2 ? 2 : 1;
    if (dtype != LG_Q4_K && rt > 2) rt = 2;  // register budget of the Q8_0 chunk
    if (m > 16 && rt > 2) rt = 2;
    if (qk) rt = 2;  // whole heads of 128 rows per column
    while (epi && rt < 2 && (n + per * rt - 1) / (per * rt) > 64) rt *= 2;
    const uint32_t cols = (n + per * rt - 1) / (per * rt);
    // two token tiles of two row tiles take every register of a SIMD (one workgroup per
    // CU): about 9/8 workgroups per CU instead (the 32-row K/V/Q launch of the draft
    // block: 610 against 624 us per block forward with 2 per CU, 614 with 3/4 per CU)
    const uint32_t tgt = m > 16 && rt == 2 ? cus * 9 / 8 : target;
    uint32_t slices = (tgt + cols / 2) / cols;
    slices = slices < 1 ? 1 : (slices > nb ? nb : slices);
    uint32_t ch = nb ? (nb + slices - 1) / slices : 1;
    const uint32_t och = g_mm_ch.load(std::memory_order_relaxed);
    if (och) ch = och < nb ? och : (nb ? nb : 1);
    ch = ch ? ch : 1;
    return {ch, nb ? (nb + ch - 1) / ch : 1, rt};
}

template <bool Q4, int TT, bool GLU, bool NORM, bool TILED, int XM>
void launch_rt(uint32_t rt, dim3 grid, const void *x, const float *up, const MmJobs &jobs, uint32_t *cnt, uint32_t m,
               uint32_t k, uint64_t rb, uint32_t ch, hipStream_t s) {
#define LG_MM(R)                                                                                                  \
    hipLaunchKernelGGL((k_mm_mf<Q4, TT, R, GLU, NORM, TILED, XM>), grid, dim3(256), 0, s, x, up, jobs, cnt, m, k, rb, \
                       ch)
    if constexpr (Q4 && TT == 1)
        if (rt == 4) {
            LG_MM(4);
            return;
        }
    if (rt == 2) {
        LG_MM(2);
        return;
    }
    LG_MM(1);
#undef LG_MM
}

// XM (activation kind) other than plain f32 only for plain products (no pair, no norm)
template <bool Q4, bool GLU, bool NORM, int XM>
void launch_tt(uint32_t tt, bool tiled, uint32_t rt, dim3 grid, const void *x, const float *up, const MmJobs &jobs,
               uint32_t *cnt, uint32_t m, uint32_t k, uint64_t rb, uint32_t ch, hipStream_t s) {
    if (tt == 2) {
        if (tiled) launch_rt<Q4, 2, GLU, NORM, true, XM>(rt, grid, x, up, jobs, cnt, m, k, rb, ch, s);
        else launch_rt<Q4, 2, GLU, NORM, false, XM>(rt, grid, x, up, jobs, cnt, m, k, rb, ch, s);
    } else {
        if (tiled) launch_rt<Q4, 1, GLU, NORM, true, XM>(rt, grid, x, up, jobs, cnt, m, k, rb, ch, s);
        else launch_rt<Q4, 1, GLU, NORM, false, XM>(rt, grid, x, up, jobs, cnt, m, k, rb, ch, s);
    }
}

template <bool Q4>
void launch_q(int xm, bool tiled, bool glu, bool norm, uint32_t tt, const MmShape &sh, dim3 grid, const void *x,
              const float *up, const MmJobs &jobs, uint32_t *cnt, uint32_t m, uint32_t k, uint64_t rb, hipStream_t s) {
    if (xm == 1) launch_tt<Q4, false, false, 1>(tt, tiled, sh.rt, grid, x, up, jobs, cnt, m, k, rb, sh.ch, s);
    else if (xm == 2) launch_tt<Q4, false, false, 2>(tt, tiled, sh.rt, grid, x, up, jobs, cnt, m, k, rb, sh.ch, s);
    else if (glu && norm) launch_tt<Q4, true, true, 0>(tt, tiled, sh.rt, grid, x, up, jobs, cnt, m, k, rb, sh.ch, s);
    else if (glu) launch_tt<Q4, true, false, 0>(tt, tiled, sh.rt, grid, x, up, jobs, cnt, m, k, rb, sh.ch, s);
    else if (norm) launch_tt<Q4, false, true, 0>(tt, tiled, sh.rt, grid, x, up, jobs, cnt, m, k, rb, sh.ch, s);
    else launch_tt<Q4, false, false, 0>(tt, tiled, sh.rt, grid, x, up, jobs, cnt, m, k, rb, sh.ch, s);
}

int launch_mm(int dtype, int xm, bool tiled, bool glu, bool norm, uint32_t tt, const MmShape &sh, uint32_t groups,
              const void *x, const float *up, const MmJobs &jobs, uint32_t *cnt, uint32_t m, uint32_t k,
              hipStream_t s) {
    const dim3 grid(groups, sh.slices);
    const uint64_t rb = dtype == LG_Q4_K ? (uint64_t)k / QK_K * Q4K_BYTES : (uint64_t)k / QK8_0 * Q80_BYTES;
    if (dtype == LG_Q4_K) launch_q<true>(xm, tiled, glu, norm, tt, sh, grid, x, up, jobs, cnt, m, k, rb, s);
    else launch_q<false>(xm, tiled, glu, norm, tt, sh, grid, x, up, jobs, cnt, m, k, rb, s);
    return after_launch(dtype == LG_Q4_K ? "proj_q4k_mm" : "proj_q8_0_mm", s);
}

uint64_t align256(uint64_t b) { return (b + 255) & ~(uint64_t)255; }

// Workspace layout: the arrival counters at a fixed place (offset 0, one per
// workgroup column, CNT_MAX of them) so that every call finds them zero, then the
// partial sums, job after job, then the fragment records of every token tile.
constexpr uint64_t CNT_BYTES = PROJ_WS_COUNTERS;
constexpr uint32_t CNT_MAX = CNT_BYTES / 4;

// The shape of the launch over the token tiles 16 t0 .. (pairs of tiles; ml rows).
MmShape launch_shape(int w_dtype, uint32_t k, const uint32_t *n, uint32_t jobs, uint32_t ml, bool glu, bool qk,
                     bool epi) {
    uint64_t ntot = 0;
    for (uint32_t j = 0; j < jobs; j++) ntot += n[j];
    return mm_shape(w_dtype, k, glu ? n[0] : (uint32_t)ntot, ml, glu, qk, epi);
}

// Floats of one job's split-k partials (finish): per workgroup column and slice, four
// wavefronts' RT x TT tiles of 256 values (columns of 64 RT rows, or 32 RT for a gate/up
// pair, whose two jobs share the columns).
uint64_t mm_part_floats(uint32_t n, uint32_t ml, uint32_t rt, uint32_t slices, bool glu) {
    const uint32_t per = (glu ? 32u : 64u) * rt, cols = (n + per - 1) / per, tt = (ml + 15) / 16;
    return (uint64_t)slices * cols * 4 * rt * tt * 256;
}

}  // namespace

namespace lg {

// The workspace of one call: counters, partial sums of the largest tile pair, records.
static uint64_t multi_ws_bytes(uint32_t k, const uint32_t *n, uint32_t jobs, uint32_t m, int w_dtype, bool glu,
                               bool qk, bool epi) {
    if (w_dtype == LG_Q4_K_T16) w_dtype = LG_Q4_K;
    if (w_dtype == LG_Q8_0_T16) w_dtype = LG_Q8_0;
    if ((w_dtype != LG_Q4_K && w_dtype != LG_Q8_0) || k % QK_K || m == 0) return 0;
    const uint32_t ml = m < 32 ? m : 32;
    const MmShape sh = launch_shape(w_dtype, k, n, jobs, ml, glu, qk, epi);
    uint64_t b = CNT_BYTES;
    if (sh.slices > 1)
        for (uint32_t j = 0; j < jobs; j++) b += align256(mm_part_floats(n[j], ml, sh.rt, sh.slices, glu) * 4);
    return b;
}

uint64_t proj_batch_multi_ws_bytes(uint32_t k, const uint32_t *n, uint32_t jobs, uint32_t m, int w_dtype) {
    // the largest of the plain, norm-producing, gate/up (two jobs of equal n) and
    // QK-normed shapes
    uint64_t b = multi_ws_bytes(k, n, jobs, m, w_dtype, false, false, false);
    const uint64_t q = multi_ws_bytes(k, n, jobs, m, w_dtype, false, true, false);
    b = q > b ? q : b;
    const uint64_t e = multi_ws_bytes(k, n, jobs, m, w_dtype, false, false, true);
    b = e > b ? e : b;
    if (jobs == 2 && n[0] == n[1]) {
        const uint64_t g = multi_ws_bytes(k, n, jobs, m, w_dtype, true, false, false);
        b = g > b ? g : b;
    }
    return b;
}

uint64_t proj_batch_ws_bytes(uint32_t k, uint32_t n, uint32_t m, int x_dtype, int w_dtype) {
    (void)x_dtype;
    const uint64_t a = multi_ws_bytes(k, &n, 1, m, w_dtype, false, false, false);
    const uint64_t e = multi_ws_bytes(k, &n, 1, m, w_dtype, false, false, true);
    return a > e ? a : e;
}

uint32_t proj_batch_norm_cols(int w_dtype, uint32_t k, uint32_t n, uint32_t m) {
    if (w_dtype == LG_Q4_K_T16) w_dtype = LG_Q4_K;
    if (w_dtype == LG_Q8_0_T16) w_dtype = LG_Q8_0;
    const MmShape sh = mm_shape(w_dtype, k, n, m < 32 ? m : 32, false, false, true);
    return (n + 64 * sh.rt - 1) / (64 * sh.rt);
}

uint32_t proj_batch_rs_cols_max(uint32_t m) { return MM_SS_LOADS * (m > 16 ? 8u : 16u); }

bool proj_batch_mfma_ok(int w_dtype, uint32_t k, const void *w) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(w);
    if (w_dtype == LG_Q4_K_T16 || w_dtype == LG_Q8_0_T16) return k && k % QK_K == 0 && (a & 15u) == 0;
    if (w_dtype == LG_Q4_K) return k && k % QK_K == 0 && (a & 15u) == 0;
    if (w_dtype == LG_Q8_0) return k && k % QK_K == 0 && (a & 15u) == 0;  // rows staged with 16-byte loads
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
    bool fast = k && w_dtype != LG_F32 && k % QK_K == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                (!up || (reinterpret_cast<uintptr_t>(up) & 15u) == 0);
    for (uint32_t j = 0; j < njobs; j++)
        fast = fast && (w_dtype != LG_Q4_K || (reinterpret_cast<uintptr_t>(jb[j].w) & 15u) == 0) &&
               (reinterpret_cast<uintptr_t>(jb[j].w) & 1u) == 0;
    LG_REQUIRE(fast || !(norm || epi || qkn), "%s: a folded RMSNorm or QK-norm needs the matrix-core path (k a "
               "multiple of 256, aligned operands)", name);
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
    const uint64_t need = multi_ws_bytes(k, nv, njobs, m, w_dtype, glu, qkn, epi);
    void *ws = ws_given;
    if (ws) {
        LG_REQUIRE(ws_bytes >= need, "%s: workspace of %llu bytes too small (%llu needed)", name,
                   (unsigned long long)ws_bytes, (unsigned long long)need);
    } else {
        LG_TRY(stream_workspace(s, need, &ws));
    }
    const uint32_t tiles = (m + 15) / 16;
    const uint64_t xsz = x_dtype == LG_F32 ? 4 : 2;
    const int xm = x_dtype == LG_BF16 ? 1 : (up ? 2 : 0);
    for (uint32_t t0 = 0; t0 < tiles; t0 += 2) {  // pairs of 16-token tiles
        const uint32_t ml = m - 16 * t0 < 32 ? m - 16 * t0 : 32, tt = (ml + 15) / 16;
        const MmShape sh = launch_shape(w_dtype, k, nv, njobs, ml, glu, qkn, epi);
        uint32_t *cnt = static_cast<uint32_t *>(ws);
        uint8_t *pb = static_cast<uint8_t *>(ws) + CNT_BYTES;
        MmJobs jobs{};
        uint32_t groups = 0;
        for (uint32_t j = 0; j < njobs; j++) {
            const uint64_t off = (uint64_t)16 * t0 * jb[j].n;
            // a job whose rows below 16 t0 + 16 are not needed skips the pair's first tile
            const uint32_t tlo = tt == 2 && !glu && xm == 0 && !jb[j].ss && jb[j].row0 >= 16 * t0 + 16 ? 1u : 0u;
            jobs.j[j] = {static_cast<const uint8_t *>(jb[j].w), jb[j].c + off, jb[j].res ? jb[j].res + off : nullptr,
                         reinterpret_cast<float *>(pb), jb[j].y, jb[j].yw, jb[j].ss, jb[j].n, groups, jb[j].qkw, tlo};
            if (sh.slices > 1) pb += align256(mm_part_floats(jb[j].n, ml, sh.rt, sh.slices, glu) * 4);
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
        LG_REQUIRE(groups <= CNT_MAX, "%s: %u workgroup columns exceed %u", name, groups, CNT_MAX);
        const void *xt = static_cast<const uint8_t *>(x) + (uint64_t)16 * t0 * k * xsz;
        const float *ut = up ? up + (uint64_t)16 * t0 * k : nullptr;
        LG_TRY(launch_mm(w_dtype, xm, tiled, glu, pnorm, tt, sh, groups, xt, ut, jobs, cnt, ml, k, s));
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
        // quants biased to unsigned (q + 128 = q XOR 0x80), as the products take them
        const uint2 v = make_uint2((src[0] | ((uint32_t)src[1] << 16)) ^ 0x80808080u,
                                   (src[2] | ((uint32_t)src[3] << 16)) ^ 0x80808080u);
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
    const uint64_t need = lg::proj_batch_ws_bytes(k, n, m, x_dtype, w_dtype);
    LG_REQUIRE(need <= STATIC_SCRATCH_BYTES,
               "%s: k=%u n=%u m=%u needs %llu bytes of scratch, more than the %llu this entry point has", name, k, n,
               m, (unsigned long long)need, (unsigned long long)STATIC_SCRATCH_BYTES);
    int dev = 0;
    LG_HIP_TRY(hipGetDevice(&dev));
    void *ws = nullptr;
    LG_TRY(static_scratch(dev, (hipStream_t)stream, false, &ws));
    return lg::proj_batch(x, x_dtype, w, c, k, n, m, w_dtype, ws, STATIC_SCRATCH_BYTES, (hipStream_t)stream);
}

extern "C" uint64_t lg_proj_quant_batch_ws_bytes(uint32_t k, uint32_t n, uint32_t m, int w_dtype) {
    if (n == 0 || m == 0 || m > 64) return 0;
    return lg::proj_batch_ws_bytes(k, n, m, LG_F32, w_dtype);
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
