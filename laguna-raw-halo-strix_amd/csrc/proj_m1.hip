// M = 1 projections: c[i] = sum_j x[j] * W[i,j] over raw GGUF blocks.
//
// Replaces kernels/proj_q4k.comp, proj_q8_0.comp, proj.comp and activation.comp
// (one invocation per output row, per-element byte decode, uncoalesced) with
// gfx950 kernels.
//
// Q4_K (k % 256 == 0, 16-byte aligned tensor), kernels chosen by measurement:
//  * plain projections with k <= 4096: integer dot products of the raw nibbles
//    against byte digits of the activations (k_q4k_m1_dig, described there).
//  * plain projections with 4096 < k <= 16384: k_q4k_m1_wide, as the fused path below.
//  * plain projections with k > 16384: vector ALU (k_q4k_m1).  Lane p of a row
//    team (up to 4 waves, 16384 elements per pass; longer rows take several passes)
//    owns the 64-element group p of the pass; a nibble masked in place is an
//    f16 subnormal (q * 2^-24, or q * 2^-20 for a high nibble), so one AND gives two
//    operands of v_fma_mix_f32 against the f32 activations, and the block's scale
//    and min enter once per 32-element sub-block:
//        sum_j x_j ((d sc) q_j - dmin m) = d sc 2^24 S - dmin m X,
//        S = sum x q 2^-24,  X = sum x (per lane, once).
//  * the fused SiLU(gate)*up down projection: int8 matrix cores, k_q4k_m1_wide (one
//    workgroup per 16 rows holds all of k, k <= 16384; described there) or, beyond,
//    k_q4k_m1_mfma.
//    In both, the activations become exact integers (three signed byte digits per
//    element, one power-of-two scale per 256-element super-block) and the raw nibbles
//    are the other operand, so a byte product costs no decode; each (row, sub-block)
//    pair gets its scale and min once, in an f32 epilogue.  k_q4k_m1_mfma splits work
//    over workgroups by rows and by k (each workgroup computes SiLU for, and converts,
//    only its k slice); the slices of a row range are summed in slice order by
//    the last workgroup to finish.
//
// Q8_0 with k <= 4096: integer dot products against activation digits (k_q80_m1_dig,
// described there).  Q8_0 with k > 4096: vector ALU.  A "team" of TW = min(4, ceil(k/4096)) waves covers one row (in
// passes of 16384 elements beyond that): lane p of
// the team owns the 64-element group p of the row (two 34-byte blocks, 68 bytes,
// dword aligned) and keeps the 64 activations of that group in registers; the
// team's partial sums meet in a DPP/swizzle wavefront reduction (plus LDS across
// the TW waves).  A workgroup holds TEAMS teams (8 waves); each team owns RPW
// contiguous rows and issues all their loads before the activations are staged.
// Each wave loads its 64-group share of a row with coalesced 16-byte loads, writes
// it to its own LDS stage and each lane reads its 17 dwords back (stride 17 dwords:
// no bank conflicts).  Bytes are biased to unsigned (q + 128), converted with
// v_cvt_f32_ubyte and corrected by 128 X per block.
//
// Inputs outside these fast paths (k not a multiple of 256, unaligned pointers,
// element offsets that are not block aligned) go to a per-element kernel that
// follows the reference's linear addressing exactly (lin = offset + i*k + j).
#include <map>
#include <mutex>

#include "lg_common.hpp"

namespace {

using namespace lg;

std::atomic<uint32_t> g_grid_cap{0};  // 0 = automatic

constexpr int M1_RPW_MAX = 8;         // rows per team whose loads are in flight together

// ------------------------------------------------------------------------------------------
// activations

__device__ __forceinline__ float silu_mul(float g, float u) {
    // kernels/activation.comp:21-28: silu(g) * up, silu(x) = x * (1 / (1 + exp(-x)))
    return g * (1.0f / (1.0f + expf(-g))) * u;
}

// The same with the hardware exp2 and reciprocal (v_exp_f32 of -g log2(e), v_rcp_f32:
// each about 1 ulp; non-finite g gives what silu_mul gives), for the fused down
// projections, whose every workgroup stages all of k: a few instructions instead of
// the IEEE exp and divide sequences.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// The workgroup's copy of the activations, in two halves so that the row loads
// can be issued in between:
//   x_fetch: this thread's float4s of x (and up) into registers;
//   x_share: (with FUSE: silu(x) * up) into LDS, one barrier, and lane p of wave wt
//            takes elements 64p .. 64p+63 of the team's k range into registers.
// LDS rows are padded to 68 floats (64 + 4) so that the lanes' 16-byte reads
// spread over the banks.  `xs` holds TW * 64 * 68 floats.
template <int XPT, bool FUSE>
struct XFetch {
    float4 x[XPT];
    float4 u[FUSE ? XPT : 1];
};

template <int XPT, bool FUSE>
__device__ __forceinline__ void x_fetch(XFetch<XPT, FUSE> &f, const float *__restrict__ x,
                                        const float *__restrict__ up, uint32_t k) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *u4 = reinterpret_cast<const float4 *>(up);
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const uint32_t e4 = threadIdx.x + i * blockDim.x;
        if (e4 < k / 4) {
            f.x[i] = x4[e4];
            if constexpr (FUSE) f.u[i] = u4[e4];
        }
    }
}

template <int XPT, bool FUSE>
__device__ __forceinline__ void x_share(const XFetch<XPT, FUSE> &f, uint32_t k, uint32_t wt, uint32_t lane,
                                        float *xs, float (&xr)[64]) {
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const uint32_t e4 = threadIdx.x + i * blockDim.x;
        if (e4 < k / 4) {
            float4 v = f.x[i];
            if constexpr (FUSE) {
                const float4 u = f.u[i];
                v = make_float4(silu_mul_fast(v.x, u.x), silu_mul_fast(v.y, u.y), silu_mul_fast(v.z, u.z),
                                silu_mul_fast(v.w, u.w));
            }
            const uint32_t e = 4 * e4;
            *reinterpret_cast<float4 *>(xs + e + 4 * (e >> 6)) = v;
        }
    }
    __syncthreads();
    const float4 *s4 = reinterpret_cast<const float4 *>(xs + 68 * (wt * 64 + lane));
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float4 v = s4[i];
        xr[4 * i] = v.x, xr[4 * i + 1] = v.y, xr[4 * i + 2] = v.z, xr[4 * i + 3] = v.w;
    }
}


__device__ __forceinline__ float h_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }
__device__ __forceinline__ float h_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// Team sums of the RPW row partials and their stores.  TW == 1: DPP/swizzle only.
// TW > 1: every wave's wavefront sums go to LDS, one barrier, wave 0 of the team
// adds the TW partials of each row.  Every wave of the workgroup calls this once.
// A row sum that is not finite is replaced by redo(row), the wavefront's element-by-element
// sum in the reference's terms: the vector kernels' split into S and X turns an inf among
// the activations into inf - inf (NaN) where the reference's loop gives inf.  Each sum is
// taken from one lane (TW == 1) or read from LDS by every lane, so that branch is uniform.
template <int TW, int TEAMS, int RPW, class Redo>
__device__ __forceinline__ void team_store(float (&acc)[RPW], uint32_t row0, uint32_t n, float *__restrict__ y,
                                           float *red, uint32_t team, uint32_t lane, uint32_t wt, const Redo &redo) {
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = wave_sum(acc[r]);
    if constexpr (TW == 1) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float s = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(acc[r])));  // lane 0's sum
            if (row0 + r < n) {
                if (!__builtin_isfinite(s)) s = redo(row0 + r);
                if (lane == 0) y[row0 + r] = s;
            }
        }
    } else {
        float *buf = red + team * (RPW * TW);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RPW; r++) buf[r * TW + wt] = acc[r];
        }
        __syncthreads();
        if (wt == 0) {
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                if (row0 + r >= n) break;
                float s = 0.0f;
#pragma unroll
                for (int t = 0; t < TW; t++) s += buf[r * TW + t];
                if (!__builtin_isfinite(s)) s = redo(row0 + r);
                if (lane == 0) y[row0 + r] = s;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Q4_K

struct Q4Lane {
    uint32_t g;                           // group within the super-block (0..3): sub-blocks 2g, 2g+1
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

// One element of the weights decoded at the reference's linear index
// (kernels/proj_q4k.comp:67, proj_q8_0.comp:54).
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

// One lane's contribution to one row: 64 weights of super-block header `hd`
// (d, dmin, scales) and quant bytes qa (bytes 0-15 of the group) and qb (16-31).
// A nibble masked in place is read as an f16 subnormal: low nibbles as q * 2^-24,
// high nibbles as 16 q * 2^-24 = q * 2^-20 (exact; v_fma_mix_f32 keeps f16
// denormals), so one AND yields two operands and no bias has to be removed:
//     S0 = sum x q 2^-24 (sub-block 2g),  S1 = sum x q 2^-20 (sub-block 2g+1)
//     sum_j x_j ((d sc) q_j - dmin m) = d sc 2^24 S0 - dmin m X0   (and 2^20 S1, X1).
__device__ __forceinline__ float q4_dot(const uint4 &hd, const uint4 &qa, const uint4 &qb, const float (&xr)[64],
                                        float X0, float X1, const Q4Lane &L) {
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    float s0a = 0.f, s0b = 0.f, s1a = 0.f, s1b = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const uint32_t v = q[t], v8 = q[t] >> 8;
        const uint32_t l02 = v & 0x000F000Fu;   // low nibbles of bytes 4t, 4t+2  -> sub-block 2g
        const uint32_t l13 = v8 & 0x000F000Fu;  // low nibbles of bytes 4t+1, 4t+3
        const uint32_t h02 = v & 0x00F000F0u;   // high nibbles of bytes 4t, 4t+2 -> sub-block 2g+1
        const uint32_t h13 = v8 & 0x00F000F0u;  // high nibbles of bytes 4t+1, 4t+3
        s0a = __builtin_fmaf(xr[4 * t + 0], h_lo(l02), s0a);
        s0b = __builtin_fmaf(xr[4 * t + 1], h_lo(l13), s0b);
        s0a = __builtin_fmaf(xr[4 * t + 2], h_hi(l02), s0a);
        s0b = __builtin_fmaf(xr[4 * t + 3], h_hi(l13), s0b);
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
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t sc = __builtin_amdgcn_ubfe(srcA, L.sa[u], 4) | (__builtin_amdgcn_ubfe(hd.y, L.sb[u], 2) << 4);
        const uint32_t mn = __builtin_amdgcn_ubfe(srcM, L.ma[u], 4) | (__builtin_amdgcn_ubfe(hd.z, L.mb[u], 2) << 4);
        const float a = d * (float)sc * (u ? 1048576.0f : 16777216.0f);  // d sc 2^24 (low), 2^20 (high)
        const float S = u ? S1 : S0, X = u ? X1 : X0;
        acc = __builtin_fmaf(a, S, acc);
        acc = __builtin_fmaf(-(dmin * (float)mn), X, acc);
    }
    return acc;
}

// Rows row0 .. row0+RPW-1 of the team, loaded all at once (rows past n clamp to n-1
// and are not stored).  Then the activations, then one row at a time as it lands.
// k beyond one pass of the team (TW * 4096 elements) is covered in passes whose
// partial sums accumulate per row.
template <int TW, int TEAMS, int RPW, bool FUSE>
__global__ __launch_bounds__(TW *TEAMS * 64) void k_q4k_m1(const float *__restrict__ x, const float *__restrict__ up,
                                                            const uint8_t *__restrict__ w, float *__restrict__ y,
                                                            uint32_t k, uint32_t n, uint64_t row_bytes) {
    constexpr int XPT = (16 * TW + TEAMS * TW - 1) / (TEAMS * TW);
    constexpr uint32_t KPASS = TW * 64 * 64;  // elements one pass covers
    __shared__ __attribute__((aligned(16))) float xs[TW * 64 * 68];
    __shared__ float red[TW > 1 ? TEAMS * RPW * TW : 1];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t team = wave / TW, wt = wave % TW;
    const uint32_t p0 = wt * 64 + lane;
    const Q4Lane L = q4_lane(p0 & 3u);  // passes start at multiples of 256 elements: the same group parity
    const uint32_t qoff = 16 + 32 * L.g;
    const uint32_t row0 = (blockIdx.x * TEAMS + team) * RPW;

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = 0.0f;
    for (uint32_t c0 = 0; c0 < k; c0 += KPASS) {  // uniform over the workgroup
        const uint32_t kc = k - c0 < KPASS ? k - c0 : KPASS;
        const bool active = p0 < (kc >> 6);
        const uint32_t p = active ? p0 : 0;  // idle lanes read group 0 and contribute 0
        const uint64_t lane_off = (uint64_t)(c0 / QK_K + (p >> 2)) * Q4K_BYTES;
        XFetch<XPT, FUSE> xf;
        x_fetch<XPT, FUSE>(xf, x + c0, FUSE ? up + c0 : up, kc);
        uint4 hd[RPW], qa[RPW], qb[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const uint32_t row = row0 + r < n ? row0 + r : n - 1;
            const uint8_t *blk = w + (uint64_t)row * row_bytes + lane_off;
            hd[r] = *reinterpret_cast<const uint4 *>(blk);
            qa[r] = *reinterpret_cast<const uint4 *>(blk + qoff);
            qb[r] = *reinterpret_cast<const uint4 *>(blk + qoff + 16);
        }
        if (c0) __syncthreads();  // every wave has read the previous pass's activations
        float xr[64];
        x_share<XPT, FUSE>(xf, kc, wt, lane, xs, xr);
        if (!active) {
#pragma unroll
            for (int i = 0; i < 64; i++) xr[i] = 0.0f;
        }
        float X0 = 0.f, X1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) X0 += xr[i], X1 += xr[32 + i];

        // Idle lanes contribute an explicit 0, not 0 * (a scale that may be inf or NaN).
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const float v = q4_dot(hd[r], qa[r], qb[r], xr, X0, X1, L);
            acc[r] += active ? v : 0.0f;
        }
    }
    team_store<TW, TEAMS, RPW>(acc, row0, n, y, red, team, lane, wt, [&](uint32_t row) {
        float a = 0.0f;  // kernels/proj_q4k.comp:60-75 (with up: activation.comp:21-28)
        for (uint32_t j = lane; j < k; j += 64) {
            float xj = x[j];
            if constexpr (FUSE) xj = silu_mul(xj, up[j]);
            a = __builtin_fmaf(xj, q4k_elem(w, (uint64_t)row * k + j), a);
        }
        return wave_sum(a);
    });
}

// ------------------------------------------------------------------------------------------
// Q8_0

constexpr uint32_t Q8_SEG = 64 * 68;                  // bytes of one wave's 64-group share of a row
constexpr uint32_t Q8_CHUNKS = Q8_SEG / 16;           // 272 16-byte chunks
constexpr uint32_t Q8_LOADS = (Q8_CHUNKS + 63) / 64;  // 5 per lane

__device__ __forceinline__ float q8_dot(const uint32_t *__restrict__ D, const float (&xr)[64], float X0, float X1) {
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
    return d0 * __builtin_fmaf(-128.0f, X0, s0) + d1 * __builtin_fmaf(-128.0f, X1, s1);
}

// Each wave stages its share of one row at a time in its own LDS region and reads
// it back; the region is only touched by that wave, whose LDS operations execute
// in order, so no barrier is needed between the write and the reads.  Every lane
// stores all of its Q8_LOADS chunks (unconditional stores keep the row registers
// out of divergent code); chunks past the share land in the stage's tail, which no
// lane reads.
template <int TW, int TEAMS, int RPW>
__global__ __launch_bounds__(TW *TEAMS * 64) void k_q80_m1(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                            float *__restrict__ y, uint32_t k, uint32_t n,
                                                            uint64_t row_bytes) {
    constexpr int XPT = (16 * TW + TEAMS * TW - 1) / (TEAMS * TW);
    constexpr uint32_t KPASS = TW * 64 * 64;  // elements one pass of the team covers
    __shared__ __attribute__((aligned(16))) float xs[TW * 64 * 68];
    __shared__ __attribute__((aligned(16))) lg_u32x4 stage_all[TW * TEAMS][64 * Q8_LOADS];
    __shared__ float red[TW > 1 ? TEAMS * RPW * TW : 1];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t team = wave / TW, wt = wave % TW;
    const uint32_t p0 = wt * 64 + lane;
    lg_u32x4 *stage = stage_all[wave];
    const uint32_t row0 = (blockIdx.x * TEAMS + team) * RPW;
    constexpr int NL = (int)Q8_LOADS;

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = 0.0f;
    for (uint32_t c0 = 0; c0 < k; c0 += KPASS) {  // uniform over the workgroup
        const uint32_t kc = k - c0 < KPASS ? k - c0 : KPASS;
        const uint32_t P = kc >> 6;
        const bool active = p0 < P;
        // this wave's share of the pass: groups wt*64 .. min(P, wt*64+64), a multiple of 4 groups
        const uint32_t groups = P > wt * 64 ? (P - wt * 64 < 64 ? P - wt * 64 : 64) : 0;
        const uint32_t seg16 = groups * 68 / 16;
        XFetch<XPT, false> xf;
        x_fetch<XPT, false>(xf, x + c0, nullptr, kc);
        lg_u32x4 c[RPW * NL];  // native vectors: plain loads and stores, kept in registers
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const uint32_t row = row0 + r < n ? row0 + r : n - 1;
            const lg_u32x4 *src = reinterpret_cast<const lg_u32x4 *>(w + (uint64_t)row * row_bytes +
                                                                     (uint64_t)c0 / QK8_0 * Q80_BYTES +
                                                                     (uint64_t)wt * Q8_SEG);
#pragma unroll
            for (int i = 0; i < NL; i++) {
                const uint32_t ch = lane + 64 * i;
                c[r * NL + i] = src[ch < seg16 ? ch : 0];  // chunks past the share re-read chunk 0
            }
        }
        if (c0) __syncthreads();  // every wave has read the previous pass's activations
        float xr[64];
        x_share<XPT, false>(xf, kc, wt, lane, xs, xr);
        if (!active) {
#pragma unroll
            for (int i = 0; i < 64; i++) xr[i] = 0.0f;
        }
        float X0 = 0.f, X1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) X0 += xr[i], X1 += xr[32 + i];

        // Idle lanes read stage words nobody wrote: their partials are replaced by 0.
#pragma unroll
        for (int r = 0; r < RPW; r++) {
#pragma unroll
            for (int i = 0; i < NL; i++) stage[lane + 64 * i] = c[r * NL + i];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const float v = q8_dot(reinterpret_cast<const uint32_t *>(stage) + 17 * lane, xr, X0, X1);
            acc[r] += active ? v : 0.0f;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
    team_store<TW, TEAMS, RPW>(acc, row0, n, y, red, team, lane, wt, [&](uint32_t row) {
        float a = 0.0f;  // kernels/proj_q8_0.comp:47-66
        for (uint32_t j = lane; j < k; j += 64) a = __builtin_fmaf(x[j], q80_elem(w, (uint64_t)row * k + j), a);
        return wave_sum(a);
    });
}

// ------------------------------------------------------------------------------------------
// Reference-semantics fallback: one wavefront per row, each element decoded at the
// reference's linear index (q4k_elem, q80_elem).

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
// Q4_K, M = 1, on int8 matrix cores (v_mfma_i32_16x16x64_i8: D[16x16] += A[16x64] B[64x16],
// lane l supplies A row l%16 / B column l%16 at bytes 16(l/16)..+15 of k; D row 4(l/16)+r,
// column l%16 lands in lane l, register r).
//
// Activations.  Each 256-element super-block of x is scaled by 2^sh, sh chosen so
// that max|x| 2^sh lies in [2^20, 2^21), and rounded to an integer X (one fma with
// 1.5 * 2^23 leaves U = X + 2^22 in the low 23 bits).  Its bytes are the digits:
// X = s0 + 2^8 s1 + 2^16 s2 - 4161408 with s0 = u0 - 128, s1 = u1 - 128, s2 = u2
// all in int8 range.  Quant nibbles are integers 0..15, so every product is exact
// in the i32 accumulators; with C_l = sum_k s_l,k q_k and Q = sum_k q_k,
//     sum_k X_k q_k = C0 + 2^8 C1 + 128 (2^9 C2 - 32511 Q)    (exact in int32),
// and the only rounding of x is to 22 significant bits of its super-block maximum.
//
// Tile: 16 weight rows (MFMA columns n = lane & 15) by one super-block.  With
// kq = lane >> 4, column n takes the quant bytes 16kq..16kq+15 (groups 0, 1) and
// 64+16kq.. (groups 2, 3) of its row.  Group pair p takes two MFMAs into one
// accumulator:
//   #1  B = low nibbles  (k block kq: sub-block 4p + 2(kq>>1), elements 16(kq&1)..+15)
//   #2  B = high nibbles (sub-block 4p + 2(kq>>1) + 1, same elements + 32)
// A row i = 4 slot + d: slots 0 and 1 carry digit d of #1's k blocks {0,1} and
// {2,3} and are zero in #2; slots 2 and 3 likewise for #2; d = 3 is a row of ones
// (so C3 = Q).  C row 4 slot + d of column n lands in lane (n, slot): after the
// pair each lane holds C0..C3 of one (row, sub-block) pair,
// j = 4p + 2 (slot & 1) + (slot >> 1), and applies that sub-block's scale and min:
//     acc += (d sc 2^-sh) S - (dmin m) X_j,   X_j = sum of x over sub-block j.
// The A fragments come from three tables of the same layout (digits, zeros,
// ones), so every lane's fragment address moves by the same amount per step.
//
// Weights reach the MFMA operands through LDS: read straight from memory, one
// instruction would touch 16 rows 2304 bytes apart (64 bytes each), which the
// memory system serves far below streaming rate.  Instead each wave copies MQ_C
// super-blocks of its 16 rows with 16-byte loads that run along the rows (about
// two rows per instruction) into its own LDS tile (rows padded so that the 16
// columns of a fragment read fall in distinct banks), and reads the fragments
// from there.  The loads of the next chunk are in flight while a chunk is used.
//
// Work split.  Workgroup (rs, ks) owns rows [n rs / RS, n (rs+1) / RS) (equal byte
// shares) and super-blocks [nsb ks / KS, nsb (ks+1) / KS) of k (at most
// MQ_MAX_SLICE); it stages only that slice of x (digit table, sub-block sums,
// scales) in LDS.  Its rows form row groups of 16 (a partial last group repeats
// its last row in the idle columns, which are not stored), and when there are
// fewer row groups than waves each row group's slice is split into KP parts, one
// (row group, part) unit per wave.  Parts are added in part order, slices in slice
// order by the last workgroup of the row range to finish (arrival counter reset
// by that workgroup): results do not depend on timing.
//
// A slice whose activations are not finite, or whose super-block maximum is below
// 2^-100 (where 2^sh would leave the f32 range), is computed by the reference's
// per-element loop instead.

constexpr int MQ_WAVES = 8;
constexpr uint32_t MQ_MIN_ROWS = 4;     // rows per workgroup below which columns idle for nothing
constexpr uint32_t MQ_MAX_SLICE = 16;   // super-blocks of x one workgroup stages
constexpr uint32_t MQ_TAB = MQ_MAX_SLICE * 768;  // one A table: 16 chunks x 48 bytes per super-block
// The zero and ones tables start 64 and 128 bytes into a 256-byte period after the
// digits, so that the lanes of one fragment read that use different tables hit
// different banks.
constexpr uint32_t MQ_TZERO = MQ_TAB + 64, MQ_TONES = 2 * MQ_TAB + 256 + 128;
constexpr uint32_t MQ_TALL = 3 * MQ_TAB + 512;

typedef int lg_i32x4 __attribute__((ext_vector_type(4)));

template <int C>
struct MqGeom {
    static constexpr uint32_t ROW = C * 144 + 16;  // staged row stride: 16 rows at distinct banks
    static constexpr uint32_t WAVE = 16 * ROW;     // one wave's tile
    static constexpr uint32_t PIECES = 16 * C * 9;  // 16-byte pieces per chunk
    static constexpr int LOADS = (PIECES + 63) / 64;
};

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = (uint32_t)__shfl_xor((int)v, o);
        v = v > t ? v : t;
    }
    return v;
}

// Staging of one super-block of x by one wave (lane l: elements 4l..4l+3): digit
// table T (chunk c at T + 48c: digit d of elements 16c..16c+15 at +16d), sub-block
// sums X, scale 2^-sh; returns 1 if the super-block needs the per-element loop.
__device__ __forceinline__ uint32_t mq_stage(float4 v, uint32_t i, uint32_t lane, uint8_t *s_T, float *s_X,
                                             float *s_FX) {
    // max |x| on the bit patterns: NaN > inf > every finite value
    uint32_t mb = __float_as_uint(v.x) & 0x7FFFFFFFu;
    mb = max(mb, __float_as_uint(v.y) & 0x7FFFFFFFu);
    mb = max(mb, __float_as_uint(v.z) & 0x7FFFFFFFu);
    mb = max(mb, __float_as_uint(v.w) & 0x7FFFFFFFu);
    mb = wave_max_u32(mb);
    const uint32_t bad = (mb >= 0x7F800000u || (mb != 0u && mb < 0x0D800000u)) ? 1u : 0u;  // non-finite, < 2^-100
    float sum = (v.x + v.y) + (v.z + v.w);
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if ((lane & 7u) == 0) s_X[i * 8u + (lane >> 3)] = sum;
    int e = 0;
    (void)frexpf(__uint_as_float(mb), &e);
    const int sh = mb == 0u || bad ? 0 : 21 - e;
    const float scale = ldexpf(1.0f, sh);
    if (lane == 0) s_FX[i] = ldexpf(1.0f, -sh);
    const uint32_t t0 = __float_as_uint(__builtin_fmaf(v.x, scale, 12582912.0f));
    const uint32_t t1 = __float_as_uint(__builtin_fmaf(v.y, scale, 12582912.0f));
    const uint32_t t2 = __float_as_uint(__builtin_fmaf(v.z, scale, 12582912.0f));
    const uint32_t t3 = __float_as_uint(__builtin_fmaf(v.w, scale, 12582912.0f));
    // byte b of the four elements into one dword (v_perm_b32: selector 0-3 picks
    // from the second operand, 4-7 from the first, 0x0C is a zero byte)
    const uint32_t p01 = __builtin_amdgcn_perm(t1, t0, 0x05010400u), p23 = __builtin_amdgcn_perm(t3, t2, 0x05010400u);
    const uint32_t q01 = __builtin_amdgcn_perm(t1, t0, 0x0C0C0602u), q23 = __builtin_amdgcn_perm(t3, t2, 0x0C0C0602u);
    uint8_t *tp = s_T + (i * 16u + (lane >> 2)) * 48u + 4u * (lane & 3u);
    *reinterpret_cast<uint32_t *>(tp) = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;
    *reinterpret_cast<uint32_t *>(tp + 16) = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;
    *reinterpret_cast<uint32_t *>(tp + 32) = __builtin_amdgcn_perm(q23, q01, 0x05040100u);
    return bad;
}

// The reference's f16 decoder (ref_half) from the hardware conversion: the two
// differ only for exponent-0 codes with a non-zero mantissa (f16 subnormals, class
// bits 4 and 7), which the reference reads as 2^-14 + 2^-24 m instead of 2^-24 m.
__device__ __forceinline__ float mq_half(uint32_t h16) {
    const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)h16);
    const float v = (float)h;
    return v + (__builtin_amdgcn_classh(h, 0x90) ? __builtin_copysignf(0x1p-14f, v) : 0.0f);
}

// Wave-private LDS fence: the wave's own LDS writes are visible to its later reads
// (and its earlier reads are done before later writes).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row ranges and k slices of the grid, as quotients and remainders (workgroup rs
// gets rows + (rs < rows_extra) rows, slice ks gets sbs + (ks < sbs_extra)
// super-blocks).
struct MqSplit {
    uint32_t rows, rows_extra, sbs, sbs_extra;
};

// C: super-blocks per staged chunk; NCH: chunks whose loads a wave issues together.
template <bool FUSE, int C, int NCH>
__global__ __launch_bounds__(MQ_WAVES * 64) void k_q4k_m1_mfma(const float *__restrict__ x,
                                                              const float *__restrict__ up,
                                                              const uint8_t *__restrict__ w, float *__restrict__ y,
                                                              float *__restrict__ part, uint32_t *__restrict__ cnt,
                                                              uint32_t k, uint32_t n, uint64_t row_bytes, MqSplit sp) {
    using G = MqGeom<C>;
    __shared__ __attribute__((aligned(16))) uint8_t s_W[MQ_WAVES * G::WAVE];
    __shared__ __attribute__((aligned(16))) uint8_t s_T[MQ_TALL + 4 * 768];  // dropped steps of a short unit read past the slice
    __shared__ float s_X[(MQ_MAX_SLICE + C) * 8];  // dropped steps of a short unit read past the slice
    __shared__ float s_FX[MQ_MAX_SLICE + C];
    __shared__ float s_part[MQ_WAVES * 16];
    __shared__ uint32_t s_bad[MQ_WAVES];
    __shared__ uint32_t s_last;

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rs = blockIdx.x, KS = gridDim.y, ks = blockIdx.y;
    // (no integer divisions before the first loads: they would delay every one of them)
    const uint32_t rows = sp.rows + (rs < sp.rows_extra ? 1u : 0u);
    const uint32_t r_begin = rs * sp.rows + (rs < sp.rows_extra ? rs : sp.rows_extra);
    const uint32_t r_end = r_begin + rows;
    const uint32_t nsl = sp.sbs + (ks < sp.sbs_extra ? 1u : 0u);  // this workgroup's slice
    const uint32_t sbA = ks * sp.sbs + (ks < sp.sbs_extra ? ks : sp.sbs_extra);
    const uint32_t RG = (rows + 15) >> 4;
    const uint32_t lkp = RG >= 5u ? 0u : RG >= 3u ? 1u : RG == 2u ? 2u : 3u;  // KP = 2^lkp: 8/RG rounded down, U <= 8 when KP > 1
    const uint32_t KP = 1u << lkp;
    const uint32_t U = RG << lkp;
    const uint32_t nn = lane & 15u, kq = lane >> 4;

    // ---- x of this wave's first two staging super-blocks: loaded before any weight,
    // so that waiting for them never waits for the weights (loads complete in order)
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *u4 = reinterpret_cast<const float4 *>(up);
    const uint32_t ia = wave < nsl ? wave : 0u, ib = wave + MQ_WAVES < nsl ? wave + MQ_WAVES : 0u;
    float4 xa = x4[(sbA + ia) * 64u + lane], xb = x4[(sbA + ib) * 64u + lane];
    float4 ua = xa, ub = xb;
    if constexpr (FUSE) ua = u4[(sbA + ia) * 64u + lane], ub = u4[(sbA + ib) * 64u + lane];

    // ---- chunk copies: piece p = 64 j + lane of a chunk is 16 bytes of row p / (9C),
    // at 16 (p % (9C)) in the row's C super-blocks
    uint32_t goff[G::LOADS], loff[G::LOADS];
    uint32_t s0u = 0, cntu = 0, row0 = 0;
    const uint8_t *ubase = w;  // this unit's first super-block of its first row
    auto unit = [&](uint32_t u) {
        const uint32_t rg = u >> lkp, kp = u & (KP - 1u);
        s0u = (nsl * kp) >> lkp;
        cntu = ((nsl * (kp + 1u)) >> lkp) - s0u;
        row0 = r_begin + 16u * rg;
        const uint32_t last = (r_end - 1u) - row0;  // rows past the range repeat the last one
        const uint32_t sbl = cntu ? cntu - 1u : 0u;  // a unit shorter than a chunk repeats its last super-block
        ubase = w + (uint64_t)row0 * row_bytes + (uint64_t)(sbA + s0u) * Q4K_BYTES;
#pragma unroll
        for (int j = 0; j < G::LOADS; j++) {
            uint32_t p = 64u * j + lane;
            p = p < G::PIECES ? p : G::PIECES - 1u;
            const uint32_t r = p / (9u * C), q = p - r * (9u * C);
            const uint32_t sb = q / 9u, qi = q - 9u * sb;
            goff[j] = (r < last ? r : last) * (uint32_t)row_bytes + (sb < sbl ? sb : sbl) * Q4K_BYTES + 16u * qi;
            loff[j] = wave * G::WAVE + r * G::ROW + 16u * q;
        }
    };
    // First step of the chunk that holds steps c0..: the last chunk of a unit is
    // moved back to end at the unit's end (its steps before c0 are dropped).
    auto chunk_start = [&](uint32_t c0) { return c0 + C <= cntu ? c0 : (cntu >= C ? cntu - C : 0u); };
    uint4 gb[NCH][G::LOADS];
    auto fetch = [&](uint32_t r0) {  // the NCH chunks of the round starting at step r0
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const uint8_t *base = ubase + (uint64_t)chunk_start(r0 + c * C) * Q4K_BYTES;
#pragma unroll
            for (int j = 0; j < G::LOADS; j++) gb[c][j] = ld_stream16(base + goff[j]);
        }
    };
    auto put = [&](int c) {
#pragma unroll
        for (int j = 0; j < G::LOADS; j++) *reinterpret_cast<uint4 *>(s_W + loff[j]) = gb[c][j];
    };
    unit(wave < U ? wave : 0u);
    if (wave >= U) cntu = 0;
    fetch(0);

    // ---- A tables: zeros and ones, then the digits of this slice
    for (uint32_t o = MQ_TAB + threadIdx.x * 16u; o < MQ_TALL; o += MQ_WAVES * 64u * 16u)
        *reinterpret_cast<uint4 *>(s_T + o) = o < MQ_TONES - 128u ? make_uint4(0u, 0u, 0u, 0u)
                                                                 : make_uint4(0x01010101u, 0x01010101u, 0x01010101u,
                                                                              0x01010101u);
    uint32_t bad = 0;
    if constexpr (FUSE) {
        xa = make_float4(silu_mul_fast(xa.x, ua.x), silu_mul_fast(xa.y, ua.y), silu_mul_fast(xa.z, ua.z),
                         silu_mul_fast(xa.w, ua.w));
        xb = make_float4(silu_mul_fast(xb.x, ub.x), silu_mul_fast(xb.y, ub.y), silu_mul_fast(xb.z, ub.z),
                         silu_mul_fast(xb.w, ub.w));
    }
    if (wave < nsl) bad |= mq_stage(xa, wave, lane, s_T, s_X, s_FX);
    if (wave + MQ_WAVES < nsl) bad |= mq_stage(xb, wave + MQ_WAVES, lane, s_T, s_X, s_FX);
    if (lane == 0) s_bad[wave] = bad;
    __syncthreads();
    uint32_t any_bad = 0;
#pragma unroll
    for (int i = 0; i < MQ_WAVES; i++) any_bad |= s_bad[i];

    float *dst = KS > 1 ? part + (uint64_t)ks * n : y;  // this slice's sums
    if (any_bad) {  // the reference's per-element loop over this slice
        for (uint32_t r = r_begin + wave; r < r_end; r += MQ_WAVES) {
            float acc = 0.0f;
            for (uint32_t j = sbA * 256u + lane; j < (sbA + nsl) * 256u; j += 64) {
                float xj = x[j];
                if constexpr (FUSE) xj = silu_mul(xj, up[j]);
                acc = __builtin_fmaf(xj, q4k_elem(w, (uint64_t)r * k + j), acc);
            }
            acc = wave_sum(acc);
            if (lane == 0) {
                if (KS > 1) __hip_atomic_store(dst + r, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else dst[r] = acc;
            }
        }
    } else {
        // per-lane bases (byte offsets); every step adds the same immediate to all of them
        const uint32_t slot = nn >> 2, dg = nn & 3u;
        const uint32_t cb = 4u * (kq >> 1) + (kq & 1u);  // 16-element chunk of #1's k block in a super-block
        const bool v1 = slot < 2u && slot == (kq >> 1), v2 = slot >= 2u && slot - 2u == (kq >> 1);
        const uint32_t dof = dg < 3u ? dg * 16u : 0u;
        const uint32_t tab1 = v1 ? (dg < 3u ? 0u : MQ_TONES) : MQ_TZERO;
        const uint32_t tab2 = v2 ? (dg < 3u ? 0u : MQ_TONES) : MQ_TZERO;
        const uint32_t ab1 = tab1 + cb * 48u + dof, ab2 = tab2 + (cb + 2u) * 48u + dof;
        const uint32_t jl = 2u * (kq & 1u) + (kq >> 1);  // C slot kq holds sub-block 4p + jl
        const uint32_t wb = wave * G::WAVE + nn * G::ROW;  // this column's staged row
        const lg_i32x4 zero4 = {0, 0, 0, 0};

        // Steps c0 .. c0+C-1 of the current unit from the staged chunk; steps past
        // cntu are computed and dropped.
        auto consume = [&](uint32_t c0) {
            const uint32_t cs = chunk_start(c0);
            const uint32_t sl0 = s0u + cs;  // slice super-block of step 0
            const uint8_t *Ta = s_T + __mul24(sl0, 768u);
            const float *Xa = s_X + sl0 * 8u + jl;
            const float *FXa = s_FX + sl0;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < C; i++) {
                const uint4 h = *reinterpret_cast<const uint4 *>(s_W + wb + i * 144);
                const uint4 A = *reinterpret_cast<const uint4 *>(s_W + wb + i * 144 + 16 + 16 * kq);
                const uint4 B = *reinterpret_cast<const uint4 *>(s_W + wb + i * 144 + 80 + 16 * kq);
                const float d = mq_half(h.x & 0xFFFFu) * FXa[i], dm = mq_half(h.x >> 16);
                float a = 0.0f;
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const uint4 q = p ? B : A;
                    const lg_i32x4 b1 = {(int)(q.x & 0x0F0F0F0Fu), (int)(q.y & 0x0F0F0F0Fu), (int)(q.z & 0x0F0F0F0Fu),
                                         (int)(q.w & 0x0F0F0F0Fu)};
                    const lg_i32x4 b2 = {(int)((q.x >> 4) & 0x0F0F0F0Fu), (int)((q.y >> 4) & 0x0F0F0F0Fu),
                                         (int)((q.z >> 4) & 0x0F0F0F0Fu), (int)((q.w >> 4) & 0x0F0F0F0Fu)};
                    const lg_i32x4 x1 = *reinterpret_cast<const lg_i32x4 *>(Ta + ab1 + i * 768 + p * 384);
                    const lg_i32x4 x2 = *reinterpret_cast<const lg_i32x4 *>(Ta + ab2 + i * 768 + p * 384);
                    lg_i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, b1, zero4, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(x2, b2, c, 0, 0, 0);
                    // scale and min of sub-block j = 4p + jl (kernels/proj_q4k.comp:46-58)
                    uint32_t sc, mn;
                    if (p == 0) {
                        sc = __builtin_amdgcn_ubfe(h.y, 8u * jl, 6);
                        mn = __builtin_amdgcn_ubfe(h.z, 8u * jl, 6);
                    } else {
                        sc = __builtin_amdgcn_ubfe(h.w, 8u * jl, 4) | (__builtin_amdgcn_ubfe(h.y, 8u * jl + 6u, 2) << 4);
                        mn = __builtin_amdgcn_ubfe(h.w, 8u * jl + 4u, 4) |
                             (__builtin_amdgcn_ubfe(h.z, 8u * jl + 6u, 2) << 4);
                    }
                    const int lo = c[0] + (c[1] << 8);
                    const int hi = __mul24(c[3], -32511) + (c[2] << 9);
                    const float S = __builtin_fmaf(128.0f, (float)hi, (float)lo);
                    a = __builtin_fmaf(d * (float)sc, S, a);
                    a = __builtin_fmaf(-(dm * (float)mn), Xa[i * 8 + 4 * p], a);
                }
                acc += cs + i >= c0 && cs + i < cntu ? a : 0.0f;
            }
            return acc;
        };
        auto finish = [&](uint32_t u, float acc) {
            acc += __shfl_xor(acc, 16);
            acc += __shfl_xor(acc, 32);
            if (KP == 1) {
                if (kq == 0 && row0 + nn < r_end) {
                    if (KS > 1) __hip_atomic_store(dst + row0 + nn, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else dst[row0 + nn] = acc;
                }
            } else if (kq == 0) {
                s_part[u * 16u + nn] = acc;
            }
        };
        // One round: the loads of its NCH chunks are in flight; each chunk goes to the
        // wave's LDS tile as soon as it has landed and is used from there.
        auto round = [&](uint32_t r0) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; c++) {
                if (r0 + c * C < cntu) {
                    wave_lds_fence();
                    put(c);
                    wave_lds_fence();
                    acc += consume(r0 + c * C);
                }
            }
            return acc;
        };
        // The first round of the first unit is straight-line code after the loads
        // issued before staging, so each chunk waits only for its own loads.
        if (wave < U) {
            float acc = round(0);
            for (uint32_t r0 = NCH * C; r0 < cntu; r0 += NCH * C) {
                fetch(r0);
                acc += round(r0);
            }
            finish(wave, acc);
        }
        for (uint32_t u = wave + MQ_WAVES; u < U; u += MQ_WAVES) {
            unit(u);
            float acc = 0.0f;
            for (uint32_t r0 = 0; r0 < cntu; r0 += NCH * C) {
                fetch(r0);
                acc += round(r0);
            }
            finish(u, acc);
        }
        if (KP > 1) {
            __syncthreads();
            for (uint32_t t = threadIdx.x; t < rows; t += blockDim.x) {
                const uint32_t rg = t >> 4, c = t & 15u;
                float s = 0.0f;
                for (uint32_t kp = 0; kp < KP; kp++) s += s_part[((rg << lkp) + kp) * 16u + c];
                if (KS > 1) __hip_atomic_store(dst + r_begin + t, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else dst[r_begin + t] = s;
            }
        }
    }
    if (KS == 1) return;
    // the last workgroup of the row range to arrive adds the slices
    if (!arrive_last(&cnt[rs], KS, &s_last)) return;
    for (uint32_t t = threadIdx.x; t < rows; t += blockDim.x) {
        const uint32_t r = r_begin + t;
        float s = 0.0f;
        for (uint32_t q0 = 0; q0 < KS; q0 += 8) {  // eight slices' loads in flight, added in slice order
            float pv[8];
#pragma unroll
            for (int g = 0; g < 8; g++)
                pv[g] = q0 + g < KS ? __hip_atomic_load(part + (uint64_t)(q0 + g) * n + r, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : 0.0f;
#pragma unroll
            for (int g = 0; g < 8; g++)
                if (q0 + g < KS) s += pv[g];
        }
        y[r] = s;
    }
}

// ------------------------------------------------------------------------------------------
// The activation digits shared by the k <= 4096 integer-dot kernels.  A workgroup of
// 256 threads converts x once: thread t takes elements 16t .. 16t+15 (group t/4,
// quarter t%4; threads past k/16 read element 0 and fill table entries that only idle
// lanes read) into the LDS table dg_tab (per group: digit planes 0, 1, 2 x 16 dwords)
// and dg_xf (per group: the sums of elements 0-31 and 32-63, and 2^-sh).
// Group p's 48 digit dwords start at dword 52 p: lane p's 16-byte reads of its group
// then fall on distinct banks over each 16 lanes (at 48 p, every fourth lane shares
// banks: 16-way conflicts on the read back).
constexpr uint32_t DIG_STRIDE = 52;
struct DigLds {
    uint32_t tab[64 * DIG_STRIDE];
    float xf[64 * 4];
    uint32_t bad;
};

__device__ __forceinline__ void dig_load_x(const float *__restrict__ x, uint32_t k, float4 (&xv)[4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t e4 = 4 * threadIdx.x + j;
        xv[j] = reinterpret_cast<const float4 *>(x)[e4 < k / 4 ? e4 : 0];
    }
}

// After a barrier that follows dg.bad = 0; flags dg.bad when some live group cannot be
// scaled (non-finite, >= 2^21, nonzero below 2^-60).  A barrier must follow before
// dig_read.  Threads past the first 256 (workgroups of eight wavefronts) convert nothing.
__device__ __forceinline__ void dig_convert(const float4 (&xv)[4], uint32_t k, DigLds &dg) {
    const uint32_t tid = threadIdx.x;
    if (tid >= 256) return;  // uniform over the wavefront
    float v[16];
#pragma unroll
    for (int j = 0; j < 4; j++) v[4 * j] = xv[j].x, v[4 * j + 1] = xv[j].y, v[4 * j + 2] = xv[j].z, v[4 * j + 3] = xv[j].w;
    uint32_t mb = 0;
#pragma unroll
    for (int j = 0; j < 16; j++) mb = max(mb, __float_as_uint(v[j]) & 0x7FFFFFFFu);
    // the group's maximum over its four threads (a quad)
    mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
    mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
    const bool outside = mb >= 0x4A000000u || (mb != 0u && mb < 0x21800000u);  // >= 2^21 or NaN/inf; < 2^-60
    const int E = (int)(mb >> 23) - 127;
    const int sh = (mb == 0u || outside) ? 0 : 20 - E;
    const float scale = __uint_as_float((uint32_t)(127 + sh) << 23);
    uint32_t U[16];
#pragma unroll
    for (int j = 0; j < 16; j++) U[j] = __float_as_uint(__builtin_fmaf(v[j], scale, 12582912.0f)) - 0x4ABF7F80u;
    uint32_t *dgp = dg.tab + (tid >> 2) * DIG_STRIDE + 4 * (tid & 3u);
#pragma unroll
    for (int q = 0; q < 4; q++) {  // elements 4q .. 4q+3 of this thread's 16: one dword per digit plane
        const uint32_t lo01 = __builtin_amdgcn_perm(U[4 * q + 1], U[4 * q], 0x05010400u);
        const uint32_t lo23 = __builtin_amdgcn_perm(U[4 * q + 3], U[4 * q + 2], 0x05010400u);
        const uint32_t hi01 = __builtin_amdgcn_perm(U[4 * q + 1], U[4 * q], 0x0C0C0602u);
        const uint32_t hi23 = __builtin_amdgcn_perm(U[4 * q + 3], U[4 * q + 2], 0x0C0C0602u);
        dgp[q] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
        dgp[16 + q] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
        dgp[32 + q] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) sum += v[j];
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0xB1, 0xF, 0xF, false));
    if ((tid & 3u) == 0) dg.xf[(tid >> 2) * 4 + 0] = sum;  // elements 0-31 of the group
    if ((tid & 3u) == 2) dg.xf[(tid >> 2) * 4 + 1] = sum;  // elements 32-63
    if ((tid & 3u) == 0) dg.xf[(tid >> 2) * 4 + 2] = __uint_as_float((uint32_t)(127 - sh) << 23);
    if (tid < k / 16 && outside) dg.bad = 1u;
}

// Group p's 48 digit dwords and its X0, X1, 2^-sh into registers.
__device__ __forceinline__ void dig_read(const DigLds &dg, uint32_t p, uint32_t (&D)[48], float &X0, float &X1,
                                         float &F) {
    const uint4 *src = reinterpret_cast<const uint4 *>(dg.tab + p * DIG_STRIDE);
#pragma unroll
    for (int i = 0; i < 12; i++) {
        const uint4 u = src[i];
        D[4 * i] = u.x, D[4 * i + 1] = u.y, D[4 * i + 2] = u.z, D[4 * i + 3] = u.w;
    }
    X0 = dg.xf[p * 4], X1 = dg.xf[p * 4 + 1], F = dg.xf[p * 4 + 2];
}

// Q4_K with k <= 4096, not fused: integer dot products (v_dot4_i32_i8) of the raw
// nibbles against three signed byte digits of the activations.
//
// Each 64-element group p of x is scaled by 2^sh_p, sh_p chosen so that the group's
// max|x| 2^sh lies in [2^20, 2^21), and rounded to an integer X (one fma with
// 1.5 * 2^23: the low 24 bits of the result are X + 0x808080).  Bytes XOR 0x80 are
// signed digits with X = t0 + 2^8 t1 + 2^16 t2, so per 32-element sub-block
//     sum_j X_j q_j = C0 + 2^8 C1 + 2^16 C2,   C_l = sum_j t_l,j q_j  (exact in int32:
//     |X| <= 2^21, q <= 15),
// and the row's term is d sc 2^-sh (C0 + 2^8 C1 + 2^16 C2) - dmin m sum_j x_j.
// The rounding of x to 21 significant bits of its group maximum is the only
// approximation (|error| <= 2^-22 max|x_group| per element).  Groups holding a
// non-finite value, a magnitude >= 2^21 or a nonzero magnitude below 2^-60 cannot
// be scaled that way: if x holds one, every row takes the reference's per-element
// loop instead.
//
// Lane p of a wave owns group p of a row (k/64 <= 64 lanes); the workgroup converts
// x once into an LDS table of 48 digit dwords per group, each lane keeps its group's
// 48 dwords in registers, and the waves stride over rows R at a time with the next
// rows' loads in flight while the current rows are reduced.
//
// IN (a layer's input, k_q4k_m1_dig_in): the activations are the RMSNorm of x + xadd
// (src/target.rs:426-437, 526-532: the residual add, then the norm), each workgroup
// computing the norm's sum of squares from its own staged copy, and up to four
// products over them run as one launch (virtual rows off[j] .. off[j+1]-1 are job j's
// rows; jobs past the count start at n).  Workgroup 0 also writes x + xadd (the
// residual stream) and the normed activations where asked.  Job j's weights and
// outputs are addressed as offsets from job 0's (wofs bytes, yofs elements), each
// pointer a kernel argument of its own: a pointer read from a structure, or selected
// among several, has no known address space, and its loads become flat loads whose
// waits also wait for the LDS traffic.
//
// GLU (IN, two jobs of equal size: an FFN's gate and up): virtual row 2r is gate row
// r and 2r + 1 is up row r, so a wave's two rows are one pair, and it writes
// silu(gate) * up (kernels/activation.comp:21-28) as row r of job 0's output.
struct DigIn {
    const float *xadd;  // null: the activations are x
    const float *nw;    // null: no norm
    float *xout, *xcap;  // x + xadd, written by workgroup 0 (each may be null)
    float *nxout;        // the normed activations, written by workgroup 0 (may be null)
    const uint8_t *w0;
    float *y0;
    int64_t wofs[4], yofs[4];
    uint32_t off[4];
    float eps;
};

template <int TEAMS, int R, bool IN, int NJ = 1, bool GLU = false>
__device__ __forceinline__ void q4k_m1_dig_body(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                float *__restrict__ y, uint32_t k, uint32_t n, uint64_t row_bytes,
                                                const DigIn &in) {
    static_assert(TEAMS == 4 || (TEAMS == 8 && !IN), "the first 256 threads convert 16 of the 4096 elements each");
    static_assert(!GLU || (IN && NJ == 2 && R == 2), "GLU pairs the two rows of a wave");
    __shared__ __attribute__((aligned(16))) DigLds dg;
    __shared__ float ssq[IN ? TEAMS : 1];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, team = tid >> 6;
    const uint32_t P = k >> 6;
    const bool active = lane < P;
    const uint32_t p = active ? lane : 0u;  // idle lanes read group 0 and contribute 0
    const Q4Lane L = q4_lane(p & 3u);
    const uint32_t lane_off = (p >> 2) * Q4K_BYTES;
    const uint32_t stride = gridDim.x * TEAMS * R;

    float4 xv[4], av[4], nwv[4];
    dig_load_x(x, k, xv);
    if constexpr (IN) {
        if (in.xadd) dig_load_x(in.xadd, k, av);
        if (in.nw) dig_load_x(in.nw, k, nwv);
    }
    // IN: the job of virtual row `row` (jobs past the count start at n), selected
    // among values held in scalar registers: a dynamically indexed read of the
    // argument block would put a scalar load before every row's weight loads
    auto job = [&](uint32_t row, const uint8_t *&wj, float *&yj, uint32_t &lr) {
        int64_t wo = 0, yo = 0;
        row = __builtin_amdgcn_readfirstlane(row);  // uniform over the wave: scalar selection
        lr = row;
        if constexpr (GLU) {
            wj = in.w0 + ((row & 1u) ? in.wofs[1] : 0);
            yj = in.y0;
            lr = row >> 1;
            return;
        }
        if constexpr (NJ > 1) {
#pragma unroll
            for (int i = 1; i < NJ; i++)
                if (row >= in.off[i]) wo = in.wofs[i], yo = in.yofs[i], lr = row - in.off[i];
        }
        wj = in.w0 + wo;
        yj = in.y0 + yo;
    };
    // the first rows' weights are in flight while x is converted.  The wave's rows are
    // held in scalar registers (they are uniform over the wave): row addresses (and,
    // IN, each row's job) cost scalar instructions (8.68 -> 8.47 us on 4096 -> 14336)
    uint32_t r0 = __builtin_amdgcn_readfirstlane((blockIdx.x * TEAMS + team) * R);
    uint4 hd[2][R], qa[2][R], qb[2][R];
    auto load = [&](int b, uint32_t rr) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = min(rr + r, n - 1u);  // rows past n re-read row n-1 and are not stored
            const uint8_t *blk;
            if constexpr (IN) {
                const uint8_t *wj;
                float *yj;
                uint32_t lr;
                job(row, wj, yj, lr);
                blk = wj + (uint64_t)lr * row_bytes + lane_off;
            } else {
                blk = w + (uint64_t)row * row_bytes + lane_off;
            }
            hd[b][r] = *reinterpret_cast<const uint4 *>(blk);
            qa[b][r] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * L.g);
            qb[b][r] = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * L.g);
        }
    };
    load(0, r0);
    float rs = 1.0f;  // IN: the norm's 1 / rms
    if constexpr (IN) {
        float sq = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (in.xadd)
                xv[j] = make_float4(xv[j].x + av[j].x, xv[j].y + av[j].y, xv[j].z + av[j].z, xv[j].w + av[j].w);
            const bool live = 4 * tid + j < k / 4;
            if (live && blockIdx.x == 0) {
                if (in.xout) reinterpret_cast<float4 *>(in.xout)[4 * tid + j] = xv[j];
                if (in.xcap) reinterpret_cast<float4 *>(in.xcap)[4 * tid + j] = xv[j];
            }
            if (live)
                sq = __builtin_fmaf(xv[j].x, xv[j].x, __builtin_fmaf(xv[j].y, xv[j].y,
                     __builtin_fmaf(xv[j].z, xv[j].z, __builtin_fmaf(xv[j].w, xv[j].w, sq))));
        }
        if (in.nw) {
            sq = wave_sum(sq);
            if (lane == 0) ssq[team] = sq;
        }
    }
    if (tid == 0) dg.bad = 0u;
    __syncthreads();
    if constexpr (IN) {
        if (in.nw) {  // kernels/rmsnorm.comp:23-34: x w / sqrt(mean(x^2) + eps)
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < TEAMS; i++) t += ssq[i];
            rs = 1.0f / sqrtf(t / (float)k + in.eps);
#pragma unroll
            for (int j = 0; j < 4; j++)
                xv[j] = make_float4(xv[j].x * nwv[j].x * rs, xv[j].y * nwv[j].y * rs, xv[j].z * nwv[j].z * rs,
                                    xv[j].w * nwv[j].w * rs);
        }
        if (in.nxout && blockIdx.x == 0)
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (4 * tid + j < k / 4) reinterpret_cast<float4 *>(in.nxout)[4 * tid + j] = xv[j];
    }
    dig_convert(xv, k, dg);
    __syncthreads();
    uint32_t D[48];
    float X0, X1, F;
    dig_read(dg, p, D, X0, X1, F);
    if (dg.bad) {  // the reference's per-element loop (kernels/proj_q4k.comp:60-75)
        if constexpr (GLU) {  // pair r: gate row r and up row r, then silu(gate) * up
            for (uint32_t pr = blockIdx.x * TEAMS + team; pr < n / 2; pr += gridDim.x * TEAMS) {
                float a[2] = {0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint8_t *wj;
                    float *yj;
                    uint32_t lr;
                    job(2 * pr + u, wj, yj, lr);
                    for (uint32_t j = lane; j < k; j += 64) {
                        float xj = in.xadd ? x[j] + in.xadd[j] : x[j];
                        if (in.nw) xj = xj * in.nw[j] * rs;
                        a[u] = __builtin_fmaf(xj, q4k_elem(wj, (uint64_t)lr * k + j), a[u]);
                    }
                    a[u] = wave_sum(a[u]);
                }
                if (lane == 0) in.y0[pr] = silu_mul(a[0], a[1]);
            }
            return;
        }
        for (uint32_t rr = blockIdx.x * TEAMS + team; rr < n; rr += gridDim.x * TEAMS) {
            float a = 0.0f;
            if constexpr (IN) {
                const uint8_t *wj;
                float *yj;
                uint32_t lr;
                job(rr, wj, yj, lr);
                for (uint32_t j = lane; j < k; j += 64) {
                    float xj = in.xadd ? x[j] + in.xadd[j] : x[j];
                    if (in.nw) xj = xj * in.nw[j] * rs;
                    a = __builtin_fmaf(xj, q4k_elem(wj, (uint64_t)lr * k + j), a);
                }
                a = wave_sum(a);
                if (lane == 0) yj[lr] = a;
            } else {
                for (uint32_t j = lane; j < k; j += 64) a = __builtin_fmaf(x[j], q4k_elem(w, (uint64_t)rr * k + j), a);
                a = wave_sum(a);
                if (lane == 0) y[rr] = a;
            }
        }
        return;
    }
    auto dotrow = [&](const uint4 &h, const uint4 &A, const uint4 &B) -> float {
        const uint32_t q[8] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w};
        int c0 = 0, c1 = 0, c2 = 0, e0 = 0, e1 = 0, e2 = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int lo = (int)(q[t] & 0x0F0F0F0Fu), hi = (int)((q[t] >> 4) & 0x0F0F0F0Fu);
            c0 = __builtin_amdgcn_sdot4(lo, (int)D[t], c0, false);
            c1 = __builtin_amdgcn_sdot4(lo, (int)D[16 + t], c1, false);
            c2 = __builtin_amdgcn_sdot4(lo, (int)D[32 + t], c2, false);
            e0 = __builtin_amdgcn_sdot4(hi, (int)D[8 + t], e0, false);
            e1 = __builtin_amdgcn_sdot4(hi, (int)D[24 + t], e1, false);
            e2 = __builtin_amdgcn_sdot4(hi, (int)D[40 + t], e2, false);
        }
        const float S0 = (float)(c0 + (c1 << 8) + (c2 << 16)), S1 = (float)(e0 + (e1 << 8) + (e2 << 16));
        // scales and mins of sub-blocks 2g and 2g+1 (kernels/proj_q4k.comp:46-58)
        const bool lo = L.g < 2;
        const uint32_t srcA = lo ? h.y : h.w, srcM = lo ? h.z : h.w;
        const float d = mq_half(h.x & 0xFFFFu) * F, dmin = mq_half(h.x >> 16);
        const float sc0 = (float)(__builtin_amdgcn_ubfe(srcA, L.sa[0], 4) | (__builtin_amdgcn_ubfe(h.y, L.sb[0], 2) << 4));
        const float sc1 = (float)(__builtin_amdgcn_ubfe(srcA, L.sa[1], 4) | (__builtin_amdgcn_ubfe(h.y, L.sb[1], 2) << 4));
        const float m0 = (float)(__builtin_amdgcn_ubfe(srcM, L.ma[0], 4) | (__builtin_amdgcn_ubfe(h.z, L.mb[0], 2) << 4));
        const float m1 = (float)(__builtin_amdgcn_ubfe(srcM, L.ma[1], 4) | (__builtin_amdgcn_ubfe(h.z, L.mb[1], 2) << 4));
        const float ts = __builtin_fmaf(sc1, S1, sc0 * S0);
        const float tm = __builtin_fmaf(m1, X1, m0 * X0);
        return __builtin_fmaf(d, ts, -(dmin * tm));
    };
    // Idle lanes contribute an explicit 0, not 0 * (a scale that may be inf or NaN).
    auto reduce = [&](int b, uint32_t rr) {
        if constexpr (GLU) {  // rows rr (gate) and rr + 1 (up) of pair rr / 2
            const float g = wave_sum(active ? dotrow(hd[b][0], qa[b][0], qb[b][0]) : 0.0f);
            const float u = wave_sum(active ? dotrow(hd[b][1], qa[b][1], qb[b][1]) : 0.0f);
            if (lane == 0 && rr < n) in.y0[rr >> 1] = silu_mul(g, u);
            return;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = dotrow(hd[b][r], qa[b][r], qb[b][r]);
            v = wave_sum(active ? v : 0.0f);
            if (lane == 0 && rr + r < n) {
                if constexpr (IN) {
                    const uint8_t *wj;
                    float *yj;
                    uint32_t lr;
                    job(rr + r, wj, yj, lr);
                    yj[lr] = v;
                } else {
                    y[rr + r] = v;
                }
            }
        }
    };
    for (;;) {  // every wave leaves once its next rows start at or past n
        const uint32_t r1 = r0 + stride;
        if (r1 >= n) {
            reduce(0, r0);
            break;
        }
        load(1, r1);
        reduce(0, r0);
        const uint32_t r2 = r1 + stride;
        if (r2 >= n) {
            reduce(1, r1);
            break;
        }
        load(0, r2);
        reduce(1, r1);
        r0 = r2;
    }
}

template <int TEAMS, int R>
__global__ __launch_bounds__(TEAMS * 64) void k_q4k_m1_dig(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                            float *__restrict__ y, uint32_t k, uint32_t n,
                                                            uint64_t row_bytes) {
    q4k_m1_dig_body<TEAMS, R, false>(x, w, y, k, n, row_bytes, DigIn{});
}

template <int TEAMS, int R, int NJ, bool GLU = false>
__global__ __launch_bounds__(TEAMS * 64) void k_q4k_m1_dig_in(
    const float *__restrict__ x, const float *xadd, const float *__restrict__ nw, float *xout, float *xcap,
    float *nxout, const uint8_t *__restrict__ w0, float *y0, int64_t wo1, int64_t wo2, int64_t wo3, int64_t yo1,
    int64_t yo2, int64_t yo3, uint32_t off1, uint32_t off2, uint32_t off3, uint32_t n, float eps, uint32_t k,
    uint64_t row_bytes) {
    const DigIn in{xadd, nw, xout, xcap, nxout, w0, y0, {0, wo1, wo2, wo3}, {0, yo1, yo2, yo3}, {0u, off1, off2, off3},
                   eps};
    q4k_m1_dig_body<TEAMS, R, true, NJ, GLU>(x, nullptr, nullptr, k, n, row_bytes, in);
}

// Q8_0 with k <= 4096: the same digits against the raw int8 quants.  Lane p owns
// group p of a row (blocks 2p, 2p+1: 68 bytes at offset 68p); each wave stages a row
// through its own LDS region with coalesced 16-byte loads (as k_q80_m1) and every lane
// reads back its 17 dwords.  Per block, three v_dot4_i32_i8 sums C0, C1, C2 of the quants
// against the digit planes give sum_j X_j q_j = C0 + 2^8 C1 + 2^16 C2 (each C exact in
// int32; combined in f32, as |sum| may pass 2^31), and the row's term is
// d 2^-sh (C0 + 2^8 C1 + 2^16 C2).  Rows stride over the grid R at a time, the next
// rows' loads in flight while the current rows are reduced.
template <int TEAMS, int R>
__global__ __launch_bounds__(TEAMS * 64) void k_q80_m1_dig(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                            float *__restrict__ y, uint32_t k, uint32_t n,
                                                            uint64_t row_bytes) {
    static_assert(TEAMS == 4 || TEAMS == 8, "the first 256 threads convert 16 of the 4096 elements each");
    constexpr int NL = (int)Q8_LOADS;
    __shared__ __attribute__((aligned(16))) DigLds dg;
    __shared__ __attribute__((aligned(16))) lg_u32x4 stage_all[TEAMS][64 * NL];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, team = tid >> 6;
    const uint32_t P = k >> 6;
    const bool active = lane < P;
    const uint32_t p = active ? lane : 0u;  // idle lanes read group 0 and contribute 0
    const uint32_t seg16 = P * 68 / 16;     // a row's 16-byte chunks (P is a multiple of 4)
    const uint32_t stride = gridDim.x * TEAMS * R;
    lg_u32x4 *stage = stage_all[team];

    float4 xv[4];
    dig_load_x(x, k, xv);
    uint32_t r0 = (blockIdx.x * TEAMS + team) * R;
    lg_u32x4 c[2][R][NL];
    auto load = [&](int b, uint32_t rr) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = min(rr + r, n - 1u);  // rows past n re-read row n-1 and are not stored
            const lg_u32x4 *src = reinterpret_cast<const lg_u32x4 *>(w + (uint64_t)row * row_bytes);
#pragma unroll
            for (int i = 0; i < NL; i++) {
                const uint32_t ch = lane + 64 * i;
                // chunks past the row re-read chunk 0; nontemporal: each chunk is read once
                // (4.94 against 5.13 us on 4096 -> 4096; the Q4_K kernels, whose lanes share
                // lines, measured slower with it)
                c[b][r][i] = __builtin_nontemporal_load(&src[ch < seg16 ? ch : 0]);
            }
        }
    };
    load(0, r0);
    if (tid == 0) dg.bad = 0u;
    __syncthreads();
    dig_convert(xv, k, dg);
    __syncthreads();
    uint32_t D[48];
    float X0, X1, F;
    dig_read(dg, p, D, X0, X1, F);
    if (dg.bad) {  // the reference's per-element loop (kernels/proj_q8_0.comp:47-66)
        for (uint32_t rr = blockIdx.x * TEAMS + team; rr < n; rr += gridDim.x * TEAMS) {
            float a = 0.0f;
            for (uint32_t j = lane; j < k; j += 64) a = __builtin_fmaf(x[j], q80_elem(w, (uint64_t)rr * k + j), a);
            a = wave_sum(a);
            if (lane == 0) y[rr] = a;
        }
        return;
    }
    // Idle lanes read stage words nobody wrote: their partials are replaced by 0.
    auto dotrow = [&](const uint32_t *v) -> float {
        int c0 = 0, c1 = 0, c2 = 0, e0 = 0, e1 = 0, e2 = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            // block 0's quants start 2 bytes into the lane's 68: realign; block 1's at byte 36
            const int a = (int)__builtin_amdgcn_alignbit(v[t + 1], v[t], 16), b = (int)v[9 + t];
            c0 = __builtin_amdgcn_sdot4(a, (int)D[t], c0, false);
            c1 = __builtin_amdgcn_sdot4(a, (int)D[16 + t], c1, false);
            c2 = __builtin_amdgcn_sdot4(a, (int)D[32 + t], c2, false);
            e0 = __builtin_amdgcn_sdot4(b, (int)D[8 + t], e0, false);
            e1 = __builtin_amdgcn_sdot4(b, (int)D[24 + t], e1, false);
            e2 = __builtin_amdgcn_sdot4(b, (int)D[40 + t], e2, false);
        }
        const float S0 = __builtin_fmaf(65536.0f, (float)c2, __builtin_fmaf(256.0f, (float)c1, (float)c0));
        const float S1 = __builtin_fmaf(65536.0f, (float)e2, __builtin_fmaf(256.0f, (float)e1, (float)e0));
        const float d0 = mq_half(v[0] & 0xFFFFu), d1 = mq_half(v[8] >> 16);
        return F * __builtin_fmaf(d1, S1, d0 * S0);
    };
    auto reduce = [&](int b, uint32_t rr) {
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int i = 0; i < NL; i++) stage[lane + 64 * i] = c[b][r][i];
            wave_lds_fence();
            uint32_t v[17];
            const uint32_t *sp = reinterpret_cast<const uint32_t *>(stage) + 17 * p;
#pragma unroll
            for (int i = 0; i < 17; i++) v[i] = sp[i];
            wave_lds_fence();
            float a = dotrow(v);
            a = wave_sum(active ? a : 0.0f);
            if (lane == 0 && rr + r < n) y[rr + r] = a;
        }
    };
    for (;;) {  // every wave leaves once its next rows start at or past n
        const uint32_t r1 = r0 + stride;
        if (r1 >= n) {
            reduce(0, r0);
            break;
        }
        load(1, r1);
        reduce(0, r0);
        const uint32_t r2 = r1 + stride;
        if (r2 >= n) {
            reduce(1, r1);
            break;
        }
        load(0, r2);
        reduce(1, r1);
        r0 = r2;
    }
}

// ------------------------------------------------------------------------------------------
// Q4_K M = 1 on int8 matrix cores with k split over the waves of one workgroup
// (k_q4k_m1_wide): the fused SiLU(gate)*up down projection.
//
// A workgroup owns RG groups of 16 rows and all of k: wave v takes super-blocks
// SPC*v .. SPC*v+SPC-1, converts their activations (with FUSE, silu(gate)*up) into
// its own LDS table of byte digits, and multiplies them by the raw nibbles of its 16
// rows with v_mfma_i32_16x16x64_i8.  The waves' row sums meet in LDS once at the end,
// so no partial sum leaves the workgroup and nothing waits on other workgroups.
//
// Digits.  Each 256-element super-block is scaled by 2^sh (max|x| 2^sh in
// [2^20, 2^21)) and rounded to integers X, whose bytes XOR 0x80 are signed digits
// t0, t1, t2 with X = t0 + 2^8 t1 + 2^16 t2.  The A operand's row 4g+d holds digit
// d of the 64 elements of group g, in the k-block (lanes 16g..16g+15) where B holds
// that group's nibbles, and zeros elsewhere; so C[4g+d][n] is digit d's dot product
// with row n's group g, and lane n + 16g receives all three in registers 0..2:
//     sum_j X_j q_j = C0 + 2^8 C1 + 2^16 C2   (per sub-block, exact in int32).
// Two MFMAs per sub-block (low nibbles: bytes 0-15 and 16-31 of the group's 32) give
// sub-block 2g, two more (high nibbles) sub-block 2g+1.  The f32 epilogue per lane:
//     d 2^-sh (sc_2g S_2g + sc_2g+1 S_2g+1) - dmin (m_2g X_2g + m_2g+1 X_2g+1).
// Super-blocks holding a non-finite value, a magnitude >= 2^21 or a nonzero magnitude
// below 2^-60 cannot be scaled that way: if any does, the workgroup's rows take the
// reference's per-element loop.
constexpr uint32_t WIDE_TAB = 768;  // one super-block's digit table: 4 groups x 3 digits x 64 bytes

__host__ __device__ constexpr uint32_t wide_wave_lds(int spc) { return 2 * spc * WIDE_TAB + spc * 8 * 4 + spc * 4; }
inline uint32_t wide_lds_bytes(uint32_t waves, uint32_t rg, int spc) {
    return waves * wide_wave_lds(spc) + waves * rg * 16 * 4 + waves * 4;
}

// xor-16 / xor-32 partners through the gfx950 lane swaps
__device__ __forceinline__ uint32_t max_x16(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return p[0] > p[1] ? p[0] : p[1];
}
__device__ __forceinline__ uint32_t max_x32(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return p[0] > p[1] ? p[0] : p[1];
}
__device__ __forceinline__ float add_x16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float add_x32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int RG, int SPC, bool FUSE>
__global__ __launch_bounds__(1024) void k_q4k_m1_wide(const float *__restrict__ x, const float *__restrict__ up,
                                                      const uint8_t *__restrict__ w, float *__restrict__ y,
                                                      uint32_t n, uint32_t nsb, uint64_t row_bytes, uint32_t rpw) {
    constexpr uint32_t WLDS = wide_wave_lds(SPC);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t l = threadIdx.x & 63u, wave = threadIdx.x >> 6, KQ = blockDim.x >> 6;
    const uint32_t nn = l & 15u, g = l >> 4;
    // rows [row0, rend) of this workgroup (rpw <= 16 RG; the grid keeps row0 < n), as
    // nrg groups of 16; a partial last group repeats row rend-1 in its idle columns
    const uint32_t row0 = blockIdx.x * rpw;
    const uint32_t rend = row0 + rpw < n ? row0 + rpw : n;
    const uint32_t nrg = (rend - row0 + 15u) >> 4;
    const uint32_t sb0 = wave * SPC;
    const uint32_t cnt = sb0 < nsb ? (nsb - sb0 < (uint32_t)SPC ? nsb - sb0 : (uint32_t)SPC) : 0u;
    uint8_t *T = lds + wave * WLDS;        // digit tables
    uint8_t *Z = T + SPC * WIDE_TAB;       // zeros: the A operand's rows outside their k-block
    float *Xs = reinterpret_cast<float *>(Z + SPC * WIDE_TAB);  // sub-block sums of x
    float *Fs = Xs + SPC * 8;                                   // 2^-sh per super-block
    float *s_part = reinterpret_cast<float *>(lds + KQ * WLDS);
    uint32_t *s_bad = reinterpret_cast<uint32_t *>(s_part + KQ * RG * 16);
    // the super-block of step t (steps past this wave's share re-read a valid one; dropped)
    uint32_t sbt[SPC];
#pragma unroll
    for (int t = 0; t < SPC; t++) sbt[t] = sb0 + t < nsb ? sb0 + t : nsb - 1u;

    // activations first (loads complete in issue order), then every weight load
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *u4 = reinterpret_cast<const float4 *>(up);
    float4 xv[SPC], uv[FUSE ? SPC : 1];
#pragma unroll
    for (int t = 0; t < SPC; t++) {
        xv[t] = x4[sbt[t] * 64u + l];
        if constexpr (FUSE) uv[t] = u4[sbt[t] * 64u + l];
    }
    uint4 hd[RG][SPC], q0[RG][SPC], q1[RG][SPC];  // header and the lane's 32 quant bytes of group g
#pragma unroll
    for (int r = 0; r < RG; r++) {
        if (RG > 1 && r >= (int)nrg) break;
        const uint32_t row = row0 + 16u * r + nn < rend ? row0 + 16u * r + nn : rend - 1u;
        const uint8_t *base = w + (uint64_t)row * row_bytes;
#pragma unroll
        for (int t = 0; t < SPC; t++) {
            const uint8_t *b = base + sbt[t] * Q4K_BYTES;
            hd[r][t] = *reinterpret_cast<const uint4 *>(b);
            q0[r][t] = *reinterpret_cast<const uint4 *>(b + 16 + 32 * g);
            q1[r][t] = *reinterpret_cast<const uint4 *>(b + 32 + 32 * g);
        }
    }
#pragma unroll
    for (int i = 0; i < (int)((SPC * WIDE_TAB + 1023) / 1024); i++)
        if (l * 16u + i * 1024u < SPC * WIDE_TAB)
            *reinterpret_cast<uint4 *>(Z + l * 16u + i * 1024u) = make_uint4(0, 0, 0, 0);

    // digits: lane l converts elements 4l .. 4l+3 of each super-block
    uint32_t bad = 0;
#pragma unroll
    for (int t = 0; t < SPC; t++) {
        float4 v = xv[t];
        if constexpr (FUSE) {
            const float4 u = uv[t];
            v = make_float4(silu_mul_fast(v.x, u.x), silu_mul_fast(v.y, u.y), silu_mul_fast(v.z, u.z),
                            silu_mul_fast(v.w, u.w));
        }
        uint32_t mb = max(max(__float_as_uint(v.x) & 0x7FFFFFFFu, __float_as_uint(v.y) & 0x7FFFFFFFu),
                          max(__float_as_uint(v.z) & 0x7FFFFFFFu, __float_as_uint(v.w) & 0x7FFFFFFFu));
        mb = max(mb, dpp_u<0xB1>(mb));   // quad_perm 1,0,3,2
        mb = max(mb, dpp_u<0x4E>(mb));   // quad_perm 2,3,0,1
        mb = max(mb, dpp_u<0x124>(mb));  // row_ror 4
        mb = max(mb, dpp_u<0x128>(mb));  // row_ror 8
        mb = max_x16(mb);
        mb = max_x32(mb);
        const bool outside = mb >= 0x4A000000u || (mb != 0u && mb < 0x21800000u);  // >= 2^21 or NaN/inf; < 2^-60
        bad |= outside && t < (int)cnt ? 1u : 0u;
        const int E = (int)(mb >> 23) - 127;
        const int sh = (mb == 0u || outside) ? 0 : 20 - E;
        const float scale = __uint_as_float((uint32_t)(127 + sh) << 23);
        const uint32_t U0 = __float_as_uint(__builtin_fmaf(v.x, scale, 12582912.0f)) - 0x4ABF7F80u;
        const uint32_t U1 = __float_as_uint(__builtin_fmaf(v.y, scale, 12582912.0f)) - 0x4ABF7F80u;
        const uint32_t U2 = __float_as_uint(__builtin_fmaf(v.z, scale, 12582912.0f)) - 0x4ABF7F80u;
        const uint32_t U3 = __float_as_uint(__builtin_fmaf(v.w, scale, 12582912.0f)) - 0x4ABF7F80u;
        const uint32_t lo01 = __builtin_amdgcn_perm(U1, U0, 0x05010400u);
        const uint32_t lo23 = __builtin_amdgcn_perm(U3, U2, 0x05010400u);
        const uint32_t hi01 = __builtin_amdgcn_perm(U1, U0, 0x0C0C0602u);
        const uint32_t hi23 = __builtin_amdgcn_perm(U3, U2, 0x0C0C0602u);
        uint8_t *tp = T + t * WIDE_TAB + (l >> 4) * 192u + 4u * (l & 15u);
        *reinterpret_cast<uint32_t *>(tp) = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
        *reinterpret_cast<uint32_t *>(tp + 64) = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
        *reinterpret_cast<uint32_t *>(tp + 128) = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;
        float sum = (v.x + v.y) + (v.z + v.w);
        sum += dpp_f<0xB1>(sum);
        sum += dpp_f<0x4E>(sum);
        sum += dpp_f<0x124>(sum);  // row_ror 4 brings lane i-4: lane 8j+4 holds lanes 8j .. 8j+7
        if ((l & 7u) == 4u) Xs[t * 8 + (l >> 3)] = sum;
        if (l == 0) Fs[t] = __uint_as_float((uint32_t)(127 - sh) << 23);
    }
    wave_lds_fence();

    // lane roles for the A operand: row i = 4 slot + d, digits where slot == k-block g and d < 3
    const uint32_t slotA = (l & 15u) >> 2, dA = l & 3u;
    const uint8_t *abase = slotA == g && dA < 3u ? T + g * 192u + dA * 64u : Z;
    const Q4Lane L = q4_lane(g);  // scale / min bit positions of sub-blocks 2g, 2g+1
    const bool lo = g < 2;

    float acc[RG];
#pragma unroll
    for (int r = 0; r < RG; r++) acc[r] = 0.0f;
    const lg_i32x4 z4 = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < SPC; t++) {
        const bool live = t < (int)cnt;
        const lg_i32x4 A00 = *reinterpret_cast<const lg_i32x4 *>(abase + t * WIDE_TAB);
        const lg_i32x4 A10 = *reinterpret_cast<const lg_i32x4 *>(abase + t * WIDE_TAB + 16);
        const lg_i32x4 A01 = *reinterpret_cast<const lg_i32x4 *>(abase + t * WIDE_TAB + 32);
        const lg_i32x4 A11 = *reinterpret_cast<const lg_i32x4 *>(abase + t * WIDE_TAB + 48);
        const float2 X2 = *reinterpret_cast<const float2 *>(Xs + t * 8 + 2 * g);
        const float F = Fs[t];
#pragma unroll
        for (int r = 0; r < RG; r++) {
            if (RG > 1 && r >= (int)nrg) break;
            const uint4 a = q0[r][t], b = q1[r][t];
            const lg_i32x4 bl0 = {(int)(a.x & 0x0F0F0F0Fu), (int)(a.y & 0x0F0F0F0Fu), (int)(a.z & 0x0F0F0F0Fu),
                                  (int)(a.w & 0x0F0F0F0Fu)};
            const lg_i32x4 bl1 = {(int)(b.x & 0x0F0F0F0Fu), (int)(b.y & 0x0F0F0F0Fu), (int)(b.z & 0x0F0F0F0Fu),
                                  (int)(b.w & 0x0F0F0F0Fu)};
            const lg_i32x4 bh0 = {(int)((a.x >> 4) & 0x0F0F0F0Fu), (int)((a.y >> 4) & 0x0F0F0F0Fu),
                                  (int)((a.z >> 4) & 0x0F0F0F0Fu), (int)((a.w >> 4) & 0x0F0F0F0Fu)};
            const lg_i32x4 bh1 = {(int)((b.x >> 4) & 0x0F0F0F0Fu), (int)((b.y >> 4) & 0x0F0F0F0Fu),
                                  (int)((b.z >> 4) & 0x0F0F0F0Fu), (int)((b.w >> 4) & 0x0F0F0F0Fu)};
            lg_i32x4 cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A00, bl0, z4, 0, 0, 0);
            cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A10, bl1, cl, 0, 0, 0);
            lg_i32x4 ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(A01, bh0, z4, 0, 0, 0);
            ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(A11, bh1, ch, 0, 0, 0);
            const uint4 h = hd[r][t];
            const float Se = (float)(cl[0] + (cl[1] << 8) + (cl[2] << 16));
            const float So = (float)(ch[0] + (ch[1] << 8) + (ch[2] << 16));
            const float d = mq_half(h.x & 0xFFFFu) * F, dm = mq_half(h.x >> 16);
            const uint32_t srcA = lo ? h.y : h.w, srcM = lo ? h.z : h.w;
            const float sce = (float)(__builtin_amdgcn_ubfe(srcA, L.sa[0], 4) | (__builtin_amdgcn_ubfe(h.y, L.sb[0], 2) << 4));
            const float sco = (float)(__builtin_amdgcn_ubfe(srcA, L.sa[1], 4) | (__builtin_amdgcn_ubfe(h.y, L.sb[1], 2) << 4));
            const float me = (float)(__builtin_amdgcn_ubfe(srcM, L.ma[0], 4) | (__builtin_amdgcn_ubfe(h.z, L.mb[0], 2) << 4));
            const float mo = (float)(__builtin_amdgcn_ubfe(srcM, L.ma[1], 4) | (__builtin_amdgcn_ubfe(h.z, L.mb[1], 2) << 4));
            const float ts = __builtin_fmaf(sco, So, sce * Se);
            const float tm = __builtin_fmaf(mo, X2.y, me * X2.x);
            const float v = __builtin_fmaf(-dm, tm, d * ts);
            acc[r] += live ? v : 0.0f;
        }
    }
#pragma unroll
    for (int r = 0; r < RG; r++) {
        if (RG > 1 && r >= (int)nrg) break;
        acc[r] = add_x32(add_x16(acc[r]));  // the 4 groups of row nn
        if (g == 0) s_part[wave * (RG * 16) + 16 * r + nn] = acc[r];
    }
    if (l == 0) s_bad[wave] = bad;
    __syncthreads();
    uint32_t any_bad = 0;
    for (uint32_t i = 0; i < KQ; i++) any_bad |= s_bad[i];
    if (!any_bad) {
        if (row0 + threadIdx.x < rend) {
            float sum = 0.0f;
            for (uint32_t i = 0; i < KQ; i++) sum += s_part[i * (RG * 16) + threadIdx.x];
            y[row0 + threadIdx.x] = sum;
        }
        return;
    }
    // the reference's per-element loop (kernels/proj_q4k.comp:60-75, activation.comp:21-28)
    for (uint32_t rr = wave; rr < RG * 16u; rr += KQ) {
        const uint32_t row = row0 + rr;
        if (row >= rend) break;
        float a = 0.0f;
        for (uint32_t j = l; j < nsb * QK_K; j += 64u) {
            float xj = x[j];
            if constexpr (FUSE) xj = silu_mul(xj, up[j]);
            a = __builtin_fmaf(xj, q4k_elem(w, (uint64_t)row * nsb * QK_K + j), a);
        }
        a = wave_sum(a);
        if (l == 0) y[row] = a;
    }
}

__global__ __launch_bounds__(256) void k_fill_zero(float *__restrict__ c, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) c[i] = 0.0f;
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


// Rows per team: enough that the grid covers the CUs once (or the tuning cap on
// workgroups), at most M1_RPW_MAX; larger n simply launches more workgroups.
uint32_t rows_per_team(uint32_t n, uint32_t teams) {
    uint64_t wgs = (uint64_t)device_cus();
    const uint32_t cap = g_grid_cap.load(std::memory_order_relaxed);
    if (cap && cap < wgs) wgs = cap;
    uint64_t rpw = (n + wgs * teams - 1) / (wgs * teams);
    if (rpw < 1) rpw = 1;
    if (rpw > (uint64_t)M1_RPW_MAX) rpw = M1_RPW_MAX;
    return (uint32_t)rpw;
}

// Launch shape of k_q4k_m1_mfma: KS slices of k times RS row ranges, about one
// workgroup per CU.  More slices mean less activation staging per workgroup (each
// stages k/KS elements; the fused SiLU adds two transcendentals per element) but
// more partial sums and a longer reduction by the last workgroup of a row range.
std::atomic<uint32_t> g_m1_split{0};  // 0 = automatic

void mq_shape(uint32_t k, uint32_t n, bool fuse, uint32_t &rs, uint32_t &ks) {
    uint32_t G = (uint32_t)device_cus();
    const uint32_t cap = g_grid_cap.load(std::memory_order_relaxed);
    if (cap && cap < G) G = cap;
    const uint32_t nsb = k / QK_K;
    uint32_t s = g_m1_split.load(std::memory_order_relaxed);
    if (!s) {
        // staging cost per workgroup ~ k/KS, product work ~ n k / G: keep their ratio small
        const double per = (fuse ? 14.0 : 8.0) * 4096.0 / (double)n * (double)G / 256.0;
        s = per < 1.0 ? 1u : (uint32_t)(per + 0.5);
    }
    const uint32_t smin = (nsb + MQ_MAX_SLICE - 1) / MQ_MAX_SLICE;  // the staged x slice fits LDS
    s = s < smin ? smin : s;
    s = s > nsb ? nsb : s;
    s = s > G ? (G > smin ? G : smin) : s;
    ks = s < 1 ? 1 : s;
    uint32_t r = G / ks;
    const uint32_t rmax = (n + MQ_MIN_ROWS - 1) / MQ_MIN_ROWS;
    r = r > rmax ? rmax : r;
    rs = r < 1 ? 1 : r;
}

template <bool FUSE>
int launch_q4k_mfma(const float *x, const float *up, const uint8_t *w, float *y, uint32_t k, uint32_t n,
                    hipStream_t s) {
    uint32_t rs = 1, ks = 1;
    mq_shape(k, n, FUSE, rs, ks);
    float *part = nullptr;
    uint32_t *cnt = nullptr;
    if (ks > 1) {
        LG_REQUIRE(rs <= PROJ_WS_COUNTERS / 4, "proj_q4k_m1: %u row ranges exceed the arrival counters", rs);
        void *ws = nullptr;
        const int st = stream_workspace(s, PROJ_WS_COUNTERS + (uint64_t)ks * n * 4, &ws);
        if (st != LG_OK) return st;
        cnt = static_cast<uint32_t *>(ws);
        part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + PROJ_WS_COUNTERS);
    }
    // longest unit of any workgroup decides the chunk: 2 super-blocks for short units
    const uint32_t nsb = k / QK_K, rows = (n + rs - 1) / rs, rg = (rows + 15) / 16;
    const uint32_t kp = rg >= 5u ? 1u : rg >= 3u ? 2u : rg == 2u ? 4u : 8u;
    const uint32_t steps = ((nsb + ks - 1) / ks + kp - 1) / kp;
    const dim3 grid(rs, ks), block(MQ_WAVES * 64);
    const uint64_t rb = (uint64_t)k / QK_K * Q4K_BYTES;
    const MqSplit sp{n / rs, n % rs, nsb / ks, nsb % ks};
    if (steps <= 2)
        hipLaunchKernelGGL((k_q4k_m1_mfma<FUSE, 2, 1>), grid, block, 0, s, x, up, w, y, part, cnt, k, n, rb, sp);
    else if (steps <= 4)
        hipLaunchKernelGGL((k_q4k_m1_mfma<FUSE, 2, 2>), grid, block, 0, s, x, up, w, y, part, cnt, k, n, rb, sp);
    else
        hipLaunchKernelGGL((k_q4k_m1_mfma<FUSE, 2, 4>), grid, block, 0, s, x, up, w, y, part, cnt, k, n, rb, sp);
    return after_launch(FUSE ? "proj_q4k_m1_silu" : "proj_q4k_m1", s);
}

// k_q4k_m1_wide launch shapes (k <= 16384):
//  * k <= 4096: one super-block per wave (k / 256 waves) and up to four groups of 16
//    rows per workgroup: ceil(n / G) rows per workgroup (G = the CU count, or the grid
//    cap) clamped to 16 .. 64, each wave holding its rows' loads in flight at once.
//    Selected by lg_set_m1_kernel(2) only: on 4096 -> 14336 its 16-row loads stream
//    slower than the integer-dot kernel's whole-row loads.
//  * above: four super-blocks per wave (ceil(k / 1024) waves), 16 rows per workgroup,
//    its LDS allowed past the 64 KiB default once per device.
constexpr int WIDE_SPC = 4;
constexpr uint32_t WIDE_MAX_SB = 16 * WIDE_SPC;
constexpr int WIDE_RG1 = 4;  // row groups per workgroup at one super-block per wave

std::atomic<uint32_t> g_m1_kernel{0};  // 0 = automatic, 1 = vector ALU / integer dot, 2 = matrix cores

std::mutex g_wide_mu;
bool g_wide_attr[64][2] = {};

template <bool FUSE>
int launch_q4k_wide(const float *x, const float *up, const uint8_t *w, float *y, uint32_t k, uint32_t n,
                    hipStream_t s) {
    const uint32_t nsb = k / QK_K;
    const uint64_t rb = (uint64_t)nsb * Q4K_BYTES;
    if (nsb <= 16) {
        uint32_t G = (uint32_t)device_cus();
        const uint32_t cap = g_grid_cap.load(std::memory_order_relaxed);
        if (cap && cap < G) G = cap;
        uint64_t rpw = ((uint64_t)n + G - 1) / G;
        rpw = rpw < 16 ? 16 : rpw > 16u * WIDE_RG1 ? 16u * WIDE_RG1 : rpw;
        const uint32_t grid = (uint32_t)(((uint64_t)n + rpw - 1) / rpw);
        hipLaunchKernelGGL((k_q4k_m1_wide<WIDE_RG1, 1, FUSE>), dim3(grid), dim3(nsb * 64),
                           wide_lds_bytes(nsb, WIDE_RG1, 1), s, x, up, w, y, n, nsb, rb, (uint32_t)rpw);
        return after_launch(FUSE ? "proj_q4k_m1_silu" : "proj_q4k_m1", s);
    }
    int dev = 0;
    LG_HIP_TRY(hipGetDevice(&dev));
    LG_REQUIRE(dev >= 0 && dev < 64, "proj_q4k_m1: device %d", dev);
    {
        std::lock_guard<std::mutex> lk(g_wide_mu);
        if (!g_wide_attr[dev][FUSE]) {
            LG_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_q4k_m1_wide<1, WIDE_SPC, FUSE>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)wide_lds_bytes(16, 1, WIDE_SPC)));
            g_wide_attr[dev][FUSE] = true;
        }
    }
    const uint32_t waves = (nsb + WIDE_SPC - 1) / WIDE_SPC;
    hipLaunchKernelGGL((k_q4k_m1_wide<1, WIDE_SPC, FUSE>), dim3((n + 15) / 16), dim3(waves * 64),
                       wide_lds_bytes(waves, 1, WIDE_SPC), s, x, up, w, y, n, nsb, rb, 16u);
    return after_launch(FUSE ? "proj_q4k_m1_silu" : "proj_q4k_m1", s);
}

template <int TW, int TEAMS, int RPW, bool FUSE>
void launch_q4k_r(const float *x, const float *up, const uint8_t *w, float *y, uint32_t k, uint32_t n,
                  hipStream_t s) {
    const uint32_t grid = (n + TEAMS * RPW - 1) / (TEAMS * RPW);
    const uint64_t rb = (uint64_t)k / QK_K * Q4K_BYTES;
    hipLaunchKernelGGL((k_q4k_m1<TW, TEAMS, RPW, FUSE>), dim3(grid), dim3(TW * TEAMS * 64), 0, s, x, up, w, y, k,
                       n, rb);
}

template <int TW, int TEAMS, bool FUSE>
int launch_q4k_t(const float *x, const float *up, const uint8_t *w, float *y, uint32_t k, uint32_t n,
                 hipStream_t s) {
    switch (rows_per_team(n, TEAMS)) {
    case 1: launch_q4k_r<TW, TEAMS, 1, FUSE>(x, up, w, y, k, n, s); break;
    case 2: launch_q4k_r<TW, TEAMS, 2, FUSE>(x, up, w, y, k, n, s); break;
    case 3: launch_q4k_r<TW, TEAMS, 3, FUSE>(x, up, w, y, k, n, s); break;
    case 4: launch_q4k_r<TW, TEAMS, 4, FUSE>(x, up, w, y, k, n, s); break;
    case 5: launch_q4k_r<TW, TEAMS, 5, FUSE>(x, up, w, y, k, n, s); break;
    case 6: launch_q4k_r<TW, TEAMS, 6, FUSE>(x, up, w, y, k, n, s); break;
    case 7: launch_q4k_r<TW, TEAMS, 7, FUSE>(x, up, w, y, k, n, s); break;
    default: launch_q4k_r<TW, TEAMS, 8, FUSE>(x, up, w, y, k, n, s); break;
    }
    return after_launch(FUSE ? "proj_q4k_m1_silu" : "proj_q4k_m1", s);
}

template <bool FUSE>
int launch_q4k(const float *x, const float *up, const uint8_t *w, float *y, uint32_t k, uint32_t n, hipStream_t s) {
    const uint32_t P = k / 64;
    if (P <= 64 && !FUSE) {
        const uint32_t gc = g_grid_cap.load(std::memory_order_relaxed), cus = (uint32_t)device_cus();
        if (n <= 16 * cus) {
            // at most two rows per wavefront: one 8-wavefront workgroup per CU (half the
            // conversions of x), the wave's two rows in flight from the start.  Measured
            // on 4096 -> 4096: 4.60 against 5.14 us for the layout below.
            constexpr int TEAMS = 8, R = 1;
            uint32_t grid = (n + TEAMS * R - 1) / (TEAMS * R);
            const uint32_t cap = gc ? gc : cus;
            grid = grid < cap ? grid : cap;
            hipLaunchKernelGGL((k_q4k_m1_dig<TEAMS, R>), dim3(grid), dim3(TEAMS * 64), 0, s, x, w, y, k, n,
                               (uint64_t)k / QK_K * Q4K_BYTES);
            return after_launch("proj_q4k_m1", s);
        }
        constexpr int TEAMS = 4, R = 2;
        uint32_t grid = (n + TEAMS * R - 1) / (TEAMS * R);
        const uint32_t cap = gc ? gc : 2 * cus;  // two workgroups per CU: measured best for 14336 rows
        grid = grid < cap ? grid : cap;
        hipLaunchKernelGGL((k_q4k_m1_dig<TEAMS, R>), dim3(grid), dim3(TEAMS * 64), 0, s, x, w, y, k, n,
                           (uint64_t)k / QK_K * Q4K_BYTES);
        return after_launch("proj_q4k_m1", s);
    }
    if (P <= 64) return launch_q4k_t<1, 8, FUSE>(x, up, w, y, k, n, s);
    if (P <= 128) return launch_q4k_t<2, 4, FUSE>(x, up, w, y, k, n, s);
    if (P <= 192) return launch_q4k_t<3, 2, FUSE>(x, up, w, y, k, n, s);
    return launch_q4k_t<4, 2, FUSE>(x, up, w, y, k, n, s);
}

template <int TW, int TEAMS, int RPW>
void launch_q80_r(const float *x, const uint8_t *w, float *y, uint32_t k, uint32_t n, hipStream_t s) {
    const uint32_t grid = (n + TEAMS * RPW - 1) / (TEAMS * RPW);
    const uint64_t rb = (uint64_t)k / QK8_0 * Q80_BYTES;
    hipLaunchKernelGGL((k_q80_m1<TW, TEAMS, RPW>), dim3(grid), dim3(TW * TEAMS * 64), 0, s, x, w, y, k, n, rb);
}

template <int TW, int TEAMS>
int launch_q80_t(const float *x, const uint8_t *w, float *y, uint32_t k, uint32_t n, hipStream_t s) {
    switch (rows_per_team(n, TEAMS)) {
    case 1: launch_q80_r<TW, TEAMS, 1>(x, w, y, k, n, s); break;
    case 2: launch_q80_r<TW, TEAMS, 2>(x, w, y, k, n, s); break;
    case 3: launch_q80_r<TW, TEAMS, 3>(x, w, y, k, n, s); break;
    case 4: launch_q80_r<TW, TEAMS, 4>(x, w, y, k, n, s); break;
    case 5: launch_q80_r<TW, TEAMS, 5>(x, w, y, k, n, s); break;
    case 6: launch_q80_r<TW, TEAMS, 6>(x, w, y, k, n, s); break;
    case 7: launch_q80_r<TW, TEAMS, 7>(x, w, y, k, n, s); break;
    default: launch_q80_r<TW, TEAMS, 8>(x, w, y, k, n, s); break;
    }
    return after_launch("proj_q8_0_m1", s);
}

int launch_q80(const float *x, const uint8_t *w, float *y, uint32_t k, uint32_t n, hipStream_t s) {
    const uint32_t P = k / 64;
    if (P <= 64) {
        const uint32_t gc = g_grid_cap.load(std::memory_order_relaxed), cus = (uint32_t)device_cus();
        if (n <= 16 * cus) {
            // as for Q4_K: one 8-wavefront workgroup per CU, at most two rows a wave.
            // Measured on 4096 -> 4096: 5.10 against 5.53 us (and 6.27 with both rows
            // of a wave loaded at once)
            constexpr int TEAMS = 8, R = 1;
            uint32_t grid = (n + TEAMS * R - 1) / (TEAMS * R);
            const uint32_t cap = gc ? gc : cus;
            grid = grid < cap ? grid : cap;
            hipLaunchKernelGGL((k_q80_m1_dig<TEAMS, R>), dim3(grid), dim3(TEAMS * 64), 0, s, x, w, y, k, n,
                               (uint64_t)k / QK8_0 * Q80_BYTES);
            return after_launch("proj_q8_0_m1", s);
        }
        constexpr int TEAMS = 4, R = 2;
        uint32_t grid = (n + TEAMS * R - 1) / (TEAMS * R);
        const uint32_t cap = gc ? gc : cus;  // one per CU: measured best for 4096 rows (5.62 us, 512: 5.73)
        grid = grid < cap ? grid : cap;
        hipLaunchKernelGGL((k_q80_m1_dig<TEAMS, R>), dim3(grid), dim3(TEAMS * 64), 0, s, x, w, y, k, n,
                           (uint64_t)k / QK8_0 * Q80_BYTES);
        return after_launch("proj_q8_0_m1", s);
    }
    if (P <= 128) return launch_q80_t<2, 4>(x, w, y, k, n, s);
    if (P <= 192) return launch_q80_t<3, 2>(x, w, y, k, n, s);
    return launch_q80_t<4, 2>(x, w, y, k, n, s);
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
    if (k == 0) {  // empty sum: c = 0 (a fill kernel, which graph capture records safely)
        LG_EXTENT(c, (uint64_t)n * 4, name);
        hipLaunchKernelGGL(k_fill_zero, dim3((n + 255) / 256), dim3(256), 0, s, c, n);
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
    const bool vec_ok = aligned16(x) && (!fuse || aligned16(up)) && k % QK_K == 0;
    if (dtype == LG_Q4_K && vec_ok && expert_offset % QK_K == 0) {
        const uint8_t *wbase = wb + (uint64_t)expert_offset / QK_K * Q4K_BYTES;
        if (aligned16(wbase)) {
            // Measured on MI355X (4096 -> 14336 / 14336 -> 4096): k <= 4096 plain, the
            // integer dot kernel (8.8 us; k_q4k_m1_wide 9.8); up to 16384, all of k in one
            // workgroup on int8 matrix cores (plain 10.5 us against 13.8 for the vector
            // kernel; fused 11.4-11.8 against 13.9 split over workgroups); beyond, the
            // vector kernel in passes (plain) or the split matrix-core kernel (fused).
            const bool wide = k / QK_K <= WIDE_MAX_SB;
            const uint32_t kind = g_m1_kernel.load(std::memory_order_relaxed);
            if (!fuse) {
                const bool mc = kind == 2 ? wide : kind == 1 ? false : wide && k > 4096;
                return mc ? launch_q4k_wide<false>(x, nullptr, wbase, c, k, n, s)
                          : launch_q4k<false>(x, nullptr, wbase, c, k, n, s);
            }
            if (kind == 1) return launch_q4k<true>(x, up, wbase, c, k, n, s);
            return wide ? launch_q4k_wide<true>(x, up, wbase, c, k, n, s)
                        : launch_q4k_mfma<true>(x, up, wbase, c, k, n, s);
        }
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

namespace lg {

bool proj_m1_in_ok(uint32_t k, const float *x, const M1In &in) {
    auto a16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (k == 0 || k > 4096 || k % QK_K || in.count < 1 || in.count > 4 || !a16(x) || !a16(in.xadd) || !a16(in.nw) ||
        !a16(in.xout) || !a16(in.xcap) || !a16(in.nxout))
        return false;
    for (uint32_t j = 0; j < in.count; j++)
        if (in.type[j] != LG_Q4_K || !in.w[j] || !in.y[j] || !a16(in.w[j])) return false;
    return !in.glu || (in.count == 2 && in.n[0] == in.n[1]);
}

int proj_m1_in(const float *x, const M1In &in, uint32_t k, hipStream_t s) {
    const char *name = "proj_q4k_m1_in";
    LG_REQUIRE(proj_m1_in_ok(k, x, in), "%s: k=%u or its operands are outside the integer-dot path", name, k);
    const uint8_t *w[4] = {};
    float *y[4] = {};
    uint32_t off[4] = {}, n = 0;
    for (uint32_t j = 0; j < in.count; j++) {
        w[j] = static_cast<const uint8_t *>(in.w[j]);
        y[j] = in.y[j];
        off[j] = n;
        n += in.n[j];
    }
    for (uint32_t j = in.count; j < 4; j++) off[j] = n;  // past the count: never selected
    if (n == 0) return LG_OK;
    constexpr int TEAMS = 4, R = 2;
    uint32_t grid = (n + TEAMS * R - 1) / (TEAMS * R);
    const uint32_t gc = g_grid_cap.load(std::memory_order_relaxed);
    const uint32_t cap = gc ? gc : 512;
    grid = grid < cap ? grid : cap;
    int64_t wo[4] = {}, yo[4] = {};
    for (uint32_t j = 1; j < in.count; j++) {  // byte and element offsets from job 0's
        wo[j] = (int64_t)(reinterpret_cast<uintptr_t>(w[j]) - reinterpret_cast<uintptr_t>(w[0]));
        yo[j] = (int64_t)(reinterpret_cast<uintptr_t>(y[j]) - reinterpret_cast<uintptr_t>(y[0])) / 4;
        LG_REQUIRE(((reinterpret_cast<uintptr_t>(y[j]) - reinterpret_cast<uintptr_t>(y[0])) & 3u) == 0,
                   "%s: output %u is not float-aligned with output 0", name, j);
    }
#define LG_DIG_IN(NJ, GLU)                                                                                   \
    hipLaunchKernelGGL((k_q4k_m1_dig_in<TEAMS, R, NJ, GLU>), dim3(grid), dim3(TEAMS * 64), 0, s, x, in.xadd, in.nw, in.xout, \
                       in.xcap, in.nxout, w[0], y[0], wo[1], wo[2], wo[3], yo[1], yo[2], yo[3], off[1], off[2], off[3], \
                       n, in.eps, k, (uint64_t)k / QK_K * Q4K_BYTES)
    if (in.count == 1) LG_DIG_IN(1, false);
    else if (in.glu) LG_DIG_IN(2, true);
    else if (in.count == 2) LG_DIG_IN(2, false);
    else LG_DIG_IN(4, false);
#undef LG_DIG_IN
    return after_launch(name, s);
}

}  // namespace lg

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
    hipStream_t s = (hipStream_t)stream;
    // the result lands in this stream's workspace, after its arrival counters (the f32
    // projection itself uses no workspace), and is copied to the host from there
    void *ws = nullptr;
    LG_TRY(stream_workspace(s, PROJ_WS_COUNTERS + (uint64_t)n * 4, &ws));
    float *tmp = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + PROJ_WS_COUNTERS);
    LG_TRY(lg_dispatch_proj_row(x, w, tmp, k, n, 0, stream));
    LG_HIP_TRY(hipMemcpyAsync(out, tmp, (uint64_t)n * 4, hipMemcpyDeviceToHost, s));
    LG_HIP_TRY(hipStreamSynchronize(s));
    return LG_OK;
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
    g_grid_cap.store(cap, std::memory_order_relaxed);
    return LG_OK;
}

// Number of k slices of the Q4_K M=1 kernel (0 = automatic).  A tuning hook like
// the cap above; results meet the same parity bound for every value and are
// repeatable for a fixed one.
int lg_set_m1_split(uint32_t slices) {
    g_m1_split.store(slices, std::memory_order_relaxed);
    return LG_OK;
}

// Kernel family of the Q4_K M=1 projections (0 = automatic, 1 = vector ALU /
// integer dot products, 2 = int8 matrix cores where k <= 16384).  A tuning hook
// like the two above.
int lg_set_m1_kernel(uint32_t kind) {
    clear_error();
    LG_REQUIRE(kind <= 2, "lg_set_m1_kernel: kind %u (0, 1 or 2)", kind);
    g_m1_kernel.store(kind, std::memory_order_relaxed);
    return LG_OK;
}

}  // extern "C"
