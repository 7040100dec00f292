// DFlash draft model glue and block forward on gfx950.
//
// The reference runs the draft one token at a time through per-op Vulkan
// dispatches with host round trips (K/V sequence rebuilt on the host,
// src/dflash.rs:945-952; softplus on the host, :956-958).  Here a block of m
// tokens goes through the layers on one stream, every intermediate stays in HBM,
// and the projections read the raw GGUF blocks (lg_dispatch_proj_quant_batch).
//
//   rmsnorm / enc_aux_norm      one workgroup per row (or row chunk)
//   qk_norm_rope                one wavefront per (row, head)
//   attention (head_dim 128)    flash-decoding: one workgroup per (kv head, 64
//                               positions); the 64 queries of a kv head (m tokens x
//                               n_q/n_kv heads) against the chunk's keys and values
//                               with v_mfma_f32_16x16x32_bf16, every f32 operand split
//                               exactly into three bf16 parts and the six significant
//                               part products accumulated (f32-grade); per-chunk
//                               maxima, sums and partial outputs merged by a second
//                               kernel
//   attention (other head_dim)  one wavefront per (row, head), online softmax
//   softplus gate, add          elementwise
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "lg_common.hpp"

namespace {

using namespace lg;


typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// f16 parts of f32 values: hi = x rounded to f16 (nearest even), lo = x - hi rounded
// to f16.  hi + lo holds x to about 22 bits while 2^-3 <= |x| < 65504 (below that lo
// is subnormal: absolute error at most 2^-25).  x - hi is one v_fma_mix_f32 (hi's half
// as an f16 operand of an f32 fma, exact), which the compiler forms from fma(hi, neg1,
// x) only while it cannot fold neg1 = -1 into a subtraction: callers pass -1.0f from
// neg_one().
__device__ __forceinline__ float neg_one() {
    float v = -1.0f;
    asm("" : "+s"(v));  // no instruction: hides the constant from the optimizer
    return v;
}
__device__ __forceinline__ void f16_parts2(float a, float b, float neg1, uint32_t &hi, uint32_t &lo) {
    const f16x2 h = __builtin_convertvector((f32x2){a, b}, f16x2);
    const f32x2 d = {__builtin_fmaf((float)h[0], neg1, a), __builtin_fmaf((float)h[1], neg1, b)};
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(d, f16x2));
}
__device__ __forceinline__ void f16_parts8(const float4 &a, const float4 &b, float neg1, f16x8 &hi, f16x8 &lo) {
    uint4 h, l;
    f16_parts2(a.x, a.y, neg1, h.x, l.x);
    f16_parts2(a.z, a.w, neg1, h.y, l.y);
    f16_parts2(b.x, b.y, neg1, h.z, l.z);
    f16_parts2(b.z, b.w, neg1, h.w, l.w);
    hi = __builtin_bit_cast(f16x8, h);
    lo = __builtin_bit_cast(f16x8, l);
}
__device__ __forceinline__ void f16_parts4(float a, float b, float c, float d, float neg1, f16x4 &hi,
                                           f16x4 &lo) {
    uint2 h, l;
    f16_parts2(a, b, neg1, h.x, l.x);
    f16_parts2(c, d, neg1, h.y, l.y);
    hi = __builtin_bit_cast(f16x4, h);
    lo = __builtin_bit_cast(f16x4, l);
}
// max(acc, |x|) over the eight values of a and b: v_max3_f32 with |x| operands (as
// asm, since fmaxf would first quiet every operand; a NaN operand may give NaN, and
// callers treat a NaN maximum as out of range)
__device__ __forceinline__ float absmax3(float acc, float a, float b) {
    float d;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(d) : "v"(acc), "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ float absmax8(float acc, const float4 &a, const float4 &b) {
    acc = absmax3(acc, a.x, a.y);
    acc = absmax3(acc, a.z, a.w);
    acc = absmax3(acc, b.x, b.y);
    return absmax3(acc, b.z, b.w);
}


// Sum over the threads of a workgroup of THREADS; every thread receives it.
template <int THREADS>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < THREADS / 64; w++) s += red[w];
    __syncthreads();
    return s;
}

// ------------------------------------------------------------------------------------------
// RMSNorm (kernels/rmsnorm.comp:23-34, kernels/enc_aux_norm.comp:21-43)

// Row `blockIdx.x` of `x` (n floats, row stride ldx): out = x * w * (mean(x^2)+eps)^-1/2.
// blockIdx.y selects a chunk of n floats inside the row (enc_aux_norm: chunk aux of a
// token's n_aux * n_feat features, weights w + aux * n).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, const float *__restrict__ w, float *out, uint32_t n,
                                                 uint32_t ldx, float eps) {
    __shared__ float red[4];
    const uint64_t base = (uint64_t)blockIdx.x * ldx + (uint64_t)blockIdx.y * n;
    const float *xr = x + base;
    const float *wr = w + (uint64_t)blockIdx.y * n;
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) s = __builtin_fmaf(xr[i], xr[i], s);
    const float ms = block_sum<256>(s, red) / (float)n;
    const float rms = 1.0f / sqrtf(ms + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 256) out[base + i] = xr[i] * wr[i] * rms;
}

// The same for rows of n = 1024 * V4 floats (16-byte aligned): each thread keeps its
// V4 float4 of the row in registers (one load each, all in flight together).
template <int V4>
__global__ __launch_bounds__(256) void k_rmsnorm4(const float *x, const float *__restrict__ w, float *out,
                                                  uint32_t n, uint32_t ldx, float eps) {
    __shared__ float red[4];
    const uint64_t base = (uint64_t)blockIdx.x * ldx + (uint64_t)blockIdx.y * n;
    const float4 *xr = reinterpret_cast<const float4 *>(x + base);
    const float4 *wr = reinterpret_cast<const float4 *>(w + (uint64_t)blockIdx.y * n);
    float4 v[V4], wv[V4];
#pragma unroll
    for (int i = 0; i < V4; i++) {
        v[i] = xr[i * 256 + threadIdx.x];
        wv[i] = wr[i * 256 + threadIdx.x];
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V4; i++)
        s = __builtin_fmaf(v[i].x, v[i].x, __builtin_fmaf(v[i].y, v[i].y,
            __builtin_fmaf(v[i].z, v[i].z, __builtin_fmaf(v[i].w, v[i].w, s))));
    const float ms = block_sum<256>(s, red) / (float)n;
    const float rms = 1.0f / sqrtf(ms + eps);
    float4 *o = reinterpret_cast<float4 *>(out + base);
#pragma unroll
    for (int i = 0; i < V4; i++)
        o[i * 256 + threadIdx.x] = make_float4(v[i].x * wv[i].x * rms, v[i].y * wv[i].y * rms, v[i].z * wv[i].z * rms,
                                               v[i].w * wv[i].w * rms);
}

// The block forward's norms folded into its projections (the products apply the
// norm's weight and 1/rms around them; csrc/proj_batch.hip).  What stays outside
// runs in one launch at the start of the block, workgroup (row, j):
//  * j < run.count: the encoder's output norm of row `row` and layer run.w[j]'s
//    attention norm of it (the injected rows are the same in every layer):
//      xe = x w / rms(x) (stored by j = 0),   out_j = xe run.w[j] / rms(xe),
//    with the arithmetic of k_rmsnorm4, so the rows equal the two norms run apart;
//  * j = run.count (when tok is given): token row `row` entering layer 0:
//    xt = tok, yt = tok * wt (layer 0's attention-norm weight, its 1/rms left to the
//    products), and the sum of tok^2 in slot 0 of the row's `cols` slots of ss (the
//    others zero): the layout the products' norm epilogue writes.
constexpr uint32_t NORM_RUN = 8;
struct NormRun {
    const float *w[NORM_RUN];
    float *out[NORM_RUN];
    uint32_t count;
    const float *tok, *wt;
    float *xt, *yt, *ss;
    uint32_t cols;
    float *rope;        // with freq (64 entries): the rotation table of positions pos0 + p,
    const float *freq;  // p < 2 * rows: rope[p][i] = cos (i < 64) or sin (i >= 64) of
    uint32_t pos0;      // freq[i % 64] * (pos0 + p), as k_qk_norm_rope computes them
};

// Rows of n floats, n a multiple of 4 up to 1024 V4: thread i holds float4s i,
// i + 256, ... of the row (zeros past its end).
template <int V4>
__device__ __forceinline__ void load_row4(const float *__restrict__ r, uint32_t n, float4 (&v)[V4]) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const uint32_t e = i * 256 + threadIdx.x;
        v[i] = e < n / 4 ? reinterpret_cast<const float4 *>(r)[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int V4>
__device__ __forceinline__ void store_row4(float *__restrict__ r, uint32_t n, const float4 (&v)[V4]) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const uint32_t e = i * 256 + threadIdx.x;
        if (e < n / 4) reinterpret_cast<float4 *>(r)[e] = v[i];
    }
}

template <int V4>
__device__ __forceinline__ float sum_sq4(const float4 (&v)[V4], float *red) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V4; i++)
        s = __builtin_fmaf(v[i].x, v[i].x, __builtin_fmaf(v[i].y, v[i].y,
            __builtin_fmaf(v[i].z, v[i].z, __builtin_fmaf(v[i].w, v[i].w, s))));
    return block_sum<256>(s, red);
}

__device__ __forceinline__ float4 mul4(float4 a, float4 b, float c) {
    return make_float4(a.x * b.x * c, a.y * b.y * c, a.z * b.z * c, a.w * b.w * c);
}

template <int V4>
__global__ __launch_bounds__(256) void k_norms_in(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ xe, NormRun run, uint32_t n, float eps) {
    __shared__ float red[4];
    const uint64_t base = (uint64_t)blockIdx.x * n;
    const uint32_t j = blockIdx.y;
    float4 v[V4], wv[V4];
    if (run.rope && j == run.count + (run.tok ? 1u : 0u)) {  // two positions of the rotation table
        const uint32_t p = 2 * blockIdx.x + (threadIdx.x >> 7), i = threadIdx.x & 127u;
        const float ang = run.freq[i & 63u] * (float)(run.pos0 + p);
        run.rope[(uint64_t)p * 128 + i] = i < 64 ? cosf(ang) : sinf(ang);
        return;
    }
    if (j == run.count) {  // a token row
        load_row4<V4>(run.tok + base, n, v);
        load_row4<V4>(run.wt, n, wv);
        store_row4<V4>(run.xt + base, n, v);
#pragma unroll
        for (int i = 0; i < V4; i++) wv[i] = mul4(v[i], wv[i], 1.0f);
        store_row4<V4>(run.yt + base, n, wv);
        const float s = sum_sq4<V4>(v, red);
        for (uint32_t p = threadIdx.x; p < run.cols; p += 256)
            run.ss[(uint64_t)blockIdx.x * run.cols + p] = p == 0 ? s : 0.0f;
        return;
    }
    load_row4<V4>(x + base, n, v);
    load_row4<V4>(w, n, wv);
    const float rms = 1.0f / sqrtf(sum_sq4<V4>(v, red) / (float)n + eps);
#pragma unroll
    for (int i = 0; i < V4; i++) v[i] = mul4(v[i], wv[i], rms);
    if (j == 0) store_row4<V4>(xe + base, n, v);
    const float rms2 = 1.0f / sqrtf(sum_sq4<V4>(v, red) / (float)n + eps);
    load_row4<V4>(run.w[j], n, wv);
#pragma unroll
    for (int i = 0; i < V4; i++) wv[i] = mul4(v[i], wv[i], rms2);
    store_row4<V4>(run.out[j] + base, n, wv);
}

// ------------------------------------------------------------------------------------------
// QK-norm + NeoX RoPE (kernels/qk_norm_rope.comp:23-67): one wavefront per (row, head).

// One tensor's share of a launch: rows x n_heads heads of hd floats, row r at
// position pos0 + r.  In place (out == x) is allowed: a wavefront reads its head
// before writing it.
struct QkJob {
    const float *x, *w;
    float *out;
    uint32_t n_heads, pos0, units, blocks;
};

// The forward's attention gate of the tokens, when its weights are raw Q4_K blocks:
// out[r][h] = sum_j x[r][j] W[h][j] (src/dflash.rs:942-944), one wavefront per
// (row, head), lane p taking the 64-element groups p, p + 64, ... of the row.
// With ss (the folded attention norm: x arrives with the norm's weight applied),
// row r's result is multiplied by (sum_{p < cols} ss[r * cols + p] / k + eps)^-1/2,
// cols <= 64.
struct GateJob {
    const float *x;
    const uint8_t *w;
    float *out;
    uint32_t n_heads, k, units, blocks;
    const float *ss;
    uint32_t cols;
    float eps;
};

// Unit (row, head) = (unit / n_heads, unit % n_heads), unit < units: every lane
// receives the result.
__device__ __forceinline__ float gate_value(const GateJob &g, uint32_t unit, uint32_t lane) {
    const uint32_t row = unit / g.n_heads, head = unit % g.n_heads;
    const float *xr = g.x + (uint64_t)row * g.k;
    const uint8_t *wr = g.w + (uint64_t)head * (g.k / QK_K) * Q4K_BYTES;
    float acc = 0.0f;
    for (uint32_t p = lane; p < g.k / 64; p += 64) {
        const uint8_t *blk = wr + (uint64_t)(p >> 2) * Q4K_BYTES;
        const uint32_t gi = p & 3u;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * gi);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * gi);
        const float4 *x4 = reinterpret_cast<const float4 *>(xr + 64 * p);
        float xv[64];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 t = x4[i];
            xv[4 * i] = t.x, xv[4 * i + 1] = t.y, xv[4 * i + 2] = t.z, xv[4 * i + 3] = t.w;
        }
        const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float slo = 0.0f, shi = 0.0f, xlo = 0.0f, xhi = 0.0f;  // sub-blocks 2gi (low nibbles), 2gi+1 (high)
#pragma unroll
        for (int b = 0; b < 32; b++) {
            const uint32_t byte = (qw[b >> 2] >> (8 * (b & 3))) & 0xFFu;
            slo = __builtin_fmaf(xv[b], (float)(byte & 15u), slo);
            shi = __builtin_fmaf(xv[32 + b], (float)(byte >> 4), shi);
            xlo += xv[b];
            xhi += xv[32 + b];
        }
        uint32_t sc0, m0, sc1, m1;
        scale_min_k4(2 * gi, hd.y, hd.z, hd.w, sc0, m0);
        scale_min_k4(2 * gi + 1, hd.y, hd.z, hd.w, sc1, m1);
        const float d = ref_half(hd.x & 0xFFFFu), dmin = ref_half(hd.x >> 16);
        acc += (d * (float)sc0) * slo - (dmin * (float)m0) * xlo + (d * (float)sc1) * shi - (dmin * (float)m1) * xhi;
    }
    acc = wave_sum(acc);
    if (g.ss) {
        const float p = lane < g.cols ? g.ss[(uint64_t)row * g.cols + lane] : 0.0f;
        acc *= 1.0f / sqrtf(wave_sum(p) / (float)g.k + g.eps);
    }
    return acc;
}

__device__ __forceinline__ void gate_dot(const GateJob &g, uint32_t unit, uint32_t lane) {
    if (unit >= g.units) return;
    const float acc = gate_value(g, unit, lane);
    if (lane == 0) g.out[unit] = acc;
}

// Job a takes workgroups 0 .. a.blocks-1, job b the next b.blocks (the forward's K
// and Q), and the gate job the rest.
__global__ __launch_bounds__(256) void k_qk_norm_rope(QkJob a, QkJob b, const float *__restrict__ freq, uint32_t hd,
                                                      uint32_t rope_dim, float eps, GateJob gj) {
    __shared__ float nrm[4][256];
    if (blockIdx.x >= a.blocks + b.blocks) {  // uniform over the workgroup
        gate_dot(gj, (blockIdx.x - a.blocks - b.blocks) * 4 + (threadIdx.x >> 6), threadIdx.x & 63u);
        return;
    }
    const bool second = blockIdx.x >= a.blocks;
    const QkJob &jb = second ? b : a;
    const float *x = jb.x, *__restrict__ w = jb.w;
    float *out = jb.out;
    const uint32_t n_heads = jb.n_heads, pos0 = jb.pos0, units = jb.units;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t unit = (blockIdx.x - (second ? a.blocks : 0u)) * 4 + wave;  // (row, head)
    const bool live = unit < units;
    const uint32_t row = live ? unit / n_heads : 0, head = live ? unit % n_heads : 0;
    const float *xh = x + (uint64_t)row * n_heads * hd + (uint64_t)head * hd;
    float v[4];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t d = lane + 64 * j;
        v[j] = (live && d < hd) ? xh[d] : 0.0f;
        s = __builtin_fmaf(v[j], v[j], s);
    }
    const float ms = wave_sum(s) / (float)hd;
    const float rms = 1.0f / sqrtf(ms + eps);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t d = lane + 64 * j;
        if (d < hd) nrm[wave][d] = v[j] * w[d] * rms;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (!live) return;
    const uint32_t half = rope_dim / 2, hd2 = hd / 2;
    const float fpos = (float)(pos0 + row);
    float *oh = out + (uint64_t)row * n_heads * hd + (uint64_t)head * hd;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t d = lane + 64 * j;
        if (d >= hd) continue;
        const float n = nrm[wave][d];
        if (d >= rope_dim) {
            oh[d] = n;
            continue;
        }
        const float ang = freq[d % half] * fpos;
        const float c = cosf(ang), sn = sinf(ang);
        oh[d] = d < half ? n * c - nrm[wave][d + hd2] * sn : n * c + nrm[wave][d - hd2] * sn;
    }
}

// ------------------------------------------------------------------------------------------
// Attention, head_dim 128, matrix cores.
//
// Sequence: positions p < n0 come from (k0, v0) row p, positions n0 <= p < S from
// (k1, v1) row p - n0 (the reference's K/V sequence without the host copy).  Query qi
// of kv head h is (row t = qi / G, q head h*G + qi % G), at position qpos0 + t.

constexpr uint32_t AHD = 128;  // head dim of the matrix-core path
constexpr uint32_t ACH = 64;   // positions per chunk of the few-query kernels (k_attn_decode, k_attn_token)
constexpr uint32_t AQ = 64;    // queries per kv head handled by one workgroup

// Max over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows), in every lane.
__device__ __forceinline__ float rows4_max(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Chunks of k_attn_split: the sequence's ceil(S / 16) position tiles split into nch
// runs of consecutive tiles, chunk c taking tiles [c nt / nch, (c + 1) nt / nch).
// floor(c nt / nch) in 32-bit steps (c <= nch < 2^16): c floor(nt / nch) + floor(c (nt mod
// nch) / nch) -- a 64-bit division by a runtime value is a long software loop on the GPU.
__host__ __device__ inline uint32_t attn_tile0(uint32_t c, uint32_t nt, uint32_t nch) {
    const uint32_t q = nt / nch, r = nt - q * nch;
    return c * q + c * r / nch;
}

__device__ __forceinline__ float softplus_gate(float g) { return g > 20.0f ? g : logf(1.0f + expf(g)); }  // src/dflash.rs:957

// The chunk partials for a few queries (rows * G <= ADQ: one token's
// query heads), straight from memory in f32: no bf16 parts, no LDS tiles.  One
// workgroup per (64-position chunk, kv head); wave w takes positions 16w .. 16w+15.
//   scores: lane (p, quarter) dots the 32 dims 32 quarter .. of K row p with every
//           query (held in LDS), the four quarters meet in two lane swaps;
//   softmax: wave w takes queries w, w + 4 over the chunk's 64 scores;
//   P V: each wave adds its 16 positions for every query (lane = dims 2l, 2l+1), and
//        the four waves' sums meet in LDS in wave order.
// Every K and V load of the chunk is issued at the start.  Partials per (kv head,
// chunk, query): the unnormalised O (AHD floats), and the chunk's max and sum.
constexpr uint32_t ADQ = 8;

__global__ __launch_bounds__(256) void k_attn_decode(const float *__restrict__ q, const float *__restrict__ k0,
                                                     const float *__restrict__ v0, uint32_t n0,
                                                     const float *__restrict__ k1, const float *__restrict__ v1,
                                                     uint32_t S, uint32_t rows, uint32_t n_q, uint32_t n_kv,
                                                     uint32_t qpos0, int causal, float scale, uint32_t nch,
                                                     float *__restrict__ part_o, float *__restrict__ part_ml) {
    __shared__ float4 lq[ADQ][AHD / 4];
    __shared__ float lp[ADQ][ACH];
    __shared__ float lo[4][ADQ][AHD];
    const uint32_t h = blockIdx.y, c = blockIdx.x;
    const uint32_t G = n_q / n_kv, nq = rows * G;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kvld = n_kv * AHD;
    auto kv_row = [&](const float *a0, const float *a1, uint32_t p) {  // position p of the sequence (p < S)
        return p < n0 ? a0 + (uint64_t)p * kvld : a1 + (uint64_t)(p - n0) * kvld;
    };
    // K: position 16 wave + (lane & 15), dims 32 (lane >> 4) ..; V: position 16 wave + j, dims 2 lane ..
    const uint32_t pk = c * ACH + 16 * wave + (lane & 15u), qd = lane >> 4;
    float4 kr[8];
    {
        const float *kp = kv_row(k0, k1, pk < S ? pk : S - 1) + h * AHD + 32 * qd;
#pragma unroll
        for (int i = 0; i < 8; i++) kr[i] = reinterpret_cast<const float4 *>(kp)[i];
    }
    float2 vr[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t p = c * ACH + 16 * wave + j;
        vr[j] = reinterpret_cast<const float2 *>(kv_row(v0, v1, p < S ? p : S - 1) + h * AHD)[lane];
    }
    for (uint32_t e = tid; e < nq * (AHD / 4); e += 256) {
        const uint32_t qi = e / (AHD / 4), t = qi / G, hq = h * G + qi % G;
        lq[qi][e % (AHD / 4)] = reinterpret_cast<const float4 *>(q + (uint64_t)t * n_q * AHD + hq * AHD)[e % (AHD / 4)];
    }
    __syncthreads();
    // scores of position pk for every query
    for (uint32_t qi = 0; qi < nq; qi++) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 qv = lq[qi][8 * qd + i];
            d = __builtin_fmaf(kr[i].x, qv.x, __builtin_fmaf(kr[i].y, qv.y,
                __builtin_fmaf(kr[i].z, qv.z, __builtin_fmaf(kr[i].w, qv.w, d))));
        }
        d = lane_add_x32(lane_add_x16(d));  // the four quarters
        const uint32_t qpos = qpos0 + qi / G;
        const bool ok = pk < S && (!causal || pk <= qpos);
        if (qd == 0) lp[qi][16 * wave + (lane & 15u)] = ok ? d * scale : -INFINITY;
    }
    __syncthreads();
    // softmax over the chunk: wave w, queries w and w + 4
    for (uint32_t qi = wave; qi < nq; qi += 4) {
        const float sv = lp[qi][lane];
        float m = sv;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float mu = m == -INFINITY ? 0.0f : m;  // a fully masked chunk has P = 0
        const float pv = expf(sv - mu);
        lp[qi][lane] = pv;
        const float l = wave_sum(pv);
        if (lane == 0) {
            const uint64_t pi = ((uint64_t)h * nch + c) * AQ + qi;
            part_ml[2 * pi] = m;
            part_ml[2 * pi + 1] = l;
        }
    }
    __syncthreads();
    // P V over this wave's 16 positions, every query
    for (uint32_t qi = 0; qi < nq; qi++) {
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float pw = lp[qi][16 * wave + j];
            o0 = __builtin_fmaf(pw, vr[j].x, o0);
            o1 = __builtin_fmaf(pw, vr[j].y, o1);
        }
        lo[wave][qi][2 * lane] = o0;
        lo[wave][qi][2 * lane + 1] = o1;
    }
    __syncthreads();
    for (uint32_t e = tid; e < nq * AHD; e += 256) {
        const uint32_t qi = e / AHD, d = e % AHD;
        const uint64_t pi = ((uint64_t)h * nch + c) * AQ + qi;
        part_o[pi * AHD + d] = ((lo[0][qi][d] + lo[1][qi][d]) + lo[2][qi][d]) + lo[3][qi][d];
    }
}

// One token's attention over a cache (the dense target, src/target.rs:443-507):
// QK-norm + NeoX RoPE of the token's query heads as each workgroup stages them, and of
// its key (row S-1 of the K sequence, normed in place by the workgroup whose chunk
// holds it, so the cache keeps it normed), then the chunk partials of k_attn_decode
// for k_attn_combine.  The norms follow k_qk_norm_rope (one head per wavefront, lane d
// holding dims d and d + 64).  Combining the chunks in the last workgroup of each kv
// head to finish (an arrival counter) instead of a second launch measured slower
// (440 against 413 us per target token): its loads of every chunk's partials sit on
// the critical path.
struct TokAttn {
    const float *q;            // [n_q][128], as projected
    const float *qn_w, *kn_w;  // QK-norm weights [128]
    const float *freq;         // RoPE table (64 entries) when rope_dim is 128
    uint32_t rope, pos;        // rope_dim is 128 (1) or 0; the token's position
    float eps, scale;
    float *k;                  // [S][n_kv][128]: rows below S-1 normed and roped, row S-1 as projected
    const float *v;            // [S][n_kv][128]
    uint32_t S, n_q, n_kv, nch;
    float *part_o, *part_ml;   // per (kv head, chunk, query): as k_attn_decode writes them
};

// A head (128 floats, lane d: dims d and d + 64) normed with weights (w0, w1) and
// rotated at `pos` by the lane's frequency fr.
__device__ __forceinline__ void head_norm_rope(float &a, float &b, float w0, float w1, float fr, const TokAttn &t) {
    float s = __builtin_fmaf(a, a, 0.0f);
    s = __builtin_fmaf(b, b, s);
    const float rms = 1.0f / sqrtf(wave_sum(s) / (float)AHD + t.eps);
    const float n0 = a * w0 * rms, n1 = b * w1 * rms;
    if (!t.rope) {
        a = n0, b = n1;
        return;
    }
    const float ang = fr * (float)t.pos;
    const float c = cosf(ang), sn = sinf(ang);
    a = n0 * c - n1 * sn;
    b = n1 * c + n0 * sn;
}

__global__ __launch_bounds__(256) void k_attn_token(TokAttn t) {
    constexpr uint32_t QW = ADQ / 4;  // query heads per wavefront
    __shared__ float lq[ADQ][AHD];
    __shared__ float lkn[AHD];
    __shared__ float lp[ADQ][ACH];
    __shared__ float lo[4][ADQ][AHD];
    const uint32_t h = blockIdx.y, c = blockIdx.x;
    const uint32_t G = t.n_q / t.n_kv, nq = G;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kvld = t.n_kv * AHD, S = t.S, self = S - 1;
    const bool owner = self / ACH == c;  // this chunk holds the token's own key
    const bool kown = owner && wave == 3;
    const uint32_t pk = c * ACH + 16 * wave + (lane & 15u), qd = lane >> 4;
    // The wave's query heads (qi = wave, wave + 4), the norm weights, the lane's
    // rotation frequency and (kown) the token's key are loaded ahead of the cache
    // rows: loads complete in issue order, so the norms then wait only for these.
    float qa[QW], qb[QW];
#pragma unroll
    for (uint32_t r = 0; r < QW; r++) {
        const uint32_t qi = wave + 4 * r < nq ? wave + 4 * r : 0;  // branch-free: unused heads read head 0
        const float *qp = t.q + (uint64_t)(h * G + qi) * AHD;
        qa[r] = qp[lane];
        qb[r] = qp[64 + lane];
    }
    const float wq0 = t.qn_w[lane], wq1 = t.qn_w[64 + lane];
    const float fr = t.rope ? t.freq[lane] : 0.0f;
    float ka = 0.0f, kb = 0.0f, wk0 = 0.0f, wk1 = 0.0f;
    float *kself = t.k + (uint64_t)self * kvld + h * AHD;
    if (kown) {
        ka = kself[lane], kb = kself[64 + lane];
        wk0 = t.kn_w[lane], wk1 = t.kn_w[64 + lane];
    }
    asm volatile("" ::: "memory");  // keep these loads issued before the cache rows
    float4 kr[8];
    {
        const float *kp = t.k + (uint64_t)(pk < S ? pk : S - 1) * kvld + h * AHD + 32 * qd;
#pragma unroll
        for (int i = 0; i < 8; i++) kr[i] = reinterpret_cast<const float4 *>(kp)[i];
    }
    float2 vr[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t p = c * ACH + 16 * wave + j;
        vr[j] = reinterpret_cast<const float2 *>(t.v + (uint64_t)(p < S ? p : S - 1) * kvld + h * AHD)[lane];
    }
    // the query heads of this kv head, and (owner) the token's key, normed and rotated
#pragma unroll
    for (uint32_t r = 0; r < QW; r++) {
        const uint32_t qi = wave + 4 * r;
        if (qi >= nq) break;  // uniform over the wave
        float a = qa[r], b = qb[r];
        head_norm_rope(a, b, wq0, wq1, fr, t);
        lq[qi][lane] = a;
        lq[qi][64 + lane] = b;
    }
    if (kown) {
        head_norm_rope(ka, kb, wk0, wk1, fr, t);
        lkn[lane] = ka;
        lkn[64 + lane] = kb;
        kself[lane] = ka;  // the cache keeps the normed key (no other workgroup reads this row)
        kself[64 + lane] = kb;
    }
    __syncthreads();
    if (owner && pk == self)
#pragma unroll
        for (int i = 0; i < 8; i++) kr[i] = reinterpret_cast<const float4 *>(lkn)[8 * qd + i];
    // scores of position pk for every query (causal: every position up to the token's)
    for (uint32_t qi = 0; qi < nq; qi++) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 qv = reinterpret_cast<const float4 *>(lq[qi])[8 * qd + i];
            d = __builtin_fmaf(kr[i].x, qv.x, __builtin_fmaf(kr[i].y, qv.y,
                __builtin_fmaf(kr[i].z, qv.z, __builtin_fmaf(kr[i].w, qv.w, d))));
        }
        d = lane_add_x32(lane_add_x16(d));
        if (qd == 0) lp[qi][16 * wave + (lane & 15u)] = pk < S ? d * t.scale : -INFINITY;
    }
    __syncthreads();
    const uint64_t pbase = ((uint64_t)h * t.nch + c) * AQ;
    for (uint32_t qi = wave; qi < nq; qi += 4) {
        const float sv = lp[qi][lane];
        float m = sv;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float mu = m == -INFINITY ? 0.0f : m;
        const float pv = expf(sv - mu);
        lp[qi][lane] = pv;
        const float l = wave_sum(pv);
        if (lane == 0) {
            t.part_ml[2 * (pbase + qi)] = m;
            t.part_ml[2 * (pbase + qi) + 1] = l;
        }
    }
    __syncthreads();
    for (uint32_t qi = 0; qi < nq; qi++) {
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float pw = lp[qi][16 * wave + j];
            o0 = __builtin_fmaf(pw, vr[j].x, o0);
            o1 = __builtin_fmaf(pw, vr[j].y, o1);
        }
        lo[wave][qi][2 * lane] = o0;
        lo[wave][qi][2 * lane + 1] = o1;
    }
    __syncthreads();
    for (uint32_t e = tid; e < nq * AHD; e += 256) {
        const uint32_t qi = e / AHD, d = e % AHD;
        t.part_o[(pbase + qi) * AHD + d] = ((lo[0][qi][d] + lo[1][qi][d]) + lo[2][qi][d]) + lo[3][qi][d];
    }
}

// With the few-query chunk kernels, the block's own positions (the `tail`, at most
// ATAIL, after the n0 context positions that those chunks cover) are attended here,
// in f32: wave w takes tail positions 16w .. 16w+15 and forms a partial like a chunk's.
constexpr uint32_t ATAIL = 64;

// out[t][hq][d] = sum_c e^(m_c - M) O_c[d] / sum_c e^(m_c - M) l_c.  One workgroup per
// query: wave w takes its part of the tail, then its share of the chunks (their
// partials loaded CB at a time, all in flight together), merged into one partial
// relative to the wave's own max; the four meet in LDS, each scaled to the overall
// max, added in wave order.  With `gate` ([rows][n_q]), the result of head hq of
// row t is then multiplied by softplus(gate[t][hq]) (gmode 1: the draft forward's
// attention gate, src/dflash.rs:956-959; gmode 2: kernels/gate_attn.comp:27, the
// target's, log(1 + exp(g)) with no threshold).  With gj.units > 0 the gate is
// computed here instead (the draft's Q4_K gate, unit t * n_q + hq), by wave 3,
// which then has no share of the chunks, nor of the tail while it fits waves 0-2.
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part_o,
                                                      const float *__restrict__ part_ml, float *__restrict__ out,
                                                      uint32_t rows, uint32_t n_q, uint32_t n_kv, uint32_t nch,
                                                      const float *__restrict__ gate, const float *__restrict__ q,
                                                      const float *__restrict__ k1, const float *__restrict__ v1,
                                                      uint32_t T, uint32_t n0, uint32_t qpos0, int causal,
                                                      float scale, int gmode, GateJob gj) {
    constexpr uint32_t CB = 12, TW = ATAIL / 4;
    __shared__ float sm[4], sl[4], so[4][AHD], sg;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t gq = blockIdx.x;  // over n_kv * AQ
    const uint32_t G = n_q / n_kv;
    const uint32_t h = gq / AQ, qi = gq % AQ;
    if (h >= n_kv || qi >= rows * G) return;  // uniform over the workgroup
    const uint64_t q0 = (uint64_t)h * nch * AQ + qi;  // partial index of chunk c: q0 + c * AQ
    // the chunks over waves 0-3, or 0-2 when wave 3 computes the gate
    const uint32_t nw = gj.units ? 3 : 4, per = (nch + nw - 1) / nw;
    const uint32_t cb0 = wave < nw ? wave * per : nch, cb1 = cb0 + per < nch ? cb0 + per : nch;
    if (gj.units && wave == 3) {  // uniform over the wave
        const float gv = gate_value(gj, (qi / G) * n_q + h * G + qi % G, lane);
        if (lane == 0) sg = gv;
    }
    // this wave's tail partial (tm, tl, t0, t1): scores made uniform over the wave
    float tm = -INFINITY, tl = 0.0f, t0 = 0.0f, t1 = 0.0f;
    if (T > wave * TW) {
        const uint32_t t = qi / G, hq = h * G + qi % G, qpos = qpos0 + t, kvld = n_kv * AHD;
        const float *qp = q + (uint64_t)t * n_q * AHD + hq * AHD;
        const float qa = qp[lane], qb = qp[64 + lane];
        float ka[TW], kb[TW], va[TW], vb[TW];
#pragma unroll
        for (uint32_t j = 0; j < TW; j++) {  // branch-free: positions past T read position T-1 (masked below)
            const uint32_t jj = wave * TW + j < T ? wave * TW + j : T - 1;
            const uint64_t o = (uint64_t)jj * kvld + h * AHD;
            ka[j] = k1[o + lane], kb[j] = k1[o + 64 + lane];
            va[j] = v1[o + lane], vb[j] = v1[o + 64 + lane];
        }
        float sc[TW];
#pragma unroll
        for (uint32_t j = 0; j < TW; j++) {
            const uint32_t jj = wave * TW + j;
            const float d = wave_sum(__builtin_fmaf(qa, ka[j], qb * kb[j]));
            const float sv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(d))) * scale;
            const bool ok = jj < T && (!causal || n0 + jj <= qpos);
            sc[j] = ok ? sv : -INFINITY;
            tm = fmaxf(tm, sc[j]);
        }
        if (tm != -INFINITY) {
#pragma unroll
            for (uint32_t j = 0; j < TW; j++) {  // tail order
                const float w = expf(sc[j] - tm);
                tl += w;
                t0 = __builtin_fmaf(w, va[j], t0);
                t1 = __builtin_fmaf(w, vb[j], t1);
            }
        }
    }
    // This wave's chunks, CB at a time with every load in flight, merged into the
    // wave's (M, L, o0, o1) after its tail partial: what is merged so far is rescaled
    // to the batch's max (exactly 1 when the max does not move).
    float M = tm, L = tl, o0 = t0, o1 = t1;
    for (uint32_t c0 = cb0; c0 < cb1; c0 += CB) {
        float mc[CB], lc[CB], a0[CB], a1[CB];
#pragma unroll
        for (uint32_t b = 0; b < CB; b++) {
            const uint32_t c = c0 + b < cb1 ? c0 + b : cb1 - 1;
            const uint64_t pq = q0 + (uint64_t)c * AQ;
            const float2 ml = *reinterpret_cast<const float2 *>(part_ml + 2 * pq);
            mc[b] = c0 + b < cb1 ? ml.x : -INFINITY;
            lc[b] = ml.y;
            a0[b] = part_o[pq * AHD + lane];
            a1[b] = part_o[pq * AHD + 64 + lane];
        }
        float mn = M;
#pragma unroll
        for (uint32_t b = 0; b < CB; b++) mn = fmaxf(mn, mc[b]);
        const float f = M == -INFINITY ? 0.0f : expf(M - mn);
        L *= f, o0 *= f, o1 *= f;
#pragma unroll
        for (uint32_t b = 0; b < CB; b++) {  // chunk order
            const float wgt = mc[b] == -INFINITY ? 0.0f : expf(mc[b] - mn);
            L = __builtin_fmaf(wgt, lc[b], L);
            o0 = __builtin_fmaf(wgt, a0[b], o0);
            o1 = __builtin_fmaf(wgt, a1[b], o1);
        }
        M = mn;
    }
    if (lane == 0) sm[wave] = M, sl[wave] = L;
    so[wave][lane] = o0;
    so[wave][64 + lane] = o1;
    __syncthreads();
    if (wave != 0) return;
    // the four waves in wave order, each scaled to the overall max
    const float Mx = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float f = sm[w] == -INFINITY ? 0.0f : expf(sm[w] - Mx);
        L = __builtin_fmaf(f, sl[w], L);
        o0 = __builtin_fmaf(f, so[w][lane], o0);
        o1 = __builtin_fmaf(f, so[w][64 + lane], o1);
    }
    const uint32_t t = qi / G, hq = h * G + qi % G;
    float *o = out + (uint64_t)t * n_q * AHD + hq * AHD;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (gate || gj.units) {
        const float gv = gj.units ? sg : gate[(uint64_t)t * n_q + hq];
        const float g = gmode == 2 ? logf(1.0f + expf(gv)) : softplus_gate(gv);
        o[lane] = (o0 * inv) * g;
        o[64 + lane] = (o1 * inv) * g;
    } else {
        o[lane] = o0 * inv;
        o[64 + lane] = o1 * inv;
    }
}

// Many queries (rows * G > ADQ), one launch.  Workgroup (kv head h, query group qg,
// chunk c) takes queries 16 qg .. 16 qg + 15 of kv head h (query qi: row qi / G, q head
// h G + qi % G) over chunk c of the sequence's 16-position tiles, its wavefront w the
// tiles tb + w, tb + w + 4, ...  K and V stream from memory straight into matrix
// products, whose k index runs over dims / positions in the order the lanes load them:
//   S^T = K Q^T   A = K: lane (position l16, kg) holds dims 16b + 4kg .. +3 of its row
//                 in one float4 (kr[b]); B = Q^T likewise;
//   P = exp(S - running max) per query (lane l16's query, four positions per lane);
//   O^T += V^T P^T  A = V^T: lane (l16, kg) loads dims 64hh + 4 l16 .. +3 of position
//                 4kg + s, and component cc feeds output tile 4hh + cc (dim 64hh + 4i
//                 + cc of its row i); B = P^T, the lane's own probabilities.
// Each product is three f16 matrix products over the operands' f16 parts, hi hi + hi lo
// + lo hi (f16_parts2: every f16 product is exact in f32, and the dropped lo lo is below
// 2^-21 of hi hi): S on v_mfma_f32_16x16x32_f16 (blocks 2j, 2j + 1 of kr form the eight
// halves of k step j), P V on v_mfma_f32_16x16x16f16 (halves s = 0..3: positions 4kg +
// s).  A tile whose K or V (or a query) has a magnitude f16 cannot hold, or whose V is
// all below 2^-4 (where lo's subnormal floor would show), takes that product in f32 on
// v_mfma_f32_16x16x4f32 instead (k steps over the same lanes' values).  No LDS for K
// and V.  The four wavefronts
// meet in LDS (one partial per workgroup), the partial goes to the workspace, and the
// last workgroup of the (h, qg) group to arrive merges the chunks in chunk order,
// applies the gate and writes the result.  Workgroups sharing (h, c) sit on one XCD
// (workgroup ids 8 apart) so that their K and V reads meet in its L2.
constexpr uint32_t AQG = 16;  // queries per workgroup of k_attn_split

struct SplitAttn {
    const float *q, *k0, *v0, *k1, *v1;
    uint32_t n0, S, rows, n_q, n_kv, qpos0, ngq, nch;
    int causal, gmode;
    float scale;
    float *part_o, *part_ml, *gbuf;  // [group][chunk][16][128], [group][chunk][16][2], [group][16]
    uint32_t *cnt;                   // one arrival counter per group, zero between calls
    float *out;
    const float *gate;
    GateJob gj;
};

__device__ __forceinline__ float f4c(const float4 &v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }

__global__ __launch_bounds__(256) void k_attn_split(SplitAttn a) {
    constexpr uint32_t OST = AHD + 4;  // LDS row stride of a wavefront's O
    __shared__ __attribute__((aligned(16))) float so[4][AQG][OST];
    __shared__ float sm[4][AQG], sl[4][AQG];
    __shared__ uint32_t last;
    const uint32_t id = blockIdx.x, slot = id / 8;
    const uint32_t qg = slot % a.ngq, r = (slot / a.ngq) * 8 + id % 8;
    if (r >= a.n_kv * a.nch) return;  // uniform over the workgroup
    const uint32_t h = r / a.nch, c = r % a.nch, grp = h * a.ngq + qg;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l16 = lane & 15u, kg = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = a.n_q / a.n_kv, nq = a.rows * G, kvld = a.n_kv * AHD;
    // the group's gate units, spread over wavefronts 2-3 of its workgroups (wavefront 0
    // takes a chunk's extra tile, when it has one)
    auto gate_units = [&]() {
        if (a.gj.units && wave >= 2)
            for (uint32_t j = c + a.nch * (wave - 2); j < AQG; j += 2 * a.nch) {
                const uint32_t qj = AQG * qg + j;
                if (qj >= nq) break;  // uniform over the wavefront
                const float gv = gate_value(a.gj, (qj / G) * a.n_q + h * G + qj % G, lane);
                if (lane == 0)
                    __hip_atomic_store(a.gbuf + grp * AQG + j, gv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
    };
    // the lane's query: dims 16b + 4kg .. +3 in qf[b] (a dead query column reads the
    // group's first query; its scores are masked).  Once the first tiles' loads are
    // issued it is held as f16 parts (k step j: blocks 2j, 2j + 1), used while every
    // query of the wavefront lies in f16's range; the f32 products read it again.
    const uint32_t qi = AQG * qg + l16;
    const bool qlive = qi < nq;
    const uint32_t qc = qlive ? qi : AQG * qg, qt = qc / G, qpos = a.qpos0 + qt;
    const float *qp = a.q + (uint64_t)qt * a.n_q * AHD + (h * G + qc % G) * AHD + 4 * kg;
    float4 qf[8];
#pragma unroll
    for (int b = 0; b < 8; b++) qf[b] = *reinterpret_cast<const float4 *>(qp + 16 * b);
    const float neg1 = neg_one();
    f16x8 qh[4], ql[4];
    bool q16 = true;
    auto split_q = [&]() {
        float qmx = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            f16_parts8(qf[2 * j], qf[2 * j + 1], neg1, qh[j], ql[j]);
            qmx = absmax8(qmx, qf[2 * j], qf[2 * j + 1]);
        }
        q16 = !__builtin_amdgcn_ballot_w64(!(qmx < 65504.0f));
    };
    const uint32_t nt = (a.S + 15) / 16, tb = attn_tile0(c, nt, a.nch), te = attn_tile0(c + 1, nt, a.nch);
    const uint32_t nmine = te > tb + wave ? (te - tb - wave + 3) / 4 : 0;
    const uint32_t tlast = tb + wave + 4 * (nmine ? nmine - 1 : 0);  // the wavefront's last tile
    // position p's row of K or V (positions past S read row S - 1, masked)
    auto kvrow = [&](const float *b0, const float *b1, uint32_t p) {
        const uint32_t pc = p < a.S ? p : a.S - 1;
        return (pc < a.n0 ? b0 + (uint64_t)pc * kvld : b1 + (uint64_t)(pc - a.n0) * kvld) + h * AHD;
    };
    auto load_k = [&](float4 (&kr)[8], uint32_t tile) {
        const float *kp = kvrow(a.k0, a.k1, 16 * tile + l16) + 4 * kg;
#pragma unroll
        for (int b = 0; b < 8; b++) kr[b] = *reinterpret_cast<const float4 *>(kp + 16 * b);
    };
    auto load_v = [&](float4 (&vr)[8], uint32_t tile) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const float *vp = kvrow(a.v0, a.v1, 16 * tile + 4 * kg + s) + 4 * l16;
            vr[2 * s] = *reinterpret_cast<const float4 *>(vp);
            vr[2 * s + 1] = *reinterpret_cast<const float4 *>(vp + 64);
        }
    };
    f32x4 Od[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) Od[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.0f;  // running max (base-2 units) and sum of the lane's query
    const float sl2 = a.scale * 1.44269504088896341f;
    // One tile: S^T from kr, then kr refilled with tile `next` (two tiles ahead), the
    // softmax, P V from vr, then vr refilled with tile `next`.  Every load is
    // unconditional (past the wavefront's last tile: the last tile again), so that
    // each product waits for its own operands only.
    auto tile_step = [&](float4 (&kr)[8], float4 (&vr)[8], uint32_t tile, uint32_t next) {
        f32x4 sc[4];  // four independent chains
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        float kmx = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; b += 2) kmx = absmax8(kmx, kr[b], kr[b + 1]);
        if (q16 && !__builtin_amdgcn_ballot_w64(!(kmx < 65504.0f))) {
#pragma unroll
            for (int j = 0; j < 4; j++) {  // chain j: k step j, the small products first
                f16x8 kh, kl;
                f16_parts8(kr[2 * j], kr[2 * j + 1], neg1, kh, kl);
                sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[j], sc[j], 0, 0, 0);
                sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[j], sc[j], 0, 0, 0);
                sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[j], sc[j], 0, 0, 0);
            }
        } else {  // chain b mod 4: blocks b, b + 4
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const float4 qb = *reinterpret_cast<const float4 *>(qp + 16 * b);
#pragma unroll
                for (int s = 0; s < 4; s++)
                    sc[b & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4c(kr[b], s), f4c(qb, s), sc[b & 3], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_k(kr, next);
        __builtin_amdgcn_sched_barrier(0);
        // scores in base-2 units: s log2(e) / sqrt(d), so that P = 2^(s - max)
        float sv[4], tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = 16 * tile + 4 * kg + i;
            const bool ok = qlive && p < a.S && (!a.causal || p <= qpos);
            sv[i] = ok ? ((sc[0][i] + sc[1][i]) + (sc[2][i] + sc[3][i])) * sl2 : -INFINITY;
            tmax = fmaxf(tmax, sv[i]);
        }
        tmax = rows4_max(tmax);
        const float mn = fmaxf(m, tmax), mu = mn == -INFINITY ? 0.0f : mn;
        if (__builtin_amdgcn_ballot_w64(mn != m)) {  // some query's max moved: rescale (2^-inf = 0)
            const float f = __builtin_amdgcn_exp2f(m - mu);
            lsum *= f;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) Od[dt] *= f;
        }
        m = mn;
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pv[i] = __builtin_amdgcn_exp2f(sv[i] - mu);
            lsum += pv[i];
        }
        float vmx = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; b += 2) vmx = absmax8(vmx, vr[b], vr[b + 1]);
        if (!__builtin_amdgcn_ballot_w64(!(vmx < 65504.0f)) && __builtin_amdgcn_ballot_w64(vmx >= 0.0625f)) {
            f16x4 ph, pl;
            f16_parts4(pv[0], pv[1], pv[2], pv[3], neg1, ph, pl);
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    f16x4 vh, vl;
                    f16_parts4(f4c(vr[hh], cc), f4c(vr[2 + hh], cc), f4c(vr[4 + hh], cc), f4c(vr[6 + hh], cc),
                               neg1, vh, vl);
                    f32x4 &o = Od[4 * hh + cc];
                    o = __builtin_amdgcn_mfma_f32_16x16x16f16(vl, ph, o, 0, 0, 0);
                    o = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, pl, o, 0, 0, 0);
                    o = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, ph, o, 0, 0, 0);
                }
        } else {
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
#pragma unroll
                    for (int cc = 0; cc < 4; cc++)
                        Od[4 * hh + cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(f4c(vr[2 * s + hh], cc), pv[s],
                                                                              Od[4 * hh + cc], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_v(vr, next);
        __builtin_amdgcn_sched_barrier(0);
    };
    // the wavefront's tiles, two sets of K and V registers in turn: each tile's loads
    // are issued two tiles ahead
    if (nmine) {
        float4 ka[8], va[8], kb[8], vb[8];
        const uint32_t t0 = tb + wave;
        auto tile_at = [&](uint32_t i) { return i < nmine ? t0 + 4 * i : tlast; };
        load_k(ka, t0);
        load_v(va, t0);
        load_k(kb, tile_at(1));
        load_v(vb, tile_at(1));
        __builtin_amdgcn_sched_barrier(0);
        split_q();
        gate_units();  // its loads after the first tiles'
        for (uint32_t i = 0; i < nmine; i += 2) {
            tile_step(ka, va, t0 + 4 * i, tile_at(i + 2));
            if (i + 1 >= nmine) break;
            tile_step(kb, vb, t0 + 4 * i + 4, tile_at(i + 3));
        }
    } else {
        gate_units();
    }
    lsum = lane_add_x32(lane_add_x16(lsum));
    // the wavefronts' partials meet in LDS: lane (query l16, kg) holds dims
    // 64hh + 16kg + 4i + cc in Od[4hh + cc][i]
    if (kg == 0) sm[wave][l16] = m, sl[wave][l16] = lsum;
#pragma unroll
    for (int hh = 0; hh < 2; hh++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<float4 *>(&so[wave][l16][64 * hh + 16 * kg + 4 * i]) =
                make_float4(Od[4 * hh][i], Od[4 * hh + 1][i], Od[4 * hh + 2][i], Od[4 * hh + 3][i]);
    __syncthreads();
    // thread (query mq, dims md .. md + 7): the workgroup's partial, waves in order
    const uint32_t mq = tid >> 4, md = 8 * (tid & 15u);
    float M = fmaxf(fmaxf(sm[0][mq], sm[1][mq]), fmaxf(sm[2][mq], sm[3][mq])), L = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float f = sm[w][mq] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm[w][mq] - M);
        L = __builtin_fmaf(f, sl[w][mq], L);
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = __builtin_fmaf(f, so[w][mq][md + e], o[e]);
    }
    // the group's partials: byte offsets within part_o (< 2^31: the workspace bound)
    const __amdgpu_buffer_rsrc_t ro = dev_rsrc(a.part_o + (uint64_t)grp * a.nch * AQG * AHD),
                                 rm = dev_rsrc(a.part_ml + (uint64_t)grp * a.nch * AQG * 2);
    {
        const uint32_t pi = c * AQG + mq;
        dev_st4(ro, 4 * (pi * AHD + md), make_float4(o[0], o[1], o[2], o[3]));
        dev_st4(ro, 4 * (pi * AHD + md + 4), make_float4(o[4], o[5], o[6], o[7]));
        if ((tid & 15u) == 0) dev_st2(rm, 8 * pi, make_float2(M, L));
    }
    // the last workgroup of the group to arrive merges its chunks, in chunk order
    if (!arrive_last(a.cnt + grp, a.nch, &last)) return;
    constexpr uint32_t CB = 8;
    M = -INFINITY, L = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = 0.0f;
    for (uint32_t c0 = 0; c0 < a.nch; c0 += CB) {
        float mc[CB], lc[CB];
        float4 oc[CB][2];
#pragma unroll
        for (uint32_t b = 0; b < CB; b++) {
            const uint32_t pi = (c0 + b < a.nch ? c0 + b : a.nch - 1) * AQG + mq;
            const float2 ml = dev_ld2(rm, 8 * pi);
            oc[b][0] = dev_ld4(ro, 4 * (pi * AHD + md));
            oc[b][1] = dev_ld4(ro, 4 * (pi * AHD + md + 4));
            mc[b] = c0 + b < a.nch ? ml.x : -INFINITY;
            lc[b] = ml.y;
        }
        float mn = M;
#pragma unroll
        for (uint32_t b = 0; b < CB; b++) mn = fmaxf(mn, mc[b]);
        const float f = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mn);
        L *= f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] *= f;
#pragma unroll
        for (uint32_t b = 0; b < CB; b++) {  // chunk order
            const float w = mc[b] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc[b] - mn);
            L = __builtin_fmaf(w, lc[b], L);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                o[e] = __builtin_fmaf(w, f4c(oc[b][0], e), o[e]);
                o[4 + e] = __builtin_fmaf(w, f4c(oc[b][1], e), o[4 + e]);
            }
        }
        M = mn;
    }
    const uint32_t qo = AQG * qg + mq;
    if (qo >= nq) return;
    const uint32_t t = qo / G, hq = h * G + qo % G;
    float sc = L > 0.0f ? 1.0f / L : 0.0f;
    if (a.gate || a.gj.units) {
        const float gv = a.gj.units
                             ? __hip_atomic_load(a.gbuf + grp * AQG + mq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : a.gate[(uint64_t)t * a.n_q + hq];
        const float g = a.gmode == 2 ? logf(1.0f + expf(gv)) : softplus_gate(gv);
        float *op = a.out + (uint64_t)t * a.n_q * AHD + hq * AHD + md;
        *reinterpret_cast<float4 *>(op) =
            make_float4((o[0] * sc) * g, (o[1] * sc) * g, (o[2] * sc) * g, (o[3] * sc) * g);
        *reinterpret_cast<float4 *>(op + 4) =
            make_float4((o[4] * sc) * g, (o[5] * sc) * g, (o[6] * sc) * g, (o[7] * sc) * g);
    } else {
        float *op = a.out + (uint64_t)t * a.n_q * AHD + hq * AHD + md;
        *reinterpret_cast<float4 *>(op) = make_float4(o[0] * sc, o[1] * sc, o[2] * sc, o[3] * sc);
        *reinterpret_cast<float4 *>(op + 4) = make_float4(o[4] * sc, o[5] * sc, o[6] * sc, o[7] * sc);
    }
}

// Any head_dim <= 256: one wavefront per (row, q head), online softmax as mha_attn.comp.
__global__ __launch_bounds__(256) void k_attn_simple(const float *__restrict__ q, const float *__restrict__ k0,
                                                     const float *__restrict__ v0, uint32_t n0,
                                                     const float *__restrict__ k1, const float *__restrict__ v1,
                                                     uint32_t S, uint32_t rows, uint32_t n_q, uint32_t n_kv,
                                                     uint32_t hd, uint32_t qpos0, int causal, float scale,
                                                     float *__restrict__ out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t unit = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= rows * n_q) return;
    const uint32_t r = unit / n_q, hq = unit % n_q, kh = hq * n_kv / n_q;
    const float *qh = q + (uint64_t)r * n_q * hd + hq * hd;
    float qv[4], acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; j++) qv[j] = lane + 64 * j < hd ? qh[lane + 64 * j] : 0.0f;
    const uint32_t end = causal ? (qpos0 + r + 1 < S ? qpos0 + r + 1 : S) : S;
    float m = -INFINITY, l = 0.0f;
    for (uint32_t p = 0; p < end; p++) {
        const bool s0 = p < n0;
        const uint64_t off = (uint64_t)(s0 ? p : p - n0) * n_kv * hd + kh * hd;
        const float *kp = (s0 ? k0 : k1) + off, *vp = (s0 ? v0 : v1) + off;
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j < hd) d = __builtin_fmaf(qv[j], kp[lane + 64 * j], d);
        const float s = wave_sum(d) * scale;
        const float mn = fmaxf(m, s);
        const float corr = expf(m - mn), wgt = expf(s - mn);
        l = l * corr + wgt;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j < hd) acc[j] = acc[j] * corr + wgt * vp[lane + 64 * j];
        m = mn;
    }
    float *oh = out + (uint64_t)r * n_q * hd + hq * hd;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (lane + 64 * j < hd) oh[lane + 64 * j] = l > 0.0f ? acc[j] / l : 0.0f;
}

// ------------------------------------------------------------------------------------------
// elementwise

__global__ __launch_bounds__(256) void k_gate_mul(const float *v, const float *__restrict__ gate, float *out, uint32_t n_heads, uint32_t hd,
                                                  uint64_t total, int softplus) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const uint64_t row = i / ((uint64_t)n_heads * hd);
    const uint32_t head = (uint32_t)(i % ((uint64_t)n_heads * hd)) / hd;
    const float g = gate[row * n_heads + head];
    // softplus 1: the draft's host softplus (src/dflash.rs:957); 2: kernels/gate_attn.comp:27,
    // log(1 + exp(g)) with no threshold (infinite for g above about 88.7)
    out[i] = v[i] * (softplus == 1 ? softplus_gate(g) : softplus == 2 ? logf(1.0f + expf(g)) : g);
}

__global__ __launch_bounds__(256) void k_add(const float *a, const float *b, float *out, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void k_copy(const float *__restrict__ src, float *__restrict__ dst, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

inline unsigned blocks_for(uint64_t n) { return (unsigned)((n + 255) / 256); }

// ------------------------------------------------------------------------------------------
// launchers shared by the C entry points and the forward

int run_rmsnorm(const float *x, const float *w, float *out, uint32_t n, uint32_t rows, uint32_t chunks, uint32_t ldx,
                float eps, hipStream_t s) {
    const bool vec = n % 1024 == 0 && ldx % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                                         reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
    const dim3 grid(rows, chunks);
    if (vec && n == 4096)
        hipLaunchKernelGGL(k_rmsnorm4<4>, grid, dim3(256), 0, s, x, w, out, n, ldx, eps);
    else if (vec && n == 2048)
        hipLaunchKernelGGL(k_rmsnorm4<2>, grid, dim3(256), 0, s, x, w, out, n, ldx, eps);
    else if (vec && n == 1024)
        hipLaunchKernelGGL(k_rmsnorm4<1>, grid, dim3(256), 0, s, x, w, out, n, ldx, eps);
    else if (vec && n == 8192)
        hipLaunchKernelGGL(k_rmsnorm4<8>, grid, dim3(256), 0, s, x, w, out, n, ldx, eps);
    else
        hipLaunchKernelGGL(k_rmsnorm, grid, dim3(256), 0, s, x, w, out, n, ldx, eps);
    return after_launch("rmsnorm", s);
}

// Rows of n floats, n a multiple of 4 up to 8192 (the folded norms' kernels).
bool fan_width_ok(uint32_t n) { return n && n % 4 == 0 && n <= 8192; }

int run_norms_in(const float *x, const float *w, float *xe, const NormRun &run, uint32_t n, uint32_t rows, float eps,
                 hipStream_t s) {
    const dim3 grid(rows, run.count + (run.tok ? 1 : 0) + (run.rope ? 1 : 0));
    if (n <= 1024) hipLaunchKernelGGL(k_norms_in<1>, grid, dim3(256), 0, s, x, w, xe, run, n, eps);
    else if (n <= 2048) hipLaunchKernelGGL(k_norms_in<2>, grid, dim3(256), 0, s, x, w, xe, run, n, eps);
    else if (n <= 4096) hipLaunchKernelGGL(k_norms_in<4>, grid, dim3(256), 0, s, x, w, xe, run, n, eps);
    else hipLaunchKernelGGL(k_norms_in<8>, grid, dim3(256), 0, s, x, w, xe, run, n, eps);
    return after_launch("encoder, attention and token-row norms", s);
}

QkJob qk_job(const float *x, const float *w, float *out, uint32_t n_heads, uint32_t pos, uint32_t rows) {
    const uint32_t units = rows * n_heads;
    return {x, w, out, n_heads, pos, units, (units + 3) / 4};
}

// One or two tensors (b.blocks == 0: none) in one launch, and the attention gate
// when gj.blocks > 0.
int run_qk_norm_rope(const QkJob &a, const QkJob &b, const float *freq, uint32_t hd, uint32_t rope_dim, float eps,
                     hipStream_t s, const GateJob &gj = GateJob{}) {
    if (a.blocks + b.blocks + gj.blocks == 0) return LG_OK;
    hipLaunchKernelGGL(k_qk_norm_rope, dim3(a.blocks + b.blocks + gj.blocks), dim3(256), 0, s, a, b, freq, hd,
                       rope_dim, eps, gj);
    return after_launch("qk_norm_rope", s);
}

bool aligned16_ptr(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Chunks per (kv head, query group) of k_attn_split: about one workgroup per CU over
// the `groups` groups, each chunk at least four tiles (one per wavefront) when S allows.
uint32_t attn_split_chunks(uint32_t S, uint32_t groups) {
    const uint32_t nt = (S + 15) / 16, per = (uint32_t)device_cus() / groups, cap = (nt + 3) / 4;
    const uint32_t nch = per < cap ? per : cap;
    return nch ? nch : 1;
}

// The attention workspace: arrival counters first (k_attn_split's, one per query group,
// zero between calls), then the partials of whichever kernel runs.
uint32_t attn_cnt_floats(uint32_t n_kv) { return (4 * n_kv + 63) / 64 * 64; }

size_t attn_partial_floats(uint32_t S, uint32_t n_kv) {
    const uint32_t nch = (S + ACH - 1) / ACH, cus = (uint32_t)device_cus();
    const size_t decode = (size_t)n_kv * nch * AQ * (AHD + 2);
    // k_attn_split: groups <= 4 n_kv (at most AQ queries per kv head), groups * chunks <= max(CUs, groups)
    const size_t gc = cus > 4 * n_kv ? cus : 4 * n_kv;
    const size_t split = gc * AQG * (AHD + 2) + (size_t)4 * n_kv * AQG;
    return attn_cnt_floats(n_kv) + (decode > split ? decode : split);
}

// `part` holds attn_partial_floats(S, n_kv) floats when the matrix-core path applies,
// zeroed before its first use; `cnt` (when given) replaces its counters.  With `gate`
// ([rows][n_q]) each head's result is multiplied by softplus of its gate.
int run_attention(const float *q, const float *k0, const float *v0, uint32_t n0, const float *k1, const float *v1,
                  uint32_t S, uint32_t rows, uint32_t n_q, uint32_t n_kv, uint32_t hd, uint32_t qpos0, int causal,
                  float *out, float *part, hipStream_t s, const float *gate = nullptr, int gmode = 1,
                  const GateJob *gj = nullptr, uint32_t *cnt = nullptr) {
    const float scale = 1.0f / sqrtf((float)hd);  // src/dflash.rs:1173
    const uint32_t G = n_q / n_kv;
    const bool al = aligned16_ptr(q) && aligned16_ptr(k0) && aligned16_ptr(v0) &&
                    (!k1 || (aligned16_ptr(k1) && aligned16_ptr(v1)));
    if (part && hd == AHD && rows * G <= AQ && al && rows * G > ADQ) {
        const uint32_t ngq = (rows * G + AQG - 1) / AQG, groups = n_kv * ngq, nch = attn_split_chunks(S, groups);
        SplitAttn a{};
        a.q = q, a.k0 = k0, a.v0 = v0, a.k1 = k1, a.v1 = v1;
        a.n0 = n0, a.S = S, a.rows = rows, a.n_q = n_q, a.n_kv = n_kv, a.qpos0 = qpos0, a.ngq = ngq, a.nch = nch;
        a.causal = causal, a.gmode = gmode, a.scale = scale;
        a.part_o = part + attn_cnt_floats(n_kv);
        a.part_ml = a.part_o + (size_t)groups * nch * AQG * AHD;
        a.gbuf = a.part_ml + (size_t)groups * nch * AQG * 2;
        a.cnt = cnt ? cnt : reinterpret_cast<uint32_t *>(part);
        a.out = out, a.gate = gate, a.gj = gj ? *gj : GateJob{};
        const uint32_t R = n_kv * nch;
        hipLaunchKernelGGL(k_attn_split, dim3((R + 7) / 8 * 8 * ngq), dim3(256), 0, s, a);
        return after_launch("attn_split", s);
    }
    if (part && hd == AHD && rows * G <= ADQ && al) {
        // Few queries: the chunks cover the context; a short run of positions after it
        // (the block's own keys in k1) is attended by the combine, so that the chunk
        // grid does not spill a few workgroups into a second round.
        part += attn_cnt_floats(n_kv);
        const uint32_t T = k1 && S > n0 && S - n0 <= ATAIL ? S - n0 : 0, Sc = T ? n0 : S;
        const uint32_t nch = (Sc + ACH - 1) / ACH;
        float *part_ml = part + (size_t)n_kv * nch * AQ * AHD;
        if (nch) {
            hipLaunchKernelGGL(k_attn_decode, dim3(nch, n_kv), dim3(256), 0, s, q, k0, v0, n0, k1, v1, Sc,
                               rows, n_q, n_kv, qpos0, causal, scale, nch, part, part_ml);
            LG_TRY(after_launch("attn_decode", s));
        }
        hipLaunchKernelGGL(k_attn_combine, dim3(n_kv * AQ), dim3(256), 0, s, part, part_ml, out, rows, n_q,
                           n_kv, nch, gate, q, k1, v1, T, n0, qpos0, causal, scale, gmode, gj ? *gj : GateJob{});
        return after_launch("attn_combine", s);
    }
    if (gj) {  // the gate by itself, ahead of the attention that it scales
        LG_TRY(run_qk_norm_rope(QkJob{}, QkJob{}, nullptr, hd, 0, 0.0f, s, *gj));
        gate = gj->out;
    }
    hipLaunchKernelGGL(k_attn_simple, dim3((rows * n_q + 3) / 4), dim3(256), 0, s, q, k0, v0, n0, k1, v1, S, rows,
                       n_q, n_kv, hd, qpos0, causal, scale, out);
    LG_TRY(after_launch("attn_simple", s));
    if (!gate) return LG_OK;
    const uint64_t total = (uint64_t)rows * n_q * hd;
    hipLaunchKernelGGL(k_gate_mul, dim3(blocks_for(total)), dim3(256), 0, s, out, gate, out, n_q, hd, total, gmode);
    return after_launch("softplus_gate_mul", s);
}

// ------------------------------------------------------------------------------------------
// forward

constexpr uint64_t FREQ_BYTES = 1024;  // rope_dim <= head_dim <= 256: at most 128 frequencies

// Device workspace of one block forward: every intermediate, the RoPE table, the
// attention partials and the small-M product workspace.  The eager entry points
// share one per device (grown on demand); a graph owns its own, since a captured
// graph keeps the addresses it was recorded with.
// ny, ssa, ssb: the folded norms (forward_folded): per layer the [2m][E] attention
// input (injected rows normalised, token rows with the norm's weight applied), and
// the token rows' sums of squares ahead of the attention and FFN norms.
struct FwdLayout {
    float *xe, *nxe, *kk, *vv, *q, *att, *gate, *o, *h, *g, *u, *feat_n, *part, *ny, *ssa, *ssb, *rope, *freq;
    void *pws;
    uint64_t pws_bytes, total;
};

uint64_t layout(const lg_dflash_hparams &hp, uint32_t m, uint32_t ctx_len, uint8_t *base, FwdLayout &L) {
    const uint64_t E = hp.n_embd, QD = (uint64_t)hp.n_heads * hp.head_dim, KVD = (uint64_t)hp.n_kv_heads * hp.head_dim;
    const uint64_t FF = hp.n_ff, A = (uint64_t)hp.n_aux * hp.n_embd;
    const uint32_t S = ctx_len + 2 * m;
    const uint64_t ss_floats = (uint64_t)m * ((E + 63) / 64);  // at most one partial per 64 rows
    const uint64_t floats[] = {2 * m * E, 2 * m * E, 2 * m * KVD, 2 * m * KVD,  2 * m * QD, m * QD,
                               2 * (uint64_t)m * hp.n_heads,      m * E,        m * E,  m * FF, m * FF, m * A,
                               attn_partial_floats(S, hp.n_kv_heads), (uint64_t)hp.n_layers * 2 * m * E,
                               ss_floats, ss_floats, 2 * (uint64_t)m * 128};
    float **dst[] = {&L.xe, &L.nxe, &L.kk, &L.vv, &L.q, &L.att, &L.gate, &L.o, &L.h, &L.g, &L.u, &L.feat_n, &L.part,
                     &L.ny, &L.ssa, &L.ssb, &L.rope};
    // The RoPE table and the small-M product workspace (whose arrival counters come
    // first) sit at fixed offsets whatever (m, ctx_len) are: an uploaded table stays
    // valid, and the counters stay zero, across calls that lay the rest out differently.
    // Its size: the largest over the forward's product shapes (k, n, rows).
    uint64_t pw = 0;
    const uint32_t shapes[][3] = {{(uint32_t)E, (uint32_t)KVD, 2 * m}, {(uint32_t)E, (uint32_t)QD, m},
                                  {(uint32_t)E, hp.n_heads, m},         {(uint32_t)QD, (uint32_t)E, m},
                                  {(uint32_t)E, (uint32_t)FF, m},       {(uint32_t)FF, (uint32_t)E, m},
                                  {(uint32_t)A, (uint32_t)E, m}};
    const uint32_t qkvg[] = {(uint32_t)KVD, (uint32_t)KVD, (uint32_t)QD, hp.n_heads}, gu[] = {(uint32_t)FF, (uint32_t)FF};
    for (int wt : {LG_Q4_K, LG_Q8_0}) {
        for (const auto &sh : shapes) {
            const uint64_t c = proj_batch_ws_bytes(sh[0], sh[1], sh[2], LG_F32, wt);
            pw = c > pw ? c : pw;
        }
        const uint64_t c1 = proj_batch_multi_ws_bytes((uint32_t)E, qkvg, 4, 2 * m, wt);
        const uint64_t c3 = proj_batch_multi_ws_bytes((uint32_t)E, qkvg, 3, 2 * m, wt);  // gate apart
        pw = c3 > pw ? c3 : pw;
        const uint64_t c2 = proj_batch_multi_ws_bytes((uint32_t)E, gu, 2, m, wt);
        pw = c1 > pw ? c1 : pw;
        pw = c2 > pw ? c2 : pw;
    }
    pw = pw > PROJ_WS_COUNTERS ? pw : PROJ_WS_COUNTERS;
    L.freq = reinterpret_cast<float *>(base);
    L.pws = base + FREQ_BYTES;
    L.pws_bytes = pw;
    uint64_t off = FREQ_BYTES + ((pw + 255) & ~(uint64_t)255);
    for (size_t i = 0; i < sizeof(floats) / sizeof(floats[0]); i++) {
        *dst[i] = reinterpret_cast<float *>(base + off);
        off += (floats[i] * 4 + 255) & ~(uint64_t)255;
    }
    L.total = off;
    return L.total;
}

// f32 RoPE frequency table exactly as the reference computes it on the host
// (src/dflash.rs:898-904: 1.0 / base.powf((2.0 * i as f32) / rope_dim as f32)).
std::vector<float> rope_table(const lg_dflash_hparams &hp) {
    std::vector<float> f(hp.rope_dim / 2 + 1, 0.0f);
    glue_rope_table(hp.rope_dim, hp.rope_base > 0.0f ? hp.rope_base : 500000.0f, f.data());
    return f;
}

// A graph's own workspace, with its table uploaded for (rope_dim, rope_base).
struct Ws {
    uint8_t *base = nullptr;
    uint64_t bytes = 0;
    uint32_t rope_dim = 0xFFFFFFFFu;
    float rope_base = 0.0f;
};

int ws_alloc(Ws &w, uint64_t need) {
    if (w.bytes >= need) return LG_OK;
    if (w.base) {
        LG_HIP_TRY(hipDeviceSynchronize());  // earlier launches may still use it
        LG_HIP_TRY(hipFree(w.base));
    }
    w = Ws();
    const uint64_t sz = (need + (1u << 20) - 1) & ~(uint64_t)((1u << 20) - 1);
    void *p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) {
        (void)hipGetLastError();
        return fail(LG_ENOMEM, "draft forward workspace (%llu bytes)", (unsigned long long)sz);
    }
    LG_HIP_TRY(hipMemset(p, 0, sz));  // the small-M products' arrival counters start at zero
    w.base = static_cast<uint8_t *>(p);
    w.bytes = sz;
    return LG_OK;
}

// The f32 RoPE table at L.freq, uploaded unless the (rope_dim, rope_base) in tag already is.
int upload_table(uint64_t (&tag)[2], const lg_dflash_hparams &hp, const FwdLayout &L, hipStream_t s) {
    uint32_t bb = 0;
    std::memcpy(&bb, &hp.rope_base, 4);
    if (tag[0] == hp.rope_dim && tag[1] == bb) return LG_OK;
    {  // a new table is a host copy and a synchronise, which a capturing stream cannot take
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        LG_HIP_TRY(hipStreamIsCapturing(s, &cs));
        LG_REQUIRE(cs == hipStreamCaptureStatusNone, "the RoPE table of this model cannot be uploaded while the stream "
                   "is being captured; make the same call once before capturing");
    }
    const std::vector<float> f = rope_table(hp);
    LG_HIP_TRY(hipMemcpyAsync(L.freq, f.data(), f.size() * 4, hipMemcpyHostToDevice, s));
    LG_HIP_TRY(hipStreamSynchronize(s));  // f is released on return
    tag[0] = hp.rope_dim;
    tag[1] = bb;
    return LG_OK;
}

int ws_table(Ws &w, const lg_dflash_hparams &hp, const FwdLayout &L, hipStream_t s) {
    uint64_t tag[2] = {w.rope_dim, 0};
    std::memcpy(&tag[1], &w.rope_base, 4);
    LG_TRY(upload_table(tag, hp, L, s));
    w.rope_dim = hp.rope_dim;
    w.rope_base = hp.rope_base;
    return LG_OK;
}

// The eager workspace of stream s laid out for (hp, m, ctx_len), table uploaded.
// Eager calls on one stream share it; calls on different streams never do.
int eager_ws(const lg_dflash_hparams &hp, uint32_t m, uint32_t ctx_len, FwdLayout &L, hipStream_t s) {
    BufLease lease;
    LG_TRY(stream_buffer(BUF_DRAFT, s, layout(hp, m, ctx_len, nullptr, L), lease, "draft forward"));
    layout(hp, m, ctx_len, static_cast<uint8_t *>(lease.buf->ptr), L);
    return upload_table(lease.buf->tag, hp, L, s);
}

// with_layers = false checks what the encoder needs only.
int check_model(const lg_dflash_model *md, uint32_t m, const char *name, bool with_layers = true) {
    LG_REQUIRE(md, "%s: null model", name);
    const lg_dflash_hparams &hp = md->hp;
    LG_REQUIRE(m >= 1 && m <= 32, "%s: m = %u (1..32)", name, m);
    LG_REQUIRE(hp.n_embd && hp.n_aux, "%s: zero n_embd or n_aux", name);
    LG_REQUIRE(md->enc_aux_norm && md->fc && md->enc_output_norm, "%s: missing encoder tensor", name);
    if (!with_layers) return LG_OK;
    LG_REQUIRE(md->layers && hp.n_layers, "%s: no layers", name);
    LG_REQUIRE(hp.n_heads && hp.n_kv_heads && hp.head_dim && hp.n_ff, "%s: zero hyperparameter", name);
    LG_REQUIRE(hp.n_heads % hp.n_kv_heads == 0, "%s: n_heads %u not a multiple of n_kv_heads %u", name, hp.n_heads,
               hp.n_kv_heads);
    LG_REQUIRE(hp.head_dim <= 256 && hp.head_dim % 2 == 0 && (hp.rope_dim == 0 || hp.rope_dim == hp.head_dim),
               "%s: head_dim %u / rope_dim %u unsupported (rope_dim must be 0 or head_dim)", name, hp.head_dim,
               hp.rope_dim);
    for (uint32_t l = 0; l < hp.n_layers; l++) {
        const lg_dflash_layer &L = md->layers[l];
        LG_REQUIRE(L.attn_norm && L.attn_q_norm && L.attn_k_norm && L.ffn_norm && L.attn_q && L.attn_k && L.attn_v &&
                       L.attn_gate && L.attn_output && L.ffn_gate && L.ffn_up && L.ffn_down,
                   "%s: layer %u is missing a tensor", name, l);
    }
    return LG_OK;
}

// c = W x, or c = res + W x
// A job over the forward's 2m rows [injected; tokens] whose result is read for the
// token rows only (the queries, the attention gate).
BatchJob tok_rows(BatchJob b, uint32_t m) {
    b.row0 = m;
    return b;
}

int proj(const FwdLayout &W, const float *x, const void *w, int type, float *c, uint32_t k, uint32_t n, uint32_t m,
         hipStream_t s, const float *res = nullptr) {
    return proj_batch(x, LG_F32, w, c, k, n, m, type, W.pws, W.pws_bytes, s, res);
}

// DFlashModel::encode (src/dflash.rs:157-234) on m feature rows.
int encode(const lg_dflash_model *md, const FwdLayout &W, const float *features, uint32_t m, float *out,
           hipStream_t s) {
    const lg_dflash_hparams &hp = md->hp;
    const uint32_t E = hp.n_embd, A = hp.n_aux * hp.n_embd;
    LG_TRY(run_rmsnorm(features, md->enc_aux_norm, W.feat_n, E, m, hp.n_aux, A, hp.rms_eps, s));
    LG_TRY(proj(W, W.feat_n, md->fc, md->fc_type, W.o, A, E, m, s));
    return run_rmsnorm(W.o, md->enc_output_norm, out, E, m, 1, E, hp.rms_eps, s);
}

int forward_folded(const lg_dflash_model *md, const FwdLayout &W, const float *features, const float *tokens,
                   uint32_t m, uint32_t ctx_len, float *out, hipStream_t s);

// Whether every norm but the output norm can fold into the products around it: all
// eight projections of every layer on the matrix-core path, rows of a width the fan
// kernels take, and per-token partial-sum counts within what the consumers load.
std::atomic<uint32_t> g_fold_norms{1};  // lg_set_fold_norms

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool norms_foldable(const lg_dflash_model *md, const float *tokens, uint32_t m) {
    const lg_dflash_hparams &hp = md->hp;
    const uint32_t E = hp.n_embd, QD = hp.n_heads * hp.head_dim, FF = hp.n_ff;
    if (!g_fold_norms.load(std::memory_order_relaxed) || !fan_width_ok(E) || !aligned16(tokens) ||
        !aligned16(md->enc_output_norm))
        return false;
    for (uint32_t li = 0; li < hp.n_layers; li++) {
        const lg_dflash_layer &L = md->layers[li];
        const bool ok = proj_batch_mfma_ok(L.attn_q_type, E, L.attn_q) && proj_batch_mfma_ok(L.attn_k_type, E, L.attn_k) &&
                        proj_batch_mfma_ok(L.attn_v_type, E, L.attn_v) &&
                        proj_batch_mfma_ok(L.attn_gate_type, E, L.attn_gate) &&
                        proj_batch_mfma_ok(L.attn_output_type, QD, L.attn_output) &&
                        proj_batch_mfma_ok(L.ffn_gate_type, E, L.ffn_gate) &&
                        proj_batch_mfma_ok(L.ffn_up_type, E, L.ffn_up) &&
                        proj_batch_mfma_ok(L.ffn_down_type, FF, L.ffn_down) && aligned16(L.attn_norm);
        if (!ok) return false;
        // the attention norm's sums come from the previous layer's down projection (the
        // gate job's wave reads at most 64), the FFN norm's from o_proj
        const uint32_t ca = li ? proj_batch_norm_cols(md->layers[li - 1].ffn_down_type, FF, E, m) : 1u;
        const uint32_t cb = proj_batch_norm_cols(L.attn_output_type, QD, E, m);
        if (ca > proj_batch_rs_cols_max(2 * m) || ca > 64 || cb > proj_batch_rs_cols_max(m)) return false;
    }
    return true;
}

// Block generalisation of DFlashModel::forward_injected_decode_hidden
// (src/dflash.rs:877-976): m tokens over ctx_len cached positions.
int forward(const lg_dflash_model *md, const FwdLayout &W, const float *features, const float *tokens, uint32_t m,
            uint32_t ctx_len, float *out, hipStream_t s) {
    if (norms_foldable(md, tokens, m)) return forward_folded(md, W, features, tokens, m, ctx_len, out, s);
    const lg_dflash_hparams &hp = md->hp;
    const uint32_t E = hp.n_embd, H = hp.n_heads, KV = hp.n_kv_heads, HD = hp.head_dim, FF = hp.n_ff;
    const uint32_t QD = H * HD, KVD = KV * HD;
    const uint64_t mE = (uint64_t)m * E;
    // rows 0..m-1 of xe: encoder output (fixed over the layers), rows m..2m-1: the hidden x
    LG_TRY(encode(md, W, features, m, W.xe, s));
    float *x = W.xe + mE;
    hipLaunchKernelGGL(k_copy, dim3(blocks_for(mE)), dim3(256), 0, s, tokens, x, mE);
    LG_TRY(after_launch("copy tokens", s));
    for (uint32_t li = 0; li < hp.n_layers; li++) {
        const lg_dflash_layer &L = md->layers[li];
        const float *nx = W.nxe + mE;
        // attn_norm of the injected rows and the tokens in one launch (src/dflash.rs:917-923, :927)
        LG_TRY(run_rmsnorm(W.xe, L.attn_norm, W.nxe, E, 2 * m, 1, E, hp.rms_eps, s));
        // K, V of [injected; tokens] at positions ctx_len .. ctx_len + 2m - 1 (src/dflash.rs:924-941),
        // Q and the attention gate of the tokens (src/dflash.rs:942-944).  With one weight
        // type the four share a launch over all 2m rows (Q and the gate over the token
        // rows' tile only, where the rows split into 16-row tiles: BatchJob::row0).
        float *q = W.q, *gate = W.gate;
        GateJob gj{};
        const bool kvq = L.attn_k_type == L.attn_v_type && L.attn_k_type == L.attn_q_type;
        if (kvq && L.attn_k_type == L.attn_gate_type) {
            const BatchJob jb[4] = {{L.attn_k, W.kk, nullptr, KVD}, {L.attn_v, W.vv, nullptr, KVD},
                                    tok_rows({L.attn_q, W.q, nullptr, QD}, m),
                                    tok_rows({L.attn_gate, W.gate, nullptr, H}, m)};
            LG_TRY(proj_batch_multi(W.nxe, LG_F32, nullptr, jb, 4, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s));
            q = W.q + (uint64_t)m * QD;
            gate = W.gate + (uint64_t)m * H;
        } else if (kvq && L.attn_gate_type == LG_Q4_K && E % QK_K == 0 &&
                   (reinterpret_cast<uintptr_t>(L.attn_gate) & 15u) == 0) {
            // K, V, Q in one launch; the raw gate (H rows) is computed with the QK norms
            // below, which keeps the grouped launch's workgroups to whole rounds
            const BatchJob jb[3] = {{L.attn_k, W.kk, nullptr, KVD}, {L.attn_v, W.vv, nullptr, KVD},
                                    tok_rows({L.attn_q, W.q, nullptr, QD}, m)};
            LG_TRY(proj_batch_multi(W.nxe, LG_F32, nullptr, jb, 3, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s));
            q = W.q + (uint64_t)m * QD;
            gate = W.gate + (uint64_t)m * H;
            gj = {nx, static_cast<const uint8_t *>(L.attn_gate), gate, H, E, m * H, (m * H + 3) / 4};
        } else {
            LG_TRY(proj(W, W.nxe, L.attn_k, L.attn_k_type, W.kk, E, KVD, 2 * m, s));
            LG_TRY(proj(W, W.nxe, L.attn_v, L.attn_v_type, W.vv, E, KVD, 2 * m, s));
            LG_TRY(proj(W, nx, L.attn_q, L.attn_q_type, W.q, E, QD, m, s));
            LG_TRY(proj(W, nx, L.attn_gate, L.attn_gate_type, W.gate, E, H, m, s));
        }
        LG_TRY(run_qk_norm_rope(qk_job(W.kk, L.attn_k_norm, W.kk, KV, ctx_len, 2 * m),
                                qk_job(q, L.attn_q_norm, q, H, ctx_len + m, m), W.freq, HD, hp.rope_dim, hp.qk_eps, s,
                                gj));
        // causal attention over [context; injected; tokens] (src/dflash.rs:945-954), each head
        // scaled by softplus of its gate (src/dflash.rs:956-959)
        LG_TRY(run_attention(q, L.k_ctx, L.v_ctx, ctx_len, W.kk, W.vv, ctx_len + 2 * m, m, H, KV, HD, ctx_len + m, 1,
                             W.att, W.part, s, gate, 1, nullptr, static_cast<uint32_t *>(W.pws)));
        LG_TRY(proj(W, W.att, L.attn_output, L.attn_output_type, x, QD, E, m, s, x));  // x += o_proj
        // SwiGLU FFN (src/dflash.rs:962-968)
        LG_TRY(run_rmsnorm(x, L.ffn_norm, W.h, E, m, 1, E, hp.rms_eps, s));
        const BatchJob dj{L.ffn_down, x, x, E};
        if (L.ffn_gate_type == L.ffn_up_type) {
            // W.g = silu(gate) * up: each workgroup computes the same rows of both products
            const BatchJob jb[2] = {{L.ffn_gate, W.g, nullptr, FF}, {L.ffn_up, W.u, nullptr, FF}};
            LG_TRY(proj_batch_multi(W.h, LG_F32, nullptr, jb, 2, E, m, L.ffn_gate_type, W.pws, W.pws_bytes, s, true));
            // x += ffn_down(silu(gate) * up)
            LG_TRY(proj_batch_multi(W.g, LG_F32, nullptr, &dj, 1, FF, m, L.ffn_down_type, W.pws, W.pws_bytes, s));
        } else {
            LG_TRY(proj(W, W.h, L.ffn_gate, L.ffn_gate_type, W.g, E, FF, m, s));
            LG_TRY(proj(W, W.h, L.ffn_up, L.ffn_up_type, W.u, E, FF, m, s));
            // x += ffn_down(silu(gate) * up), the activation computed while staging the product's input
            LG_TRY(proj_batch_multi(W.g, LG_F32, W.u, &dj, 1, FF, m, L.ffn_down_type, W.pws, W.pws_bytes, s));
        }
    }
    if (md->output_norm) return run_rmsnorm(x, md->output_norm, out, E, m, 1, E, hp.rms_eps, s);
    hipLaunchKernelGGL(k_copy, dim3(blocks_for(mE)), dim3(256), 0, s, x, out, mE);
    return after_launch("copy hidden", s);
}

// The same forward with the attention and FFN norms folded into the products around
// them (rmsnorm(x) W^T = (x w) W^T / rms(x)): the product that writes the residual
// stream x also writes x w for the next norm and the sums of x^2 per workgroup column;
// the next product takes x w and scales its results by 1/rms.  The encoder's output
// norm and every layer's attention norm of the (fixed) injected rows run in one launch.
int forward_folded(const lg_dflash_model *md, const FwdLayout &W, const float *features, const float *tokens,
                   uint32_t m, uint32_t ctx_len, float *out, hipStream_t s) {
    const lg_dflash_hparams &hp = md->hp;
    const uint32_t E = hp.n_embd, H = hp.n_heads, KV = hp.n_kv_heads, HD = hp.head_dim, FF = hp.n_ff;
    const uint32_t QD = H * HD, KVD = KV * HD, A = hp.n_aux * hp.n_embd;
    const uint64_t mE = (uint64_t)m * E, ly = 2 * mE;  // W.ny: one [2m][E] attention input per layer
    const float eps = hp.rms_eps;
    // encoder (src/dflash.rs:157-234), then layer l's attention norm of its rows into
    // rows 0..m-1 of W.ny + l ly (src/dflash.rs:917-923)
    LG_TRY(run_rmsnorm(features, md->enc_aux_norm, W.feat_n, E, m, hp.n_aux, A, eps, s));
    LG_TRY(proj(W, W.feat_n, md->fc, md->fc_type, W.o, A, E, m, s));
    // and the token rows entering layer 0: x = tokens, with layer 0's x attn_norm and
    // sums of squares
    float *x = W.xe + mE;  // the tokens' residual stream
    // QK-norm and RoPE inside the K/V/Q launch (whole heads per workgroup column), the
    // gate inside the attention's combine: for heads of 128 rotated in full, at most 32
    // rows per launch and a Q4_K gate; the rotation table of the 2m positions is built
    // with the first norms
    const bool qkf = HD == AHD && hp.rope_dim == AHD && 2 * m <= 32;
    for (uint32_t l0 = 0; l0 < hp.n_layers; l0 += NORM_RUN) {
        NormRun run{};
        run.count = hp.n_layers - l0 < NORM_RUN ? hp.n_layers - l0 : NORM_RUN;
        for (uint32_t j = 0; j < run.count; j++) {
            run.w[j] = md->layers[l0 + j].attn_norm;
            run.out[j] = W.ny + (l0 + j) * ly;
        }
        if (l0 == 0) {
            run.tok = tokens;
            run.wt = md->layers[0].attn_norm;
            run.xt = x;
            run.yt = W.ny + mE;
            run.ss = W.ssa;
            run.cols = 1;
            if (qkf) {
                run.rope = W.rope;
                run.freq = W.freq;
                run.pos0 = ctx_len;
            }
        }
        LG_TRY(run_norms_in(W.o, md->enc_output_norm, W.xe, run, E, m, eps, s));
    }
    uint32_t cols_a = 1;  // partial sums per token row in W.ssa
    for (uint32_t li = 0; li < hp.n_layers; li++) {
        const lg_dflash_layer &L = md->layers[li];
        const float *Y = W.ny + li * ly, *ny = Y + mE;
        const RowScale ra{W.ssa, cols_a, m, eps};  // over Y's 2m rows: the token rows scaled
        const RowScale rt{W.ssa, cols_a, 0, eps};  // over the token rows alone
        // K, V of [injected; tokens], Q and the gate of the tokens (src/dflash.rs:924-944),
        // grouped as in forward()
        float *q = W.q, *gate = W.gate;
        GateJob gj{};
        const bool kvq = L.attn_k_type == L.attn_v_type && L.attn_k_type == L.attn_q_type;
        if (qkf && kvq && L.attn_gate_type == L.attn_k_type) {
            // the gate as a fourth job of the K/V/Q launch (token rows, no QK-norm)
            BatchJob jb[4] = {{L.attn_k, W.kk, nullptr, KVD}, {L.attn_v, W.vv, nullptr, KVD},
                              tok_rows({L.attn_q, W.q, nullptr, QD}, m),
                              tok_rows({L.attn_gate, W.gate, nullptr, H}, m)};
            jb[0].qkw = L.attn_k_norm;
            jb[2].qkw = L.attn_q_norm;
            const QkRope qk{W.rope, hp.qk_eps};
            LG_TRY(proj_batch_multi(Y, LG_F32, nullptr, jb, 4, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s, false,
                                    &ra, &qk));
            q = W.q + (uint64_t)m * QD;
            gate = W.gate + (uint64_t)m * H;
            LG_TRY(run_attention(q, L.k_ctx, L.v_ctx, ctx_len, W.kk, W.vv, ctx_len + 2 * m, m, H, KV, HD, ctx_len + m,
                                 1, W.att, W.part, s, gate, 1, nullptr, static_cast<uint32_t *>(W.pws)));
        } else if (qkf && kvq && L.attn_gate_type == LG_Q4_K) {
            BatchJob jb[3] = {{L.attn_k, W.kk, nullptr, KVD}, {L.attn_v, W.vv, nullptr, KVD},
                              tok_rows({L.attn_q, W.q, nullptr, QD}, m)};
            jb[0].qkw = L.attn_k_norm;
            jb[2].qkw = L.attn_q_norm;
            const QkRope qk{W.rope, hp.qk_eps};
            LG_TRY(proj_batch_multi(Y, LG_F32, nullptr, jb, 3, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s, false,
                                    &ra, &qk));
            q = W.q + (uint64_t)m * QD;
            gj = {ny, static_cast<const uint8_t *>(L.attn_gate), W.gate + (uint64_t)m * H, H, E, m * H, (m * H + 3) / 4,
                  W.ssa, cols_a, eps};
            LG_TRY(run_attention(q, L.k_ctx, L.v_ctx, ctx_len, W.kk, W.vv, ctx_len + 2 * m, m, H, KV, HD, ctx_len + m,
                                 1, W.att, W.part, s, nullptr, 1, &gj, static_cast<uint32_t *>(W.pws)));
        } else {
            if (kvq && L.attn_k_type == L.attn_gate_type) {
                const BatchJob jb[4] = {{L.attn_k, W.kk, nullptr, KVD}, {L.attn_v, W.vv, nullptr, KVD},
                                        tok_rows({L.attn_q, W.q, nullptr, QD}, m),
                                        tok_rows({L.attn_gate, W.gate, nullptr, H}, m)};
                LG_TRY(proj_batch_multi(Y, LG_F32, nullptr, jb, 4, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s,
                                        false, &ra));
                q = W.q + (uint64_t)m * QD;
                gate = W.gate + (uint64_t)m * H;
            } else if (kvq && L.attn_gate_type == LG_Q4_K) {
                const BatchJob jb[3] = {{L.attn_k, W.kk, nullptr, KVD}, {L.attn_v, W.vv, nullptr, KVD},
                                        tok_rows({L.attn_q, W.q, nullptr, QD}, m)};
                LG_TRY(proj_batch_multi(Y, LG_F32, nullptr, jb, 3, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s,
                                        false, &ra));
                q = W.q + (uint64_t)m * QD;
                gate = W.gate + (uint64_t)m * H;
                gj = {ny, static_cast<const uint8_t *>(L.attn_gate), gate, H, E, m * H, (m * H + 3) / 4,
                      W.ssa, cols_a, eps};
            } else {
                const BatchJob k1{L.attn_k, W.kk, nullptr, KVD}, v1{L.attn_v, W.vv, nullptr, KVD};
                const BatchJob q1{L.attn_q, W.q, nullptr, QD}, g1{L.attn_gate, W.gate, nullptr, H};
                LG_TRY(proj_batch_multi(Y, LG_F32, nullptr, &k1, 1, E, 2 * m, L.attn_k_type, W.pws, W.pws_bytes, s,
                                        false, &ra));
                LG_TRY(proj_batch_multi(Y, LG_F32, nullptr, &v1, 1, E, 2 * m, L.attn_v_type, W.pws, W.pws_bytes, s,
                                        false, &ra));
                LG_TRY(proj_batch_multi(ny, LG_F32, nullptr, &q1, 1, E, m, L.attn_q_type, W.pws, W.pws_bytes, s,
                                        false, &rt));
                LG_TRY(proj_batch_multi(ny, LG_F32, nullptr, &g1, 1, E, m, L.attn_gate_type, W.pws, W.pws_bytes, s,
                                        false, &rt));
            }
            LG_TRY(run_qk_norm_rope(qk_job(W.kk, L.attn_k_norm, W.kk, KV, ctx_len, 2 * m),
                                    qk_job(q, L.attn_q_norm, q, H, ctx_len + m, m), W.freq, HD, hp.rope_dim,
                                    hp.qk_eps, s, gj));
            LG_TRY(run_attention(q, L.k_ctx, L.v_ctx, ctx_len, W.kk, W.vv, ctx_len + 2 * m, m, H, KV, HD, ctx_len + m,
                                 1, W.att, W.part, s, gate, 1, nullptr, static_cast<uint32_t *>(W.pws)));
        }
        // x += o_proj, writing x ffn_norm and the sums of x^2 for the FFN norm (src/dflash.rs:960-962)
        const uint32_t cols_b = proj_batch_norm_cols(L.attn_output_type, QD, E, m);
        const BatchJob oj{L.attn_output, x, x, E, W.h, L.ffn_norm, W.ssb};
        LG_TRY(proj_batch_multi(W.att, LG_F32, nullptr, &oj, 1, QD, m, L.attn_output_type, W.pws, W.pws_bytes, s));
        const RowScale rb{W.ssb, cols_b, 0, eps};
        // SwiGLU FFN (src/dflash.rs:962-968); x += ffn_down, writing the next layer's
        // attention input rows and sums of x^2
        const bool next = li + 1 < hp.n_layers;
        const BatchJob dj{L.ffn_down, x, x, E, next ? W.ny + (li + 1) * ly + mE : nullptr,
                          next ? md->layers[li + 1].attn_norm : nullptr, next ? W.ssa : nullptr};
        if (L.ffn_gate_type == L.ffn_up_type) {
            const BatchJob jb[2] = {{L.ffn_gate, W.g, nullptr, FF}, {L.ffn_up, W.u, nullptr, FF}};
            LG_TRY(proj_batch_multi(W.h, LG_F32, nullptr, jb, 2, E, m, L.ffn_gate_type, W.pws, W.pws_bytes, s, true,
                                    &rb));
            LG_TRY(proj_batch_multi(W.g, LG_F32, nullptr, &dj, 1, FF, m, L.ffn_down_type, W.pws, W.pws_bytes, s));
        } else {
            const BatchJob g1{L.ffn_gate, W.g, nullptr, FF}, u1{L.ffn_up, W.u, nullptr, FF};
            LG_TRY(proj_batch_multi(W.h, LG_F32, nullptr, &g1, 1, E, m, L.ffn_gate_type, W.pws, W.pws_bytes, s, false,
                                    &rb));
            LG_TRY(proj_batch_multi(W.h, LG_F32, nullptr, &u1, 1, E, m, L.ffn_up_type, W.pws, W.pws_bytes, s, false,
                                    &rb));
            LG_TRY(proj_batch_multi(W.g, LG_F32, W.u, &dj, 1, FF, m, L.ffn_down_type, W.pws, W.pws_bytes, s));
        }
        if (next) cols_a = proj_batch_norm_cols(L.ffn_down_type, FF, E, m);
    }
    if (md->output_norm) return run_rmsnorm(x, md->output_norm, out, E, m, 1, E, hp.rms_eps, s);
    hipLaunchKernelGGL(k_copy, dim3(blocks_for(mE)), dim3(256), 0, s, x, out, mE);
    return after_launch("copy hidden", s);
}

struct Graph {
    hipGraph_t g = nullptr;
    hipGraphExec_t exec = nullptr;
    Ws ws;
};

void graph_free(Graph *G) {
    if (G->exec) (void)hipGraphExecDestroy(G->exec);
    if (G->g) (void)hipGraphDestroy(G->g);
    if (G->ws.base) (void)hipFree(G->ws.base);
    delete G;
}

int check_forward(const lg_dflash_model *md, const float *features, const float *tokens, uint32_t m,
                  uint32_t ctx_len, float *out, const char *name) {
    LG_TRY(check_model(md, m, name));
    LG_REQUIRE(features && tokens && out, "%s: null input or output", name);
    if (ctx_len)
        for (uint32_t l = 0; l < md->hp.n_layers; l++)
            LG_REQUIRE(md->layers[l].k_ctx && md->layers[l].v_ctx, "%s: layer %u has no context cache", name, l);
    return LG_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// the launchers, for the target forward (one row each unless stated)

namespace lg {

int glue_rmsnorm(const float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps, hipStream_t s) {
    return run_rmsnorm(x, w, out, n, rows, 1, n, eps, s);
}

int glue_qk_norm_rope(const float *x, const float *w, float *out, uint32_t n_heads, uint32_t head_dim,
                      uint32_t rope_dim, uint32_t pos, const float *freq, float eps, hipStream_t s) {
    return run_qk_norm_rope(qk_job(x, w, out, n_heads, pos, 1), QkJob{}, freq, head_dim, rope_dim, eps, s);
}

int glue_qk_norm_rope2(const float *q, const float *wq, float *q_out, uint32_t n_q, const float *k, const float *wk,
                       float *k_out, uint32_t n_kv, uint32_t head_dim, uint32_t rope_dim, uint32_t pos,
                       const float *freq, float eps, hipStream_t s) {
    return run_qk_norm_rope(qk_job(q, wq, q_out, n_q, pos, 1), qk_job(k, wk, k_out, n_kv, pos, 1), freq, head_dim,
                            rope_dim, eps, s);
}

uint64_t glue_attn_partial_bytes(uint32_t seq_len, uint32_t n_kv) { return attn_partial_floats(seq_len, n_kv) * 4; }

int glue_attention(const float *q, const float *k, const float *v, uint32_t seq_len, uint32_t q_pos, uint32_t n_q,
                   uint32_t n_kv, uint32_t head_dim, float *out, float *part, hipStream_t s, const float *gate) {
    return run_attention(q, k, v, seq_len, nullptr, nullptr, seq_len, 1, n_q, n_kv, head_dim, q_pos, 1, out, part, s,
                         gate, 2);
}

bool glue_attention_token_ok(uint32_t head_dim, uint32_t n_q, uint32_t n_kv, uint32_t rope_dim) {
    return head_dim == AHD && n_kv && n_q % n_kv == 0 && n_q / n_kv <= ADQ && (rope_dim == 0 || rope_dim == AHD);
}

int glue_attention_token(const float *q, const float *qn_w, const float *kn_w, const float *freq, uint32_t rope_dim,
                         uint32_t pos, float eps, float *k, const float *v, uint32_t seq_len, uint32_t n_q,
                         uint32_t n_kv, uint32_t head_dim, const float *gate, float *out, float *part, hipStream_t s) {
    LG_REQUIRE(glue_attention_token_ok(head_dim, n_q, n_kv, rope_dim) && seq_len && part &&
                   aligned16_ptr(k) && aligned16_ptr(v),
               "attention_token: shape (head_dim %u, %u / %u heads, rope_dim %u) or operands outside the kernel",
               head_dim, n_q, n_kv, rope_dim);
    TokAttn t{};
    t.q = q, t.qn_w = qn_w, t.kn_w = kn_w, t.freq = freq, t.rope = rope_dim ? 1u : 0u, t.pos = pos, t.eps = eps;
    t.scale = 1.0f / sqrtf((float)head_dim);  // src/dflash.rs:1173
    t.k = k, t.v = v, t.S = seq_len, t.n_q = n_q, t.n_kv = n_kv, t.nch = (seq_len + ACH - 1) / ACH;
    t.part_o = part + attn_cnt_floats(n_kv);
    t.part_ml = part + (size_t)n_kv * t.nch * AQ * AHD;
    hipLaunchKernelGGL(k_attn_token, dim3(t.nch, n_kv), dim3(256), 0, s, t);
    LG_TRY(after_launch("attention_token", s));
    hipLaunchKernelGGL(k_attn_combine, dim3(n_kv * AQ), dim3(256), 0, s, t.part_o, t.part_ml, out, 1u, n_q, n_kv,
                       t.nch, gate, q, nullptr, nullptr, 0u, 0u, 0u, 1, t.scale, 2, GateJob{});
    return after_launch("attn_combine", s);
}

int glue_gate_attn(const float *attn, const float *gate, float *out, uint32_t n_heads, uint32_t head_dim,
                   hipStream_t s) {
    const uint64_t total = (uint64_t)n_heads * head_dim;
    hipLaunchKernelGGL(k_gate_mul, dim3(blocks_for(total)), dim3(256), 0, s, attn, gate, out, n_heads, head_dim, total,
                       2);
    return after_launch("gate_attn", s);
}

int glue_add(const float *a, const float *b, float *out, uint64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_add, dim3(blocks_for(n)), dim3(256), 0, s, a, b, out, n);
    return after_launch("add", s);
}

int glue_copy(const float *src, float *dst, uint64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_copy, dim3(blocks_for(n)), dim3(256), 0, s, src, dst, n);
    return after_launch("copy", s);
}

void glue_rope_table(uint32_t rope_dim, float base, float *out) {
    for (uint32_t i = 0; i < rope_dim / 2; i++) out[i] = 1.0f / std::pow(base, (2.0f * (float)i) / (float)rope_dim);
}

}  // namespace lg

extern "C" {

int lg_dispatch_rmsnorm(const float *w, const float *x, float *out, uint32_t n, uint32_t rows, float eps,
                        void *stream) {
    clear_error();
    if (n == 0 || rows == 0) return LG_OK;
    LG_REQUIRE(w && x && out, "lg_dispatch_rmsnorm: null pointer");
    LG_EXTENT(x, (uint64_t)n * rows * 4, "lg_dispatch_rmsnorm x");
    LG_EXTENT(out, (uint64_t)n * rows * 4, "lg_dispatch_rmsnorm out");
    LG_EXTENT(w, (uint64_t)n * 4, "lg_dispatch_rmsnorm w");
    return run_rmsnorm(x, w, out, n, rows, 1, n, eps, (hipStream_t)stream);
}

int lg_dispatch_enc_aux_norm(const float *x, const float *aux_norm_w, float *out, uint32_t n_feat, uint32_t n_aux,
                             uint32_t n_total, void *stream) {
    clear_error();
    if (n_feat == 0 || n_aux == 0 || n_total == 0) return LG_OK;
    LG_REQUIRE(x && aux_norm_w && out, "lg_dispatch_enc_aux_norm: null pointer");
    const uint64_t per = (uint64_t)n_feat * n_aux;
    LG_REQUIRE(n_total % per == 0, "lg_dispatch_enc_aux_norm: n_total=%u is not a whole number of tokens of %llu",
               n_total, (unsigned long long)per);
    const uint32_t n_tokens = (uint32_t)(n_total / per);
    LG_EXTENT(x, (uint64_t)n_total * 4, "lg_dispatch_enc_aux_norm x");
    LG_EXTENT(out, (uint64_t)n_total * 4, "lg_dispatch_enc_aux_norm out");
    LG_EXTENT(aux_norm_w, per * 4, "lg_dispatch_enc_aux_norm w");
    return run_rmsnorm(x, aux_norm_w, out, n_feat, n_tokens, n_aux, n_feat * n_aux, 1e-5f, (hipStream_t)stream);
}

int lg_dispatch_qk_norm_rope(const float *x, const float *norm_w, const float *freq, float *out, uint32_t n_heads,
                             uint32_t head_dim, uint32_t rope_dim, uint32_t pos, uint32_t rows, float eps,
                             void *stream) {
    clear_error();
    if (n_heads == 0 || rows == 0 || head_dim == 0) return LG_OK;
    LG_REQUIRE(x && norm_w && out && (freq || rope_dim == 0), "lg_dispatch_qk_norm_rope: null pointer");
    LG_REQUIRE(head_dim <= 256 && head_dim % 2 == 0 && (rope_dim == 0 || rope_dim == head_dim),
               "lg_dispatch_qk_norm_rope: head_dim %u / rope_dim %u unsupported (rope_dim must be 0 or head_dim)",
               head_dim, rope_dim);
    const uint64_t tot = (uint64_t)rows * n_heads * head_dim * 4;
    LG_EXTENT(x, tot, "lg_dispatch_qk_norm_rope x");
    LG_EXTENT(out, tot, "lg_dispatch_qk_norm_rope out");
    LG_EXTENT(norm_w, (uint64_t)head_dim * 4, "lg_dispatch_qk_norm_rope norm_w");
    return run_qk_norm_rope(qk_job(x, norm_w, out, n_heads, pos, rows), QkJob{}, freq, head_dim, rope_dim, eps,
                            (hipStream_t)stream);
}

int lg_dispatch_mha_attn(const float *q, const float *k_seq, const float *v_seq, float *out, uint32_t n_q_heads,
                         uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq_len, uint32_t q_pos, uint32_t rows,
                         int causal, void *stream) {
    clear_error();
    const char *name = "lg_dispatch_mha_attn";
    if (rows == 0 || n_q_heads == 0) return LG_OK;
    LG_REQUIRE(q && out && (seq_len == 0 || (k_seq && v_seq)), "%s: null pointer", name);
    LG_REQUIRE(n_kv_heads && n_q_heads % n_kv_heads == 0, "%s: n_q %u, n_kv %u", name, n_q_heads, n_kv_heads);
    LG_REQUIRE(head_dim && head_dim <= 256, "%s: head_dim %u unsupported", name, head_dim);
    LG_EXTENT(q, (uint64_t)rows * n_q_heads * head_dim * 4, name);
    LG_EXTENT(out, (uint64_t)rows * n_q_heads * head_dim * 4, name);
    if (seq_len) {
        LG_EXTENT(k_seq, (uint64_t)seq_len * n_kv_heads * head_dim * 4, name);
        LG_EXTENT(v_seq, (uint64_t)seq_len * n_kv_heads * head_dim * 4, name);
    }
    hipStream_t s = (hipStream_t)stream;
    float *part = nullptr;
    const uint32_t G = n_q_heads / n_kv_heads;
    if (head_dim == AHD && rows * G <= AQ && seq_len) {
        void *p = nullptr;
        BufLease lease;
        LG_TRY(stream_buffer(BUF_ATTN, s, attn_partial_floats(seq_len, n_kv_heads) * 4, lease, "lg_dispatch_mha_attn"));
        p = lease.buf->ptr;
        part = static_cast<float *>(p);
    }
    return run_attention(q, k_seq, v_seq, seq_len, nullptr, nullptr, seq_len, rows, n_q_heads, n_kv_heads, head_dim,
                         q_pos, causal, out, part, s);
}

// dispatch_gate_mul / the softplus gate (src/dflash.rs:1236-1266, 956-959):
// attn_out[i] = v_rep[i] * g(gate[i / head_dim]) for i < n_hd, g = identity or
// softplus.  As in kernels/gate_mul.comp, n_heads does not enter the result.
static int gate_mul(float *attn_out, const float *v_rep, const float *gate, uint32_t n_hd, uint32_t n_heads,
                    uint32_t head_dim, int softplus, void *stream, const char *name) {
    clear_error();
    (void)n_heads;
    if (n_hd == 0) return LG_OK;
    LG_REQUIRE(attn_out && v_rep && gate, "%s: null pointer", name);
    LG_REQUIRE(head_dim, "%s: head_dim = 0", name);
    LG_EXTENT(v_rep, (uint64_t)n_hd * 4, name);
    LG_EXTENT(attn_out, (uint64_t)n_hd * 4, name);
    LG_EXTENT(gate, (uint64_t)((n_hd + head_dim - 1) / head_dim) * 4, name);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_gate_mul, dim3(blocks_for(n_hd)), dim3(256), 0, s, v_rep, gate, attn_out, 1u, head_dim,
                       (uint64_t)n_hd, softplus);
    return after_launch(name, s);
}

int lg_dispatch_gate_mul(float *attn_out, const float *v_rep, const float *gate, uint32_t n_hd, uint32_t n_heads,
                         uint32_t head_dim, void *stream) {
    return gate_mul(attn_out, v_rep, gate, n_hd, n_heads, head_dim, 0, stream, "lg_dispatch_gate_mul");
}

int lg_dispatch_softplus_gate_mul(float *attn_out, const float *v_rep, const float *gate, uint32_t n_hd,
                                  uint32_t n_heads, uint32_t head_dim, void *stream) {
    return gate_mul(attn_out, v_rep, gate, n_hd, n_heads, head_dim, 1, stream, "lg_dispatch_softplus_gate_mul");
}

int lg_dispatch_gate_attn(const float *attn_out, const float *gate, float *result, uint32_t n_heads,
                          uint32_t head_dim, void *stream) {
    clear_error();
    const char *name = "lg_dispatch_gate_attn";
    const uint64_t n = (uint64_t)n_heads * head_dim;
    if (n == 0) return LG_OK;
    LG_REQUIRE(attn_out && gate && result, "%s: null pointer", name);
    LG_EXTENT(attn_out, n * 4, name);
    LG_EXTENT(result, n * 4, name);
    LG_EXTENT(gate, (uint64_t)n_heads * 4, name);
    return glue_gate_attn(attn_out, gate, result, n_heads, head_dim, (hipStream_t)stream);
}

int lg_dispatch_add(const float *a, const float *b, float *out, uint32_t n, void *stream) {
    clear_error();
    if (n == 0) return LG_OK;
    LG_REQUIRE(a && b && out, "lg_dispatch_add: null pointer");
    LG_EXTENT(a, (uint64_t)n * 4, "lg_dispatch_add a");
    LG_EXTENT(b, (uint64_t)n * 4, "lg_dispatch_add b");
    LG_EXTENT(out, (uint64_t)n * 4, "lg_dispatch_add out");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_add, dim3(blocks_for(n)), dim3(256), 0, s, a, b, out, (uint64_t)n);
    return after_launch("lg_dispatch_add", s);
}

int lg_dflash_encode(const lg_dflash_model *model, const float *features, uint32_t m, float *out, void *stream) {
    clear_error();
    LG_TRY(check_model(model, m, "lg_dflash_encode", false));
    LG_REQUIRE(features && out, "lg_dflash_encode: null pointer");
    hipStream_t s = (hipStream_t)stream;
    FwdLayout W;
    LG_TRY(eager_ws(model->hp, m, 0, W, s));
    int st;
    {
        DeferSync d;
        st = encode(model, W, features, m, out, s);
    }
    return st != LG_OK ? st : after_launch("lg_dflash_encode", s);
}

int lg_dflash_forward_block(const lg_dflash_model *model, const float *features, const float *tokens, uint32_t m,
                            uint32_t ctx_len, float *out, void *stream) {
    clear_error();
    LG_TRY(check_forward(model, features, tokens, m, ctx_len, out, "lg_dflash_forward_block"));
    hipStream_t s = (hipStream_t)stream;
    FwdLayout W;
    LG_TRY(eager_ws(model->hp, m, ctx_len, W, s));
    int st;
    {
        DeferSync d;
        st = forward(model, W, features, tokens, m, ctx_len, out, s);
    }
    return st != LG_OK ? st : after_launch("lg_dflash_forward_block", s);
}

int lg_dflash_graph_create(const lg_dflash_model *model, const float *features, const float *tokens, uint32_t m,
                           uint32_t ctx_len, float *out, void *stream, void **graph) {
    clear_error();
    const char *name = "lg_dflash_graph_create";
    LG_REQUIRE(graph, "%s: null graph", name);
    LG_REQUIRE(stream, "%s: capture needs a created stream (not the null stream)", name);
    LG_TRY(check_forward(model, features, tokens, m, ctx_len, out, name));
    hipStream_t s = (hipStream_t)stream;
    Graph *G = new Graph();
    FwdLayout W;
    int st = ws_alloc(G->ws, layout(model->hp, m, ctx_len, nullptr, W));
    if (st == LG_OK) {
        layout(model->hp, m, ctx_len, G->ws.base, W);
        st = ws_table(G->ws, model->hp, W, s);
    }
    if (st == LG_OK) {  // one eager pass: every lazy set-up happens before capture
        DeferSync d;
        st = forward(model, W, features, tokens, m, ctx_len, out, s);
    }
    if (st == LG_OK && hipStreamSynchronize(s) != hipSuccess) st = fail(LG_EHIP, "%s: warm-up run failed", name);
    if (st != LG_OK) {
        graph_free(G);
        return st;
    }
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        graph_free(G);
        return fail(LG_EHIP, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    }
    st = forward(model, W, features, tokens, m, ctx_len, out, s);
    e = hipStreamEndCapture(s, &G->g);
    if (st != LG_OK || e != hipSuccess) {
        graph_free(G);
        if (st != LG_OK) return st;
        return fail(LG_EHIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    }
    e = hipGraphInstantiate(&G->exec, G->g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        graph_free(G);
        return fail(LG_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    *graph = G;
    return LG_OK;
}

int lg_dflash_graph_launch(void *graph, void *stream) {
    clear_error();
    LG_REQUIRE(graph, "lg_dflash_graph_launch: null graph");
    hipStream_t s = (hipStream_t)stream;
    LG_HIP_TRY(hipGraphLaunch(static_cast<Graph *>(graph)->exec, s));
    return after_launch("lg_dflash_graph_launch", s);
}

int lg_dflash_graph_destroy(void *graph) {
    clear_error();
    if (!graph) return LG_OK;
    graph_free(static_cast<Graph *>(graph));
    return LG_OK;
}

}  // extern "C"

namespace lg {
bool fold_norms() { return g_fold_norms.load(std::memory_order_relaxed) != 0; }
}  // namespace lg

// The forwards' RMSNorms (and the target's residual adds) folded into the products
// around them (1, the default, where the model allows it) or run as their own
// launches (0): a switch for A/B measurement; both meet the same parity bound.
extern "C" int lg_set_fold_norms(uint32_t folded) {
    g_fold_norms.store(folded ? 1u : 0u, std::memory_order_relaxed);
    return LG_OK;
}
