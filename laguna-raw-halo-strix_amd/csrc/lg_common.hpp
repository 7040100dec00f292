// Shared host/device helpers of the gfx950 projection library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "laguna_hip.h"
#include "laguna_hip_tuning.h"

namespace lg {

// ---- error state (thread-local text, status codes; nothing crosses the ABI as an exception)
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Extent check: if p lies inside an allocation made by lg_buf_alloc, the
// range [p, p+bytes) must lie inside it too.  Unknown pointers pass.
bool extent_ok(const void *p, uint64_t bytes);
bool blocking();

#define LG_HIP_TRY(expr)                                                                  \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return ::lg::fail(LG_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));     \
    } while (0)

// Check a launch and honour blocking mode (no wait while the stream is being captured).
int after_launch(const char *what, hipStream_t s);
// Compute units of the current device.
int device_cus();

// While one lives, after_launch on this thread does not wait in blocking mode: a
// multi-launch entry point waits once, at its end.
struct DeferSync {
    DeferSync();
    ~DeferSync();
};

// Return the status of a call that fails.
#define LG_TRY(expr)                                                                                                   \
    do {                                                                                                               \
        const int st_ = (expr);                                                                                        \
        if (st_ != LG_OK) return st_;                                                                                  \
    } while (0)

#define LG_REQUIRE(cond, ...)                                                             \
    do {                                                                                  \
        if (!(cond)) return ::lg::fail(LG_EINVAL, __VA_ARGS__);                           \
    } while (0)

#define LG_EXTENT(ptr, bytes, name)                                                       \
    LG_REQUIRE(::lg::extent_ok((ptr), (bytes)),                                           \
               "%s: %llu bytes at %p run past the end of its lg_buf_alloc allocation",     \
               name, (unsigned long long)(bytes), (const void *)(ptr))

// A product workspace starts with PROJ_WS_COUNTERS bytes of arrival counters that
// every call expects to find zero (and leaves zero); callers that lay other data out
// after a workspace keep that region at a fixed place.
constexpr uint64_t PROJ_WS_COUNTERS = 65536;

// Device memory the library owns for one purpose on one stream of one device, so
// that calls on different streams never share it.  It grows on demand: the stream
// is synchronised and the old allocation freed, unless a graph captured from that
// stream may still use it (then it is kept until the process ends).  It cannot grow
// while the stream is being captured (LG_EINVAL: make the same call once on that
// stream before capturing).  New memory is zeroed on the stream.  The lease holds
// the registry lock; `tag` is free for the purpose's own bookkeeping.
enum BufPurpose { BUF_PRODUCT = 0, BUF_ATTN = 1, BUF_DRAFT = 2, BUF_TARGET = 3 };
struct StreamBuf {
    void *ptr = nullptr;
    uint64_t bytes = 0;
    bool captured = false;
    uint64_t tag[2] = {~0ull, ~0ull};
};
struct BufLease {
    StreamBuf *buf = nullptr;
    void *lock = nullptr;  // std::unique_lock<std::mutex>, released by the destructor
    BufLease() = default;
    BufLease(const BufLease &) = delete;
    BufLease &operator=(const BufLease &) = delete;
    ~BufLease();
};
int stream_buffer(int purpose, hipStream_t s, uint64_t need, BufLease &lease, const char *what);
// The product kernels' workspace on stream s (arrival counters first, then partial
// sums): at least `need` bytes.  Every call finds the counters zero and leaves them
// zero.
int stream_workspace(hipStream_t s, uint64_t need, void **out);

// 16- and 8-byte loads and stores coherent across the device (sc1: written through to,
// and read from, the device's coherence point), for partial results that one
// workgroup writes and another reads back; buffer offsets in bytes, below 2^31.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const float *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ float4 dev_ld4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CPOL_SC1));
}
__device__ __forceinline__ float2 dev_ld2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, CPOL_SC1));
}
__device__ __forceinline__ void dev_st4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, byte_off, 0, CPOL_SC1);
}
__device__ __forceinline__ void dev_st2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, byte_off, 0, CPOL_SC1);
}

// Split-k arrival, called by every thread of a (one-dimensional) workgroup after it
// has stored its partial results with device-coherent stores (dev_st4, or relaxed
// agent-scope atomics: written through to the device's coherence point).  True in
// every thread of the last workgroup to arrive at *cnt (of `total`), which resets the
// counter; that workgroup reads the partial results back with device-coherent loads.  Each
// wave waits for its own stores to complete (vmcnt 0, in an asm statement with a
// memory clobber, so the compiler keeps every store before it) before the barrier
// that precedes the arrival, so every partial result is at the coherence point
// before the counter can reach `total`.  (Release and acquire fences at agent scope
// would order the same accesses through an L2 write-back and invalidate in every
// wave; measured on MI355X they made the split-k products 3 to 5 times slower.)
__device__ __forceinline__ bool arrive_last(uint32_t *cnt, uint32_t total, uint32_t *s_flag) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        *s_flag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1 ? 1u : 0u;
    __syncthreads();
    if (*s_flag == 0u) return false;
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Small-M product behind lg_dispatch_proj_quant_batch: c = W x, or c = res + W x
// when res is given (res may be c).  ws == nullptr uses stream s's workspace;
// otherwise ws holds at least proj_batch_ws_bytes(k, n, m, x_dtype, w_dtype) bytes
// owned by the caller, zeroed before its first use and used by one call at a time
// (graphs capture it, so it must outlive them).
uint64_t proj_batch_ws_bytes(uint32_t k, uint32_t n, uint32_t m, int x_dtype, int w_dtype);
// Sets up the allocation-free product's scratch on device `dev` (current); lg_init
// calls it, and the entry point's first call on a device does otherwise.
int static_scratch_setup(int dev);
int proj_batch(const void *x, int x_dtype, const void *w, float *c, uint32_t k, uint32_t n, uint32_t m, int w_dtype,
               void *ws, uint64_t ws_bytes, hipStream_t s, const float *res = nullptr);

// Up to 4 small-M products over the same activations in one launch: job j computes
// c_j = W_j x (+ res_j) with W_j of n_j rows; all weights share k and w_dtype.
// With `up` (f32 activations only), x is replaced by silu(x) * up (SiLU FFN input).
// With `glu`, the two jobs are an FFN's gate and up products (equal n, f32 x, no
// residuals): job 0's output receives silu(gate) * up and job 1's is scratch.
//
// An RMSNorm between two products runs inside them (m <= 32, Q4_K / Q8_0 weights on
// the matrix-core path, f32 activations, not with `up`):
//  * job fields y, yw, ss (not glu): also y = c * yw[row] (c the job's output, e.g. the
//    residual stream with res = c) and ss[t * cols + g] = sum of c[t][row]^2 over the
//    rows of workgroup column g, cols = proj_batch_norm_cols(w_dtype, k, n, m);
//  * RowScale on the consuming call (x = such a y): the results of activation rows
//    t >= tok0 are multiplied by (sum_g ss[(t - tok0) * cols + g] / k + eps)^-1/2, the
//    norm's 1/rms (rows below tok0 arrive normalised).  cols <= proj_batch_rs_cols_max(m).
//  * job field qkw with a QkRope on the call: the job's rows are heads of 128, and
//    each head of each activation row t is written QK-normed with weights qkw and
//    rotated (NeoX, all 128 dims) at row t's angles: table[t][0..63] the cosines and
//    table[t][64..127] the sines of freq[i] * position(t) (the whole call's m rows).
struct BatchJob {
    const void *w;
    float *c;
    const float *res;
    uint32_t n;
    float *y = nullptr;
    const float *yw = nullptr;
    float *ss = nullptr;
    const float *qkw = nullptr;
    uint32_t row0 = 0;  // rows of c below row0 are not needed (left unwritten or zero, in steps of 16)
};
struct RowScale {
    const float *ss = nullptr;
    uint32_t cols = 0, tok0 = 0;
    float eps = 0.0f;
};
struct QkRope {
    const float *table = nullptr;
    float eps = 0.0f;
};
uint64_t proj_batch_multi_ws_bytes(uint32_t k, const uint32_t *n, uint32_t jobs, uint32_t m, int w_dtype);
int proj_batch_multi(const void *x, int x_dtype, const float *up, const BatchJob *jobs, uint32_t njobs, uint32_t k,
                     uint32_t m, int w_dtype, void *ws, uint64_t ws_bytes, hipStream_t s, bool glu = false,
                     const RowScale *rs = nullptr, const QkRope *qk = nullptr);
uint32_t proj_batch_norm_cols(int w_dtype, uint32_t k, uint32_t n, uint32_t m);
uint32_t proj_batch_rs_cols_max(uint32_t m);
// Whether products with these weights (f32 activations, 16-byte aligned) take the
// matrix-core path, which the folded norm needs.
bool proj_batch_mfma_ok(int w_dtype, uint32_t k, const void *w);

// A dense layer's input on the M = 1 integer-dot path: the activations are
// RMSNorm(x + xadd) (xadd, nw may be null: no add, no norm) and up to four Q4_K
// products over them run as one launch, job j writing y[j][0..n[j]).  The first
// workgroup also writes x + xadd to xout and xcap, and the normed activations to
// nxout (each may be null); xout must not alias x or xadd.  k <= 4096, a multiple of
// 256; 16-byte aligned operands (proj_m1_in_ok says whether the call qualifies).
struct M1In {
    const void *w[4] = {};
    int type[4] = {};
    float *y[4] = {};
    uint32_t n[4] = {};
    uint32_t count = 0;
    const float *xadd = nullptr, *nw = nullptr;
    float eps = 0.0f;
    float *xout = nullptr, *xcap = nullptr, *nxout = nullptr;
    bool glu = false;  // two jobs of equal n (gate, up): y[0] = silu(gate) * up, y[1] unused
};
bool proj_m1_in_ok(uint32_t k, const float *x, const M1In &in);
// lg_set_fold_norms: whether the forwards fold their norms into the products.
bool fold_norms();
int proj_m1_in(const float *x, const M1In &in, uint32_t k, hipStream_t s);

// ---- launchers of the draft's glue kernels, used by the target forward (one row each;
// in place allowed where the kernels allow it: rmsnorm, qk_norm_rope, gate_attn, add)
int glue_rmsnorm(const float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps, hipStream_t s);
int glue_qk_norm_rope(const float *x, const float *w, float *out, uint32_t n_heads, uint32_t head_dim,
                      uint32_t rope_dim, uint32_t pos, const float *freq, float eps, hipStream_t s);
// Q (n_q heads) and K (n_kv heads) of one row in one launch.
int glue_qk_norm_rope2(const float *q, const float *wq, float *q_out, uint32_t n_q, const float *k, const float *wk,
                       float *k_out, uint32_t n_kv, uint32_t head_dim, uint32_t rope_dim, uint32_t pos,
                       const float *freq, float eps, hipStream_t s);
// Causal attention of one query row at q_pos over seq_len keys/values; `part` holds
// glue_attn_partial_bytes(seq_len, n_kv) bytes (or is null: the plain kernel).  With
// `gate` ([n_q]) each head's result is multiplied by log(1 + exp(gate[h]))
// (kernels/gate_attn.comp).
uint64_t glue_attn_partial_bytes(uint32_t seq_len, uint32_t n_kv);
int glue_attention(const float *q, const float *k, const float *v, uint32_t seq_len, uint32_t q_pos, uint32_t n_q,
                   uint32_t n_kv, uint32_t head_dim, float *out, float *part, hipStream_t s,
                   const float *gate = nullptr);
// One token's attention step over seq_len keys/values: QK-norm + NeoX RoPE at `pos`
// of the query heads and of key row seq_len - 1 (normed in place in k), the
// attention, and the gate log(1 + exp(gate[h])) when gate is given.  `part` as for
// glue_attention.
bool glue_attention_token_ok(uint32_t head_dim, uint32_t n_q, uint32_t n_kv, uint32_t rope_dim);
int glue_attention_token(const float *q, const float *qn_w, const float *kn_w, const float *freq, uint32_t rope_dim,
                         uint32_t pos, float eps, float *k, const float *v, uint32_t seq_len, uint32_t n_q,
                         uint32_t n_kv, uint32_t head_dim, const float *gate, float *out, float *part, hipStream_t s);
int glue_gate_attn(const float *attn, const float *gate, float *out, uint32_t n_heads, uint32_t head_dim,
                   hipStream_t s);
int glue_add(const float *a, const float *b, float *out, uint64_t n, hipStream_t s);
int glue_copy(const float *src, float *dst, uint64_t n, hipStream_t s);
// The reference's f32 RoPE table: out[i] = 1 / base^(2i / rope_dim), i < rope_dim / 2.
void glue_rope_table(uint32_t rope_dim, float base, float *out);

// ---- GGUF block geometry (src/gguf.rs:97,101,134,136)
constexpr uint32_t QK_K = 256, Q4K_BYTES = 144;
constexpr uint32_t QK8_0 = 32, Q80_BYTES = 34;

constexpr uint32_t Q4K_TILE = 16 * Q4K_BYTES;      // LG_Q4_K_T16: 16 rows x one super-block
constexpr uint32_t Q80_TILE = 16 * 8 * Q80_BYTES;  // LG_Q8_0_T16: 16 rows x 8 blocks

// Bytes of a k x n tensor repacked into 16-row tiles (rows padded to a multiple of
// 16; dtype the raw type or its tiled id).
inline uint64_t tiled_bytes(int dtype, uint32_t k, uint32_t n) {
    const bool q4 = dtype == LG_Q4_K || dtype == LG_Q4_K_T16;
    return (uint64_t)(n + 15) / 16 * (k / 256) * (q4 ? Q4K_TILE : Q80_TILE);
}

inline uint64_t tensor_bytes(int dtype, uint64_t elems) {
    switch (dtype) {
    case LG_Q4_K: return (elems + QK_K - 1) / QK_K * Q4K_BYTES;
    case LG_Q8_0: return (elems + QK8_0 - 1) / QK8_0 * Q80_BYTES;
    case LG_F32: return elems * 4;
    case LG_F16:
    case LG_BF16: return elems * 2;
    default: return 0;
    }
}

}  // namespace lg

// ---- device helpers ------------------------------------------------------------------

// The reference's binary16 decoder (src/dflash.rs:314-329, kernels/proj_q4k.comp:28-44):
// IEEE for normals, zeros, inf and NaN (payload kept), but exponent-0 codes with a
// non-zero mantissa decode as 2^-14 * (1 + m/1024) instead of 2^-24 * m.
// Written as one add on the shifted code: bias = 112, 113 (quirk) or 224 (inf/NaN).
__device__ __forceinline__ float ref_half(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u;
    const uint32_t t = (h & 0x7FFFu) << 13;
    uint32_t bias = 112u << 23;
    if (e == 0u) bias = (h & 0x3FFu) ? (113u << 23) : 0u;
    if (e == 31u) bias = 224u << 23;
    return __uint_as_float((t + bias) | sign);
}

// ggml get_scale_min_k4 (kernels/proj_q4k.comp:46-58) on the 12 scale bytes held in
// three little-endian dwords s0 = bytes 0-3, s1 = bytes 4-7, s2 = bytes 8-11.
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &sc, uint32_t &mn) {
    if (j < 4u) {
        sc = (s0 >> (8u * j)) & 63u;
        mn = (s1 >> (8u * j)) & 63u;
    } else {
        const uint32_t sh = 8u * (j - 4u);
        const uint32_t bp = (s2 >> sh) & 0xFFu;
        sc = (bp & 15u) | (((s0 >> sh) >> 6 & 3u) << 4);
        mn = (bp >> 4) | (((s1 >> sh) >> 6 & 3u) << 4);
    }
}

// 16-byte load with the nontemporal (streaming) hint, for data read exactly once.
typedef uint32_t lg_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
    const lg_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const lg_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte I of u as float (selected into v_cvt_f32_ubyteI).
template <int I>
__device__ __forceinline__ float ubyte_f(uint32_t u) { return (float)((u >> (8 * I)) & 0xFFu); }

// v plus the v of lane i ^ 16 (lane_add_x16) or i ^ 32 (lane_add_x32), through the
// gfx950 row swaps v_permlane16_swap / v_permlane32_swap (VALU, no LDS round trip).
// With both operands v, the swap leaves one operand holding the even (lower) rows and
// the other the odd (upper) ones, so their sum is v_i + v_(i^16) in every lane: the
// same float as __shfl_xor(v, 16) + v (addition is commutative).
__device__ __forceinline__ float lane_add_x16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float lane_add_x32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Sum over each 16-lane row: DPP xor 1, xor 2 (quad_perm), then row_ror 4 and 8.
// Every lane receives its row's sum (lanes of different quads may associate the
// terms differently).
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)); // row_ror 4
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)); // row_ror 8
    return v;
}

// Sum over the 64 lanes of a wavefront; every lane receives the total: the rows
// by DPP, then the four rows with the two row swaps.
__device__ __forceinline__ float wave_sum(float v) { return lane_add_x32(lane_add_x16(row16_sum(v))); }
