// Target-side verify: argmax over rows of logits (src/lib.rs:456-464) on the device.
//
// The reference folds the logits left to right with Iterator::max_by and
// partial_cmp(..).unwrap_or(Equal): the running best is replaced by element i
// unless best > v[i], so ties go to the later index and a NaN (unordered, taken
// as Equal) becomes the best and is replaced by whatever follows it.  The fold
// over a sequence is therefore the fold over the elements after its last NaN
// (or that NaN, when it is the last element).  That makes the fold splittable
// over contiguous segments: a segment's state is (value, index, has-NaN), and
// for a left segment L and a right segment R
//     R has a NaN:  the result is R's state
//     otherwise:    the later of L and R unless L.value > R.value, has-NaN of L.
// Segments combine in index order only (never interleaved), so the result is the
// reference's index bit for bit, NaNs, infinities and signed zeros included.
//
// Launch: grid (chunks, rows); a workgroup of 256 threads takes ARG_CHUNK
// contiguous logits of one row, each thread a run of ARG_RUN.  Runs meet lane by
// lane (shuffle-down, left operand the lower lanes) and wave by wave in LDS; the
// chunk states go to the workspace, and the last workgroup of the row to arrive
// (an arrival counter, reset by it) combines them in chunk order.
#include "lg_common.hpp"

namespace {

using namespace lg;

constexpr uint32_t ARG_RUN = 16;              // contiguous logits per thread (four float4)
constexpr uint32_t ARG_CHUNK = 256 * ARG_RUN;  // logits per workgroup

constexpr uint32_t ST_VALID = 1u, ST_NAN = 2u;

struct ArgState {
    float v;
    uint32_t i, f;  // index; ST_VALID | ST_NAN bits
};

// L is the segment to the left of R.
__device__ __forceinline__ ArgState arg_combine(const ArgState &L, const ArgState &R) {
    if (!(R.f & ST_VALID)) return L;
    if (!(L.f & ST_VALID)) return R;
    if (R.f & ST_NAN) return R;
    return L.v > R.v ? L : ArgState{R.v, R.i, R.f | (L.f & ST_NAN)};
}

__device__ __forceinline__ ArgState arg_shfl_down(const ArgState &s, uint32_t d) {
    return {__shfl_down(s.v, d), __shfl_down(s.i, d), __shfl_down(s.f, d)};
}

// Lane 0 receives the ordered combination of the wave's 64 states.
__device__ __forceinline__ ArgState arg_wave(ArgState s) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const ArgState r = arg_shfl_down(s, d);
        if (lane + d < 64) s = arg_combine(s, r);
    }
    return s;
}

__global__ __launch_bounds__(256) void k_argmax_rows(const float *__restrict__ x, uint64_t ld, uint32_t n,
                                                     uint4 *part, uint32_t *cnt, uint32_t *out) {
    __shared__ ArgState ws[4];
    __shared__ uint32_t last;
    const uint32_t row = blockIdx.y, c = blockIdx.x, nch = gridDim.x;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const float *xr = x + (uint64_t)row * ld;
    const uint32_t e0 = c * ARG_CHUNK + tid * ARG_RUN;

    // this thread's run, all loads issued first (float4 when the row allows it)
    float v[ARG_RUN];
    if ((ld & 3u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && e0 + ARG_RUN <= n) {
        const float4 *p = reinterpret_cast<const float4 *>(xr + e0);
#pragma unroll
        for (uint32_t q = 0; q < ARG_RUN / 4; q++) {
            const float4 t = p[q];
            v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (uint32_t j = 0; j < ARG_RUN; j++) v[j] = e0 + j < n ? xr[e0 + j] : 0.0f;
    }
    // the reference's fold over the run (src/lib.rs:459-462)
    ArgState s{0.0f, 0u, 0u};
    if (e0 < n) {
        s = {v[0], e0, ST_VALID | (v[0] != v[0] ? ST_NAN : 0u)};
#pragma unroll
        for (uint32_t j = 1; j < ARG_RUN; j++) {
            if (e0 + j < n) {
                if (!(s.v > v[j])) s.v = v[j], s.i = e0 + j;
                if (v[j] != v[j]) s.f |= ST_NAN;
            }
        }
    }
    s = arg_wave(s);
    if (lane == 0) ws[wave] = s;
    __syncthreads();
    if (tid == 0) {
        ArgState t = ws[0];
#pragma unroll
        for (int w = 1; w < 4; w++) t = arg_combine(t, ws[w]);
        if (nch == 1) {
            out[row] = t.i;
        } else {
            const uint4 st = make_uint4(__float_as_uint(t.v), t.i, t.f, 0u);
            uint32_t *pw = reinterpret_cast<uint32_t *>(part + (uint64_t)row * nch + c);
            __hip_atomic_store(pw, st.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pw + 1, st.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pw + 2, st.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (nch == 1) return;
    // the last workgroup of the row to arrive combines the chunk states
    if (!arrive_last(&cnt[row], nch, &last) || wave != 0) return;
    // the chunk states in chunk order, 64 at a time
    ArgState acc{0.0f, 0u, 0u};
    for (uint32_t c0 = 0; c0 < nch; c0 += 64) {
        ArgState t{0.0f, 0u, 0u};
        if (c0 + lane < nch) {
            const uint32_t *pr = reinterpret_cast<const uint32_t *>(part + (uint64_t)row * nch + c0 + lane);
            t.v = __uint_as_float(__hip_atomic_load(pr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            t.i = __hip_atomic_load(pr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            t.f = __hip_atomic_load(pr + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        t = arg_wave(t);
        acc = arg_combine(acc, ArgState{__shfl(t.v, 0), __shfl(t.i, 0), __shfl(t.f, 0)});
    }
    if (lane == 0) out[row] = acc.i;
}

__global__ void k_zero_u32(uint32_t *out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = 0u;
}

}  // namespace

extern "C" int lg_dispatch_argmax(const float *logits, uint32_t n, uint32_t rows, uint64_t ld, uint32_t *out,
                                  void *stream) {
    clear_error();
    if (rows == 0) return LG_OK;
    LG_REQUIRE(out, "lg_dispatch_argmax: null output");
    hipStream_t s = (hipStream_t)stream;
    if (n == 0) {  // unwrap_or(0) on an empty slice (a kernel, not a memset: the call may be captured)
        hipLaunchKernelGGL(k_zero_u32, dim3((rows + 255) / 256), dim3(256), 0, s, out, rows);
        return after_launch("lg_dispatch_argmax", s);
    }
    LG_REQUIRE(logits, "lg_dispatch_argmax: null logits");
    LG_REQUIRE(ld >= n, "lg_dispatch_argmax: row stride %llu < n=%u", (unsigned long long)ld, n);
    LG_REQUIRE(n <= 0x7FFFFFFFu, "lg_dispatch_argmax: n=%u too large", n);
    LG_REQUIRE(rows <= PROJ_WS_COUNTERS / 4 && rows <= 65535u, "lg_dispatch_argmax: %u rows (at most %llu)", rows,
               (unsigned long long)(PROJ_WS_COUNTERS / 4 < 65535 ? PROJ_WS_COUNTERS / 4 : 65535));
    LG_EXTENT(logits, ((uint64_t)(rows - 1) * ld + n) * 4, "lg_dispatch_argmax logits");
    LG_EXTENT(out, (uint64_t)rows * 4, "lg_dispatch_argmax out");
    const uint32_t nch = (n + ARG_CHUNK - 1) / ARG_CHUNK;
    void *ws = nullptr;
    if (nch > 1) LG_TRY(stream_workspace(s, PROJ_WS_COUNTERS + (uint64_t)rows * nch * 16, &ws));
    uint32_t *cnt = static_cast<uint32_t *>(ws);
    uint4 *part = ws ? reinterpret_cast<uint4 *>(static_cast<uint8_t *>(ws) + PROJ_WS_COUNTERS) : nullptr;
    hipLaunchKernelGGL(k_argmax_rows, dim3(nch, rows), dim3(256), 0, s, logits, ld, n, part, cnt, out);
    return after_launch("lg_dispatch_argmax", s);
}
