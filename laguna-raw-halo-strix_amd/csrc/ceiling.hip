// Ceiling kernels for measurement (no counterpart in the reference): an empty
// kernel and plain streaming reads.  Timed next to the projections, they give what
// one launch and one read of the same bytes cost on this device, so that each
// projection's time can be read against both.
#include "lg_common.hpp"

using namespace lg;

// Written only if a read's checksum hits a magic value (never, in practice); external
// linkage keeps the store, and so the loads feeding it, in the kernel.
__device__ uint32_t lg_bench_sink;

namespace {

__global__ __launch_bounds__(256) void k_empty() {}

// A streaming read of n16 16-byte words in chunks of T * L words: every thread issues
// its L loads of a chunk at once, thread t of the chunk reading words t, t + T, ...
// One-shot (PERSIST false): workgroup b reads chunk b.  Persistent: the grid holds a
// fixed number of workgroups per compute unit and workgroup b reads chunks b,
// b + gridDim.x, ...  NT reads with the nontemporal (streaming) hint.  Indices past
// the end re-read the last word.
template <int T, int L, bool NT, bool PERSIST>
__global__ __launch_bounds__(T) void k_read(const uint4 *__restrict__ p, uint64_t n16) {
    const uint64_t per = (uint64_t)T * L, nch = (n16 + per - 1) / per;
    uint32_t s = 0;
    for (uint64_t c = blockIdx.x; c < nch; c += PERSIST ? gridDim.x : nch) {
        const uint64_t base = c * per + threadIdx.x;
        uint4 v[L];
#pragma unroll
        for (int i = 0; i < L; i++) {
            const uint64_t j = base + (uint64_t)i * T;
            const uint4 *q = p + (j < n16 ? j : n16 - 1);
            v[i] = NT ? ld_stream16(q) : *q;
        }
#pragma unroll
        for (int i = 0; i < L; i++) s ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (s == 0x9E3779B9u) lg_bench_sink = s;
}

template <int T, int L, bool NT>
void launch_read(const uint4 *p, uint64_t n16, uint32_t per_cu, hipStream_t s) {
    const uint64_t nch = (n16 + (uint64_t)T * L - 1) / ((uint64_t)T * L);
    if (per_cu) {
        const uint64_t g = (uint64_t)per_cu * device_cus();
        hipLaunchKernelGGL((k_read<T, L, NT, true>), dim3((uint32_t)(g < nch ? g : nch)), dim3(T), 0, s, p, n16);
    } else {
        hipLaunchKernelGGL((k_read<T, L, NT, false>), dim3((uint32_t)nch), dim3(T), 0, s, p, n16);
    }
}

template <int T, bool NT>
int read_l(const uint4 *p, uint64_t n16, uint32_t loads, uint32_t per_cu, hipStream_t s) {
    switch (loads) {
    case 2: launch_read<T, 2, NT>(p, n16, per_cu, s); return LG_OK;
    case 4: launch_read<T, 4, NT>(p, n16, per_cu, s); return LG_OK;
    case 8: launch_read<T, 8, NT>(p, n16, per_cu, s); return LG_OK;
    case 16: launch_read<T, 16, NT>(p, n16, per_cu, s); return LG_OK;
    default: return fail(LG_EINVAL, "lg_bench_read_shape: %u loads per thread (2, 4, 8 or 16)", loads);
    }
}

}  // namespace

extern "C" int lg_bench_empty(uint32_t workgroups, void *stream) {
    clear_error();
    LG_REQUIRE(workgroups >= 1 && workgroups <= 65535u, "lg_bench_empty: %u workgroups (1..65535)", workgroups);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_empty, dim3(workgroups), dim3(256), 0, s);
    return after_launch("lg_bench_empty", s);
}

extern "C" int lg_bench_read_shape(const void *buf, uint64_t bytes, uint32_t threads, uint32_t loads,
                                   uint32_t per_cu, uint32_t nontemporal, void *stream) {
    clear_error();
    const char *name = "lg_bench_read_shape";
    LG_REQUIRE(buf, "%s: null buffer", name);
    LG_REQUIRE(bytes >= 16 && bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(buf) & 15u) == 0,
               "%s: %llu bytes (a positive multiple of 16, 16-byte aligned)", name, (unsigned long long)bytes);
    LG_REQUIRE(per_cu <= 8, "%s: %u workgroups per compute unit (0 = one-shot grid, else 1..8)", name, per_cu);
    LG_EXTENT(buf, bytes, name);
    const uint64_t n16 = bytes / 16;
    LG_REQUIRE(n16 / threads / 2 <= 0x7FFFFFFFu, "%s: %llu bytes is too large", name, (unsigned long long)bytes);
    const uint4 *p = static_cast<const uint4 *>(buf);
    hipStream_t s = (hipStream_t)stream;
    int st;
    switch (threads) {
    case 256: st = nontemporal ? read_l<256, true>(p, n16, loads, per_cu, s) : read_l<256, false>(p, n16, loads, per_cu, s); break;
    case 512: st = nontemporal ? read_l<512, true>(p, n16, loads, per_cu, s) : read_l<512, false>(p, n16, loads, per_cu, s); break;
    case 1024: st = nontemporal ? read_l<1024, true>(p, n16, loads, per_cu, s) : read_l<1024, false>(p, n16, loads, per_cu, s); break;
    default: return fail(LG_EINVAL, "%s: %u threads per workgroup (256, 512 or 1024)", name, threads);
    }
    LG_TRY(st);
    return after_launch(name, s);
}

extern "C" int lg_bench_read(const void *buf, uint64_t bytes, void *stream) {
    return lg_bench_read_shape(buf, bytes, 256, 8, 0, 0, stream);
}
